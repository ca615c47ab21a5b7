// Minimal safetensors reader for the MoE parameters (the format
// candle_core::safetensors::load reads in weights.rs:112-115, through the
// `safetensors` crate 0.8.0 that candle-core 0.11.1 depends on, Cargo.lock:185
// and :1293-1296): an 8-byte little-endian
// header length, a JSON header mapping tensor names to
// {"dtype", "shape", "data_offsets": [begin, end]}, then the payload.
//
// The whole header is validated before anything is allocated for a tensor,
// following the format's published rules: the header is at most 100,000,000
// bytes and fits in the file; every entry has a known dtype, non-negative
// dims whose element count times the dtype size neither overflows nor
// differs from end - begin; and the entries tile the payload exactly, in
// offset order, with no hole and no overlap ("the byte buffer needs to be
// entirely indexed, and cannot contain holes").  Any violation is
// NOMAS_ERR_IO with the message "loading <path>: <reason>", the form of
// load_dit's error (weights.rs:112-115).  Only the requested tensors are
// read from disk.  The JSON itself is held to what the crate's serde_json
// parse accepts: strict JSON, `__metadata__` null or an object of strings, at
// most 128 nested containers; the parser is iterative, so no header can
// exhaust the stack.
#include <sys/types.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <memory>
#include <utility>

#include "host.hpp"

namespace nomas {

namespace {

struct Entry {
    std::string dtype;
    std::vector<int64_t> shape;
    int64_t begin = -1, end = -1;
};

// Small JSON parser covering the safetensors header.
class Json {
public:
    explicit Json(const std::string& s) : s_(s) {}

    bool parse_header(std::map<std::string, Entry>* out) {
        ws();
        if (!eat('{')) return false;
        ws();
        if (eat('}')) {
            ws();
            return p_ == s_.size();
        }
        for (;;) {
            std::string key;
            ws();
            if (!str(&key)) return false;
            ws();
            if (!eat(':')) return false;
            ws();
            if (key == "__metadata__") {
                if (!metadata()) return false;
            } else {
                Entry e;
                if (!entry(&e)) return false;
                (*out)[key] = e;
            }
            ws();
            if (eat(',')) continue;
            if (eat('}')) {
                ws();  // the header may be padded with whitespace, nothing else
                return p_ == s_.size();
            }
            return false;
        }
    }

private:
    // Most containers nested in a header, its top-level object included
    // (serde_json's default recursion limit, which the safetensors crate's
    // header parse runs under).
    static constexpr int kMaxDepth = 128;
    const std::string& s_;
    size_t p_ = 0;

    void ws() {
        while (p_ < s_.size() && (s_[p_] == ' ' || s_[p_] == '\n' || s_[p_] == '\t' || s_[p_] == '\r'))
            ++p_;
    }
    bool eat(char c) {
        if (p_ < s_.size() && s_[p_] == c) { ++p_; return true; }
        return false;
    }
    // Four hex digits of a \u escape at p_.
    bool hex4(uint32_t* v) {
        if (s_.size() - p_ < 4) return false;
        uint32_t x = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = s_[p_ + i];
            const int d = c >= '0' && c <= '9' ? c - '0'
                        : c >= 'a' && c <= 'f' ? c - 'a' + 10
                        : c >= 'A' && c <= 'F' ? c - 'A' + 10 : -1;
            if (d < 0) return false;
            x = x * 16 + (uint32_t)d;
        }
        p_ += 4;
        *v = x;
        return true;
    }
    static void utf8(uint32_t cp, std::string* out) {
        if (cp < 0x80) {
            out->push_back((char)cp);
        } else if (cp < 0x800) {
            out->push_back((char)(0xC0 | (cp >> 6)));
            out->push_back((char)(0x80 | (cp & 0x3F)));
        } else if (cp < 0x10000) {
            out->push_back((char)(0xE0 | (cp >> 12)));
            out->push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            out->push_back((char)(0x80 | (cp & 0x3F)));
        } else {
            out->push_back((char)(0xF0 | (cp >> 18)));
            out->push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
            out->push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            out->push_back((char)(0x80 | (cp & 0x3F)));
        }
    }
    // A JSON string, unescaped into *out.  Raw control characters, unknown
    // escapes, malformed \u escapes and unpaired surrogates are errors (as in
    // serde_json, which the safetensors crate parses its header with).
    bool str(std::string* out) {
        if (!eat('"')) return false;
        out->clear();
        while (p_ < s_.size() && s_[p_] != '"') {
            const unsigned char b = (unsigned char)s_[p_];
            if (b < 0x20) return false;
            if (b != '\\') {
                out->push_back(s_[p_++]);
                continue;
            }
            if (++p_ >= s_.size()) return false;
            const char c = s_[p_++];
            switch (c) {
            case '"': case '\\': case '/': out->push_back(c); break;
            case 'b': out->push_back('\b'); break;
            case 'f': out->push_back('\f'); break;
            case 'n': out->push_back('\n'); break;
            case 'r': out->push_back('\r'); break;
            case 't': out->push_back('\t'); break;
            case 'u': {
                uint32_t cp;
                if (!hex4(&cp)) return false;
                if (cp >= 0xDC00 && cp < 0xE000) return false;  // lone low surrogate
                if (cp >= 0xD800 && cp < 0xDC00) {               // high: a low one must follow
                    uint32_t lo;
                    if (!eat('\\') || !eat('u') || !hex4(&lo) || lo < 0xDC00 || lo >= 0xE000)
                        return false;
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                }
                utf8(cp, out);
                break;
            }
            default: return false;
            }
        }
        return eat('"');
    }
    bool integer(int64_t* v) {
        ws();
        size_t q = p_;
        bool neg = false;
        if (q < s_.size() && s_[q] == '-') { neg = true; ++q; }
        if (q >= s_.size() || s_[q] < '0' || s_[q] > '9') return false;
        // JSON has no leading zeros
        if (s_[q] == '0' && q + 1 < s_.size() && s_[q + 1] >= '0' && s_[q + 1] <= '9') return false;
        int64_t x = 0;
        while (q < s_.size() && s_[q] >= '0' && s_[q] <= '9') {
            if (__builtin_mul_overflow(x, (int64_t)10, &x) ||
                __builtin_add_overflow(x, (int64_t)(s_[q] - '0'), &x))
                return false;  // beyond int64: no valid dim or offset
            ++q;
        }
        p_ = q;
        *v = neg ? -x : x;
        return true;
    }
    bool int_array(std::vector<int64_t>* v) {
        ws();
        if (!eat('[')) return false;
        ws();
        if (eat(']')) return true;
        for (;;) {
            int64_t x;
            if (!integer(&x)) return false;
            v->push_back(x);
            ws();
            if (eat(',')) continue;
            if (eat(']')) return true;
            return false;
        }
    }
    bool entry(Entry* e) {
        if (!eat('{')) return false;
        for (;;) {
            ws();
            std::string k;
            if (!str(&k)) return false;
            ws();
            if (!eat(':')) return false;
            ws();
            if (k == "dtype") {
                if (!str(&e->dtype)) return false;
            } else if (k == "shape") {
                if (!int_array(&e->shape)) return false;
            } else if (k == "data_offsets") {
                std::vector<int64_t> o;
                if (!int_array(&o) || o.size() != 2) return false;
                e->begin = o[0];
                e->end = o[1];
            } else if (!skip(kMaxDepth - 2)) {  // inside the header and the entry
                return false;
            }
            ws();
            if (eat(',')) continue;
            if (eat('}')) return true;
            return false;
        }
    }
    // A JSON number (RFC 8259 grammar: -?(0|[1-9][0-9]*)(.[0-9]+)?([eE][+-]?[0-9]+)?).
    bool number() {
        auto digits = [&]() {
            const size_t q = p_;
            while (p_ < s_.size() && s_[p_] >= '0' && s_[p_] <= '9') ++p_;
            return p_ > q;
        };
        eat('-');
        if (eat('0')) {
        } else if (!digits()) {
            return false;
        }
        if (eat('.') && !digits()) return false;
        if (p_ < s_.size() && (s_[p_] == 'e' || s_[p_] == 'E')) {
            ++p_;
            if (!eat('+')) eat('-');
            if (!digits()) return false;
        }
        return true;
    }
    bool literal(const char* w) {
        const size_t n = std::strlen(w);
        if (s_.compare(p_, n, w) != 0) return false;
        p_ += n;
        return true;
    }
    // `"__metadata__"`'s value: null or an object of string values (the
    // safetensors crate reads it as Option<HashMap<String, String>>).
    bool metadata() {
        if (literal("null")) return true;
        if (!eat('{')) return false;
        ws();
        if (eat('}')) return true;
        for (;;) {
            std::string k, v;
            ws();
            if (!str(&k)) return false;
            ws();
            if (!eat(':')) return false;
            ws();
            if (!str(&v)) return false;
            ws();
            if (eat(',')) continue;
            return eat('}');
        }
    }
    // Any JSON value, skipped, holding at most max_depth nested containers.
    // Iterative, so no header can exhaust the stack; anything that is not
    // JSON fails.
    bool skip(int max_depth) {
        char open[kMaxDepth];  // '{' or '[' of each open container
        if (max_depth > kMaxDepth) max_depth = kMaxDepth;
        int depth = 0;
        for (;;) {
            // one value
            ws();
            if (p_ >= s_.size()) return false;
            const char c = s_[p_];
            bool opened = false;
            if (c == '"') {
                std::string t;
                if (!str(&t)) return false;
            } else if (c == '{' || c == '[') {
                if (depth >= max_depth) return false;
                open[depth++] = c;
                ++p_;
                ws();
                if (eat(c == '{' ? '}' : ']')) {
                    --depth;  // empty container: a complete value
                } else {
                    opened = true;
                }
            } else if (c == 't' || c == 'f' || c == 'n') {
                if (!literal(c == 't' ? "true" : c == 'f' ? "false" : "null")) return false;
            } else if (!number()) {
                return false;
            }
            // after a complete value: close containers or go on to the next member
            for (;;) {
                if (depth == 0) return true;
                if (opened) break;  // the first member of a just-opened container
                ws();
                if (eat(',')) break;
                if (!eat(open[depth - 1] == '{' ? '}' : ']')) return false;
                --depth;
            }
            if (open[depth - 1] == '{') {  // a member: "key": value
                ws();
                std::string t;
                if (!str(&t)) return false;
                ws();
                if (!eat(':')) return false;
            }
        }
    }
};

int64_t dtype_bytes(const std::string& d) {
    if (d == "F64" || d == "I64" || d == "U64") return 8;
    if (d == "F32" || d == "I32" || d == "U32") return 4;
    if (d == "BF16" || d == "F16" || d == "I16" || d == "U16") return 2;
    if (d == "U8" || d == "I8" || d == "BOOL" || d == "F8_E4M3" || d == "F8_E5M2") return 1;
    return -1;
}

}  // namespace

namespace {

struct FileCloser {
    void operator()(FILE* f) const { std::fclose(f); }
};

// Checks one header entry on its own: known dtype, non-negative dims and
// offsets, element count x dtype size == end - begin without overflow.
// Returns nullptr or what is wrong.
const char* entry_problem(const Entry& e) {
    const int64_t eb = dtype_bytes(e.dtype);
    if (eb < 0) return "unknown dtype";
    if (e.begin < 0 || e.end < 0) return "missing or negative data_offsets";
    if (e.end < e.begin) return "data_offsets end before begin";
    int64_t numel = 1;
    for (int64_t d : e.shape) {
        if (d < 0) return "negative dimension";
        if (__builtin_mul_overflow(numel, d, &numel)) return "element count overflows";
    }
    int64_t bytes = 0;
    if (__builtin_mul_overflow(numel, eb, &bytes)) return "byte size overflows";
    if (bytes != e.end - e.begin) return "byte size does not match shape and dtype";
    return nullptr;
}

// Parses and validates the header of `f` (file `path`); on success fills
// `entries` and the payload's file offset.
int read_header(FILE* f, const std::string& path, std::map<std::string, Entry>* entries,
                int64_t* data0) {
    constexpr uint64_t kMaxHeader = 100000000;  // the format's header limit
    if (fseeko(f, 0, SEEK_END) != 0)
        return set_error(NOMAS_ERR_IO, "loading %s: cannot seek", path.c_str());
    const int64_t fsize = (int64_t)ftello(f);
    if (fsize < 8 || fseeko(f, 0, SEEK_SET) != 0)
        return set_error(NOMAS_ERR_IO, "loading %s: truncated header", path.c_str());
    uint8_t hb[8];
    if (std::fread(hb, 1, 8, f) != 8)
        return set_error(NOMAS_ERR_IO, "loading %s: truncated header", path.c_str());
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | hb[i];
    if (hlen > kMaxHeader)
        return set_error(NOMAS_ERR_IO, "loading %s: header too large (%llu bytes)", path.c_str(),
                         (unsigned long long)hlen);
    if ((int64_t)hlen > fsize - 8)
        return set_error(NOMAS_ERR_IO, "loading %s: truncated header", path.c_str());
    std::string hdr(hlen, '\0');
    if (hlen > 0 && std::fread(&hdr[0], 1, hlen, f) != hlen)
        return set_error(NOMAS_ERR_IO, "loading %s: truncated header", path.c_str());
    Json js(hdr);
    if (!js.parse_header(entries))
        return set_error(NOMAS_ERR_IO, "loading %s: malformed safetensors header", path.c_str());
    const int64_t payload = fsize - 8 - (int64_t)hlen;
    // every entry well-formed, and together they cover [0, payload) in
    // offset order with no hole or overlap
    std::vector<std::pair<std::pair<int64_t, int64_t>, const std::string*>> spans;
    spans.reserve(entries->size());
    for (const auto& kv : *entries) {
        if (const char* why = entry_problem(kv.second))
            return set_error(NOMAS_ERR_IO, "loading %s: tensor %s: %s", path.c_str(),
                             kv.first.c_str(), why);
        spans.push_back({{kv.second.begin, kv.second.end}, &kv.first});
    }
    std::sort(spans.begin(), spans.end());
    int64_t at = 0;
    for (const auto& sp : spans) {
        if (sp.first.first != at)
            return set_error(NOMAS_ERR_IO, "loading %s: tensor %s: data_offsets %s the previous tensor",
                             path.c_str(), sp.second->c_str(),
                             sp.first.first < at ? "overlap" : "leave a hole after");
        at = sp.first.second;
    }
    if (at != payload)
        return set_error(NOMAS_ERR_IO,
                         "loading %s: tensors cover %lld payload bytes, the file holds %lld",
                         path.c_str(), (long long)at, (long long)payload);
    *data0 = 8 + (int64_t)hlen;
    return NOMAS_OK;
}

}  // namespace

int read_safetensors(const std::vector<std::string>& files, const std::vector<std::string>& names,
                     std::map<std::string, StTensor>* out) {
    for (const std::string& path : files) {
        std::unique_ptr<FILE, FileCloser> f(std::fopen(path.c_str(), "rb"));
        if (!f) return set_error(NOMAS_ERR_IO, "loading %s: cannot open file", path.c_str());
        std::map<std::string, Entry> entries;
        int64_t data0 = 0;
        int rc = read_header(f.get(), path, &entries, &data0);
        if (rc != NOMAS_OK) return rc;
        for (const std::string& n : names) {
            auto it = entries.find(n);
            if (it == entries.end()) continue;
            const Entry& e = it->second;  // validated: 0 <= begin <= end <= payload
            StTensor t;
            t.dtype = e.dtype;
            t.shape = e.shape;
            t.data.resize((size_t)(e.end - e.begin));
            if (fseeko(f.get(), (off_t)(data0 + e.begin), SEEK_SET) != 0 ||
                std::fread(t.data.data(), 1, t.data.size(), f.get()) != t.data.size())
                return set_error(NOMAS_ERR_IO, "loading %s: truncated payload of %s", path.c_str(),
                                 n.c_str());
            (*out)[n] = std::move(t);
        }
    }
    return NOMAS_OK;
}

int st_to_f32(const StTensor& t, std::vector<float>* out) {
    const size_t n = t.data.size() / (size_t)std::max<int64_t>(1, dtype_bytes(t.dtype));
    out->resize(n);
    const uint8_t* p = t.data.data();
    if (t.dtype == "F32") {
        std::memcpy(out->data(), p, n * 4);
    } else if (t.dtype == "F64") {
        for (size_t i = 0; i < n; ++i) {
            double d;
            std::memcpy(&d, p + 8 * i, 8);
            (*out)[i] = (float)d;
        }
    } else if (t.dtype == "BF16") {
        for (size_t i = 0; i < n; ++i) {
            uint16_t b;
            std::memcpy(&b, p + 2 * i, 2);
            (*out)[i] = bf16_bits_to_f32(b);
        }
    } else if (t.dtype == "F16") {
        for (size_t i = 0; i < n; ++i) {
            uint16_t b;
            std::memcpy(&b, p + 2 * i, 2);
            (*out)[i] = f16_bits_to_f32(b);
        }
    } else {
        return set_error(NOMAS_ERR_INVALID_ARGUMENT, "unsupported safetensors dtype %s",
                         t.dtype.c_str());
    }
    return NOMAS_OK;
}

}  // namespace nomas
