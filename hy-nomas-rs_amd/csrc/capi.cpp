// extern "C" entry points declared in include/nomas_moe.h.
//
// Each one validates its arguments before touching the GPU, so configuration
// errors are reported the same way on hosts without a device.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "host.hpp"

using nomas::DType;
using nomas::LinF32;
using nomas::MoeLayer;
using nomas::MoeParamsF32;
using nomas::set_error;

struct nomas_moe {
    std::unique_ptr<MoeLayer> layer;
};

namespace {

// Runs the body of an int-returning entry point.  No C++ exception crosses the
// C ABI: one that escapes the body becomes a status (bad_alloc ->
// OUT_OF_MEMORY, anything else -> INTERNAL) with the entry point's name.
template <typename F>
int guarded(const char* fn, F&& body) noexcept {
    try {
        return body();
    } catch (const std::bad_alloc&) {
        return set_error(NOMAS_ERR_OUT_OF_MEMORY, "%s: host allocation failed", fn);
    } catch (const std::exception& e) {
        return set_error(NOMAS_ERR_INTERNAL, "%s: %s", fn, e.what());
    } catch (...) {
        return set_error(NOMAS_ERR_INTERNAL, "%s: unexpected exception", fn);
    }
}

int make_layer(const nomas_moe_config* cfg, int64_t dim, int64_t hidden, int dtype, int device,
               std::unique_ptr<MoeLayer>* out) {
    int rc = MoeLayer::check_shape(*cfg, dim, hidden, dtype);
    if (rc != NOMAS_OK) return rc;
    int ndev = 0;
    hipError_t e = hipGetDeviceCount(&ndev);
    if (e != hipSuccess || ndev <= 0)
        return set_error(NOMAS_ERR_HIP, "no HIP device available (%s)",
                         e == hipSuccess ? "0 devices" : hipGetErrorString(e));
    if (device < 0 || device >= ndev)
        return set_error(NOMAS_ERR_INVALID_ARGUMENT, "device %d out of range (%d devices)", device, ndev);
    try {
        out->reset(new MoeLayer(*cfg, dim, hidden, static_cast<DType>(dtype), device));
    } catch (const std::bad_alloc&) {
        return set_error(NOMAS_ERR_OUT_OF_MEMORY, "host allocation failed");
    }
    return NOMAS_OK;
}

// Lin::random (mod.rs:80-95): xavier weight seeded by path_seed(seed, path), zero bias.
LinF32 random_lin(uint64_t seed, const std::string& path, int64_t in_f, int64_t out_f, bool bias) {
    LinF32 l;
    l.w.resize((size_t)(in_f * out_f));
    nomas::randn_affine(nomas::path_seed(seed, path.c_str()), 0.0,
                        std::sqrt(2.0 / (double)(out_f + in_f)), in_f * out_f, l.w.data());
    if (bias) l.b.assign((size_t)out_f, 0.0f);
    return l;
}

// One Lin to read from a checkpoint: `key`.weight (out_f, in_f) and, with
// `bias`, `key`.bias (out_f,).
struct Want {
    std::string key;
    int64_t out_f, in_f;
    bool bias;
};

// Lin::load over the named files (weights.rs:105-145): every wanted tensor
// must be present (missing keys are one error listing the first few in sorted
// order, weights.rs:117-127) and have the wanted shape.
int load_lins(const char* const* files, int64_t n_files, const std::vector<Want>& want,
              std::vector<LinF32>* lins) {
    std::vector<std::string> names;
    for (const Want& w : want) {
        names.push_back(w.key + ".weight");
        if (w.bias) names.push_back(w.key + ".bias");
    }
    std::vector<std::string> fl;
    for (int64_t i = 0; i < n_files; ++i) {
        if (!files[i]) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "files[%lld] is null", (long long)i);
        fl.emplace_back(files[i]);
    }
    std::map<std::string, nomas::StTensor> ts;
    int rc = nomas::read_safetensors(fl, names, &ts);
    if (rc != NOMAS_OK) return rc;
    std::vector<std::string> missing;
    for (const std::string& n : names)
        if (!ts.count(n)) missing.push_back(n);
    std::sort(missing.begin(), missing.end());
    if (!missing.empty()) {
        std::string list;
        for (size_t i = 0; i < missing.size() && i < 5; ++i) list += (i ? ", " : "") + missing[i];
        return set_error(NOMAS_ERR_WEIGHT_KEY, "checkpoint is missing %zu model keys, first few: [%s]",
                         missing.size(), list.c_str());
    }
    lins->assign(want.size(), LinF32());
    for (size_t i = 0; i < want.size(); ++i) {
        const Want& w = want[i];
        LinF32* l = &(*lins)[i];
        const nomas::StTensor& tw = ts[w.key + ".weight"];
        if (tw.shape.size() != 2 || tw.shape[0] != w.out_f || tw.shape[1] != w.in_f)
            return set_error(NOMAS_ERR_WEIGHT_KEY, "%s.weight: expected shape (%lld, %lld)",
                             w.key.c_str(), (long long)w.out_f, (long long)w.in_f);
        rc = nomas::st_to_f32(tw, &l->w);
        if (rc != NOMAS_OK) return rc;
        if (w.bias) {
            const nomas::StTensor& tb = ts[w.key + ".bias"];
            if (tb.shape.size() != 1 || tb.shape[0] != w.out_f)
                return set_error(NOMAS_ERR_WEIGHT_KEY, "%s.bias: expected shape (%lld,)",
                                 w.key.c_str(), (long long)w.out_f);
            rc = nomas::st_to_f32(tb, &l->b);
            if (rc != NOMAS_OK) return rc;
        }
    }
    return NOMAS_OK;
}

// The dense feed-forward is checked like a one-expert MoE.
const nomas_moe_config kDenseCfg = {1, 1, 0.0, 0};

int make_dense(int64_t dim, int64_t hidden, int dtype, int device, std::unique_ptr<MoeLayer>* out) {
    int rc = MoeLayer::check_shape(kDenseCfg, dim, hidden, dtype);
    if (rc != NOMAS_OK) return rc;
    int ndev = 0;
    hipError_t e = hipGetDeviceCount(&ndev);
    if (e != hipSuccess || ndev <= 0)
        return set_error(NOMAS_ERR_HIP, "no HIP device available (%s)",
                         e == hipSuccess ? "0 devices" : hipGetErrorString(e));
    if (device < 0 || device >= ndev)
        return set_error(NOMAS_ERR_INVALID_ARGUMENT, "device %d out of range (%d devices)", device, ndev);
    try {
        out->reset(new MoeLayer(MoeLayer::DenseTag{}, dim, hidden, static_cast<DType>(dtype), device));
    } catch (const std::bad_alloc&) {
        return set_error(NOMAS_ERR_OUT_OF_MEMORY, "host allocation failed");
    }
    return NOMAS_OK;
}

int finish(std::unique_ptr<MoeLayer> layer, nomas_moe_t** out) {
    try {
        *out = new nomas_moe{std::move(layer)};
    } catch (const std::bad_alloc&) {
        return set_error(NOMAS_ERR_OUT_OF_MEMORY, "host allocation failed");
    }
    return NOMAS_OK;
}

}  // namespace

extern "C" {

int nomas_moe_config_validate(const nomas_moe_config* cfg) {
    return guarded(__func__, [&]() -> int {
        nomas::clear_error();
        if (!cfg) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "cfg must be non-null");
        if (cfg->top_k < 1 || cfg->top_k > cfg->experts)
            return set_error(NOMAS_ERR_INVALID_CONFIG, "invalid MoE top_k/experts");
        return NOMAS_OK;
    });
}

int nomas_moe_from_random(const nomas_moe_config* cfg, const char* path, int64_t dim,
                          int64_t hidden, int dtype, uint64_t seed, int device, nomas_moe_t** out) {
    return guarded(__func__, [&]() -> int {
        nomas::clear_error();
        if (!cfg || !path || !out) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "null argument");
        *out = nullptr;
        std::unique_ptr<MoeLayer> layer;
        int rc = make_layer(cfg, dim, hidden, dtype, device, &layer);
        if (rc != NOMAS_OK) return rc;
        MoeParamsF32 p;
        const std::string base(path);
        try {
            p.router = random_lin(seed, base + ".router", dim, cfg->experts, false);
            for (int64_t e = 0; e < cfg->experts; ++e) {
                const std::string ep = base + ".experts." + std::to_string(e);
                p.gate.push_back(random_lin(seed, ep + ".gate", dim, hidden, true));
                p.up.push_back(random_lin(seed, ep + ".up", dim, hidden, true));
                p.down.push_back(random_lin(seed, ep + ".down", hidden, dim, true));
            }
            if (cfg->shared_dense > 0.0) {
                p.has_dense = true;
                p.dgate = random_lin(seed, base + ".dense.gate", dim, hidden, true);
                p.dup = random_lin(seed, base + ".dense.up", dim, hidden, true);
                p.ddown = random_lin(seed, base + ".dense.down", hidden, dim, true);
            }
        } catch (const std::bad_alloc&) {
            return set_error(NOMAS_ERR_OUT_OF_MEMORY, "host allocation failed");
        }
        rc = layer->upload_f32(p);
        if (rc != NOMAS_OK) return rc;
        return finish(std::move(layer), out);
    });
}

int nomas_moe_from_safetensors(const nomas_moe_config* cfg, const char* const* files,
                               int64_t n_files, const char* path, int64_t dim, int64_t hidden,
                               int dtype, int device, nomas_moe_t** out) {
    return guarded(__func__, [&]() -> int {
        nomas::clear_error();
        if (!cfg || !files || n_files < 1 || !path || !out)
            return set_error(NOMAS_ERR_INVALID_ARGUMENT, "null argument or no files");
        *out = nullptr;
        int rc = MoeLayer::check_shape(*cfg, dim, hidden, dtype);
        if (rc != NOMAS_OK) return rc;
        const std::string base(path);
        const bool dense = cfg->shared_dense > 0.0;
        std::vector<Want> want;
        want.push_back({base + ".router", cfg->experts, dim, false});
        for (int64_t e = 0; e < cfg->experts; ++e) {
            const std::string ep = base + ".experts." + std::to_string(e);
            want.push_back({ep + ".gate", hidden, dim, true});
            want.push_back({ep + ".up", hidden, dim, true});
            want.push_back({ep + ".down", dim, hidden, true});
        }
        if (dense) {
            want.push_back({base + ".dense.gate", hidden, dim, true});
            want.push_back({base + ".dense.up", hidden, dim, true});
            want.push_back({base + ".dense.down", dim, hidden, true});
        }
        std::vector<LinF32> lins;
        rc = load_lins(files, n_files, want, &lins);
        if (rc != NOMAS_OK) return rc;
        MoeParamsF32 p;
        size_t wi = 0;
        p.router = std::move(lins[wi++]);
        for (int64_t e = 0; e < cfg->experts; ++e) {
            p.gate.push_back(std::move(lins[wi++]));
            p.up.push_back(std::move(lins[wi++]));
            p.down.push_back(std::move(lins[wi++]));
        }
        if (dense) {
            p.has_dense = true;
            p.dgate = std::move(lins[wi++]);
            p.dup = std::move(lins[wi++]);
            p.ddown = std::move(lins[wi++]);
        }
        lins.clear();
        std::unique_ptr<MoeLayer> layer;
        rc = make_layer(cfg, dim, hidden, dtype, device, &layer);
        if (rc != NOMAS_OK) return rc;
        rc = layer->upload_f32(p);
        if (rc != NOMAS_OK) return rc;
        return finish(std::move(layer), out);
    });
}

int nomas_moe_from_host(const nomas_moe_config* cfg, int64_t dim, int64_t hidden, int dtype,
                        int device, const void* router_w, const void* gate_w, const void* gate_b,
                        const void* up_w, const void* up_b, const void* down_w, const void* down_b,
                        const void* dense_gate_w, const void* dense_gate_b, const void* dense_up_w,
                        const void* dense_up_b, const void* dense_down_w, const void* dense_down_b,
                        nomas_moe_t** out) {
    return guarded(__func__, [&]() -> int {
        nomas::clear_error();
        if (!cfg || !out) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "null argument");
        *out = nullptr;
        if (!router_w || !gate_w || !up_w || !down_w)
            return set_error(NOMAS_ERR_INVALID_ARGUMENT, "router/gate/up/down weights must be non-null");
        int rc = MoeLayer::check_shape(*cfg, dim, hidden, dtype);
        if (rc != NOMAS_OK) return rc;
        if (cfg->shared_dense > 0.0 && (!dense_gate_w || !dense_up_w || !dense_down_w))
            return set_error(NOMAS_ERR_INVALID_ARGUMENT, "shared_dense > 0 needs the dense weights");
        std::unique_ptr<MoeLayer> layer;
        rc = make_layer(cfg, dim, hidden, dtype, device, &layer);
        if (rc != NOMAS_OK) return rc;
        rc = layer->upload(router_w, gate_w, gate_b, up_w, up_b, down_w, down_b, dense_gate_w,
                           dense_gate_b, dense_up_w, dense_up_b, dense_down_w, dense_down_b);
        if (rc != NOMAS_OK) return rc;
        return finish(std::move(layer), out);
    });
}

int nomas_moe_forward(nomas_moe_t* h, const void* x, void* y, int64_t rows, void* stream) {
    return guarded(__func__, [&]() -> int {
        nomas::clear_error();
        if (!h) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "null handle");
        return h->layer->forward(x, y, rows, static_cast<hipStream_t>(stream));
    });
}

int nomas_moe_forward_noalloc(nomas_moe_t* h, const void* x, void* y, int64_t rows, void* stream) {
    return guarded(__func__, [&]() -> int {
        nomas::clear_error();
        if (!h) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "null handle");
        return h->layer->forward_noalloc(x, y, rows, static_cast<hipStream_t>(stream));
    });
}

int nomas_moe_forward_block(nomas_moe_t* h, const void* x, void* out, int64_t rows, int64_t seq,
                            const float* norm_w, double eps, const float* shift,
                            const float* scale, const float* gate, void* stream) {
    return guarded(__func__, [&]() -> int {
        nomas::clear_error();
        if (!h) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "null handle");
        MoeLayer::BlockArgs b;
        b.seq = seq;
        b.norm_w = norm_w;
        b.eps = eps;
        b.shift = shift;
        b.scale = scale;
        b.gate = gate;
        return h->layer->forward_block(x, out, rows, b, static_cast<hipStream_t>(stream));
    });
}

int nomas_moe_forward_host(nomas_moe_t* h, const void* x, void* y, int64_t rows) {
    return guarded(__func__, [&]() -> int {
        nomas::clear_error();
        if (!h) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "null handle");
        return h->layer->forward_host(x, y, rows);
    });
}

int64_t nomas_moe_n_params(const nomas_moe_t* h) { return h ? h->layer->n_params() : -1; }

int nomas_moe_routing(nomas_moe_t* h, int32_t* idx, float* w, int32_t* counts, float* gap) {
    return guarded(__func__, [&]() -> int {
        nomas::clear_error();
        if (!h) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "null handle");
        return h->layer->routing(idx, w, counts, gap);
    });
}

int nomas_moe_dims(const nomas_moe_t* h, int64_t* dim, int64_t* hidden, int64_t* experts,
                   int64_t* top_k, int* dtype) {
    return guarded(__func__, [&]() -> int {
        nomas::clear_error();
        if (!h) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "null handle");
        if (dim) *dim = h->layer->dim();
        if (hidden) *hidden = h->layer->hidden();
        if (experts) *experts = h->layer->experts();
        if (top_k) *top_k = h->layer->top_k();
        if (dtype) *dtype = static_cast<int>(h->layer->dtype());
        return NOMAS_OK;
    });
}

int nomas_moe_set_profiling(nomas_moe_t* h, int enable) {
    return guarded(__func__, [&]() -> int {
        nomas::clear_error();
        if (!h) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "null handle");
        return h->layer->set_profiling(enable != 0);
    });
}

int nomas_moe_stage_times(nomas_moe_t* h, float* ms6) {
    return guarded(__func__, [&]() -> int {
        nomas::clear_error();
        if (!h) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "null handle");
        return h->layer->stage_times(ms6);
    });
}

int nomas_moe_uses_mfma(const nomas_moe_t* h) { return h && h->layer->uses_mfma() ? 1 : 0; }

void nomas_moe_destroy(nomas_moe_t* h) { delete h; }

// ---- dense SwiGLU feed-forward (mlp.rs:9-59) ----------------------------------

struct nomas_ffn {
    std::unique_ptr<MoeLayer> layer;
};

static int finish_ffn(std::unique_ptr<MoeLayer> layer, nomas_ffn_t** out) {
    try {
        *out = new nomas_ffn{std::move(layer)};
    } catch (const std::bad_alloc&) {
        return set_error(NOMAS_ERR_OUT_OF_MEMORY, "host allocation failed");
    }
    return NOMAS_OK;
}

int nomas_ffn_from_random(const char* path, int64_t dim, int64_t hidden, int dtype, uint64_t seed,
                          int device, nomas_ffn_t** out) {
    return guarded(__func__, [&]() -> int {
        nomas::clear_error();
        if (!path || !out) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "null argument");
        *out = nullptr;
        std::unique_ptr<MoeLayer> layer;
        int rc = make_dense(dim, hidden, dtype, device, &layer);
        if (rc != NOMAS_OK) return rc;
        MoeParamsF32 p;
        const std::string base(path);
        try {
            p.gate.push_back(random_lin(seed, base + ".gate", dim, hidden, true));
            p.up.push_back(random_lin(seed, base + ".up", dim, hidden, true));
            p.down.push_back(random_lin(seed, base + ".down", hidden, dim, true));
        } catch (const std::bad_alloc&) {
            return set_error(NOMAS_ERR_OUT_OF_MEMORY, "host allocation failed");
        }
        rc = layer->upload_f32(p);
        if (rc != NOMAS_OK) return rc;
        return finish_ffn(std::move(layer), out);
    });
}

int nomas_ffn_from_safetensors(const char* const* files, int64_t n_files, const char* path,
                               int64_t dim, int64_t hidden, int dtype, int device,
                               nomas_ffn_t** out) {
    return guarded(__func__, [&]() -> int {
        nomas::clear_error();
        if (!files || n_files < 1 || !path || !out)
            return set_error(NOMAS_ERR_INVALID_ARGUMENT, "null argument or no files");
        *out = nullptr;
        int rc = MoeLayer::check_shape(kDenseCfg, dim, hidden, dtype);
        if (rc != NOMAS_OK) return rc;
        const std::string base(path);
        const std::vector<Want> want = {{base + ".gate", hidden, dim, true},
                                        {base + ".up", hidden, dim, true},
                                        {base + ".down", dim, hidden, true}};
        std::vector<LinF32> lins;
        rc = load_lins(files, n_files, want, &lins);
        if (rc != NOMAS_OK) return rc;
        MoeParamsF32 p;
        p.gate.push_back(std::move(lins[0]));
        p.up.push_back(std::move(lins[1]));
        p.down.push_back(std::move(lins[2]));
        lins.clear();
        std::unique_ptr<MoeLayer> layer;
        rc = make_dense(dim, hidden, dtype, device, &layer);
        if (rc != NOMAS_OK) return rc;
        rc = layer->upload_f32(p);
        if (rc != NOMAS_OK) return rc;
        return finish_ffn(std::move(layer), out);
    });
}

int nomas_ffn_from_host(int64_t dim, int64_t hidden, int dtype, int device, const void* gate_w,
                        const void* gate_b, const void* up_w, const void* up_b, const void* down_w,
                        const void* down_b, nomas_ffn_t** out) {
    return guarded(__func__, [&]() -> int {
        nomas::clear_error();
        if (!out) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "null argument");
        *out = nullptr;
        if (!gate_w || !up_w || !down_w)
            return set_error(NOMAS_ERR_INVALID_ARGUMENT, "gate/up/down weights must be non-null");
        int rc = MoeLayer::check_shape(kDenseCfg, dim, hidden, dtype);
        if (rc != NOMAS_OK) return rc;
        std::unique_ptr<MoeLayer> layer;
        rc = make_dense(dim, hidden, dtype, device, &layer);
        if (rc != NOMAS_OK) return rc;
        rc = layer->upload(nullptr, gate_w, gate_b, up_w, up_b, down_w, down_b, nullptr, nullptr,
                           nullptr, nullptr, nullptr, nullptr);
        if (rc != NOMAS_OK) return rc;
        return finish_ffn(std::move(layer), out);
    });
}

int nomas_ffn_forward(nomas_ffn_t* h, const void* x, void* y, int64_t rows, void* stream) {
    return guarded(__func__, [&]() -> int {
        nomas::clear_error();
        if (!h) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "null handle");
        return h->layer->forward(x, y, rows, static_cast<hipStream_t>(stream));
    });
}

int nomas_ffn_forward_host(nomas_ffn_t* h, const void* x, void* y, int64_t rows) {
    return guarded(__func__, [&]() -> int {
        nomas::clear_error();
        if (!h) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "null handle");
        return h->layer->forward_host(x, y, rows);
    });
}

int64_t nomas_ffn_n_params(const nomas_ffn_t* h) { return h ? h->layer->n_params() : -1; }

int nomas_ffn_set_profiling(nomas_ffn_t* h, int enable) {
    return guarded(__func__, [&]() -> int {
        nomas::clear_error();
        if (!h) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "null handle");
        return h->layer->set_profiling(enable != 0);
    });
}

int nomas_ffn_stage_times(nomas_ffn_t* h, float* ms6) {
    return guarded(__func__, [&]() -> int {
        nomas::clear_error();
        if (!h) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "null handle");
        return h->layer->stage_times(ms6);
    });
}

int nomas_ffn_uses_mfma(const nomas_ffn_t* h) { return h && h->layer->uses_mfma() ? 1 : 0; }

void nomas_ffn_destroy(nomas_ffn_t* h) { delete h; }

namespace {

int check_seam_args(int dtype, const void* a, const void* b, const void* c, int64_t rows,
                    int64_t dim, int64_t seq) {
    if (dtype < 0 || dtype > 2) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "unknown dtype %d", dtype);
    if (rows < 0) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "rows must be >= 0");
    if (dim <= 0 || dim % 8 != 0 || dim > (1 << 24))
        return set_error(NOMAS_ERR_INVALID_ARGUMENT, "dim must be a positive multiple of 8 (got %lld)",
                         (long long)dim);
    if (seq < 1 || rows % seq != 0)
        return set_error(NOMAS_ERR_INVALID_ARGUMENT,
                         "rows=%lld must be a whole number of sequences of seq=%lld",
                         (long long)rows, (long long)seq);
    if (rows == 0) return NOMAS_OK;
    if (!a || !b || !c) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "null tensor pointer");
    if ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
         reinterpret_cast<uintptr_t>(c)) & 15)
        return set_error(NOMAS_ERR_INVALID_ARGUMENT, "tensors must be 16-byte aligned");
    return NOMAS_OK;
}

}  // namespace

int nomas_norm_modulate(int dtype, const void* x, void* h, int64_t rows, int64_t dim, int64_t seq,
                        const float* norm_w, double eps, const float* shift, const float* scale,
                        void* stream) {
    return guarded(__func__, [&]() -> int {
        nomas::clear_error();
        int rc = check_seam_args(dtype, x, h, shift, rows, dim, seq);
        if (rc != NOMAS_OK || rows == 0) return rc;
        if (!scale) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "scale must be non-null");
        if ((reinterpret_cast<uintptr_t>(scale) | reinterpret_cast<uintptr_t>(norm_w)) & 15)
            return set_error(NOMAS_ERR_INVALID_ARGUMENT, "scale and norm_w must be 16-byte aligned");
        if (!(eps >= 0.0)) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "eps must be >= 0");
        nomas::SeamArgs a;
        a.x = x;
        a.h = h;
        a.rows = rows;
        a.D = (int)dim;
        a.seq = seq;
        a.norm_w = norm_w;
        a.eps = eps;
        a.shift = shift;
        a.scale = scale;
        hipError_t e = nomas::launch_seam_h(static_cast<DType>(dtype), a, static_cast<hipStream_t>(stream));
        if (e != hipSuccess)
            return set_error(NOMAS_ERR_HIP, "norm/modulate launch failed: %s", hipGetErrorString(e));
        return NOMAS_OK;
    });
}

int nomas_gated_residual(int dtype, const void* x, const void* y, const float* gate, void* out,
                         int64_t rows, int64_t dim, int64_t seq, void* stream) {
    return guarded(__func__, [&]() -> int {
        nomas::clear_error();
        int rc = check_seam_args(dtype, x, y, out, rows, dim, seq);
        if (rc != NOMAS_OK || rows == 0) return rc;
        if (!gate) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "gate must be non-null");
        if (reinterpret_cast<uintptr_t>(gate) & 15)
            return set_error(NOMAS_ERR_INVALID_ARGUMENT, "gate must be 16-byte aligned");
        hipError_t e = nomas::launch_gated_residual(static_cast<DType>(dtype), x, y, gate, out, rows,
                                                    (int)dim, seq, static_cast<hipStream_t>(stream));
        if (e != hipSuccess)
            return set_error(NOMAS_ERR_HIP, "gated residual launch failed: %s", hipGetErrorString(e));
        return NOMAS_OK;
    });
}

const char* nomas_moe_last_error(void) { return nomas::last_error(); }

uint64_t nomas_path_seed(uint64_t seed, const char* path) {
    return path ? nomas::path_seed(seed, path) : 0;
}

void nomas_randn_affine(uint64_t seed, double mean, double std, int64_t n, float* out) {
    if (out && n > 0) nomas::randn_affine(seed, mean, std, n, out);
}

void nomas_f32_to_bf16(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = nomas::f32_to_bf16_bits(in[i]);
}

void nomas_f32_to_f16(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = nomas::f32_to_f16_bits(in[i]);
}

}  // extern "C"
