// MoeLayer: the object behind the C ABI (hy-nomas-rs modules/moe.rs:16-115).
//
// Owns the device copies of the router and expert parameters and a workspace
// sized for the largest row count seen, and runs the six-stage forward
// (router, scan, dispatch, gate/up GEMM, down GEMM, combine) on the caller's
// stream.  The reference's dense evaluation (every expert on every row) and
// this sparse evaluation give the same result: the reference multiplies the
// rows of unselected experts by a zero gate (moe.rs:3-7,97-102).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "host.hpp"

namespace nomas {

StageTiming*& stage_timing() {
    thread_local StageTiming* t = nullptr;
    return t;
}

// ---- errors ---------------------------------------------------------------

namespace {
// a fixed buffer: recording an error never allocates (or throws)
thread_local char g_last_error[1024];

struct DeviceGuard {
    int prev = -1;
    bool ok = false;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        ok = hipSetDevice(dev) == hipSuccess;
    }
    ~DeviceGuard() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

inline size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// The end-of-forward event only orders a later forward on another stream of
// the same device after this one: a device-scope release is enough (the
// default system-scope release writes back and invalidates the caches and
// idled the GPU for about 6 us per forward).  The stage-timing events take a
// device-scope release for the same reason.
constexpr unsigned kDoneFlags = hipEventDisableTiming | hipEventReleaseToDevice;
}  // namespace

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

const char* last_error() { return g_last_error; }
void clear_error() { g_last_error[0] = '\0'; }

#define HIP_TRY(expr)                                                                        \
    do {                                                                                     \
        hipError_t _e = (expr);                                                              \
        if (_e != hipSuccess)                                                                \
            return set_error(_e == hipErrorOutOfMemory ? NOMAS_ERR_OUT_OF_MEMORY : NOMAS_ERR_HIP, \
                             "%s failed: %s", #expr, hipGetErrorString(_e));                 \
    } while (0)

// ---- construction ---------------------------------------------------------

int MoeLayer::check_shape(const nomas_moe_config& cfg, int64_t dim, int64_t hidden, int dtype) {
    if (cfg.experts < 1 || cfg.top_k < 1 || cfg.top_k > cfg.experts)
        return set_error(NOMAS_ERR_INVALID_CONFIG, "invalid MoE top_k/experts (top_k=%lld, experts=%lld)",
                         (long long)cfg.top_k, (long long)cfg.experts);
    if (cfg.experts > kMaxExperts)
        return set_error(NOMAS_ERR_INVALID_CONFIG, "experts=%lld exceeds the supported maximum %d",
                         (long long)cfg.experts, kMaxExperts);
    {
        const bool dense = cfg.shared_dense > 0.0;
        const int ecols = (int)cfg.experts + (dense ? 1 : 0), kslots = (int)cfg.top_k + (dense ? 1 : 0);
        if (!dispatch_supported(ecols, kslots))
            return set_error(NOMAS_ERR_INVALID_CONFIG,
                             "top_k=%lld with experts=%lld exceeds the dispatch kernel's LDS",
                             (long long)cfg.top_k, (long long)cfg.experts);
    }
    if (dtype < 0 || dtype > 2)
        return set_error(NOMAS_ERR_INVALID_CONFIG, "unknown dtype code %d", dtype);
    if (dim < 8 || dim % 8 != 0)
        return set_error(NOMAS_ERR_INVALID_CONFIG,
                         "dim=%lld must be a positive multiple of 8 (16-byte rows)", (long long)dim);
    if (hidden < 1)
        return set_error(NOMAS_ERR_INVALID_CONFIG, "hidden=%lld must be positive", (long long)hidden);
    if (dim > (1 << 24) || hidden > (1 << 24))
        return set_error(NOMAS_ERR_INVALID_CONFIG, "dim/hidden beyond the supported range");
    return NOMAS_OK;
}

MoeLayer::MoeLayer(const nomas_moe_config& cfg, int64_t dim, int64_t hidden, DType dt, int device)
    : D_(dim), H_(hidden), E_(cfg.experts), k_(cfg.top_k), shared_dense_(cfg.shared_dense),
      dt_(dt), device_(device) {
    const bool dense = cfg.shared_dense > 0.0;
    Ecols_ = E_ + (dense ? 1 : 0);
    kslots_ = k_ + (dense ? 1 : 0);
    mfma_ = D_ % kMfmaBN == 0 && H_ % (kMfmaBN / 2) == 0;
    BM_ = mfma_ ? kMfmaBM : kSimtBM;
}

MoeLayer::MoeLayer(DenseTag, int64_t dim, int64_t hidden, DType dt, int device)
    : D_(dim), H_(hidden), E_(1), k_(1), shared_dense_(0.0), dt_(dt), device_(device) {
    Ecols_ = 1;
    kslots_ = 1;
    dense_only_ = true;
    mfma_ = D_ % kMfmaBN == 0 && H_ % (kMfmaBN / 2) == 0;
    BM_ = mfma_ ? kMfmaBM : kSimtBM;
}

MoeLayer::~MoeLayer() {
    DeviceGuard g(device_);
    free_workspace();
    if (hs_copy_) (void)hipStreamSynchronize(hs_copy_);
    if (hs_comp_) (void)hipStreamSynchronize(hs_comp_);
    for (void* p : {d_wr_, d_w1_, (void*)d_b1_, d_w2_, (void*)d_b2_, d_hio_, d_route_})
        if (p) (void)hipFree(p);
    for (hipEvent_t e : events_) (void)hipEventDestroy(e);
    for (int i = 0; i < kHostMaxPieces; ++i) {
        if (hev_in_[i]) (void)hipEventDestroy(hev_in_[i]);
        if (hev_fw_[i]) (void)hipEventDestroy(hev_fw_[i]);
    }
    for (hipStream_t s : {hs_copy_, hs_comp_})
        if (s) (void)hipStreamDestroy(s);
    if (done_) (void)hipEventDestroy(done_);
}

int64_t MoeLayer::n_params() const {
    // gate, up, down with biases (mlp.rs:50-58)
    const int64_t ffn = 2 * (H_ * D_ + H_) + (D_ * H_ + D_);
    if (dense_only_) return ffn;
    // router (no bias) + experts; dense excluded (moe.rs:112-114).
    return E_ * D_ + E_ * ffn;
}

int MoeLayer::upload(const void* router_w, const void* gate_w, const void* gate_b,
                     const void* up_w, const void* up_b, const void* down_w, const void* down_b,
                     const void* dg_w, const void* dg_b, const void* du_w, const void* du_b,
                     const void* dd_w, const void* dd_b) {
    if ((!router_w && !dense_only_) || !gate_w || !up_w || !down_w)
        return set_error(NOMAS_ERR_INVALID_ARGUMENT, "router/gate/up/down weights must be non-null");
    const bool dense = Ecols_ > E_;
    if (dense && (!dg_w || !du_w || !dd_w))
        return set_error(NOMAS_ERR_INVALID_ARGUMENT,
                         "shared_dense > 0 needs the dense gate/up/down weights");
    const size_t es = dtype_size(dt_);
    const int64_t D = D_, H = H_;
    auto to_f32 = [&](const void* p, int64_t i) -> float {
        const uint8_t* b = static_cast<const uint8_t*>(p) + i * es;
        if (dt_ == DType::F32) { float f; std::memcpy(&f, b, 4); return f; }
        uint16_t h;
        std::memcpy(&h, b, 2);
        return dt_ == DType::BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
    };
    // Per-expert source pointers (dense branch appended as the last expert).
    auto wsrc = [&](const void* moe, const void* dn, int64_t e, int64_t per) -> const uint8_t* {
        if (e < E_) return static_cast<const uint8_t*>(moe) + e * per * es;
        return static_cast<const uint8_t*>(dn);
    };
    auto bsrc = [&](const void* moe, const void* dn, int64_t e, int64_t per, int64_t i) -> float {
        const void* base = e < E_ ? moe : dn;
        if (!base) return 0.0f;
        return to_f32(base, (e < E_ ? e * per : 0) + i);
    };

    DeviceGuard g(device_);
    if (!g.ok) return set_error(NOMAS_ERR_HIP, "hipSetDevice(%d) failed", device_);
    // the end-of-forward event, made here so that no forward creates anything
    if (!done_) HIP_TRY(hipEventCreateWithFlags(&done_, kDoneFlags));

    // gate/up
    std::vector<uint8_t> w1((size_t)(Ecols_ * 2 * H * D) * es);
    std::vector<float> b1((size_t)(Ecols_ * 2 * H));
    for (int64_t e = 0; e < Ecols_; ++e) {
        const uint8_t* gw = wsrc(gate_w, dg_w, e, H * D);
        const uint8_t* uw = wsrc(up_w, du_w, e, H * D);
        for (int64_t p = 0; p < 2 * H; ++p) {
            int64_t src_row;
            bool is_up;
            if (mfma_) {  // rows 64g..64g+31 gate 32g.., rows 64g+32.. up 32g..
                const int64_t grp = p / 64, w = p % 64;
                is_up = w >= 32;
                src_row = grp * 32 + (w % 32);
            } else {      // [gate rows][up rows]
                is_up = p >= H;
                src_row = p % H;
            }
            const uint8_t* src = (is_up ? uw : gw) + src_row * D * es;
            if (mfma_) {  // K-blocked: (e, p, k) at ((e * D/KB + k/KB) * 2H + p) * KB + k % KB
                const int64_t KB = kKBlockBytes / (int64_t)es, nkb = D / KB;
                for (int64_t kb = 0; kb < nkb; ++kb)
                    std::memcpy(&w1[(size_t)(((e * nkb + kb) * 2 * H + p) * KB) * es],
                                src + kb * KB * es, (size_t)KB * es);
            } else {
                std::memcpy(&w1[(size_t)((e * 2 * H + p) * D) * es], src, (size_t)D * es);
            }
            b1[(size_t)(e * 2 * H + p)] = is_up ? bsrc(up_b, du_b, e, H, src_row)
                                                : bsrc(gate_b, dg_b, e, H, src_row);
        }
    }
    // down
    std::vector<uint8_t> w2((size_t)(Ecols_ * D * H) * es);
    std::vector<float> b2((size_t)(Ecols_ * D));
    for (int64_t e = 0; e < Ecols_; ++e) {
        const uint8_t* src = wsrc(down_w, dd_w, e, D * H);
        if (mfma_) {  // K-blocked: (e, n, k) at ((e * H/KB + k/KB) * D + n) * KB + k % KB
            const int64_t KB = kKBlockBytes / (int64_t)es, nkb = H / KB;
            for (int64_t n = 0; n < D; ++n)
                for (int64_t kb = 0; kb < nkb; ++kb)
                    std::memcpy(&w2[(size_t)(((e * nkb + kb) * D + n) * KB) * es],
                                src + (n * H + kb * KB) * es, (size_t)KB * es);
        } else {
            std::memcpy(&w2[(size_t)(e * D * H) * es], src, (size_t)(D * H) * es);
        }
        for (int64_t d = 0; d < D; ++d) b2[(size_t)(e * D + d)] = bsrc(down_b, dd_b, e, D, d);
    }

    for (void* p : {d_wr_, d_w1_, (void*)d_b1_, d_w2_, (void*)d_b2_})
        if (p) (void)hipFree(p);
    d_wr_ = d_w1_ = d_w2_ = nullptr;
    d_b1_ = d_b2_ = nullptr;
    if (!dense_only_) HIP_TRY(hipMalloc(&d_wr_, (size_t)(E_ * D) * es));
    HIP_TRY(hipMalloc(&d_w1_, w1.size()));
    HIP_TRY(hipMalloc((void**)&d_b1_, b1.size() * sizeof(float)));
    HIP_TRY(hipMalloc(&d_w2_, w2.size()));
    HIP_TRY(hipMalloc((void**)&d_b2_, b2.size() * sizeof(float)));
    if (!dense_only_) HIP_TRY(hipMemcpy(d_wr_, router_w, (size_t)(E_ * D) * es, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(d_w1_, w1.data(), w1.size(), hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(d_b1_, b1.data(), b1.size() * sizeof(float), hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(d_w2_, w2.data(), w2.size(), hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(d_b2_, b2.data(), b2.size() * sizeof(float), hipMemcpyHostToDevice));
    return NOMAS_OK;
}

int MoeLayer::upload_f32(const MoeParamsF32& p) {
    const size_t es = dtype_size(dt_);
    auto cvt = [&](const std::vector<float>& v, std::vector<uint8_t>* out) {
        out->resize(v.size() * es);
        if (dt_ == DType::F32) {
            std::memcpy(out->data(), v.data(), v.size() * 4);
            return;
        }
        uint16_t* o = reinterpret_cast<uint16_t*>(out->data());
        for (size_t i = 0; i < v.size(); ++i)
            o[i] = dt_ == DType::BF16 ? f32_to_bf16_bits(v[i]) : f32_to_f16_bits(v[i]);
    };
    auto cat = [&](const std::vector<LinF32>& ls, bool bias, int64_t per) {
        std::vector<float> all;
        all.reserve(ls.size() * per);
        for (const LinF32& l : ls) {
            const std::vector<float>& src = bias ? l.b : l.w;
            if (src.empty()) all.insert(all.end(), per, 0.0f);
            else all.insert(all.end(), src.begin(), src.end());
        }
        return all;
    };
    const int64_t D = D_, H = H_;
    std::vector<uint8_t> r, gw, gb, uw, ub, dw, db, xgw, xgb, xuw, xub, xdw, xdb;
    if (!dense_only_) cvt(p.router.w, &r);
    cvt(cat(p.gate, false, H * D), &gw);
    cvt(cat(p.gate, true, H), &gb);
    cvt(cat(p.up, false, H * D), &uw);
    cvt(cat(p.up, true, H), &ub);
    cvt(cat(p.down, false, D * H), &dw);
    cvt(cat(p.down, true, D), &db);
    const bool dense = Ecols_ > E_ && p.has_dense;
    if (dense) {
        cvt(p.dgate.w, &xgw);
        cvt(p.dgate.b.empty() ? std::vector<float>(H, 0.0f) : p.dgate.b, &xgb);
        cvt(p.dup.w, &xuw);
        cvt(p.dup.b.empty() ? std::vector<float>(H, 0.0f) : p.dup.b, &xub);
        cvt(p.ddown.w, &xdw);
        cvt(p.ddown.b.empty() ? std::vector<float>(D, 0.0f) : p.ddown.b, &xdb);
    }
    return upload(dense_only_ ? nullptr : r.data(), gw.data(), gb.data(), uw.data(), ub.data(), dw.data(), db.data(),
                  dense ? xgw.data() : nullptr, dense ? xgb.data() : nullptr,
                  dense ? xuw.data() : nullptr, dense ? xub.data() : nullptr,
                  dense ? xdw.data() : nullptr, dense ? xdb.data() : nullptr);
}

// ---- workspace --------------------------------------------------------------

int MoeLayer::max_tiles(int64_t rows) const {
    const int64_t A = rows * kslots_;
    return (int)((A + BM_ - 1) / BM_ + Ecols_);
}

size_t MoeLayer::layout(int64_t cap, bool block, uint8_t* base, Workspace* w) const {
    const int64_t A = cap * kslots_;
    const size_t es = dtype_size(dt_);
    const int mt = max_tiles(cap);
    size_t off = 0;
    auto take = [&](size_t bytes) -> uint8_t* {
        const size_t o = off;
        off += align256(bytes);
        return base ? base + o : nullptr;
    };
    Workspace v;
    v.cap_rows = cap;
    // First, at fixed offsets: the split-tile counters, then the partials.  The
    // counters' bytes are reserved in every layout (also where no GEMM splits)
    // so that nothing else ever writes there: in the shared scratch array they
    // stay zero from one forward to the next, whichever layer ran before.
    v.split_cnt = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * kSplitUnits));
    if (mfma_)
        v.split_ws = reinterpret_cast<float*>(take(sizeof(float) * kSplitUnitFloats * kSplitUnits));
    v.idx = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * A));
    v.w = reinterpret_cast<float*>(take(sizeof(float) * A));
    v.gap = reinterpret_cast<float*>(take(sizeof(float) * cap));
    v.pos = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * A));
    // one histogram per router block, of at least kMinRouterBlockRows rows
    v.chunk_counts = reinterpret_cast<int32_t*>(
        take(sizeof(int32_t) * (cap / kMinRouterBlockRows) * Ecols_));
    v.expert_count = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * Ecols_));
    v.expert_off = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * (Ecols_ + 1)));
    v.tiles = reinterpret_cast<TileInfo*>(take(sizeof(TileInfo) * mt));
    v.tile_total = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * 3));  // + tail counters
    v.xperm = take(es * A * D_);
    v.h = take(es * A * H_);
    if (!dense_only_) v.yperm = take(es * A * D_);  // dense: the down GEMM writes y
    if (block) v.block_h = take(es * cap * D_);
    if (w) *w = v;
    return off;
}

void MoeLayer::free_workspace() {
    if (d_ws_) (void)hipFree(d_ws_);
    d_ws_ = nullptr;
    ws_ = Workspace();
    if (!last_in_scratch_) last_rows_ = -1;  // the last forward's routing went with the buffers
}

int MoeLayer::ensure_workspace(int64_t rows) {
    if (rows <= ws_.cap_rows && (!want_block_ || ws_.block_h)) return NOMAS_OK;
    int64_t cap = std::max<int64_t>(rows, ws_.cap_rows + ws_.cap_rows / 2);
    cap = (cap + kRouterRows - 1) / kRouterRows * kRouterRows;
    const size_t bytes = layout(cap, want_block_, nullptr, nullptr);
    free_workspace();
    void* ws = nullptr;
    HIP_TRY(hipMalloc(&ws, bytes));
    d_ws_ = ws;
    layout(cap, want_block_, static_cast<uint8_t*>(ws), &ws_);
    if (mfma_) {
        // the split-tile counters start at zero; the GEMMs keep them there.
        // Finished before any stream (blocking or not) can use the workspace.
        HIP_TRY(hipMemset(ws_.split_cnt, 0, sizeof(int32_t) * kSplitUnits));
        HIP_TRY(hipDeviceSynchronize());
    }
    return NOMAS_OK;
}

// ---- forward ------------------------------------------------------------------

int MoeLayer::check_forward(const void* x, const void* y, int64_t rows) const {
    if (rows < 0) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "rows must be >= 0 (got %lld)", (long long)rows);
    if (rows == 0) return NOMAS_OK;
    if (!x || !y) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "x and y must be non-null");
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15)
        return set_error(NOMAS_ERR_INVALID_ARGUMENT, "x and y must be 16-byte aligned");
    if (!d_w1_) return set_error(NOMAS_ERR_STATE, "weights have not been uploaded");
    if (rows * kslots_ > 0x7fffffffLL || rows * kslots_ * std::max(D_, H_) > (1LL << 40))
        return set_error(NOMAS_ERR_INVALID_ARGUMENT, "rows=%lld exceed the supported range", (long long)rows);
    return NOMAS_OK;
}

int MoeLayer::forward(const void* x, void* y, int64_t rows, hipStream_t s) {
    return forward_impl(x, y, rows, s, nullptr);
}

int MoeLayer::forward_block(const void* x, void* out, int64_t rows, const BlockArgs& b,
                            hipStream_t s) {
    if (!b.shift || !b.scale || !b.gate)
        return set_error(NOMAS_ERR_INVALID_ARGUMENT, "shift, scale and gate must be non-null");
    if (b.seq < 1 || rows % b.seq != 0)
        return set_error(NOMAS_ERR_INVALID_ARGUMENT,
                         "rows=%lld must be a whole number of sequences of seq=%lld",
                         (long long)rows, (long long)b.seq);
    if (!(b.eps >= 0.0)) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "eps must be >= 0");
    if ((reinterpret_cast<uintptr_t>(b.shift) | reinterpret_cast<uintptr_t>(b.scale) |
         reinterpret_cast<uintptr_t>(b.gate) | reinterpret_cast<uintptr_t>(b.norm_w)) & 15)
        return set_error(NOMAS_ERR_INVALID_ARGUMENT,
                         "shift, scale, gate and norm_w must be 16-byte aligned");
    want_block_ = true;  // the next workspace layout holds h
    return forward_impl(x, out, rows, s, &b);
}

int MoeLayer::forward_impl(const void* x, void* y, int64_t rows, hipStream_t s,
                           const BlockArgs* blk) {
    int rc = check_forward(x, y, rows);
    if (rc != NOMAS_OK) return rc;
    if (rows == 0) { last_rows_ = 0; last_in_scratch_ = false; return NOMAS_OK; }
    DeviceGuard g(device_);
    if (!g.ok) return set_error(NOMAS_ERR_HIP, "hipSetDevice(%d) failed", device_);
    rc = ensure_workspace(rows);
    if (rc != NOMAS_OK) return rc;
    if (done_recorded_ && s != last_stream_) HIP_TRY(hipStreamWaitEvent(s, done_, 0));
    if (dense_only_) {
        if (blk) return set_error(NOMAS_ERR_STATE, "the fused block is implemented for the MoE layer");
        return forward_dense(x, y, rows, s);
    }
    rc = run_routed(x, y, rows, s, blk, ws_);
    if (rc != NOMAS_OK) {
        last_rows_ = -1;  // a failed forward may have overwritten the last one's routing
        return rc;
    }
    last_in_scratch_ = false;
    return finish_forward(rows, s, ws_);
}

int MoeLayer::forward_noalloc(const void* x, void* y, int64_t rows, hipStream_t s) {
    if (dense_only_)
        return set_error(NOMAS_ERR_STATE, "the no-allocation forward is implemented for the MoE layer");
    int rc = check_forward(x, y, rows);
    if (rc != NOMAS_OK) return rc;
    if (rows == 0) { last_rows_ = 0; last_in_scratch_ = false; return NOMAS_OK; }
    const int64_t cap = (rows + kRouterRows - 1) / kRouterRows * kRouterRows;
    const size_t need = layout(cap, false, nullptr, nullptr);
    if (need > kScratchBytes) {
        // the most rows that fit, for the message
        int64_t lo = 0, hi = cap / kRouterRows;
        while (lo < hi) {
            const int64_t mid = (lo + hi + 1) / 2;
            if (layout(mid * kRouterRows, false, nullptr, nullptr) <= kScratchBytes) lo = mid;
            else hi = mid - 1;
        }
        return set_error(NOMAS_ERR_INVALID_ARGUMENT,
                         "rows=%lld need %zu bytes of device scratch; the no-allocation forward "
                         "holds %zu (at most %lld rows for this layer): use nomas_moe_forward",
                         (long long)rows, need, kScratchBytes, (long long)(lo * kRouterRows));
    }
    DeviceGuard g(device_);
    if (!g.ok) return set_error(NOMAS_ERR_HIP, "hipSetDevice(%d) failed", device_);
    void* base = nullptr;
    uint64_t gen = 0;
    rc = scratch_acquire(device_, s, &base, &gen);
    if (rc != NOMAS_OK) return rc;
    Workspace w;
    layout(cap, false, static_cast<uint8_t*>(base), &w);
    if (done_recorded_ && s != last_stream_) HIP_TRY(hipStreamWaitEvent(s, done_, 0));
    rc = run_routed(x, y, rows, s, nullptr, w);
    if (rc != NOMAS_OK) {
        last_rows_ = -1;  // as in forward_impl
        return rc;
    }
    last_in_scratch_ = true;
    last_scratch_gen_ = gen;
    return finish_forward(rows, s, w);
}

int MoeLayer::finish_forward(int64_t rows, hipStream_t s, const Workspace& w) {
    // done_ is created with the weights; recording it allocates nothing
    HIP_TRY(hipEventRecord(done_, s));
    done_recorded_ = true;
    host_pieces_ = 0;  // routing() reads this forward's workspace
    last_rows_ = rows;
    last_stream_ = s;
    last_ws_ = w;
    return NOMAS_OK;
}

int MoeLayer::run_routed(const void* x, void* y, int64_t rows, hipStream_t s,
                         const BlockArgs* blk, const Workspace& w) {
    int rc;
    const int nch = (int)((rows + kRouterRows - 1) / kRouterRows);
    const int mt = max_tiles(rows);
    const int64_t a_cap = w.cap_rows * kslots_;
    hipEvent_t* ev = nullptr;
    uint8_t* empty = nullptr;
    if (profiling_) {
        ev = &events_[(size_t)(recorded_ % kRing) * kProfEvents];
        empty = &stage_empty_[(size_t)(recorded_ % kRing) * kProfStages];
        ++recorded_;
    }
    StageClock clock(ev, empty, s);
    auto mark = [&](int i) -> int {
        HIP_TRY(clock.mark(i));
        return NOMAS_OK;
    };
#define STAGE(call, what)                                                                  \
    do {                                                                                   \
        hipError_t _e = (call);                                                            \
        if (_e != hipSuccess)                                                              \
            return set_error(NOMAS_ERR_HIP, "%s launch failed: %s", what, hipGetErrorString(_e)); \
    } while (0)

    if ((rc = mark(0))) return rc;
    const void* xr = x;  // what the router and the dispatch read: x, or h in a block
    if (blk) {
        SeamArgs sm;
        sm.x = x;
        sm.h = w.block_h;
        sm.rows = rows;
        sm.D = (int)D_;
        sm.seq = blk->seq;
        sm.norm_w = blk->norm_w;
        sm.eps = blk->eps;
        sm.shift = blk->shift;
        sm.scale = blk->scale;
        STAGE(launch_seam_h(dt_, sm, s), "norm/modulate");
        xr = w.block_h;
    }
    RouterArgs ra;
    ra.x = xr;
    ra.wr = d_wr_;
    ra.rows = rows;
    ra.D = (int)D_;
    ra.E = (int)E_;
    ra.k = (int)k_;
    ra.k_slots = (int)kslots_;
    ra.dense_coef = (float)shared_dense_;
    ra.topk_idx = w.idx;
    ra.topk_w = w.w;
    ra.gap = w.gap;
    ra.chunk_counts = w.chunk_counts;
    ra.block_rows = router_block_rows(dt_, rows, (int)D_, (int)E_);
    STAGE(launch_router(dt_, ra, s), "router");
    if ((rc = mark(1))) return rc;

    // the scan of the chunk histograms is part of the dispatch kernel: the
    // "scan" stage is empty
    if ((rc = mark(2))) return rc;

    DispatchArgs da;
    da.x = xr;
    da.rows = rows;
    da.D = (int)D_;
    da.E_cols = (int)Ecols_;
    da.k_slots = (int)kslots_;
    da.topk_idx = w.idx;
    da.chunk_counts = w.chunk_counts;
    da.nchunks = nch;
    da.count_rows = ra.block_rows;
    da.BM = BM_;
    da.max_tiles = mt;
    da.expert_count = w.expert_count;
    da.expert_off = w.expert_off;
    da.tiles = w.tiles;
    da.tile_total = w.tile_total;
    da.tok_pos = w.pos;
    da.x_perm = w.xperm;
    da.a_cap = a_cap;
    da.kblocked = mfma_ ? 1 : 0;
    STAGE(launch_dispatch(dt_, da, s), "dispatch");
    if ((rc = mark(3))) return rc;

    GemmArgs g1;
    g1.X = w.xperm;
    g1.W = d_w1_;
    g1.bias = d_b1_;
    g1.out = w.h;
    g1.tiles = w.tiles;
    g1.tile_total = w.tile_total;
    g1.max_tiles = mt;
    g1.N = (int)(2 * H_);
    g1.K = (int)D_;
    g1.num_experts = (int)Ecols_;
    g1.a_cap = a_cap;
    g1.split_ws = w.split_ws;
    g1.split_cnt = w.split_cnt;
    g1.tail_cnt = w.tile_total + 1;
    STAGE(mfma_ ? launch_gemm_gate_up_mfma(dt_, g1, s) : launch_gemm_gate_up_simt(dt_, g1, s),
          "gate/up GEMM");
    if ((rc = mark(4))) return rc;

    GemmArgs g2 = g1;
    g2.X = w.h;
    g2.W = d_w2_;
    g2.bias = d_b2_;
    g2.out = w.yperm;
    g2.tail_cnt = w.tile_total + 2;
    g2.N = (int)D_;
    g2.K = (int)H_;
    g2.out_nt = rows * kslots_ * D_ * (int64_t)dtype_size(dt_) > kLastLevelCacheBytes;
    STAGE(mfma_ ? launch_gemm_down_mfma(dt_, g2, s) : launch_gemm_down_simt(dt_, g2, s),
          "down GEMM");
    if ((rc = mark(5))) return rc;

    CombineArgs ca;
    ca.y_perm = w.yperm;
    ca.tok_pos = w.pos;
    ca.topk_w = w.w;
    ca.rows = rows;
    ca.D = (int)D_;
    ca.k_slots = (int)kslots_;
    ca.out = y;
    ca.a_cap = a_cap;
    ca.resid_x = blk ? x : nullptr;
    ca.gate = blk ? blk->gate : nullptr;
    ca.seq = blk ? blk->seq : 1;
    ca.out_nt = g2.out_nt;
    STAGE(launch_combine(dt_, ca, s), "combine");
    if ((rc = mark(6))) return rc;
#undef STAGE
    return NOMAS_OK;
}

// Dense feed-forward: the stages of the routed forward that remain.  Stage
// slots for profiling: router (none), scan = tile table, dispatch = K-blocked
// copy of x (MFMA path only), gate/up, down (written straight into y), combine
// (none).
int MoeLayer::forward_dense(const void* x, void* y, int64_t rows, hipStream_t s) {
    int rc;
    const Workspace& w = ws_;
    const int mt = max_tiles(rows);
    hipEvent_t* ev = nullptr;
    uint8_t* empty = nullptr;
    if (profiling_) {
        ev = &events_[(size_t)(recorded_ % kRing) * kProfEvents];
        empty = &stage_empty_[(size_t)(recorded_ % kRing) * kProfStages];
        ++recorded_;
    }
    StageClock clock(ev, empty, s);
    auto mark = [&](int i) -> int {
        HIP_TRY(clock.mark(i));
        return NOMAS_OK;
    };
#define STAGE(call, what)                                                                  \
    do {                                                                                   \
        hipError_t _e = (call);                                                            \
        if (_e != hipSuccess)                                                              \
            return set_error(NOMAS_ERR_HIP, "%s launch failed: %s", what, hipGetErrorString(_e)); \
    } while (0)
    if ((rc = mark(0))) return rc;
    if ((rc = mark(1))) return rc;
    STAGE(launch_dense_tiles(rows, BM_, mt, w.tiles, w.tile_total, s), "tile table");
    if ((rc = mark(2))) return rc;
    // the MFMA GEMMs read K-blocked rows; the general path reads x in place
    if (mfma_) STAGE(launch_kblock(dt_, x, w.xperm, rows, (int)D_, w.cap_rows, s), "K-blocked copy");
    if ((rc = mark(3))) return rc;

    GemmArgs g1;
    g1.X = mfma_ ? w.xperm : x;
    g1.W = d_w1_;
    g1.bias = d_b1_;
    g1.out = w.h;
    g1.tiles = w.tiles;
    g1.tile_total = w.tile_total;
    g1.max_tiles = mt;
    g1.N = (int)(2 * H_);
    g1.K = (int)D_;
    g1.num_experts = 1;
    // MFMA: the K-blocked buffers' row capacity; general: rows of x (row-major)
    g1.a_cap = mfma_ ? w.cap_rows : rows;
    g1.split_ws = w.split_ws;
    g1.split_cnt = w.split_cnt;
    g1.tail_cnt = w.tile_total + 1;
    STAGE(mfma_ ? launch_gemm_gate_up_mfma(dt_, g1, s) : launch_gemm_gate_up_simt(dt_, g1, s),
          "gate/up GEMM");
    if ((rc = mark(4))) return rc;

    GemmArgs g2 = g1;
    g2.X = w.h;
    g2.W = d_w2_;
    g2.bias = d_b2_;
    g2.out = y;  // rows stay in order: the output is y itself
    g2.tail_cnt = w.tile_total + 2;
    g2.N = (int)D_;
    g2.K = (int)H_;
    STAGE(mfma_ ? launch_gemm_down_mfma(dt_, g2, s) : launch_gemm_down_simt(dt_, g2, s),
          "down GEMM");
    if ((rc = mark(5))) return rc;
    if ((rc = mark(6))) return rc;
#undef STAGE
    last_in_scratch_ = false;
    return finish_forward(rows, s, w);
}

int MoeLayer::forward_host(const void* x, void* y, int64_t rows) {
    if (rows < 0) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "rows must be >= 0");
    if (rows == 0) { last_rows_ = 0; return NOMAS_OK; }
    if (!x || !y) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "x and y must be non-null");
    DeviceGuard g(device_);
    if (!g.ok) return set_error(NOMAS_ERR_HIP, "hipSetDevice(%d) failed", device_);
    const size_t bytes = (size_t)(rows * D_) * dtype_size(dt_);
    // device copies of x and y live with the handle: an allocation and a
    // free per call cost more than the copies
    if (bytes > hio_bytes_) {
        const size_t half = align256(std::max(bytes, hio_bytes_ + hio_bytes_ / 2));
        if (d_hio_) HIP_TRY(hipFree(d_hio_));
        d_hio_ = nullptr;
        hio_bytes_ = 0;
        HIP_TRY(hipMalloc(&d_hio_, 2 * half));
        hio_bytes_ = half;
    }
    void* dx = d_hio_;
    void* dy = static_cast<uint8_t*>(d_hio_) + hio_bytes_;
    const int np = rows >= 2 * kHostPieceRows
                       ? (int)std::min<int64_t>(kHostMaxPieces, rows / kHostPieceRows)
                       : 1;
    if (np == 1) {
        host_pieces_ = 0;
        int rc = stager_.to_device(dx, x, bytes, nullptr);
        if (rc == NOMAS_OK) rc = forward(dx, dy, rows, nullptr);
        if (rc == NOMAS_OK) rc = stager_.to_host(y, dy, bytes, nullptr);
        return rc;
    }
    return forward_host_pieces(x, y, rows, np, dx, dy);
}

int MoeLayer::host_pipe_setup() {
    if (hs_comp_) return NOMAS_OK;
    for (hipStream_t* s : {&hs_copy_, &hs_comp_})
        if (!*s) HIP_TRY(hipStreamCreateWithFlags(s, hipStreamNonBlocking));
    for (int i = 0; i < kHostMaxPieces; ++i) {
        if (!hev_in_[i]) HIP_TRY(hipEventCreateWithFlags(&hev_in_[i], hipEventDisableTiming));
        if (!hev_fw_[i]) HIP_TRY(hipEventCreateWithFlags(&hev_fw_[i], hipEventDisableTiming));
    }
    return NOMAS_OK;
}

// A large host-tensor forward in np row pieces (whole multiples of 64 rows,
// the last one shorter): every piece's input is copied in first, each on the
// copy stream, and the compute stream runs piece p's forward once its input
// has landed; then every piece's output is copied out once its forward is
// done.  The host thread stages piece p + 1 in while the GPU computes piece
// p, and piece p out while it computes p + 1.  Each piece is an ordinary
// forward: rows are independent, so the results are those of a forward over
// the piece's rows (a K-split GEMM tile can round differently than in one
// forward over all rows, within the same bars).  The routing of every piece
// is kept, so routing() reads the whole call back.
int MoeLayer::forward_host_pieces(const void* x, void* y, int64_t rows, int np, void* dx, void* dy) {
    int rc = host_pipe_setup();
    if (rc != NOMAS_OK) return rc;
    const size_t rb = (size_t)D_ * dtype_size(dt_);  // bytes per row
    const int64_t per = ((rows + np - 1) / np + kRouterRows - 1) / kRouterRows * kRouterRows;
    const size_t route = dense_only_ ? 0 : (size_t)rows * kslots_ * 8 + (size_t)rows * 4 +
                                               (size_t)np * Ecols_ * 4;
    if (route > route_bytes_) {
        if (hs_comp_) HIP_TRY(hipStreamSynchronize(hs_comp_));
        if (d_route_) HIP_TRY(hipFree(d_route_));
        d_route_ = nullptr;
        route_bytes_ = 0;
        HIP_TRY(hipMalloc(&d_route_, route));
        route_bytes_ = route;
    }
    // the pieces' routing (a dense feed-forward has none, and no d_route_)
    int32_t* r_idx = nullptr;
    float *r_w = nullptr, *r_gap = nullptr;
    int32_t* r_cnt = nullptr;
    if (!dense_only_) {
        r_idx = static_cast<int32_t*>(d_route_);
        r_w = reinterpret_cast<float*>(r_idx + rows * kslots_);
        r_gap = r_w + rows * kslots_;
        r_cnt = reinterpret_cast<int32_t*>(r_gap + rows);
    }
    auto fail = [&](int code) {  // nothing in flight outlives the call
        (void)hipStreamSynchronize(hs_copy_);
        (void)hipStreamSynchronize(hs_comp_);
        host_pieces_ = 0;
        return code;
    };
    int n_pieces = 0;
    for (int p = 0; p < np; ++p) {
        const int64_t off = p * per, n = std::min(per, rows - off);
        if (n <= 0) break;
        n_pieces = p + 1;
        const size_t o = (size_t)off * rb;
        rc = stager_.to_device(static_cast<uint8_t*>(dx) + o, static_cast<const uint8_t*>(x) + o,
                               (size_t)n * rb, hs_copy_);
        if (rc != NOMAS_OK) return fail(rc);
        if (hipEventRecord(hev_in_[p], hs_copy_) != hipSuccess ||
            hipStreamWaitEvent(hs_comp_, hev_in_[p], 0) != hipSuccess)
            return fail(set_error(NOMAS_ERR_HIP, "host piece %d: event failed", p));
        rc = forward(static_cast<uint8_t*>(dx) + o, static_cast<uint8_t*>(dy) + o, n, hs_comp_);
        if (rc != NOMAS_OK) return fail(rc);
        if (!dense_only_) {
            const Workspace& w = last_ws_;
            const hipMemcpyKind d2d = hipMemcpyDeviceToDevice;
            if (hipMemcpyAsync(r_idx + off * kslots_, w.idx, sizeof(int32_t) * n * kslots_, d2d, hs_comp_) ||
                hipMemcpyAsync(r_w + off * kslots_, w.w, sizeof(float) * n * kslots_, d2d, hs_comp_) ||
                hipMemcpyAsync(r_gap + off, w.gap, sizeof(float) * n, d2d, hs_comp_) ||
                hipMemcpyAsync(r_cnt + (int64_t)p * Ecols_, w.expert_count, sizeof(int32_t) * Ecols_, d2d,
                               hs_comp_))
                return fail(set_error(NOMAS_ERR_HIP, "host piece %d: routing copy failed", p));
        }
        if (hipEventRecord(hev_fw_[p], hs_comp_) != hipSuccess)
            return fail(set_error(NOMAS_ERR_HIP, "host piece %d: event failed", p));
    }
    for (int p = 0; p < n_pieces; ++p) {
        const int64_t off = p * per, n = std::min(per, rows - off);
        const size_t o = (size_t)off * rb;
        if (hipStreamWaitEvent(hs_copy_, hev_fw_[p], 0) != hipSuccess)
            return fail(set_error(NOMAS_ERR_HIP, "host piece %d: event failed", p));
        rc = stager_.to_host(static_cast<uint8_t*>(y) + o, static_cast<const uint8_t*>(dy) + o,
                             (size_t)n * rb, hs_copy_);
        if (rc != NOMAS_OK) return fail(rc);
    }
    // the copy-out of the last piece has finished on the host; the routing
    // copies are ordered before the events it waited for
    host_pieces_ = n_pieces;
    last_rows_ = rows;
    return NOMAS_OK;
}

int MoeLayer::routing(int32_t* idx, float* w, int32_t* counts, float* gap) {
    if (dense_only_) return set_error(NOMAS_ERR_STATE, "a dense feed-forward has no routing");
    if (last_rows_ < 0) return set_error(NOMAS_ERR_STATE, "no forward has run on this handle");
    if (last_in_scratch_ && last_rows_ > 0 && scratch_generation(device_) != last_scratch_gen_)
        return set_error(NOMAS_ERR_STATE,
                         "the routing of this handle's last (no-allocation) forward was overwritten "
                         "by a later no-allocation forward on device %d", device_);
    DeviceGuard g(device_);
    HIP_TRY(hipStreamSynchronize(last_stream_));
    const int64_t rows = last_rows_;
    if (rows == 0) {
        if (counts) std::memset(counts, 0, sizeof(int32_t) * E_);
        return NOMAS_OK;
    }
    // a pieced host-tensor forward keeps its routing in d_route_
    const int32_t* s_idx = last_ws_.idx;
    const float* s_w = last_ws_.w;
    const float* s_gap = last_ws_.gap;
    if (host_pieces_ > 0) {
        s_idx = static_cast<const int32_t*>(d_route_);
        s_w = reinterpret_cast<const float*>(s_idx + rows * kslots_);
        s_gap = s_w + rows * kslots_;
    }
    if (idx || w) {
        std::vector<int32_t> hi((size_t)(rows * kslots_));
        std::vector<float> hw((size_t)(rows * kslots_));
        HIP_TRY(hipMemcpy(hi.data(), s_idx, hi.size() * sizeof(int32_t), hipMemcpyDeviceToHost));
        HIP_TRY(hipMemcpy(hw.data(), s_w, hw.size() * sizeof(float), hipMemcpyDeviceToHost));
        for (int64_t r = 0; r < rows; ++r)
            for (int64_t j = 0; j < k_; ++j) {
                if (idx) idx[r * k_ + j] = hi[(size_t)(r * kslots_ + j)];
                if (w) w[r * k_ + j] = hw[(size_t)(r * kslots_ + j)];
            }
    }
    if (counts) {
        if (host_pieces_ > 0) {  // the pieces' counts, added
            std::vector<int32_t> pc((size_t)host_pieces_ * Ecols_);
            HIP_TRY(hipMemcpy(pc.data(), s_gap + rows, pc.size() * sizeof(int32_t), hipMemcpyDeviceToHost));
            for (int64_t e = 0; e < E_; ++e) {
                int64_t c = 0;
                for (int p = 0; p < host_pieces_; ++p) c += pc[(size_t)p * Ecols_ + e];
                counts[e] = (int32_t)c;
            }
        } else {
            HIP_TRY(hipMemcpy(counts, last_ws_.expert_count, sizeof(int32_t) * E_, hipMemcpyDeviceToHost));
        }
    }
    if (gap) HIP_TRY(hipMemcpy(gap, s_gap, sizeof(float) * rows, hipMemcpyDeviceToHost));
    return NOMAS_OK;
}

int MoeLayer::set_profiling(bool on) {
    DeviceGuard g(device_);
    if (on && events_.empty()) {
        events_.resize((size_t)kRing * kProfEvents);
        stage_empty_.assign((size_t)kRing * kProfStages, 0);
        for (hipEvent_t& e : events_) HIP_TRY(hipEventCreateWithFlags(&e, hipEventReleaseToDevice));
    }
    profiling_ = on;
    recorded_ = 0;
    return NOMAS_OK;
}

int MoeLayer::stage_times(float* ms6) {
    if (!ms6) return set_error(NOMAS_ERR_INVALID_ARGUMENT, "ms6 must be non-null");
    if (!profiling_ || recorded_ == 0)
        return set_error(NOMAS_ERR_STATE, "no profiled forward recorded");
    DeviceGuard g(device_);
    const int n = std::min(recorded_, kRing);
    double sum[6] = {0, 0, 0, 0, 0, 0};
    for (int i = 0; i < n; ++i) {
        const int set = (recorded_ - 1 - i) % kRing;
        hipEvent_t* ev = &events_[(size_t)set * kProfEvents];
        const uint8_t* empty = &stage_empty_[(size_t)set * kProfStages];
        // the last stage's last recorded event
        HIP_TRY(hipEventSynchronize(ev[empty[kProfStages - 1] ? kProfEvents - 2 : kProfEvents - 1]));
        for (int st = 0; st < kProfStages; ++st) {
            if (empty[st]) continue;  // no kernel: zero
            float ms = 0.0f;
            HIP_TRY(hipEventElapsedTime(&ms, ev[2 * st], ev[2 * st + 1]));
            sum[st] += ms;
        }
    }
    for (int st = 0; st < 6; ++st) ms6[st] = (float)(sum[st] / n);
    recorded_ = 0;
    return NOMAS_OK;
}

}  // namespace nomas
