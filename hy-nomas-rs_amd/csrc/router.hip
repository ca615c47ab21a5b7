// Router: logits = x . Wr^T, softmax, top-k and renormalised gates, fused in
// one kernel (hy-nomas-rs moe.rs:67-95).
//
// One block = 8 waves = one chunk of 64 rows; each wave routes 8 rows, as two
// passes of 4 rows over x.
//  - Logits accumulate in f64.  Every product of two bf16/f16 inputs is exact
//    in f32 and of two f32 inputs in the f64 fma, so the only rounding is the
//    f64 sum: indices are then
//    decided far below the 1e-6 logit near-tie threshold.  The kernel reads
//    x once (T*D*b bytes): HBM-bound.
//  - Lanes split D in 16-byte chunks; each lane keeps 4 rows x 8 experts of
//    partial sums, then a butterfly reduce-scatter (5 halving xor-shuffle
//    steps + 1 full step: 32 shuffles instead of 32*6) leaves every sum on one
//    lane pair.
//  - Selection is wave-parallel over experts: max / sum / k rounds of argmax
//    are xor-shuffle reductions across the wave.  Ties go to the lowest
//    expert index, the reference's first-max-wins argmax (moe.rs:78-80).
//  - Gates: p = exp(l - max) / sum_E exp(l - max), w = p / (sum_selected p + 1e-9)
//    (moe.rs:68,92-95), evaluated in f64 and stored as f32.
//  - Output per row: k experts in ascending index with their gates, the
//    logit gap between the k-th selected and the best unselected expert, and
//    (block level) the chunk's per-expert histogram for the dispatch scan.
//    With a shared dense branch the row gets one more slot: expert E with
//    gate `dense_coef` (moe.rs:103-106 adds it after the experts).
#include "kernels.hpp"

namespace nomas {

namespace {

constexpr int kRouterThreads = 512;  // 8 waves; each routes 8 rows as 2 passes of 4
constexpr int kRowsPerPass = 4;
constexpr int kRowsPerWave = kRouterRows / (kRouterThreads / kWave);
constexpr int kExpGroup = 8;

__device__ __forceinline__ double wave_max(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmax(v, __shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// acc + x * w with the product exact: a product of two 16-bit floats fits the
// 24-bit f32 significand, two f32 need the f64 fma.
template <typename T>
__device__ __forceinline__ double acc_exact(float x, float w, double acc) {
    if constexpr (sizeof(T) == 2) return acc + (double)(x * w);
    else return __builtin_fma((double)x, (double)w, acc);
}

template <typename T>
__global__ __launch_bounds__(kRouterThreads) void router_kernel(
    const T* __restrict__ x, const T* __restrict__ wr, int64_t rows, int D, int E, int k,
    int k_slots, float dense_coef, int32_t* __restrict__ topk_idx, float* __restrict__ topk_w,
    float* __restrict__ gap, int32_t* __restrict__ chunk_counts) {
    extern __shared__ double s_logit[];  // [kRouterRows][E]
    int* s_cnt = reinterpret_cast<int*>(s_logit + kRouterRows * E);  // [E + 1]
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int E_cols = E + (k_slots > k ? 1 : 0);
    for (int e = tid; e < E_cols; e += kRouterThreads) s_cnt[e] = 0;

    constexpr int EPC = 16 / sizeof(T);
    const int nchunk = D / EPC;
    const int64_t chunk_row0 = (int64_t)blockIdx.x * kRouterRows;

    for (int pass = 0; pass < kRowsPerWave / kRowsPerPass; ++pass) {
        const int lr0 = wave * kRowsPerWave + pass * kRowsPerPass;
        bool valid[kRowsPerPass];
        const T* xr[kRowsPerPass];
#pragma unroll
        for (int r = 0; r < kRowsPerPass; ++r) {
            const int64_t row = chunk_row0 + lr0 + r;
            valid[r] = row < rows;
            xr[r] = x + (valid[r] ? row : 0) * (int64_t)D;
        }
        if (!valid[0]) break;  // wave-uniform: no row of this pass exists
        for (int e0 = 0; e0 < E; e0 += kExpGroup) {
            double v[kRowsPerPass * kExpGroup];  // partial sums, index r * kExpGroup + g
#pragma unroll
            for (int i = 0; i < kRowsPerPass * kExpGroup; ++i) v[i] = 0.0;
            for (int c = lane; c < nchunk; c += kWave) {
                float xv[kRowsPerPass][EPC];
#pragma unroll
                for (int r = 0; r < kRowsPerPass; ++r) {
                    if (valid[r]) {
                        load16(xr[r] + (int64_t)c * EPC, xv[r]);
                    } else {
#pragma unroll
                        for (int i = 0; i < EPC; ++i) xv[r][i] = 0.0f;
                    }
                }
#pragma unroll
                for (int g = 0; g < kExpGroup; ++g) {
                    if (e0 + g < E) {
                        float wv[EPC];
                        load16(wr + (int64_t)(e0 + g) * D + (int64_t)c * EPC, wv);
#pragma unroll
                        for (int i = 0; i < EPC; ++i)
#pragma unroll
                            for (int r = 0; r < kRowsPerPass; ++r)
                                v[r * kExpGroup + g] = acc_exact<T>(xv[r][i], wv[i], v[r * kExpGroup + g]);
                    }
                }
            }
            // Butterfly reduce-scatter of the 32 partial sums over the 64 lanes.
#pragma unroll
            for (int step = 0; step < 5; ++step) {
                const int o = 32 >> step;
                const int half = 16 >> step;
                const bool upper = (lane & o) != 0;
#pragma unroll
                for (int i = 0; i < half; ++i) {
                    const double send = upper ? v[i] : v[i + half];
                    const double keep = upper ? v[i + half] : v[i];
                    v[i] = keep + __shfl_xor(send, o);
                }
            }
            v[0] += __shfl_xor(v[0], 1);
            // Lane l now holds the full sum of value index (l >> 1) & 31.
            if ((lane & 1) == 0) {
                const int vi = (lane >> 1) & 31;
                const int r = vi / kExpGroup, g = vi % kExpGroup;
                if (e0 + g < E) s_logit[(lr0 + r) * E + e0 + g] = v[0];
            }
        }
    }
    __syncthreads();

    const int per_lane = (E + kWave - 1) / kWave;  // experts per lane (<= 4 for E <= 256)
    for (int r = 0; r < kRowsPerWave; ++r) {
        const int lr = wave * kRowsPerWave + r;
        const int64_t row = chunk_row0 + lr;
        if (row >= rows) break;  // wave-uniform
        const double* lg = s_logit + lr * E;
        double m = -INFINITY;
        for (int j = 0; j < per_lane; ++j) {
            const int e = lane + j * kWave;
            if (e < E) m = fmax(m, lg[e]);
        }
        m = wave_max(m);
        double s = 0.0;
        for (int j = 0; j < per_lane; ++j) {
            const int e = lane + j * kWave;
            if (e < E) s += exp(lg[e] - m);
        }
        s = wave_sum(s);

        uint32_t sel = 0;
        double kth = INFINITY;
        for (int it = 0; it < k; ++it) {
            double bv = 0.0;
            int bi = -1;
            for (int j = 0; j < per_lane; ++j) {
                const int e = lane + j * kWave;
                if (e < E && !((sel >> j) & 1u)) {
                    const double lv = lg[e];
                    if (bi < 0 || lv > bv) { bv = lv; bi = e; }
                }
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                const double ov = __shfl_xor(bv, o);
                const int oi = __shfl_xor(bi, o);
                if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) { bv = ov; bi = oi; }
            }
            if ((bi & (kWave - 1)) == lane) sel |= 1u << (bi / kWave);
            kth = bv;
        }
        double best_un = -INFINITY, psel = 0.0;
        for (int j = 0; j < per_lane; ++j) {
            const int e = lane + j * kWave;
            if (e >= E) continue;
            if ((sel >> j) & 1u) psel += exp(lg[e] - m) / s;
            else best_un = fmax(best_un, lg[e]);
        }
        best_un = wave_max(best_un);
        psel = wave_sum(psel);

        int base = 0;
        for (int j = 0; j < per_lane; ++j) {
            const bool is_sel = (sel >> j) & 1u;
            const uint64_t bal = __ballot(is_sel);
            if (is_sel) {
                const int e = lane + j * kWave;
                const int rank = base + __popcll(bal & ((1ull << lane) - 1ull));
                const double p = exp(lg[e] - m) / s;
                topk_idx[row * k_slots + rank] = e;
                topk_w[row * k_slots + rank] = (float)(p / (psel + 1e-9));
                atomicAdd(&s_cnt[e], 1);
            }
            base += __popcll(bal);
        }
        if (lane == 0) {
            gap[row] = (k == E) ? INFINITY : (float)(kth - best_un);
            if (k_slots > k) {
                topk_idx[row * k_slots + k] = E;
                topk_w[row * k_slots + k] = dense_coef;
                atomicAdd(&s_cnt[E], 1);
            }
        }
    }
    __syncthreads();
    for (int e = tid; e < E_cols; e += kRouterThreads)
        chunk_counts[(int64_t)blockIdx.x * E_cols + e] = s_cnt[e];
}

template <typename T>
hipError_t launch_router_t(const RouterArgs& a, hipStream_t s) {
    const int nblk = (int)((a.rows + kRouterRows - 1) / kRouterRows);
    const size_t lds = sizeof(double) * kRouterRows * a.E + sizeof(int) * (a.E + 1);
    if (lds > 65536) {
        hipError_t err = hipFuncSetAttribute((const void*)router_kernel<T>,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (err != hipSuccess) return err;
    }
    hipLaunchKernelGGL(router_kernel<T>, dim3(nblk), dim3(kRouterThreads), lds, s,
                       (const T*)a.x, (const T*)a.wr, a.rows, a.D, a.E, a.k, a.k_slots,
                       a.dense_coef, a.topk_idx, a.topk_w, a.gap, a.chunk_counts);
    return hipGetLastError();
}

}  // namespace

size_t router_lds_bytes(int E) { return sizeof(double) * kRouterRows * E + sizeof(int) * (E + 1); }

hipError_t launch_router(DType dt, const RouterArgs& a, hipStream_t s) {
    switch (dt) {
        case DType::F32: return launch_router_t<float>(a, s);
        case DType::BF16: return launch_router_t<__bf16>(a, s);
        case DType::F16: return launch_router_t<_Float16>(a, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace nomas
