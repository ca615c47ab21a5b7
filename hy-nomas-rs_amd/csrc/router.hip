// Router: logits = x . Wr^T, softmax, top-k and renormalised gates, fused in
// one kernel (hy-nomas-rs moe.rs:67-95).
//
// One block = 16 waves = one chunk of 64 rows.
//  - Logits.  bf16/f16 inputs: one v_mfma_f32_16x16x32 per 32 k (products
//    exact in f32, 32 of them summed in f32), the per-MFMA sums added in f64
//    in k order; the logit error is a few f32 ulps of a 32-term partial sum
//    (~1e-8 on unit-scale logits).  f32 inputs: f64 matrix products
//    (v_mfma_f64_16x16x4_f64, exact products, f64 sums).  Either way expert
//    choice is decided far below the 1e-6 logit near-tie threshold.
//  - Wave (g, q) computes rows 16g..16g+15 of the chunk against 16 NB experts
//    per pass over x (NB = 1, 2, 4 blocks of 16 for up to 16, 32, more
//    experts) over the q-th quarter of D; the four quarters are added into the
//    logit slots in a fixed order (q = 0, 1, 2, 3), so results do not depend
//    on timing.
//    Each lane loads 16 contiguous bytes of its row (and of its expert's
//    weights) per step and feeds them to consecutive MFMAs: the k index of
//    MFMA i, lane group lg is k0 + lg * EPC + i, the same assignment for both
//    operands, so the 4-deep MFMA k dimension reads whole 16-byte chunks.
//  - Selection: with E <= 16 four lanes take a row (waves 0-3, one per SIMD),
//    with E <= 64 sixteen lanes (all waves), each lane a share of the row's
//    experts, combined by xor shuffles; with more experts it is wave-parallel
//    over experts (max / sum / k rounds of argmax as xor-shuffle reductions
//    across the wave).  Ties go to the
//    lowest expert index, the reference's first-max-wins argmax (moe.rs:78-80).
//  - Gates: p = exp(l - max) / sum_E exp(l - max), w = p / (sum_selected p + 1e-9)
//    (moe.rs:68,92-95), evaluated in f64 and stored as f32.
//  - Output per row: k experts in ascending index with their gates, the
//    logit gap between the k-th selected and the best unselected expert, and
//    (block level) the chunk's per-expert histogram for the dispatch scan.
//    With a shared dense branch the row gets one more slot: expert E with
//    gate `dense_coef` (moe.rs:103-106 adds it after the experts).
//  The kernel reads x once (T*D*b bytes) and the router weights from L2.
#include "kernels.hpp"

#include <type_traits>

namespace nomas {

namespace {

constexpr int kRouterThreads = 1024;  // 16 waves
constexpr int kGroups = 4;            // row groups of 16 rows
constexpr int kParts = 4;             // quarters of D
constexpr int kRowsPerWave = kRouterRows / (kRouterThreads / kWave);
static_assert(kGroups * 16 == kRouterRows, "4 groups of 16 rows per chunk");
static_assert(kGroups * kParts * kWave == kRouterThreads, "one wave per (group, part)");

typedef double d4 __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

// v_mfma_f32_16x16x32_{bf16,f16} on raw 16-byte operands, C = 0: lane l gives
// row l % 16 of A (x) and column l % 16 of B (weights) at k 8 (l / 16) .. +7;
// the result lane l holds C[4 (l / 16) + r][l % 16], r = 0..3.
template <typename T> struct Mfma16;
template <> struct Mfma16<__bf16> {
    static __device__ __forceinline__ f32x4_t run(const uint4& a, const uint4& b) {
        bf16x8_t av, bv;
        __builtin_memcpy(&av, &a, 16);
        __builtin_memcpy(&bv, &b, 16);
        const f32x4_t z = {0.0f, 0.0f, 0.0f, 0.0f};
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, z, 0, 0, 0);
    }
};
template <> struct Mfma16<_Float16> {
    static __device__ __forceinline__ f32x4_t run(const uint4& a, const uint4& b) {
        f16x8_t av, bv;
        __builtin_memcpy(&av, &a, 16);
        __builtin_memcpy(&bv, &b, 16);
        const f32x4_t z = {0.0f, 0.0f, 0.0f, 0.0f};
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, z, 0, 0, 0);
    }
};
template <> struct Mfma16<float> {  // not used: f32 inputs take the f64 MFMAs
    static __device__ __forceinline__ f32x4_t run(const uint4&, const uint4&) { return {}; }
};

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

// LDS layout (bytes): logits [64][E] f64, counts [E + 1] int.
__host__ __device__ inline size_t router_lds(int E) {
    return sizeof(double) * (size_t)kRouterRows * E + sizeof(int) * (E + 1);
}

// Expert blocks of 16 per pass over x: every x chunk loaded feeds NB MFMAs.
// The ring depth shrinks as NB grows so the loads in flight fit the
// registers of 16 waves per CU.
template <typename T, int NB> struct RouterPass {
    static constexpr int kPre = NB == 1 ? 4 : (NB == 2 ? 3 : 2);
};

template <typename T, int NB>
__global__ __launch_bounds__(kRouterThreads) void router_kernel(
    const T* __restrict__ x, const T* __restrict__ wr, int64_t rows, int D, int E, int k,
    int k_slots, float dense_coef, int32_t* __restrict__ topk_idx, float* __restrict__ topk_w,
    float* __restrict__ gap, int32_t* __restrict__ chunk_counts) {
    extern __shared__ double s_logit[];                                   // [kRouterRows][E]
    int* s_cnt = reinterpret_cast<int*>(s_logit + (size_t)kRouterRows * E);  // [E + 1]
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int E_cols = E + (k_slots > k ? 1 : 0);
    for (int e = tid; e < E_cols; e += kRouterThreads) s_cnt[e] = 0;

    constexpr int EPC = 16 / sizeof(T);  // elements per 16-byte chunk = MFMAs per step
    constexpr int CK = 4 * EPC;          // k per step (4 lane groups)
    const int64_t chunk_row0 = (int64_t)blockIdx.x * kRouterRows;
    const int g = wave / kParts, q = wave % kParts;
    const int r16 = lane & 15, lg = lane >> 4;
    const int64_t row = chunk_row0 + g * 16 + r16;
    const bool row_ok = row < rows;
    const T* xr = x + (row_ok ? row : 0) * (int64_t)D;
    // this part's steps: a contiguous quarter of them
    const int nstep = (D + CK - 1) / CK;
    const int s0 = (int)((int64_t)nstep * q / kParts), s1 = (int)((int64_t)nstep * (q + 1) / kParts);

    // Loads run kPre steps ahead of the MFMAs (a ring of raw 16-byte chunks
    // in registers), so the memory latency of x is paid once per pipeline
    // fill, not once per step.
    constexpr int kPre = RouterPass<T, NB>::kPre;
    auto unpack = [](const uint4& raw, int i) -> double {
        Vec16<T> t;
        __builtin_memcpy(&t, &raw, 16);
        return (double)Elt<T>::to_f32(t.v[i]);
    };
    for (int e0 = 0; e0 < E; e0 += 16 * NB) {
        // Loads are unconditional from clamped addresses (a load whose address
        // or value is chosen by a condition becomes a flat load with a
        // scratch-resident zero); chunks past this part's steps or past D are
        // zeroed where they are used.  Rows past the end and experts past E
        // read row 0 / expert 0: their logits are never used.
        const T* wrr[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int ex = e0 + 16 * b + r16;
            wrr[b] = wr + (int64_t)(ex < E ? ex : 0) * D;
        }
        auto fetch = [&](int st, uint4& xa, uint4 (&wa)[NB]) {
            const int kk = min(max(min(st, s1 - 1), 0) * CK + lg * EPC, D - EPC);
            xa = *reinterpret_cast<const uint4*>(xr + kk);
#pragma unroll
            for (int b = 0; b < NB; ++b) wa[b] = *reinterpret_cast<const uint4*>(wrr[b] + kk);
        };
        auto live = [&](int st) { return st < s1 && st * CK + lg * EPC < D; };  // D % 8 == 0
        uint4 xb[kPre], wb[kPre][NB];
#pragma unroll
        for (int p = 0; p < kPre; ++p) fetch(s0 + p, xb[p], wb[p]);
        d4 c0[NB], c1[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            c0[b] = d4{0.0, 0.0, 0.0, 0.0};
            c1[b] = d4{0.0, 0.0, 0.0, 0.0};
        }
        // whole turns of the ring: steps past s1 are zeroed, which adds exactly 0
        for (int st0 = s0; st0 < s1; st0 += kPre) {
#pragma unroll
            for (int p = 0; p < kPre; ++p) {
                if (!live(st0 + p)) {
                    xb[p] = make_uint4(0, 0, 0, 0);
#pragma unroll
                    for (int b = 0; b < NB; ++b) wb[p][b] = make_uint4(0, 0, 0, 0);
                }
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    if constexpr (sizeof(T) == 2) {
                        // one 16x16x32 MFMA per step: the 32 products are exact
                        // in f32 and summed there; each step's sums join the f64
                        // accumulators in step order
                        const f32x4_t m = Mfma16<T>::run(xb[p], wb[p][b]);
#pragma unroll
                        for (int r = 0; r < 4; ++r) c0[b][r] += (double)m[r];
                    } else {
#pragma unroll
                        for (int i = 0; i < EPC; ++i) {
                            const double xd = unpack(xb[p], i), wd = unpack(wb[p][b], i);
                            if (i & 1) c1[b] = __builtin_amdgcn_mfma_f64_16x16x4f64(xd, wd, c1[b], 0, 0, 0);
                            else c0[b] = __builtin_amdgcn_mfma_f64_16x16x4f64(xd, wd, c0[b], 0, 0, 0);
                        }
                    }
                }
                fetch(st0 + p + kPre, xb[p], wb[p]);
            }
        }
        // lane holds expert column r16 of rows 4 lg + r (16-bit inputs) or
        // lg + 4 r (f32) of the group.  logit = ((p0 + p1) + p2) + p3: the
        // parts add into the logit slots one after another.
#pragma unroll
        for (int qq = 0; qq < kParts; ++qq) {
            if (q == qq) {
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    const int ex = e0 + 16 * b + r16;
                    if (ex >= E) continue;
                    const d4 c = sizeof(T) == 2 ? c0[b] : c0[b] + c1[b];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int i = sizeof(T) == 2 ? 4 * lg + r : lg + 4 * r;
                        double* dst = &s_logit[(g * 16 + i) * E + ex];
                        *dst = qq == 0 ? c[r] : *dst + c[r];
                    }
                }
            }
            __syncthreads();
        }
    }

    if (E <= kWave) {
        // L lanes per row (4 for up to 16 experts: waves 0-3, one per SIMD;
        // 16 above: all 16 waves): lane sub of a row's group takes experts
        // sub, sub + L, ...; max, sums and argmax combine over the group with
        // xor shuffles.
        auto select_rows = [&](auto lanes) {
            constexpr int L = decltype(lanes)::value;
            if (wave >= L) return;
            const int lr = tid / L, sub = tid % L;
            const int64_t orow = chunk_row0 + lr;
            const bool ok = orow < rows;  // lanes of missing rows still shuffle
            const double* lgt = s_logit + (ok ? lr : 0) * E;
            auto group_max = [](double v) {
#pragma unroll
                for (int o = 1; o < L; o <<= 1) v = fmax(v, __shfl_xor(v, o));
                return v;
            };
            auto group_sum = [](double v) {
#pragma unroll
                for (int o = 1; o < L; o <<= 1) v += __shfl_xor(v, o);
                return v;
            };
            double m = -INFINITY;
            for (int e = sub; e < E; e += L) m = fmax(m, lgt[e]);
            m = group_max(m);
            double s = 0.0;
            for (int e = sub; e < E; e += L) s += exp(lgt[e] - m);
            s = group_sum(s);
            uint64_t sel = 0;  // all selected experts of the row (every lane of the group)
            double kth = INFINITY;
            for (int it = 0; it < k; ++it) {
                double bv = 0.0;
                int bi = -1;
                for (int e = sub; e < E; e += L)
                    if (!((sel >> e) & 1ull) && (bi < 0 || lgt[e] > bv)) { bv = lgt[e]; bi = e; }
#pragma unroll
                for (int o = 1; o < L; o <<= 1) {  // first maximum wins: lowest index
                    const double ov = __shfl_xor(bv, o);
                    const int oi = __shfl_xor(bi, o);
                    if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) { bv = ov; bi = oi; }
                }
                sel |= 1ull << bi;
                kth = bv;
            }
            double best_un = -INFINITY, psel = 0.0;
            for (int e = sub; e < E; e += L) {
                if ((sel >> e) & 1ull) psel += exp(lgt[e] - m) / s;
                else best_un = fmax(best_un, lgt[e]);
            }
            best_un = group_max(best_un);
            psel = group_sum(psel);
            if (ok) {
                for (int e = sub; e < E; e += L) {
                    if (!((sel >> e) & 1ull)) continue;
                    const int rank = __popcll(sel & ((1ull << e) - 1ull));  // ascending index
                    const double p = exp(lgt[e] - m) / s;
                    topk_idx[orow * k_slots + rank] = e;
                    topk_w[orow * k_slots + rank] = (float)(p / (psel + 1e-9));
                    atomicAdd(&s_cnt[e], 1);
                }
                if (sub == 0) {
                    gap[orow] = (k == E) ? INFINITY : (float)(kth - best_un);
                    if (k_slots > k) {
                        topk_idx[orow * k_slots + k] = E;
                        topk_w[orow * k_slots + k] = dense_coef;
                        atomicAdd(&s_cnt[E], 1);
                    }
                }
            }
        };
        if (E <= 16) select_rows(std::integral_constant<int, 4>{});
        else select_rows(std::integral_constant<int, 16>{});
        __syncthreads();
        for (int e = tid; e < E_cols; e += kRouterThreads)
            chunk_counts[(int64_t)blockIdx.x * E_cols + e] = s_cnt[e];
        return;
    }
    const int per_lane = (E + kWave - 1) / kWave;  // experts per lane (<= 4 for E <= 256)
    for (int r = 0; r < kRowsPerWave; ++r) {
        const int lr = wave * kRowsPerWave + r;
        const int64_t orow = chunk_row0 + lr;
        if (orow >= rows) break;  // wave-uniform
        const double* lgt = s_logit + lr * E;
        double m = -INFINITY;
        for (int j = 0; j < per_lane; ++j) {
            const int e = lane + j * kWave;
            if (e < E) m = fmax(m, lgt[e]);
        }
        m = wave_max(m);
        double s = 0.0;
        for (int j = 0; j < per_lane; ++j) {
            const int e = lane + j * kWave;
            if (e < E) s += exp(lgt[e] - m);
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
                    const double lv = lgt[e];
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
            if ((sel >> j) & 1u) psel += exp(lgt[e] - m) / s;
            else best_un = fmax(best_un, lgt[e]);
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
                const double p = exp(lgt[e] - m) / s;
                topk_idx[orow * k_slots + rank] = e;
                topk_w[orow * k_slots + rank] = (float)(p / (psel + 1e-9));
                atomicAdd(&s_cnt[e], 1);
            }
            base += __popcll(bal);
        }
        if (lane == 0) {
            gap[orow] = (k == E) ? INFINITY : (float)(kth - best_un);
            if (k_slots > k) {
                topk_idx[orow * k_slots + k] = E;
                topk_w[orow * k_slots + k] = dense_coef;
                atomicAdd(&s_cnt[E], 1);
            }
        }
    }
    __syncthreads();
    for (int e = tid; e < E_cols; e += kRouterThreads)
        chunk_counts[(int64_t)blockIdx.x * E_cols + e] = s_cnt[e];
}

template <typename T, int NB>
hipError_t launch_router_nb(const RouterArgs& a, hipStream_t s, int nblk) {
    const size_t lds = router_lds(a.E);
    if (lds > 65536) {
        hipError_t err = hipFuncSetAttribute((const void*)router_kernel<T, NB>,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (err != hipSuccess) return err;
    }
    hipLaunchKernelGGL((router_kernel<T, NB>), dim3(nblk), dim3(kRouterThreads), lds, s,
                       (const T*)a.x, (const T*)a.wr, a.rows, a.D, a.E, a.k, a.k_slots,
                       a.dense_coef, a.topk_idx, a.topk_w, a.gap, a.chunk_counts);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_router_t(const RouterArgs& a, hipStream_t s) {
    const int nblk = (int)((a.rows + kRouterRows - 1) / kRouterRows);
    if (nblk == 0) return hipSuccess;
    // f32 inputs (f64 MFMAs, two accumulators per block) take one block per pass
    if constexpr (sizeof(T) == 4) {
        return launch_router_nb<T, 1>(a, s, nblk);
    } else {
        if (a.E <= 16) return launch_router_nb<T, 1>(a, s, nblk);
        if (a.E <= 32) return launch_router_nb<T, 2>(a, s, nblk);
        return launch_router_nb<T, 4>(a, s, nblk);
    }
}

}  // namespace

size_t router_lds_bytes(int E) { return router_lds(E); }

hipError_t launch_router(DType dt, const RouterArgs& a, hipStream_t s) {
    switch (dt) {
        case DType::F32: return launch_router_t<float>(a, s);
        case DType::BF16: return launch_router_t<__bf16>(a, s);
        case DType::F16: return launch_router_t<_Float16>(a, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace nomas
