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
#include "lds_dma.hpp"

#include <algorithm>
#include <type_traits>

namespace nomas {

namespace {

constexpr int kRouterThreads = 1024;  // 16 waves
constexpr int kGroups = 4;            // row groups of 16 rows
constexpr int kParts = 4;             // quarters of D
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

// Logit slots: [64][E + 1] f64 (rows padded by one slot, so that rows read at
// one expert index spread over the LDS banks).
__host__ __device__ inline int logit_ld(int E) { return E + 1; }

// LDS layout of router_kernel (bytes): logits [64][E + 1] f64, counts [E + 1] int.
__host__ __device__ inline size_t router_lds(int E) {
    return sizeof(double) * (size_t)kRouterRows * logit_ld(E) + sizeof(int) * (E + 1);
}

// Reductions over a quad of lanes (4 consecutive lanes) with DPP quad
// permutes: xor 1 = quad_perm [1,0,3,2] (0xB1), xor 2 = [2,3,0,1] (0x4E).
template <int CTRL>
__device__ __forceinline__ int quad_dpp(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ double quad_dpp(double v) {
    const int64_t b = __double_as_longlong(v);
    const int lo = quad_dpp<CTRL>((int)(b & 0xffffffff)), hi = quad_dpp<CTRL>((int)(b >> 32));
    return __longlong_as_double(((int64_t)hi << 32) | (uint32_t)lo);
}
__device__ __forceinline__ double quad_max(double v) {
    v = fmax(v, quad_dpp<0xB1>(v));
    return fmax(v, quad_dpp<0x4E>(v));
}
__device__ __forceinline__ double quad_sum(double v) {
    v += quad_dpp<0xB1>(v);  // (a + b) + (c + d): the same order in every lane of the quad
    return v + quad_dpp<0x4E>(v);
}
__device__ __forceinline__ double quad_min(double v) {
    v = fmin(v, quad_dpp<0xB1>(v));
    return fmin(v, quad_dpp<0x4E>(v));
}
// Reductions over a group of L = 4 or 8 consecutive lanes: the quad steps,
// then for 8 lanes one exchange with the other quad of the 8 (row_half_mirror:
// lane i and lane 7 - i).  Every lane of a quad holds the quad's value by
// then, so the exchange completes the reduction, and a sum's last add has
// the same two operands in both quads (the same value in all 8 lanes).
constexpr int kHalfMirror = 0x141;
template <int L>
__device__ __forceinline__ double grp_max(double v) {
    v = quad_max(v);
    if constexpr (L == 8) v = fmax(v, quad_dpp<kHalfMirror>(v));
    return v;
}
template <int L>
__device__ __forceinline__ double grp_min(double v) {
    v = quad_min(v);
    if constexpr (L == 8) v = fmin(v, quad_dpp<kHalfMirror>(v));
    return v;
}
template <int L>
__device__ __forceinline__ double grp_sum(double v) {
    v = quad_sum(v);
    if constexpr (L == 8) v += quad_dpp<kHalfMirror>(v);
    return v;
}

template <int L>
__device__ __forceinline__ uint32_t grp_maxu(uint32_t v) {
    v = max(v, (uint32_t)quad_dpp<0xB1>((int)v));
    v = max(v, (uint32_t)quad_dpp<0x4E>((int)v));
    if constexpr (L == 8) v = max(v, (uint32_t)quad_dpp<kHalfMirror>((int)v));
    return v;
}
template <int L>
__device__ __forceinline__ uint32_t grp_minu(uint32_t v) {
    v = min(v, (uint32_t)quad_dpp<0xB1>((int)v));
    v = min(v, (uint32_t)quad_dpp<0x4E>((int)v));
    if constexpr (L == 8) v = min(v, (uint32_t)quad_dpp<kHalfMirror>((int)v));
    return v;
}

// The quad's best (value, index): the larger value, and the lower index of
// equal values (-1 = none).
template <int L>
__device__ __forceinline__ void grp_argmax(double& bv, int& bi) {
    auto step = [&](double ov, int oi) {
        if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) { bv = ov; bi = oi; }
    };
    step(quad_dpp<0xB1>(bv), quad_dpp<0xB1>(bi));
    step(quad_dpp<0x4E>(bv), quad_dpp<0x4E>(bi));
    if constexpr (L == 8) step(quad_dpp<kHalfMirror>(bv), quad_dpp<kHalfMirror>(bi));
}

// k rounds of argmax over a row held by a group of L lanes (lane sub: experts sub + L j,
// bit j of `valid` set where that expert exists) on the f64 logits, the first
// maximum winning (the lowest index among equal values).  Returns this lane's
// chosen experts as bits j.
template <int PL, int L>
__device__ __forceinline__ uint32_t argmax_rounds(const double (&lv)[PL], uint32_t valid, int k,
                                                  int sub) {
    uint32_t mine = 0;
    for (int it = 0; it < k; ++it) {
        const uint32_t open = valid & ~mine;
        double bv = 0.0;
        int bi = -1;
#pragma unroll
        for (int j = 0; j < PL; ++j)
            if (((open >> j) & 1u) && (bi < 0 || lv[j] > bv)) { bv = lv[j]; bi = sub + j * L; }
        grp_argmax<L>(bv, bi);
        if (bi >= 0 && bi % L == sub) mine |= 1u << (bi / L);
    }
    return mine;
}

// The same choice (up to 64 experts) on one 32-bit key per candidate: the
// logit rounded to f32, its bits made to order as unsigned integers, the low
// 6 bits replaced by 63 - expert.  A larger key is a larger value, or of
// values equal to 17 significant bits ("truncated") the lower expert; a round
// is a max over the lane's keys and the group's, and the winner's key is
// cleared.  f64 -> f32 rounding and the truncation keep the order of unequal
// values (not strictly), so with T the smallest truncated value chosen, every
// candidate above T is in the f64 choice and every one below T is not.  Those
// equal to T (when one of them was left out) are settled on their f64
// logits: argmax_rounds over just them for the places left.
template <int L>
__device__ __forceinline__ int grp_sumi(int v) {
    v += quad_dpp<0xB1>(v);
    v += quad_dpp<0x4E>(v);
    if constexpr (L == 8) v += quad_dpp<kHalfMirror>(v);
    return v;
}
template <int PL, int L>
__device__ __forceinline__ uint32_t argmax_keys(const double (&lv)[PL], uint32_t valid, int k,
                                                int sub) {
    uint32_t key[PL], trunc[PL];
#pragma unroll
    for (int j = 0; j < PL; ++j) {
        const uint32_t b = __float_as_uint((float)lv[j]);
        const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
        key[j] = (valid >> j) & 1u ? (o & ~63u) | (uint32_t)(63 - (sub + j * L)) : 0u;
        trunc[j] = o >> 6;
    }
    // (keys are distinct, so each round clears one; with at least k experts
    // a round's maximum is never 0)
    for (int it = 0; it < k; ++it) {
        uint32_t m = 0;
#pragma unroll
        for (int j = 0; j < PL; ++j) m = max(m, key[j]);
        m = grp_maxu<L>(m);
#pragma unroll
        for (int j = 0; j < PL; ++j) key[j] = key[j] == m ? 0u : key[j];
    }
    uint32_t mine = 0;  // the valid experts whose keys were cleared
#pragma unroll
    for (int j = 0; j < PL; ++j) mine |= (key[j] == 0 ? 1u : 0u) << j;
    mine &= valid;
    uint32_t kth = ~0u, un = 0;
#pragma unroll
    for (int j = 0; j < PL; ++j) {
        if ((mine >> j) & 1u) kth = min(kth, trunc[j]);
        else if ((valid >> j) & 1u) un = max(un, trunc[j]);
    }
    kth = grp_minu<L>(kth);
    if (kth > grp_maxu<L>(un)) return mine;  // (uniform over the group)
    uint32_t sure = 0, tied = 0;
#pragma unroll
    for (int j = 0; j < PL; ++j) {
        sure |= (((mine >> j) & 1u) && trunc[j] > kth ? 1u : 0u) << j;
        tied |= (((valid >> j) & 1u) && trunc[j] == kth ? 1u : 0u) << j;
    }
    const int left = k - grp_sumi<L>(__popc(sure));
    return sure | argmax_rounds<PL, L>(lv, tied, left, sub);
}

// OR of a 64-bit mask over a group of L lanes.
template <int L>
__device__ __forceinline__ uint64_t grp_or(uint64_t v) {
    auto step = [&](auto ctrl) {
        constexpr int C = decltype(ctrl)::value;
        const uint32_t lo = (uint32_t)quad_dpp<C>((int)(uint32_t)v);
        const uint32_t hi = (uint32_t)quad_dpp<C>((int)(uint32_t)(v >> 32));
        v |= ((uint64_t)hi << 32) | lo;
    };
    step(std::integral_constant<int, 0xB1>{});
    step(std::integral_constant<int, 0x4E>{});
    if constexpr (L == 8) step(std::integral_constant<int, kHalfMirror>{});
    return v;
}

// Selection for one block of RR rows from its f64 logits (block of NT
// threads; every thread calls it): softmax, k rounds of argmax (ties to the
// lowest index), gates p / (sum_sel p + 1e-9), the k-th/best-unselected logit
// gap, the dense slot, and the block's histogram (s_cnt, zeroed by the
// caller, written to counts_out).  The logits come in NP partial slot sets
// [NP][RR][logit_ld(E)] at s_logit, summed in part order.
template <int NT, int NP = 1, int RR = kRouterRows>
__device__ __forceinline__ void select_chunk(const double* s_logit, int* s_cnt, int64_t chunk_row0,
                                             int64_t rows, int E, int k, int k_slots,
                                             float dense_coef, int32_t* __restrict__ topk_idx,
                                             float* __restrict__ topk_w, float* __restrict__ gap,
                                             int32_t* __restrict__ counts_out) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int E_cols = E + (k_slots > k ? 1 : 0);
    const int part_stride = RR * logit_ld(E);
    if (E <= kWave) {
        // L lanes per row (a DPP quad, or two in blocks of 512 threads or
        // more): lane sub holds experts sub, sub + L, ... (at most PL) and
        // their logits in registers; max, sums and argmax combine over the
        // group with DPP permutes (xor 1, xor 2 and, for 8 lanes, the half-row
        // mirror).  The RR rows take RR L lanes: one pass of the block, whole
        // waves idle past them.
        // Eight lanes per row halve each lane's dependent chain, and the two
        // waves per SIMD of a 512-thread block hide each other's latencies.
        auto select_rows = [&](auto per_lane, auto lanes) {
            constexpr int PL = decltype(per_lane)::value;
            constexpr int L = decltype(lanes)::value;
            if (tid >= RR * L) return;  // whole waves
            const int lr = tid / L, sub = tid % L;
            const int64_t orow = chunk_row0 + lr;
            const bool ok = orow < rows;  // lanes of missing rows still take part
            const double* lgt = s_logit + (ok ? lr : 0) * logit_ld(E);
            double lv[PL];
            uint32_t valid = 0;  // bit j: expert sub + L j exists
#pragma unroll
            for (int j = 0; j < PL; ++j) {
                const int e = sub + j * L;
                double v = -INFINITY;
                if (e < E) {
                    v = lgt[e];
#pragma unroll
                    for (int p = 1; p < NP; ++p) v += lgt[p * part_stride + e];
                    valid |= 1u << j;
                }
                lv[j] = v;
            }
            double m = -INFINITY;
#pragma unroll
            for (int j = 0; j < PL; ++j) m = fmax(m, lv[j]);
            m = grp_max<L>(m);
            // exp(l - m) once per expert, in f32 (the difference is taken in
            // f64): the gates carry about 1e-7 of relative error from it, the
            // expert choice none (it compares the logits)
            float pe[PL];
            double s = 0.0;
#pragma unroll
            for (int j = 0; j < PL; ++j) {
                pe[j] = (valid >> j) & 1u ? expf((float)(lv[j] - m)) : 0.0f;
                s += (double)pe[j];
            }
            s = grp_sum<L>(s);
            // k rounds of argmax on 32-bit keys of the logits; where the k-th
            // and best unchosen logits are within the keys' resolution (about
            // 8e-6 relative), the f64 logits settle the candidates in between
            const uint32_t mine = argmax_keys<PL, L>(lv, valid, k, sub);  // bit j: chosen
            const double inv_s = 1.0 / s;
            double kth = INFINITY, best_un = -INFINITY, psel = 0.0;
            uint64_t sel = 0;  // the row's chosen experts (after the OR over the quad)
#pragma unroll
            for (int j = 0; j < PL; ++j) {
                const bool chosen = (mine >> j) & 1u;
                psel += chosen ? (double)pe[j] * inv_s : 0.0;
                kth = chosen ? fmin(kth, lv[j]) : kth;
                best_un = (!chosen && ((valid >> j) & 1u)) ? fmax(best_un, lv[j]) : best_un;
                sel |= chosen ? 1ull << (sub + j * L) : 0ull;
            }
            kth = grp_min<L>(kth);
            best_un = grp_max<L>(best_un);
            psel = grp_sum<L>(psel);
            sel = grp_or<L>(sel);
            if (ok) {
                const double inv_norm = 1.0 / (psel + 1e-9);
#pragma unroll
                for (int j = 0; j < PL; ++j) {
                    if (!((mine >> j) & 1u)) continue;
                    const int e = sub + j * L;
                    const int rank = __popcll(sel & ((1ull << e) - 1ull));  // ascending index
                    topk_idx[orow * k_slots + rank] = e;
                    topk_w[orow * k_slots + rank] = (float)((double)pe[j] * inv_s * inv_norm);
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
        if constexpr (NT >= 8 * RR) {
            using L8 = std::integral_constant<int, 8>;
            if (E <= 16) select_rows(std::integral_constant<int, 2>{}, L8{});
            else select_rows(std::integral_constant<int, 8>{}, L8{});
        } else {
            using L4 = std::integral_constant<int, 4>;
            if (E <= 16) select_rows(std::integral_constant<int, 4>{}, L4{});
            else select_rows(std::integral_constant<int, 16>{}, L4{});
        }
        __syncthreads();
        for (int e = tid; e < E_cols; e += NT) counts_out[e] = s_cnt[e];
        return;
    }
    constexpr int kRowsPerWave = RR / (NT / kWave);
    static_assert(kRowsPerWave * (NT / kWave) == RR, "whole rows per wave");
    const int per_lane = (E + kWave - 1) / kWave;  // experts per lane (<= 4 for E <= 256)
    for (int r = 0; r < kRowsPerWave; ++r) {
        const int lr = wave * kRowsPerWave + r;
        const int64_t orow = chunk_row0 + lr;
        if (orow >= rows) break;  // wave-uniform
        const double* lgt = s_logit + lr * logit_ld(E);  // (NP == 1 on this path)
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
    for (int e = tid; e < E_cols; e += NT) counts_out[e] = s_cnt[e];
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
    int* s_cnt = reinterpret_cast<int*>(s_logit + (size_t)kRouterRows * logit_ld(E));  // [E + 1]
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
                        double* dst = &s_logit[(g * 16 + i) * logit_ld(E) + ex];
                        *dst = qq == 0 ? c[r] : *dst + c[r];
                    }
                }
            }
            __syncthreads();
        }
    }

    select_chunk<kRouterThreads>(s_logit, s_cnt, chunk_row0, rows, E, k, k_slots, dense_coef,
                                 topk_idx, topk_w, gap, chunk_counts + (int64_t)blockIdx.x * E_cols);
}


// ---- LDS-staged logits: 16-bit inputs, up to 64 experts, D % 128 == 0 -------
//
// One block = 8 waves = RR rows (64 or 32; the histogram it writes covers its
// RR rows).  Waves 0-3 compute the logits and load the router weights;
// waves 4-7 only load x (they take the same barriers).  The selection runs on
// 8 lanes per row.
//  - The x bytes in flight bound the kernel: a block has NST - 1 stages of
//    its rows in flight, so fewer rows per block with a deeper ring keep more
//    bytes in flight when the rows alone would leave CUs idle (the plan is
//    chosen per launch, router_plan).
//  - x and the router weights stream through an LDS ring of kStages stages,
//    each 128 elements (256 bytes) of every row of the chunk and of every
//    expert row.  One direct-to-LDS load fetches 1 KB: four whole 256-byte
//    row slices, so every HBM line is fetched whole by one instruction.  The
//    16 chunks of 16 bytes of a slice are stored XOR-swizzled by row bits 0-2
//    (applied on the global side: lane l always fills slot l), so the 16-row
//    operand reads of the MFMAs (ds_read_b128) hit distinct banks.
//  - Compute wave w takes expert group eg = w % NEG (16 experts) and k part
//    kp = w / NEG (every NKP-th k step of 32, NKP = 4 / NEG) for all 64 rows:
//    per k step it reads one weight fragment and four x fragments and runs
//    four v_mfma_f32_16x16x32 (x as A: lane (r, g) row r, k 8g..8g+7 of the
//    step; the weights as B with the same k).  Each weight byte of a stage is
//    read by one wave only, each x byte by NEG waves.
//  - The MFMA accumulators chain kChain k steps (128 products) in f32 before
//    each joins an f64 accumulator: the products are exact, each chained
//    rounding is at most half an ulp of a ~128-term partial sum, so a logit
//    carries a few 1e-8 of error at unit scale -- far below the 1e-6 near-tie
//    window that expert choice is checked against.
//  - The k parts are added into the f64 logit slots in part order (the slots
//    reuse the ring), then the shared selection runs.
constexpr int kLdsComputeWaves = 4;
constexpr int kLdsThreads = 2 * kLdsComputeWaves * kWave;  // + 4 waves that load x
constexpr int kChain = 4;           // k steps accumulated in f32 per f64 add
constexpr int kLdsMaxExperts = 64;

// ROWB bytes of each row per stage, NST stages in the ring, RR rows per block
template <typename T, int NEG, int ROWB, int NST, int RR>
__global__ __launch_bounds__(kLdsThreads) void router_lds_kernel(
    const T* __restrict__ x, const T* __restrict__ wr, int64_t rows, int D, int E, int k,
    int k_slots, float dense_coef, int32_t* __restrict__ topk_idx, float* __restrict__ topk_w,
    float* __restrict__ gap, int32_t* __restrict__ chunk_counts) {
    static_assert(sizeof(T) == 2, "16-bit inputs");
    constexpr int EPC = 8;                         // elements per 16-byte chunk
    constexpr int CPR = ROWB / 16;                 // 16-byte chunks per row slice
    constexpr int KS = CPR * EPC;                  // elements per stage
    constexpr int RPI = 1024 / ROWB;               // rows per 1 KB load
    constexpr int NKP = 4 / NEG;                   // k parts
    constexpr int EP = 16 * NEG;                   // experts, padded to whole groups
    constexpr int NRG = RR / 16;                   // row groups of 16
    constexpr int XB = RR * ROWB;                  // x bytes per stage
    constexpr int SB = XB + EP * ROWB;             // stage bytes
    constexpr int QX = RR / RPI / 4;               // x loads per loading wave per stage
    constexpr int QW = EP / RPI / 4;               // weight loads per compute wave per stage
    constexpr int KPW = CPR / 4 / NKP;             // this wave's k steps per stage
    constexpr int kRing = NST * SB;
    static_assert(CPR >= 8 && QX >= 1 && QW >= 1 && KPW >= 1, "stage shape");
    static_assert(NKP * RR * (16 * NEG + 1) * sizeof(double) <= (size_t)kRing,
                  "the k parts' logit slots fit in the ring");
    static_assert(RR % 16 == 0 && RR <= kRouterRows && kRouterRows % RR == 0, "row groups of 16");
    __shared__ __attribute__((aligned(16))) unsigned char sRing[kRing];
    __shared__ int s_cnt[kLdsMaxExperts + 1];
    double* const s_logit = reinterpret_cast<double*>(sRing);  // after the k loop

    const int tid = threadIdx.x, lane = tid & 63;
    // waves 0-3 compute (and load the weights), waves 4-7 load x; `wave`
    // numbers each kind 0-3
    const int wave_all = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool x_loader = wave_all >= kLdsComputeWaves;
    const int wave = x_loader ? wave_all - kLdsComputeWaves : wave_all;
    const int eg = wave % NEG, kp = wave / NEG;
    const int r16 = lane & 15, g = lane >> 4;
    const int E_cols = E + (k_slots > k ? 1 : 0);
    for (int e = tid; e < E_cols; e += kLdsThreads) s_cnt[e] = 0;
    __syncthreads();  // (before any load is in flight: this barrier may wait for all)
    const int64_t chunk_row0 = (int64_t)blockIdx.x * RR;
    const int nvalid = (int)min<int64_t>(RR, rows - chunk_row0);
    const int nstage = D / KS;

    // Load q of a stage fills LDS bytes [q * 1 KB, +1 KB): rows RPI q ..
    // RPI q + RPI - 1, lane l row RPI q + l / CPR, slot l % CPR holding
    // logical chunk (l % CPR) ^ (row & 7).  Rows past the chunk re-read its last row, expert
    // rows past E the last expert (never used).  Byte offsets from the
    // stage's base (the chunk's first row / expert 0 at that k).
    uint32_t xoff[QX], woff[QW];
#pragma unroll
    for (int i = 0; i < QX; ++i) {
        const int r = (wave * QX + i) * RPI + lane / CPR;
        const int rr = min(r, nvalid - 1);
        xoff[i] = (uint32_t)(((int64_t)rr * D + (((lane % CPR) ^ (r & 7)) * EPC)) * 2);
    }
#pragma unroll
    for (int i = 0; i < QW; ++i) {
        const int r = (wave * QW + i) * RPI + lane / CPR;
        const int rr = min(r, E - 1);
        woff[i] = (uint32_t)(((int64_t)rr * D + (((lane % CPR) ^ (r & 7)) * EPC)) * 2);
    }
    const T* const xc = x + chunk_row0 * D;
    const uint32_t ring = lds_addr(sRing);
    auto issue = [&](int st, int slot) {  // this wave's loads of stage st
        const int sc = min(st, nstage - 1);  // past the end: re-load the last stage
        const uint32_t base = ring + slot * SB;
        if (x_loader) {
#pragma unroll
            for (int i = 0; i < QX; ++i)
                lds_dma16(xc + sc * KS, xoff[i], base + (wave * QX + i) * 1024);
        } else {
            // weight rows past E (the expert group's padding) are not loaded:
            // their LDS rows feed only MFMA columns that are never read
#pragma unroll
            for (int i = 0; i < QW; ++i)
                if ((wave * QW + i) * RPI < E)
                    lds_dma16(wr + sc * KS, woff[i], base + XB + (wave * QW + i) * 1024);
        }
    };
    // operand fragment: row `row` of a region, logical chunk c
    auto frag = [&](int slot, int region, int row, int c) -> uint4 {
        return *reinterpret_cast<const uint4*>(sRing + slot * SB + region + row * ROWB +
                                              ((c ^ (row & 7)) * 16));
    };

    typedef float f4 __attribute__((ext_vector_type(4)));
    f4 acc[NRG];
    d4 acc64[NRG];
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
        acc[rg] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        acc64[rg] = d4{0.0, 0.0, 0.0, 0.0};
    }
    auto flush = [&]() {
#pragma unroll
        for (int rg = 0; rg < NRG; ++rg) {
#pragma unroll
            for (int i = 0; i < 4; ++i) acc64[rg][i] += (double)acc[rg][i];
            acc[rg] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    };
#pragma unroll
    for (int p = 0; p < NST - 1; ++p) issue(p, p);
    if (x_loader) {
        // the compute waves' loop without the compute: the same waits and
        // barriers, so the ring turns in step
        for (int s = 0; s < nstage; ++s) {
            __builtin_amdgcn_sched_barrier(0);
            wait_vmcnt<(NST - 2) * QX>();
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            issue(s + NST - 1, (s + NST - 1) % NST);
        }
    } else
    for (int s = 0; s < nstage; ++s) {
        // this wave's loads of stage s have landed; after the bare barrier
        // everyone's have, and every wave is done reading stage s - 1 (whose
        // slot the next load refills).  __syncthreads() would also wait for
        // the later stages' loads.
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<(NST - 2) * QW>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        issue(s + NST - 1, (s + NST - 1) % NST);
        const int slot = s % NST;
#pragma unroll
        for (int jj = 0; jj < KPW; ++jj) {  // this wave's k steps of the stage
            const int j = kp + jj * NKP;
            const uint4 wf = frag(slot, XB, eg * 16 + r16, 4 * j + g);
#pragma unroll
            for (int rg = 0; rg < NRG; ++rg) {
                const uint4 xf = frag(slot, 0, rg * 16 + r16, 4 * j + g);
                typename std::conditional<std::is_same<T, __bf16>::value, bf16x8_t, f16x8_t>::type
                    av, bv;
                __builtin_memcpy(&av, &xf, 16);
                __builtin_memcpy(&bv, &wf, 16);
                if constexpr (std::is_same<T, __bf16>::value)
                    acc[rg] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc[rg], 0, 0, 0);
                else
                    acc[rg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc[rg], 0, 0, 0);
            }
            // every kChain of this wave's k steps join the f64 accumulators
            if constexpr (KPW >= kChain) {
                if ((jj + 1) % kChain == 0) flush();
            }
        }
        if constexpr (KPW < kChain) {
            if ((s + 1) % (kChain / KPW) == 0) flush();
        }
    }
    flush();  // the last, partial chain (a no-op add of zeros otherwise)
    wait_vmcnt<0>();  // the trailing re-loads, before the ring becomes the logit slots
    __syncthreads();
    // lane (r16, g) holds expert eg * 16 + r16 of rows rg * 16 + 4 g + i; each
    // k part fills its own slot set, which the selection adds in part order
    const int ex = eg * 16 + r16;
    if (!x_loader && ex < E) {
        double* part = s_logit + kp * (RR * logit_ld(E));
#pragma unroll
        for (int rg = 0; rg < NRG; ++rg)
#pragma unroll
            for (int i = 0; i < 4; ++i) part[(rg * 16 + 4 * g + i) * logit_ld(E) + ex] = acc64[rg][i];
    }
    __syncthreads();
    select_chunk<kLdsThreads, NKP, RR>(s_logit, s_cnt, chunk_row0, rows, E, k, k_slots, dense_coef,
                                       topk_idx, topk_w, gap,
                                       chunk_counts + (int64_t)blockIdx.x * E_cols);
}

template <typename T, int NB>
hipError_t launch_router_nb(const RouterArgs& a, hipStream_t s, int nblk) {
    const size_t lds = router_lds(a.E);
    if (lds > 65536) {
        hipError_t err = hipFuncSetAttribute((const void*)router_kernel<T, NB>,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (err != hipSuccess) return err;
    }
    launch_kernel((router_kernel<T, NB>), dim3(nblk), dim3(kRouterThreads), lds, s,
                  (const T*)a.x, (const T*)a.wr, a.rows, a.D, a.E, a.k, a.k_slots,
                  a.dense_coef, a.topk_idx, a.topk_w, a.gap, a.chunk_counts);
    return hipGetLastError();
}

// The LDS router's shape for a launch: RR rows per block and a ring of NST
// stages.  What bounds the stream is the x bytes the blocks have in flight
// together (NST - 1 stages of RR rows each): a block has at most one 64-row
// chunk's 4-stage ring in flight, and 64-row chunks fill the CUs only from
// 16,384 rows on.
//  - Up to 8,192 rows and 32 experts: 32-row blocks with the deepest ring one
//    block per CU holds (12 stages at 16 experts: 88 KB of x in flight, 5.5
//    times a 64-row block's).  One 4,680-row segment at 8 experts: 13.3 ->
//    10.1 us.  Past 256 such blocks the dispatch's bookkeeping needs a second
//    round trip over the histograms (+5 us at 14,232 rows against 0.6 us
//    saved here), and with more than 32 experts a stage's weight slices
//    outweigh a 32-row x slice (64 experts, 16,384 rows: 27.3 -> 29.6 us).
//  - Otherwise 64-row blocks and a 4-stage ring.
struct RouterPlan {
    int rr, nst;
};

constexpr int kRouterLdsBytes = 152 * 1024;  // ring budget of one block per CU
constexpr int kRouterSmallRows = 8192;       // 32-row blocks up to here

// Stage bytes of NEG expert groups and RR rows (256-byte row slices).
constexpr int router_stage_bytes(int rr, int neg) { return (rr + 16 * neg) * 256; }
// The deepest ring of RR-row blocks one block per CU holds.
constexpr int router_ring(int rr, int neg) {
    return std::min(12, kRouterLdsBytes / router_stage_bytes(rr, neg));
}

RouterPlan router_plan(int64_t rows, int E) {
    const int neg = E <= 16 ? 1 : (E <= 32 ? 2 : 4);
    if (rows <= kRouterSmallRows && neg < 4) return {32, router_ring(32, neg)};
    return {64, std::min(4, router_ring(64, neg))};
}

template <typename T, int NEG, int RR, int NST>
hipError_t launch_router_lds_rr(const RouterArgs& a, hipStream_t s) {
    constexpr int ROWB = 256;
    static_assert(NST * router_stage_bytes(RR, NEG) <= kRouterLdsBytes, "the ring fits");
    const int nblk = (int)((a.rows + RR - 1) / RR);
    launch_kernel((router_lds_kernel<T, NEG, ROWB, NST, RR>), dim3(nblk), dim3(kLdsThreads), 0, s,
                  (const T*)a.x, (const T*)a.wr, a.rows, a.D, a.E, a.k, a.k_slots,
                  a.dense_coef, a.topk_idx, a.topk_w, a.gap, a.chunk_counts);
    return hipGetLastError();
}

// The shapes router_plan can ask for at each NEG.
template <typename T, int NEG>
hipError_t launch_router_lds(const RouterArgs& a, hipStream_t s, const RouterPlan& p) {
    constexpr int d64 = std::min(4, router_ring(64, NEG));
    if (p.rr == 64 && p.nst == d64) return launch_router_lds_rr<T, NEG, 64, d64>(a, s);
    if constexpr (NEG < 4) {
        constexpr int d32 = router_ring(32, NEG);
        if (p.rr == 32 && p.nst == d32) return launch_router_lds_rr<T, NEG, 32, d32>(a, s);
    }
    return hipErrorInvalidValue;
}

// Whether a launch takes the LDS router (16-bit inputs, up to 64 experts,
// D % 128 == 0).
bool router_lds_applies(DType dt, int D, int E) {
    return dt != DType::F32 && E <= kLdsMaxExperts && D % 128 == 0;
}

template <typename T>
hipError_t launch_router_t(const RouterArgs& a, hipStream_t s) {
    if (a.rows <= 0) return hipSuccess;
    // f32 inputs (f64 MFMAs, two accumulators per block) take one block per pass
    if constexpr (sizeof(T) == 4) {
        if (a.block_rows != kRouterRows) return hipErrorInvalidValue;
        return launch_router_nb<T, 1>(a, s, (int)((a.rows + kRouterRows - 1) / kRouterRows));
    } else {
        // LDS-staged logits where they apply (up to 64 experts, D % 128 == 0)
        if (a.E <= kLdsMaxExperts && a.D % 128 == 0) {
            const RouterPlan p = router_plan(a.rows, a.E);
            if (a.block_rows != p.rr) return hipErrorInvalidValue;
            if (a.E <= 16) return launch_router_lds<T, 1>(a, s, p);
            if (a.E <= 32) return launch_router_lds<T, 2>(a, s, p);
            return launch_router_lds<T, 4>(a, s, p);
        }
        if (a.block_rows != kRouterRows) return hipErrorInvalidValue;
        const int nblk = (int)((a.rows + kRouterRows - 1) / kRouterRows);
        if (a.E <= 16) return launch_router_nb<T, 1>(a, s, nblk);
        if (a.E <= 32) return launch_router_nb<T, 2>(a, s, nblk);
        return launch_router_nb<T, 4>(a, s, nblk);
    }
}

}  // namespace

size_t router_lds_bytes(int E) { return router_lds(E); }

int router_block_rows(DType dt, int64_t rows, int D, int E) {
    return router_lds_applies(dt, D, E) ? router_plan(rows, E).rr : kRouterRows;
}

hipError_t launch_router(DType dt, const RouterArgs& a, hipStream_t s) {
    switch (dt) {
        case DType::F32: return launch_router_t<float>(a, s);
        case DType::BF16: return launch_router_t<__bf16>(a, s);
        case DType::F16: return launch_router_t<_Float16>(a, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace nomas
