// Grouped expert GEMMs on CDNA4 matrix cores (bf16 / f16 in, f32 accumulate).
//
// Problem per expert e (rows of x_perm / h that belong to e):
//   gate/up:  h[m, :] = silu(x W_gate^T + b_gate) * (x W_up^T + b_up)   K = D, N = 2H
//   down:     y[m, :] = h W_down^T + b_down                              K = H, N = D
// (hy-nomas-rs mlp.rs:42-46 applied to the rows routed to e).
//
// Work unit: a BM x BN output tile of one expert.  The scan kernel lists the
// experts' BM-row tiles; the grid enumerates (row tile, column tile) pairs.
//  - Operands: weights are the MFMA "A" operand (rows = output columns),
//    token rows the "B" operand, so each lane's accumulator holds 4
//    consecutive output columns of one token row (8-byte stores).
//  - v_mfma_f32_32x32x16_{bf16,f16}; 4 waves in a 2 x 2 grid, each wave a
//    (BN/2) x (BM/2) tile of 32 x 32 MFMA blocks (256 f32 accumulators per
//    lane for 256 x 256 tiles, held in AGPRs).
//  - K is walked in BK-wide steps through a ring of S LDS stages filled by
//    direct global->LDS loads (global_load_lds_dwordx4: no VGPR staging).
//    Loads run S-1 steps ahead of the MFMAs; each step waits only for its own
//    stage (partial vmcnt) and synchronises the block once.
//  - Operands are K-blocked in memory (kernels.hpp): one k step of a tile is a
//    single contiguous 16 KB run, fetched as whole 128-byte lines.
//  - LDS rows (BK * 2 bytes) keep their 16-byte chunks XOR-swizzled, so the
//    32-row MFMA operand reads (ds_read_b128) are free of bank conflicts.  The
//    swizzle is applied on the global side: lane l of a load instruction always
//    writes LDS slot l, and reads the global chunk that belongs there.
//  - Gate and up rows are interleaved in groups of 32 when the weights are
//    packed (rows 64g..64g+31 = gate 32g.., rows 64g+32.. = up 32g..), so a
//    wave holds gate and up of the same hidden unit in the same lane and the
//    SwiGLU is applied in the epilogue without an extra pass over HBM.
//  - Block ids are mapped to tiles XCD-aware (tile_map.hpp): the XCDs work on
//    one expert at a time (its weights shared through the MALL), each XCD on a
//    4 x 8 group of tiles that share panels in its own L2.
#include "kernels.hpp"
#include "tile_map.hpp"

namespace nomas {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

template <typename T> struct Mfma;
template <> struct Mfma<__bf16> {
    typedef bf16x8_t V;
    static __device__ __forceinline__ f32x16_t run(V a, V b, f32x16_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};
template <> struct Mfma<_Float16> {
    typedef f16x8_t V;
    static __device__ __forceinline__ f32x16_t run(V a, V b, f32x16_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

enum { kGateUp = 0, kDown = 1 };

constexpr int kThreads = 256;
constexpr int kBK = 32;     // k step
constexpr int kStages = 4;  // LDS ring depth

// Physical 16-byte chunk of logical chunk c in LDS row r (CH chunks per row).
template <int CH>
__device__ __forceinline__ int swz(int r) {
    if constexpr (CH == 8) return (r ^ (r >> 3)) & 7;
    else return ((r >> 1) ^ (r >> 3)) & 3;
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Direct global->LDS load of 16 bytes per lane from sbase + voff (a uniform
// 64-bit base in SGPRs plus a per-lane 32-bit byte offset): lane l's bytes
// land at LDS address lds_base + 16 * l (global_load_lds_dwordx4, M0 = LDS
// base; one wait state between the M0 write and the load).  Issued as inline
// assembly so the compiler does not track it: completion is waited for
// explicitly with wait_vmcnt, and nothing else in these kernels uses M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // M0 is clobbered on purpose, see above
__device__ __forceinline__ void lds_dma16(const void* sbase, uint32_t voff, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(sbase), "s"(lds_base)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

template <typename P>
__device__ __forceinline__ uint32_t lds_addr(P* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

template <typename T, int MODE, int BM, int BN, int BK, int S>
__global__ __launch_bounds__(kThreads, 1) void gemm_mfma_kernel(GemmArgs a) {
    using V = typename Mfma<T>::V;
    constexpr int WM = BM / 2, WN = BN / 2;       // wave tile: token rows x weight rows
    constexpr int SM = WM / 32, SN = WN / 32;     // 32x32 MFMA blocks per wave
    constexpr int CH = BK / 8;                    // 16-byte chunks per LDS row
    constexpr int RPI = kWave / CH;               // rows filled by one load instruction
    constexpr int NW = kThreads / kWave;
    constexpr int QW = BN / RPI / NW;             // load instructions per wave per k step
    constexpr int QX = BM / RPI / NW;
    constexpr int Q = QW + QX;
    static_assert(MODE == kDown || SN % 2 == 0, "gate/up pairs need an even block count");
    static_assert(S >= 3 && S <= 5, "ring depth");
    static_assert((S - 2) * Q <= 63, "vmcnt range");
    static_assert(BK == kKBlock, "operands are K-blocked by the k step");

    // One LDS object per stage: the compiler then knows a stage being read is
    // not the target of the loads in flight, and inserts no vmcnt(0) before
    // the reads.  Stage indices are compile-time after unrolling.
    __shared__ __attribute__((aligned(16))) T sW0[BN * BK], sW1[BN * BK], sW2[BN * BK],
        sW3[S > 3 ? BN * BK : 8], sW4[S > 4 ? BN * BK : 8];
    __shared__ __attribute__((aligned(16))) T sX0[BM * BK], sX1[BM * BK], sX2[BM * BK],
        sX3[S > 3 ? BM * BK : 8], sX4[S > 4 ? BM * BK : 8];
    auto stW = [&](int s) -> T* {
        return s == 0 ? sW0 : s == 1 ? sW1 : s == 2 ? sW2 : s == 3 ? sW3 : sW4;
    };
    auto stX = [&](int s) -> T* {
        return s == 0 ? sX0 : s == 1 ? sX1 : s == 2 ? sX2 : s == 3 ? sX3 : sX4;
    };

    const int N = a.N, K = a.K;
    int mt, nt;
    if (!tile_coords(blockIdx.x, N / BN, a.max_tiles, &mt, &nt)) return;
    if (mt >= *a.tile_total) return;
    const TileInfo ti = a.tiles[mt];
    const int e = ti.expert, row0 = ti.row0, nrows = ti.rows;
    if (e < 0 || e >= a.num_experts || nrows < 1 || row0 < 0 || row0 + (int64_t)nrows > a.a_cap)
        return;
    const int n0 = nt * BN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    // K-blocked operands: step kt of this tile is one contiguous block of
    // 256 rows x BK for the weights (stride N * BK between steps) and for the
    // token rows (stride a_cap * BK).
    const T* Wt = static_cast<const T*>(a.W) + ((int64_t)e * (K / BK) * N + n0) * BK;
    const T* Xt = static_cast<const T*>(a.X) + (int64_t)row0 * BK;
    const int64_t wstep = (int64_t)N * BK, xstep = a.a_cap * BK;

    // Lane l of load instruction q writes LDS bytes [q*1024 + l*16, +16): tile
    // row r = RPI*q + l/CH, stored chunk l%CH, which holds logical chunk
    // (l%CH) ^ swz(r) of that row.
    int woff[QW], xoff[QX];
#pragma unroll
    for (int i = 0; i < QW; ++i) {
        const int r = (wave * QW + i) * RPI + lane / CH;
        woff[i] = (r * BK + (((lane % CH) ^ swz<CH>(r)) * 8)) * (int)sizeof(T);  // bytes
    }
#pragma unroll
    for (int i = 0; i < QX; ++i) {
        const int r = (wave * QX + i) * RPI + lane / CH;
        const int rr = r < nrows ? r : nrows - 1;
        xoff[i] = (rr * BK + (((lane % CH) ^ swz<CH>(r)) * 8)) * (int)sizeof(T);  // bytes
    }

    f32x16_t acc[SN][SM];
#pragma unroll
    for (int i = 0; i < SN; ++i)
#pragma unroll
        for (int j = 0; j < SM; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int uwave = __builtin_amdgcn_readfirstlane(wave);  // wave-uniform (SGPR) copy
    auto issue = [&](int kt, int buf) {
        const T* ws = Wt + kt * wstep;
        const T* xs = Xt + kt * xstep;
        const uint32_t bw = lds_addr(stW(buf)) + uwave * QW * RPI * BK * (int)sizeof(T);
        const uint32_t bx = lds_addr(stX(buf)) + uwave * QX * RPI * BK * (int)sizeof(T);
#pragma unroll
        for (int i = 0; i < QW; ++i)
            lds_dma16(ws, woff[i], bw + i * RPI * BK * (int)sizeof(T));
#pragma unroll
        for (int i = 0; i < QX; ++i)
            lds_dma16(xs, xoff[i], bx + i * RPI * BK * (int)sizeof(T));
        // keep the loads ahead of the MFMAs that follow
        __builtin_amdgcn_sched_barrier(0);
    };
    const int l32 = lane & 31, lhi = lane >> 5;
    // MFMAs of stage `buf`, with the Q loads of step `ktl` into stage `bufl`
    // spread through them (one load per NMF / Q MFMAs): a burst of loads at
    // the top of the stage would stall this wave's in-order issue while the
    // memory pipeline drains, and with it the MFMAs behind them.
    constexpr int NMF = (BK / 16) * SN * SM;
    constexpr int EVERY = NMF / Q;
    static_assert(NMF % Q == 0, "loads must divide the MFMA count");
    auto compute_issue = [&](int buf, int ktl, int bufl) {
        const T* cW = stW(buf);
        const T* cX = stX(buf);
        const T* ws = Wt + ktl * wstep;
        const T* xs = Xt + ktl * xstep;
        const uint32_t bw = lds_addr(stW(bufl)) + uwave * QW * RPI * BK * (int)sizeof(T);
        const uint32_t bx = lds_addr(stX(bufl)) + uwave * QX * RPI * BK * (int)sizeof(T);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int kc = ks * 2 + lhi;
            V av[SN], bv[SM];
#pragma unroll
            for (int i = 0; i < SN; ++i) {
                const int r = wn * WN + i * 32 + l32;
                av[i] = *reinterpret_cast<const V*>(&cW[r * BK + ((kc ^ swz<CH>(r)) * 8)]);
            }
#pragma unroll
            for (int j = 0; j < SM; ++j) {
                const int r = wm * WM + j * 32 + l32;
                bv[j] = *reinterpret_cast<const V*>(&cX[r * BK + ((kc ^ swz<CH>(r)) * 8)]);
            }
#pragma unroll
            for (int i = 0; i < SN; ++i) {
#pragma unroll
                for (int j = 0; j < SM; ++j) {
                    const int m = (ks * SN + i) * SM + j;  // compile-time after unrolling
                    if (m % EVERY == 0) {
                        const int q = m / EVERY;
                        if (q < QW) lds_dma16(ws, woff[q], bw + q * RPI * BK * (int)sizeof(T));
                        else lds_dma16(xs, xoff[q - QW], bx + (q - QW) * RPI * BK * (int)sizeof(T));
                    }
                    acc[i][j] = Mfma<T>::run(av[i], bv[j], acc[i][j]);
                }
            }
        }
    };

    // K / BK is a multiple of S (checked by the launcher).  Step kt computes
    // stage kt % S.  Before it, the loads of stages <= kt must have landed:
    // this wave's by vmcnt (exactly S - 2 later stages stay in flight), every
    // wave's by the barrier.  The barrier also frees stage (kt - 1) % S, which
    // is refilled with step kt + S - 1.  Past the end the last step is loaded
    // again into that freed (never again read) stage, which keeps the loop
    // free of branches and the in-flight count constant.  A bare s_barrier is
    // used: __syncthreads() would add a full vmcnt(0) fence.
    const int KT = K / BK;
#pragma unroll
    for (int s = 0; s < S - 1; ++s) issue(s, s);
    for (int kt0 = 0; kt0 < KT; kt0 += S) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int kt = kt0 + s;
            wait_vmcnt<(S - 2) * Q>();
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            compute_issue(s, min(kt + S - 1, KT - 1), (s + S - 1) % S);
        }
    }
    // drain the trailing loads before this block's LDS can be handed on
    wait_vmcnt<0>();

    // Epilogue.  Lane (l32, lhi) of block (i, j) holds token row
    // wm*WM + j*32 + l32 and weight rows wn*WN + i*32 + 8*(r/4) + 4*lhi + r%4.
    const float* bias = a.bias + (int64_t)e * N;
    T* out = static_cast<T*>(a.out);
#pragma unroll
    for (int j = 0; j < SM; ++j) {
        const int m = wm * WM + j * 32 + l32;
        if (m >= nrows) continue;
        if (MODE == kGateUp) {
            // h is written K-blocked for the down GEMM: (row, c) at
            // ((c / 32) * a_cap + row) * 32 + c % 32
            T* hrow = out + (int64_t)(row0 + m) * kKBlock;
#pragma unroll
            for (int q = 0; q < SN / 2; ++q) {
                const int pbase = n0 + wn * WN + q * 64;  // packed row of gate unit 0 of the pair
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const int off = 8 * g4 + 4 * lhi;
                    const float4 bg = *reinterpret_cast<const float4*>(bias + pbase + off);
                    const float4 bu = *reinterpret_cast<const float4*>(bias + pbase + 32 + off);
                    const float bgv[4] = {bg.x, bg.y, bg.z, bg.w};
                    const float buv[4] = {bu.x, bu.y, bu.z, bu.w};
                    T hv[4];
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        const float g = acc[2 * q][j][g4 * 4 + s] + bgv[s];
                        const float u = acc[2 * q + 1][j][g4 * 4 + s] + buv[s];
                        hv[s] = Elt<T>::from_f32(g / (1.0f + __expf(-g)) * u);
                    }
                    uint2 raw;
                    __builtin_memcpy(&raw, hv, 8);
                    const int hc = pbase / 2 + off;  // 4 columns inside one 32-block
                    *reinterpret_cast<uint2*>(hrow + (int64_t)(hc / kKBlock) * a.a_cap * kKBlock +
                                              hc % kKBlock) = raw;
                }
            }
        } else {
            T* orow = out + (int64_t)(row0 + m) * N;
#pragma unroll
            for (int i = 0; i < SN; ++i) {
                const int nb = n0 + wn * WN + i * 32;
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const int off = 8 * g4 + 4 * lhi;
                    const float4 b = *reinterpret_cast<const float4*>(bias + nb + off);
                    const float bv4[4] = {b.x, b.y, b.z, b.w};
                    T ov[4];
#pragma unroll
                    for (int s = 0; s < 4; ++s)
                        ov[s] = Elt<T>::from_f32(acc[i][j][g4 * 4 + s] + bv4[s]);
                    uint2 raw;
                    __builtin_memcpy(&raw, ov, 8);
                    *reinterpret_cast<uint2*>(orow + nb + off) = raw;
                }
            }
        }
    }
}

template <typename T, int MODE>
hipError_t launch_mfma_t(const GemmArgs& a, hipStream_t s) {
    constexpr int BM = kMfmaBM, BN = kMfmaBN;
    if (a.N % BN != 0 || a.K % (kBK * kStages) != 0) return hipErrorInvalidValue;
    const int64_t grid = tile_grid(a.max_tiles, a.N / BN);
    if (grid <= 0) return hipSuccess;
    if (grid > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL((gemm_mfma_kernel<T, MODE, BM, BN, kBK, kStages>), dim3((unsigned)grid),
                       dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_gate_up_mfma(DType dt, const GemmArgs& a, hipStream_t s) {
    if (dt == DType::BF16) return launch_mfma_t<__bf16, kGateUp>(a, s);
    if (dt == DType::F16) return launch_mfma_t<_Float16, kGateUp>(a, s);
    return hipErrorInvalidValue;
}

hipError_t launch_gemm_down_mfma(DType dt, const GemmArgs& a, hipStream_t s) {
    if (dt == DType::BF16) return launch_mfma_t<__bf16, kDown>(a, s);
    if (dt == DType::F16) return launch_mfma_t<_Float16, kDown>(a, s);
    return hipErrorInvalidValue;
}

}  // namespace nomas
