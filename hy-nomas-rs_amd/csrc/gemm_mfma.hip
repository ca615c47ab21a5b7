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
//    (BN/2) x (BM/2) tile of 32 x 32 MFMA blocks.
//  - K is walked in 64-wide steps through double-buffered LDS tiles.  Rows of
//    128 bytes are stored with their 16-byte chunks XOR-swizzled by
//    (r ^ r >> 3) & 7, which keeps both the 16-byte row-chunk stores and the
//    32-row MFMA operand reads free of bank conflicts.
//  - Gate and up rows are interleaved in groups of 32 when the weights are
//    packed (rows 64g..64g+31 = gate 32g.., rows 64g+32.. = up 32g..), so a
//    wave holds gate and up of the same hidden unit in the same lane and the
//    SwiGLU is applied in the epilogue without an extra pass over HBM.
//  - Tiles are ordered in groups of GM row tiles (column index fastest within
//    a group) and the grid is remapped so each XCD (block i runs on XCD i % 8)
//    gets one contiguous range of that order: its concurrently running blocks
//    share weight and token panels in the XCD's own L2.
#include "kernels.hpp"

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

constexpr int kBK = 64;
constexpr int kThreads = 256;
constexpr int kGroupM = 4;

__device__ __forceinline__ int swz(int r) { return (r ^ (r >> 3)) & 7; }

// Maps the hardware block id to (row tile, column tile).
__device__ __forceinline__ void tile_coords(int pid, int G, int ntn, int max_tiles, int* mt,
                                            int* nt) {
    const int xcd = pid % kNumXcd, loc = pid / kNumXcd;
    const int per = (G + kNumXcd - 1) / kNumXcd;
    const int tall = (G % kNumXcd) == 0 ? kNumXcd : G % kNumXcd;
    const int L = xcd < tall ? xcd * per + loc : tall * per + (xcd - tall) * (per - 1) + loc;
    const int group = L / (kGroupM * ntn);
    const int first_m = group * kGroupM;
    const int gm = min(kGroupM, max_tiles - first_m);
    const int within = L - group * kGroupM * ntn;
    *mt = first_m + within % gm;
    *nt = within / gm;
}

template <typename T, int MODE, int BM, int BN>
__global__ __launch_bounds__(kThreads, 1) void gemm_mfma_kernel(GemmArgs a) {
    using V = typename Mfma<T>::V;
    constexpr int WM = BM / 2, WN = BN / 2;       // wave tile: token rows x weight rows
    constexpr int SM = WM / 32, SN = WN / 32;     // 32x32 MFMA blocks per wave
    // Direct global->LDS loads: one wave instruction fills 8 rows x 128 bytes.
    constexpr int QW = BN / 8 / (kThreads / kWave);  // load instructions per wave per k step
    constexpr int QX = BM / 8 / (kThreads / kWave);
    static_assert(MODE == kDown || SN % 2 == 0, "gate/up pairs need an even block count");

    // Two stages, each its own LDS object so the compiler can tell a stage
    // being filled from the one being read.
    __shared__ __attribute__((aligned(16))) T sW0[BN * kBK];
    __shared__ __attribute__((aligned(16))) T sX0[BM * kBK];
    __shared__ __attribute__((aligned(16))) T sW1[BN * kBK];
    __shared__ __attribute__((aligned(16))) T sX1[BM * kBK];

    const int N = a.N, K = a.K;
    int mt, nt;
    tile_coords(blockIdx.x, gridDim.x, N / BN, a.max_tiles, &mt, &nt);
    if (mt >= *a.tile_total) return;
    const TileInfo ti = a.tiles[mt];
    const int e = ti.expert, row0 = ti.row0, nrows = ti.rows;
    if (e < 0 || e >= a.num_experts || nrows < 1 || row0 < 0 || row0 + (int64_t)nrows > a.a_cap)
        return;
    const int n0 = nt * BN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    const T* Wt = static_cast<const T*>(a.W) + ((int64_t)e * N + n0) * K;
    const T* Xt = static_cast<const T*>(a.X) + (int64_t)row0 * K;

    // Lane l of load instruction q writes LDS bytes [q*1024 + l*16, +16): tile
    // row r = 8q + l/8, stored chunk l%8, which holds logical chunk
    // (l%8) ^ swz(r) of that row -- the swizzle is applied on the global side.
    int woff[QW], xoff[QX];
#pragma unroll
    for (int i = 0; i < QW; ++i) {
        const int r = (wave * QW + i) * 8 + (lane >> 3);
        woff[i] = r * K + (((lane & 7) ^ swz(r)) * 8);
    }
#pragma unroll
    for (int i = 0; i < QX; ++i) {
        const int r = (wave * QX + i) * 8 + (lane >> 3);
        const int rr = r < nrows ? r : nrows - 1;
        xoff[i] = rr * K + (((lane & 7) ^ swz(r)) * 8);
    }

    f32x16_t acc[SN][SM];
#pragma unroll
    for (int i = 0; i < SN; ++i)
#pragma unroll
        for (int j = 0; j < SM; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    auto issue = [&](int kt, T* dW, T* dX) {
        const int ko = kt * kBK;
#pragma unroll
        for (int i = 0; i < QW; ++i)
            __builtin_amdgcn_global_load_lds(
                (const void*)(Wt + woff[i] + ko),
                (__attribute__((address_space(3))) void*)(dW + (wave * QW + i) * 8 * kBK), 16, 0, 0);
#pragma unroll
        for (int i = 0; i < QX; ++i)
            __builtin_amdgcn_global_load_lds(
                (const void*)(Xt + xoff[i] + ko),
                (__attribute__((address_space(3))) void*)(dX + (wave * QX + i) * 8 * kBK), 16, 0, 0);
        // keep the loads ahead of the MFMAs that follow (the scheduler would
        // otherwise sink them to the wait at the end of the stage)
        __builtin_amdgcn_sched_barrier(0);
    };
    const int l32 = lane & 31, lhi = lane >> 5;
    auto compute = [&](const T* cW, const T* cX) {
#pragma unroll
        for (int ks = 0; ks < kBK / 16; ++ks) {
            const int kc = ks * 2 + lhi;
            V av[SN], bv[SM];
#pragma unroll
            for (int i = 0; i < SN; ++i) {
                const int r = wn * WN + i * 32 + l32;
                av[i] = *reinterpret_cast<const V*>(&cW[r * kBK + ((kc ^ swz(r)) * 8)]);
            }
#pragma unroll
            for (int j = 0; j < SM; ++j) {
                const int r = wm * WM + j * 32 + l32;
                bv[j] = *reinterpret_cast<const V*>(&cX[r * kBK + ((kc ^ swz(r)) * 8)]);
            }
#pragma unroll
            for (int i = 0; i < SN; ++i)
#pragma unroll
                for (int j = 0; j < SM; ++j) acc[i][j] = Mfma<T>::run(av[i], bv[j], acc[i][j]);
        }
    };
    // All of this wave's loads have landed, then every wave's have.
    auto land = [&]() {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    };

    const int KT = K / kBK;
    issue(0, sW0, sX0);
    land();
    int kt = 0;
    for (; kt + 2 <= KT; kt += 2) {
        issue(kt + 1, sW1, sX1);
        compute(sW0, sX0);
        land();
        if (kt + 2 < KT) issue(kt + 2, sW0, sX0);
        compute(sW1, sX1);
        land();
    }
    if (kt < KT) compute(sW0, sX0);  // odd number of k steps: the last one is staged in 0

    // Epilogue.  Lane (l32, lhi) of block (i, j) holds token row
    // wm*WM + j*32 + l32 and weight rows wn*WN + i*32 + 8*(r/4) + 4*lhi + r%4.
    const float* bias = a.bias + (int64_t)e * N;
    T* out = static_cast<T*>(a.out);
#pragma unroll
    for (int j = 0; j < SM; ++j) {
        const int m = wm * WM + j * 32 + l32;
        if (m >= nrows) continue;
        if (MODE == kGateUp) {
            const int H = N / 2;
            T* orow = out + (int64_t)(row0 + m) * H;
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
                    *reinterpret_cast<uint2*>(orow + pbase / 2 + off) = raw;
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
    if (a.N % BN != 0 || a.K % kBK != 0) return hipErrorInvalidValue;
    const int64_t grid = (int64_t)a.max_tiles * (a.N / BN);
    if (grid <= 0) return hipSuccess;
    if (grid > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL((gemm_mfma_kernel<T, MODE, BM, BN>), dim3((unsigned)grid), dim3(kThreads),
                       0, s, a);
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
