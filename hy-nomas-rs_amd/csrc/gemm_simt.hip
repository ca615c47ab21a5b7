// General grouped expert GEMMs: any dtype (f32 / bf16 / f16), any D and H.
//
// Used for f32 models (hy-nomas-rs's default DataType, config.rs:30-33) and
// for shapes the MFMA kernels do not tile (D % 256 or H % 128 non-zero).
// 64 x 64 output tile per block, 256 threads each owning a 4 x 4 sub-tile,
// K walked in 16-wide LDS steps, f32 accumulation, bounds-checked everywhere.
// Weight layout: gate/up as [E][2][H][D] (gate block then up block), down as
// the reference's [E][D][H]; biases f32 [E][2][H] and [E][D].
#include "kernels.hpp"

namespace nomas {

namespace {

enum { kGateUp = 0, kDown = 1 };
constexpr int kT = 64;   // output tile (rows and columns)
constexpr int kKs = 16;  // k step

template <typename T, int MODE>
__global__ __launch_bounds__(256) void gemm_simt_kernel(GemmArgs a) {
    __shared__ float sX[kKs][kT + 1];
    __shared__ float sA[kKs][kT + 1];
    __shared__ float sB[MODE == kGateUp ? kKs : 1][kT + 1];
    const int mt = blockIdx.x;
    if (mt >= *a.tile_total) return;
    const TileInfo ti = a.tiles[mt];
    const int e = ti.expert, row0 = ti.row0, nrows = ti.rows;
    if (e < 0 || e >= a.num_experts || nrows < 1 || row0 < 0 || row0 + (int64_t)nrows > a.a_cap)
        return;
    const int K = a.K;
    const int Nout = MODE == kGateUp ? a.N / 2 : a.N;  // columns of the output
    const int n0 = blockIdx.y * kT;
    const T* X = static_cast<const T*>(a.X) + (int64_t)row0 * K;
    const T* Wa;
    const T* Wb = nullptr;
    if (MODE == kGateUp) {
        Wa = static_cast<const T*>(a.W) + (int64_t)e * 2 * Nout * K;  // gate [H][D]
        Wb = Wa + (int64_t)Nout * K;                                  // up   [H][D]
    } else {
        Wa = static_cast<const T*>(a.W) + (int64_t)e * Nout * K;      // down [D][H]
    }
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    float accA[4][4] = {}, accB[4][4] = {};
    for (int k0 = 0; k0 < K; k0 += kKs) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = tid + 256 * i;
            const int r = idx / kKs, kk = idx % kKs;
            const bool kin = k0 + kk < K;
            sX[kk][r] = (r < nrows && kin) ? Elt<T>::to_f32(X[(int64_t)r * K + k0 + kk]) : 0.0f;
            const bool nin = n0 + r < Nout;
            sA[kk][r] = (nin && kin) ? Elt<T>::to_f32(Wa[(int64_t)(n0 + r) * K + k0 + kk]) : 0.0f;
            if (MODE == kGateUp)
                sB[kk][r] = (nin && kin) ? Elt<T>::to_f32(Wb[(int64_t)(n0 + r) * K + k0 + kk]) : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kKs; ++kk) {
            float xv[4], av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                xv[i] = sX[kk][ty * 4 + i];
                av[i] = sA[kk][tx * 4 + i];
                if (MODE == kGateUp) bv[i] = sB[kk][tx * 4 + i];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    accA[i][j] += xv[i] * av[j];
                    if (MODE == kGateUp) accB[i][j] += xv[i] * bv[j];
                }
        }
        __syncthreads();
    }
    T* out = static_cast<T*>(a.out);
    const float* bias = a.bias + (int64_t)e * (MODE == kGateUp ? 2 * Nout : Nout);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = ty * 4 + i;
        if (m >= nrows) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + tx * 4 + j;
            if (n >= Nout) continue;
            float v;
            if (MODE == kGateUp) {
                const float g = accA[i][j] + bias[n];
                const float u = accB[i][j] + bias[Nout + n];
                v = g / (1.0f + expf(-g)) * u;
            } else {
                v = accA[i][j] + bias[n];
            }
            out[(int64_t)(row0 + m) * Nout + n] = Elt<T>::from_f32(v);
        }
    }
}

template <typename T, int MODE>
hipError_t launch_simt_t(const GemmArgs& a, hipStream_t s) {
    const int Nout = MODE == kGateUp ? a.N / 2 : a.N;
    dim3 grid(a.max_tiles, (Nout + kT - 1) / kT);
    if (a.max_tiles <= 0) return hipSuccess;
    launch_kernel((gemm_simt_kernel<T, MODE>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

template <int MODE>
hipError_t launch_simt(DType dt, const GemmArgs& a, hipStream_t s) {
    switch (dt) {
        case DType::F32: return launch_simt_t<float, MODE>(a, s);
        case DType::BF16: return launch_simt_t<__bf16, MODE>(a, s);
        case DType::F16: return launch_simt_t<_Float16, MODE>(a, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_gemm_gate_up_simt(DType dt, const GemmArgs& a, hipStream_t s) {
    return launch_simt<kGateUp>(dt, a, s);
}

hipError_t launch_gemm_down_simt(DType dt, const GemmArgs& a, hipStream_t s) {
    return launch_simt<kDown>(dt, a, s);
}

}  // namespace nomas
