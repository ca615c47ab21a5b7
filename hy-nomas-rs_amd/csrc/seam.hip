// norm2 + modulate of a DiT block on gfx950 (block.rs:96):
//   h = modulate(norm2(x), shift, scale)      (norm.rs:55-65, modulate.rs:69-79)
// for rows x D activations, row r in sequence r / seq.
//
// One block takes 64 rows in two phases.
//  1. The sum of squares of each row, added in the reference's order: x*x
//     rounded to f32, then one add per element in ascending d -- a serial chain
//     of D adds per row that no reordering may shorten.  Waves 1..15 make the
//     squares, 128 columns of the 64 rows at a time, into one half of a double
//     buffer in LDS (f32, rows padded by 16 bytes so the 64 lanes' 16-byte
//     reads at one column spread over all banks); meanwhile lane r of wave 0
//     adds row r's squares out of the other half.  The chain then costs one
//     add per element and never waits on HBM.
//  2. h for the 64 rows, 16 bytes per thread, coalesced; norm_w, shift and scale
//     of the sequences the block touches come from LDS (from global memory
//     when they do not fit).
// Bytes per row: D*b read twice (the second pass mostly from cache), D*b written.
#include <algorithm>

#include "kernels.hpp"
#include "seam.hpp"

namespace nomas {

namespace {

constexpr int kSeamRows = 64;
constexpr int kSeamThreads = 1024;
constexpr int kStageCols = 128;                           // columns per stage
constexpr int kRowStride = kStageCols * 4 + 16;           // bytes, padded
constexpr int kStageBytes = kSeamRows * kRowStride;       // 33,792
constexpr int kBatch = 8;                                 // h chunks per thread in flight
constexpr size_t kMaxLds = 160 * 1024;

template <typename T>
__global__ __launch_bounds__(kSeamThreads) void seam_h_kernel(SeamArgs a) {
    // [2][64][kRowStride] stages (later the factors) in factor_lds bytes,
    // then inverse RMS [64] and sequence [64] per row
    extern __shared__ __align__(16) unsigned char s_buf[];
    float* s_inv = reinterpret_cast<float*>(s_buf + a.factor_lds);
    int* s_seqidx = reinterpret_cast<int*>(s_inv + kSeamRows);
    constexpr int EPC = 16 / sizeof(T);
    constexpr int kChunks = kSeamRows * kStageCols / EPC;   // 16-byte chunks per stage
    constexpr int kRowChunks = kStageCols / EPC;
    // waves 1..15 produce the squares, wave 0 adds them up
    constexpr int kProducers = kSeamThreads - kWave;
    constexpr int kLoads = (kChunks + kProducers - 1) / kProducers;  // 2 (16-bit) or 3 (f32)
    // stages of x in flight: ~64 KB per block, what HBM's latency under load
    // times a CU's share of its bandwidth asks for
    constexpr int kRing = kLoads == 2 ? 4 : 3;
    const T* x = static_cast<const T*>(a.x);  // h may alias x: no restrict
    T* h = static_cast<T*>(a.h);
    const int D = a.D, nck = D / EPC;  // D % 8 == 0
    const int64_t row0 = (int64_t)blockIdx.x * kSeamRows;
    const int nrows = (int)min<int64_t>(kSeamRows, a.rows - row0);
    const int tid = threadIdx.x;
    const int pi = tid - kWave;  // producer index (negative in wave 0)
    const int nstage = (D + kStageCols - 1) / kStageCols;

    // ---- phase 1: inverse RMS of each row ----
    // x arrives through a ring of kRing stages in registers (the loads of a
    // stage are issued kRing - 1 stages before its squares go to LDS).  The
    // loads are unconditional (chunks outside the rows, past D or past the
    // stage read a valid chunk instead) and the stash zeroes or skips what
    // lies outside: a load under a branch is waited for at the branch's join.
    uint4 ring[kRing][kLoads];
    auto inside = [&](int st, int j) {
        const int i = pi + j * kProducers;
        return i < kChunks && i / kRowChunks < nrows && st * kRowChunks + i % kRowChunks < nck;
    };
    auto fetch = [&](int st, uint4* ld) {
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            const int i = min(pi + j * kProducers, kChunks - 1);
            const int r = min(i / kRowChunks, nrows - 1);
            const int c = inside(st, j) ? st * kRowChunks + i % kRowChunks : 0;
            ld[j] = *reinterpret_cast<const uint4*>(x + (row0 + r) * (int64_t)D + (int64_t)c * EPC);
        }
    };
    auto stash = [&](const uint4* ld, int st) {  // the squares, rounded to f32
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            const int i = pi + j * kProducers;
            const bool in = inside(st, j);
            Vec16<T> t;
            __builtin_memcpy(&t, &ld[j], 16);
            float sq[EPC];
#pragma unroll
            for (int e = 0; e < EPC; ++e) {
                const float v = Elt<T>::to_f32(t.v[e]);
                const float q = mul_rn(v, v);
                sq[e] = in ? q : 0.0f;  // zeros: acc + 0 == acc
            }
            if (i < kChunks) {
                unsigned char* dst = s_buf + (st & 1) * kStageBytes + (i / kRowChunks) * kRowStride +
                                     (i % kRowChunks) * EPC * 4;
#pragma unroll
                for (int q = 0; q < EPC / 4; ++q)
                    *reinterpret_cast<float4*>(dst + 16 * q) =
                        make_float4(sq[4 * q], sq[4 * q + 1], sq[4 * q + 2], sq[4 * q + 3]);
            }
        }
    };
    // Producers and the adder run separate loops with the same barriers (one
    // per stage): a branch inside one loop would hide from the compiler that
    // a producer's ring slot had kRing - 1 stages of loads issued after it.
    float acc = 0.0f;
    if (tid >= kWave) {
#pragma unroll
        for (int p = 0; p < kRing; ++p) fetch(p, ring[p]);
        stash(ring[0], 0);
        fetch(kRing, ring[0]);
        __syncthreads();
        // whole ring turns; stage st sits in ring slot st % kRing, LDS half st & 1.
        // Stages past the end stash zeros nobody reads and load a valid chunk.
        for (int st0 = 0; st0 < nstage; st0 += kRing) {
#pragma unroll
            for (int p = 0; p < kRing; ++p) {
                const int st = st0 + p;
                stash(ring[(p + 1) % kRing], st + 1);
                fetch(st + 1 + kRing, ring[(p + 1) % kRing]);
                __syncthreads();
            }
        }
    } else {
        s_seqidx[tid] = (int)((row0 + min(tid, nrows - 1)) / a.seq - row0 / a.seq);
        __syncthreads();
        for (int st0 = 0; st0 < nstage; st0 += kRing) {
#pragma unroll
            for (int p = 0; p < kRing; ++p) {
                const int st = st0 + p;
                if (st < nstage) {
                    const unsigned char* rowp = s_buf + (st & 1) * kStageBytes + tid * kRowStride;
#pragma unroll 8
                    for (int c = 0; c < kStageCols / 4; ++c) {
                        const float4 q = *reinterpret_cast<const float4*>(rowp + c * 16);
                        acc = add_nc(acc, q.x);
                        acc = add_nc(acc, q.y);
                        acc = add_nc(acc, q.z);
                        acc = add_nc(acc, q.w);
                    }
                }
                __syncthreads();
            }
        }
    }
    if (tid < kWave) s_inv[tid] = seam_inv_rms(acc, D, a.eps);

    // ---- phase 2: h ----
    // norm_w and the scale / shift rows of the sequences the block touches
    // go to LDS when they fit (the stage buffers are free now), else they are
    // read from global memory; either way 16 bytes at a time.
    const int64_t b0 = row0 / a.seq;
    const int nsq = s_seqidx[nrows - 1] + 1;
    const bool lds_f = (size_t)(1 + 2 * nsq) * D * 4 <= a.factor_lds;
    float* f_w = reinterpret_cast<float*>(s_buf);  // D
    float* f_sc = f_w + D;                          // nsq x D
    float* f_sh = f_sc + (size_t)nsq * D;           // nsq x D
    if (lds_f) {
        for (int i = tid; i < D / 4; i += kSeamThreads) {
            float4 w = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
            if (a.norm_w) w = reinterpret_cast<const float4*>(a.norm_w)[i];
            reinterpret_cast<float4*>(f_w)[i] = w;
        }
        for (int i = tid; i < nsq * D / 4; i += kSeamThreads) {
            reinterpret_cast<float4*>(f_sc)[i] = reinterpret_cast<const float4*>(a.scale + b0 * D)[i];
            reinterpret_cast<float4*>(f_sh)[i] = reinterpret_cast<const float4*>(a.shift + b0 * D)[i];
        }
    }
    __syncthreads();
    // 16-byte chunks of the block's rows, kBatch per thread in flight; each
    // thread reads only the chunks it writes (h may alias x).  pw null: gain 1.
    auto rows_h = [&](const float* pw, const float* psc, const float* psh) {
        const int total = nrows * nck;
        for (int i0 = tid; i0 < total; i0 += kSeamThreads * kBatch) {
            uint4 v[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {  // past the end: the last chunk again, not stored
                const int i = min(i0 + u * kSeamThreads, total - 1);
                const int r = i / nck;
                v[u] = *reinterpret_cast<const uint4*>(x + (row0 + r) * (int64_t)D +
                                                       (int64_t)(i - r * nck) * EPC);
            }
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int i = i0 + u * kSeamThreads;
                if (i >= total) continue;
                const int r = i / nck, col = (i - r * nck) * EPC;
                const size_t fo = (size_t)s_seqidx[r] * D + col;
                const float inv = s_inv[r];
                float w[EPC], sc[EPC], sh[EPC];
                if (pw) {
                    load_f32s<EPC>(pw + col, w);
                } else {
#pragma unroll
                    for (int e = 0; e < EPC; ++e) w[e] = 1.0f;
                }
                load_f32s<EPC>(psc + fo, sc);
                load_f32s<EPC>(psh + fo, sh);
                Vec16<T> t;
                __builtin_memcpy(&t, &v[u], 16);
#pragma unroll
                for (int e = 0; e < EPC; ++e)
                    t.v[e] = Elt<T>::from_f32(seam_h<T>(Elt<T>::to_f32(t.v[e]), inv, w[e], sc[e], sh[e]));
                uint4 o;
                __builtin_memcpy(&o, &t, 16);
                *reinterpret_cast<uint4*>(h + (row0 + r) * (int64_t)D + col) = o;
            }
        }
    };
    if (lds_f)
        rows_h(f_w, f_sc, f_sh);
    else
        rows_h(a.norm_w, a.scale + b0 * D, a.shift + b0 * D);
}

template <typename T>
hipError_t launch_seam_h_t(const SeamArgs& a, hipStream_t s) {
    const int64_t nblk = (a.rows + kSeamRows - 1) / kSeamRows;
    if (nblk == 0) return hipSuccess;
    // LDS: the two stage buffers, which phase 2 reuses for the factors of up
    // to two sequences when a larger allocation is not needed for them
    SeamArgs b = a;
    const size_t want = (size_t)5 * a.D * 4;
    b.factor_lds = (int)std::max<size_t>(2 * kStageBytes, std::min<size_t>(want, kMaxLds - 512));
    const size_t lds = (size_t)b.factor_lds + 512;  // + inverse RMS and sequence per row
    hipError_t err = hipFuncSetAttribute((const void*)seam_h_kernel<T>,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (err != hipSuccess) return err;
    launch_kernel(seam_h_kernel<T>, dim3((unsigned)nblk), dim3(kSeamThreads), lds, s, b);
    return hipGetLastError();
}

// out = x + y * gate (block.rs:101) on its own, for a feed-forward whose last
// kernel does not apply it: 16 bytes of each operand per thread; each thread
// reads the elements it writes, so out may alias x or y.
template <typename T>
__global__ __launch_bounds__(256) void gated_residual_kernel(const T* x, const T* y,
                                                             const float* __restrict__ gate,
                                                             T* out, int64_t rows, int D,
                                                             int64_t seq) {
    constexpr int EPC = 16 / sizeof(T);
    const int nck = D / EPC;
    const int64_t total = rows * nck;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = i / nck;
        const int64_t off = row * D + (i % nck) * EPC;
        float xv[EPC], yv[EPC], g[EPC];
        load16(x + off, xv);
        load16(y + off, yv);
        load_f32s<EPC>(gate + row / seq * D + (i % nck) * EPC, g);
#pragma unroll
        for (int e = 0; e < EPC; ++e) xv[e] = seam_residual<T>(xv[e], yv[e], g[e]);
        store16(out + off, xv);
    }
}

template <typename T>
hipError_t launch_residual_t(const void* x, const void* y, const float* gate, void* out,
                             int64_t rows, int D, int64_t seq, hipStream_t s) {
    const int64_t total = rows * (D / (16 / (int)sizeof(T)));
    if (total == 0) return hipSuccess;
    const int64_t blocks = std::min<int64_t>((total + 255) / 256, 256 * 16);
    launch_kernel(gated_residual_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, s,
                  (const T*)x, (const T*)y, gate, (T*)out, rows, D, seq);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gated_residual(DType dt, const void* x, const void* y, const float* gate,
                                 void* out, int64_t rows, int D, int64_t seq, hipStream_t s) {
    if (!x || !y || !gate || !out || seq < 1 || D <= 0 || D % 8 != 0 || rows < 0)
        return hipErrorInvalidValue;
    switch (dt) {
        case DType::F32: return launch_residual_t<float>(x, y, gate, out, rows, D, seq, s);
        case DType::BF16: return launch_residual_t<__bf16>(x, y, gate, out, rows, D, seq, s);
        case DType::F16: return launch_residual_t<_Float16>(x, y, gate, out, rows, D, seq, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_seam_h(DType dt, const SeamArgs& a, hipStream_t s) {
    if (!a.x || !a.h || !a.shift || !a.scale || a.seq < 1 || a.D <= 0 || a.D % 8 != 0 ||
        a.rows < 0)
        return hipErrorInvalidValue;
    switch (dt) {
        case DType::F32: return launch_seam_h_t<float>(a, s);
        case DType::BF16: return launch_seam_h_t<__bf16>(a, s);
        case DType::F16: return launch_seam_h_t<_Float16>(a, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace nomas
