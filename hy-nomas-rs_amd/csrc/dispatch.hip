// Dispatch and combine: the data movement around the expert GEMMs.
//
// The reference evaluates every expert on every row and masks by the gate
// (moe.rs:97-102).  Here only the selected (row, expert) pairs are computed:
// rows are permuted into expert-contiguous order, the GEMMs run per expert,
// and combine gathers each row's k results back.  Within an expert, rows keep
// ascending row order (a stable permutation), so every run produces the same
// buffers, and combine sums a row's slots in ascending expert order, the order
// of the reference's accumulation loop (moe.rs:98-102).
#include <algorithm>

#include "kernels.hpp"
#include "seam.hpp"

namespace nomas {

namespace {

constexpr int kScanThreads = 1024;

// Exclusive scan of one int per thread across the block (1024 threads).
// Returns the exclusive prefix; *total receives the block sum.
__device__ int block_exclusive_scan(int v, int* s_wave, int* total) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(incl, o);
        if (lane >= o) incl += t;
    }
    if (lane == 63) s_wave[wave] = incl;
    __syncthreads();
    if (wave == 0) {
        int w = lane < kScanThreads / 64 ? s_wave[lane] : 0;
        int wi = w;
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
            const int t = __shfl_up(wi, o);
            if (lane >= o) wi += t;
        }
        if (lane < kScanThreads / 64) s_wave[16 + lane] = wi - w;
        if (lane == kScanThreads / 64 - 1) s_wave[32] = wi;
    }
    __syncthreads();
    const int excl = incl - v + s_wave[16 + wave];
    *total = s_wave[32];
    __syncthreads();
    return excl;
}

// Single block.  From the per-chunk expert histograms computes
//  - chunk_base[c][e]: first position of chunk c's rows of expert e,
//  - expert_count[e], expert_off[e] (exclusive scan, expert_off[E] = A),
//  - the GEMM tile table: ceil(count_e / BM) tiles of BM rows per expert.
// Each thread owns one (expert, slice of chunks) pair so the serial work is
// about sqrt(nchunks) per thread.
__global__ __launch_bounds__(kScanThreads) void scan_kernel(ScanArgs a) {
    __shared__ int s_part[kScanThreads];
    __shared__ int s_tot[kMaxExperts + 1];
    __shared__ int s_off[kMaxExperts + 1];
    __shared__ int s_tstart[kMaxExperts + 1];
    __shared__ int s_wave[40];
    const int tid = threadIdx.x;
    const int E = a.E_cols, nch = a.nchunks;
    int nsl = 1;
    while ((nsl * 2) * (nsl * 2) <= nch && (nsl * 2) * E <= kScanThreads) nsl *= 2;
    const int cps = (nch + nsl - 1) / nsl;
    const int e = tid % E, sl = tid / E;
    const bool active = sl < nsl;
    const int c0 = sl * cps, c1 = min(nch, c0 + cps);
    int sum = 0;
    if (active)
        for (int c = c0; c < c1; ++c) sum += a.chunk_counts[(int64_t)c * E + e];
    if (active) s_part[sl * E + e] = sum;
    __syncthreads();
    if (tid < E) {
        int run = 0;
        for (int q = 0; q < nsl; ++q) {
            const int v = s_part[q * E + tid];
            s_part[q * E + tid] = run;
            run += v;
        }
        s_tot[tid] = run;
    }
    __syncthreads();
    int total_rows;
    const int ex = block_exclusive_scan(tid < E ? s_tot[tid] : 0, s_wave, &total_rows);
    if (tid < E) s_off[tid] = ex;
    __syncthreads();
    if (active) {
        int run = s_off[e] + s_part[sl * E + e];
        for (int c = c0; c < c1; ++c) {
            const int64_t i = (int64_t)c * E + e;
            a.chunk_base[i] = run;
            run += a.chunk_counts[i];
        }
    }
    const int nt = tid < E ? (s_tot[tid] + a.BM - 1) / a.BM : 0;
    int total_tiles;
    const int ts = block_exclusive_scan(nt, s_wave, &total_tiles);
    if (tid < E) {
        s_tstart[tid] = ts;
        a.expert_count[tid] = s_tot[tid];
        a.expert_off[tid] = s_off[tid];
    }
    if (tid == 0) {
        a.expert_off[E] = total_rows;
        a.tile_total[0] = min(total_tiles, a.max_tiles);
    }
    __syncthreads();
    for (int i = tid; i < total_tiles && i < a.max_tiles; i += kScanThreads) {
        int lo = 0, hi = E - 1;  // last expert with tstart <= i (skipping empty ones)
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (s_tstart[mid] <= i) lo = mid; else hi = mid - 1;
        }
        while (lo > 0 && s_tstart[lo] > i) --lo;
        const int j = i - s_tstart[lo];
        TileInfo t;
        t.expert = lo;
        t.row0 = s_off[lo] + j * a.BM;
        t.rows = min(a.BM, s_tot[lo] - j * a.BM);
        t.pad = 0;
        a.tiles[i] = t;
    }
}

// One block per 64-row chunk.  Wave 0 ranks the chunk's slots: for each
// expert in ascending order, a ballot over the 64 rows gives every row its
// rank among the chunk's rows of that expert; adding the chunk base gives a
// stable position.  Then all 16 waves copy rows: each x row is read once and
// written to its k positions with 16-byte accesses.
template <typename T>
__global__ __launch_bounds__(1024) void dispatch_kernel(DispatchArgs a) {
    extern __shared__ int s_dyn[];
    const int k = a.k_slots;
    int* s_idx = s_dyn;           // 64 x k
    int* s_pos = s_dyn + 64 * k;  // 64 x k
    const int tid = threadIdx.x;
    const int64_t row0 = (int64_t)blockIdx.x * kRouterRows;
    const int nvalid = (int)min<int64_t>(kRouterRows, a.rows - row0);
    for (int i = tid; i < 64 * k; i += 1024) {
        s_idx[i] = (i / k < nvalid) ? a.topk_idx[row0 * k + i] : -1;
        s_pos[i] = -1;
    }
    __syncthreads();
    if (tid < 64) {
        const int lane = tid;
        const int* mine = s_idx + lane * k;
        const int32_t* base = a.chunk_base + (int64_t)blockIdx.x * a.E_cols;
        int cur = 0;
        for (int e = 0; e < a.E_cols; ++e) {
            const bool has = cur < k && mine[cur] == e;
            const uint64_t bal = __ballot(has);
            if (has) {
                const int p = base[e] + __popcll(bal & ((1ull << lane) - 1ull));
                s_pos[lane * k + cur] = p;
                a.tok_pos[(row0 + lane) * k + cur] = p;
                ++cur;
            }
        }
    }
    __syncthreads();
    constexpr int EPC = 16 / sizeof(T);
    const int nchunk = a.D / EPC;
    const int wave = tid >> 6, lane = tid & 63;
    const T* x = static_cast<const T*>(a.x);
    T* xp = static_cast<T*>(a.x_perm);
    for (int r = wave * 4; r < wave * 4 + 4 && r < nvalid; ++r) {
        const T* src = x + (row0 + r) * (int64_t)a.D;
        for (int c = lane; c < nchunk; c += kWave) {
            const uint4 v = *reinterpret_cast<const uint4*>(src + (int64_t)c * EPC);
            const int64_t col = (int64_t)c * EPC;
            for (int j = 0; j < k; ++j) {
                const int p = s_pos[r * k + j];
                if (p < 0 || p >= a.a_cap) continue;
                // row-major (p, col) or K-blocked ((col / 32) * a_cap + p) * 32 + col % 32
                const int64_t off = a.kblocked
                    ? ((col / kKBlock) * a.a_cap + p) * kKBlock + col % kKBlock
                    : (int64_t)p * a.D + col;
                *reinterpret_cast<uint4*>(xp + off) = v;
            }
        }
    }
}

// One wave per row: out[row] = sum_j w_j * y_perm[pos_j] over the row's slots
// in ascending expert order (then the dense slot), accumulated in f32.
template <typename T>
__global__ __launch_bounds__(256) void combine_kernel(CombineArgs a) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + wave;
    if (row >= a.rows) return;
    constexpr int EPC = 16 / sizeof(T);
    const int nchunk = a.D / EPC;
    const int k = a.k_slots;
    const T* y = static_cast<const T*>(a.y_perm);
    T* out = static_cast<T*>(a.out);
    // gated residual: the row's gate and input (block.rs:101)
    const float* grow = a.gate ? a.gate + row / a.seq * a.D : nullptr;
    const T* xrow = a.gate ? static_cast<const T*>(a.resid_x) + row * a.D : nullptr;
    for (int c = lane; c < nchunk; c += kWave) {
        float acc[EPC], xv[EPC];
        if (grow) load16(xrow + (int64_t)c * EPC, xv);  // in flight with the y loads
#pragma unroll
        for (int i = 0; i < EPC; ++i) acc[i] = 0.0f;
        for (int j = 0; j < k; ++j) {
            const int p = a.tok_pos[row * k + j];
            const float w = a.topk_w[row * k + j];
            if (p < 0 || p >= a.a_cap) continue;
            float v[EPC];
            load16(y + (int64_t)p * a.D + (int64_t)c * EPC, v);
#pragma unroll
            for (int i = 0; i < EPC; ++i) acc[i] = acc[i] + v[i] * w;
        }
        if (grow) {  // out = x + y * gate, y and each step rounded to the model dtype
            float g[EPC];
            load_f32s<EPC>(grow + (int64_t)c * EPC, g);
#pragma unroll
            for (int i = 0; i < EPC; ++i)
                acc[i] = seam_residual<T>(xv[i], Elt<T>::to_f32(Elt<T>::from_f32(acc[i])), g[i]);
        }
        store16(out + row * a.D + (int64_t)c * EPC, acc);
    }
}

// Dense feed-forward: every row goes to expert 0, in order.
__global__ void dense_tiles_kernel(int64_t rows, int BM, int max_tiles, TileInfo* tiles,
                                   int32_t* tile_total) {
    const int64_t ntiles = (rows + BM - 1) / BM;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < max_tiles; i += gridDim.x * blockDim.x) {
        TileInfo t;
        t.expert = 0;
        t.row0 = i * BM;
        t.rows = i < ntiles ? (int)min<int64_t>(BM, rows - (int64_t)i * BM) : 0;
        t.pad = 0;
        tiles[i] = t;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) *tile_total = (int32_t)min<int64_t>(ntiles, max_tiles);
}

// x (rows x D, row-major) to the K-blocked layout of the MFMA GEMMs: one
// 16-byte chunk per thread, coalesced reads, 64-byte runs written.
template <typename T>
__global__ __launch_bounds__(256) void kblock_kernel(const T* __restrict__ x, T* __restrict__ xk,
                                                     int64_t rows, int D, int64_t a_cap) {
    constexpr int EPC = 16 / sizeof(T);
    const int nchunk = D / EPC;
    const int64_t total = rows * nchunk;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / nchunk;
        const int64_t col = (i % nchunk) * EPC;
        const uint4 v = *reinterpret_cast<const uint4*>(x + r * D + col);
        *reinterpret_cast<uint4*>(xk + ((col / kKBlock) * a_cap + r) * kKBlock + col % kKBlock) = v;
    }
}

template <typename T>
hipError_t launch_dispatch_t(const DispatchArgs& a, hipStream_t s) {
    const int nblk = (int)((a.rows + kRouterRows - 1) / kRouterRows);
    const size_t lds = sizeof(int) * 2 * 64 * a.k_slots;
    if (lds > 65536) {
        hipError_t err = hipFuncSetAttribute((const void*)dispatch_kernel<T>,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (err != hipSuccess) return err;
    }
    hipLaunchKernelGGL(dispatch_kernel<T>, dim3(nblk), dim3(1024), lds, s, a);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_combine_t(const CombineArgs& a, hipStream_t s) {
    const int nblk = (int)((a.rows + 3) / 4);
    hipLaunchKernelGGL(combine_kernel<T>, dim3(nblk), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_scan(const ScanArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(kScanThreads), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_dispatch(DType dt, const DispatchArgs& a, hipStream_t s) {
    switch (dt) {
        case DType::F32: return launch_dispatch_t<float>(a, s);
        case DType::BF16: return launch_dispatch_t<__bf16>(a, s);
        case DType::F16: return launch_dispatch_t<_Float16>(a, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_dense_tiles(int64_t rows, int BM, int max_tiles, TileInfo* tiles,
                              int32_t* tile_total, hipStream_t s) {
    if (max_tiles <= 0) return hipErrorInvalidValue;
    const int nblk = (max_tiles + 255) / 256;
    hipLaunchKernelGGL(dense_tiles_kernel, dim3(nblk), dim3(256), 0, s, rows, BM, max_tiles, tiles,
                       tile_total);
    return hipGetLastError();
}

hipError_t launch_kblock(DType dt, const void* x, void* xk, int64_t rows, int D, int64_t a_cap,
                         hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (D % kKBlock != 0 || a_cap < rows) return hipErrorInvalidValue;
    const int64_t chunks = rows * (D / (16 / (int)dtype_size(dt)));
    const unsigned nblk = (unsigned)std::min<int64_t>((chunks + 255) / 256, 65536);
    switch (dt) {
        case DType::BF16:
            hipLaunchKernelGGL(kblock_kernel<__bf16>, dim3(nblk), dim3(256), 0, s,
                               (const __bf16*)x, (__bf16*)xk, rows, D, a_cap);
            break;
        case DType::F16:
            hipLaunchKernelGGL(kblock_kernel<_Float16>, dim3(nblk), dim3(256), 0, s,
                               (const _Float16*)x, (_Float16*)xk, rows, D, a_cap);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_combine(DType dt, const CombineArgs& a, hipStream_t s) {
    switch (dt) {
        case DType::F32: return launch_combine_t<float>(a, s);
        case DType::BF16: return launch_combine_t<__bf16>(a, s);
        case DType::F16: return launch_combine_t<_Float16>(a, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace nomas
