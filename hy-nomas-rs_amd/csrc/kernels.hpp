// Host-side launch interface of the MoE feed-forward kernels.
//
// Pipeline of one forward (all on one stream):
//   router  -> topk_idx / topk_w / gap per row, per-chunk expert histogram
//   dispatch-> expert counts/offsets, GEMM tile table, stable permutation
//              (tok_pos) + gather of x rows (x_perm)
//   gemm_gate_up -> h = silu(x W_gate^T + b_gate) * (x W_up^T + b_up)
//   gemm_down    -> y_perm = h W_down^T + b_down
//   combine -> out[t] = sum over the row's slots (ascending expert) of w * y_perm
#pragma once

#include <hip/hip_ext.h>

#include "common.hpp"

namespace nomas {

constexpr int kMaxExperts = 256;  // router LDS holds 64 rows x E f64 logits

// Kernel-exact stage timing.  While a layer records a profiled forward, this
// thread's stage in progress is set here, and every launch of the stage
// carries its events: the runtime stamps the start event when the stage's
// first kernel starts and the stop event when each kernel ends (the last one
// counts).  Null when not profiling.
struct StageTiming {
    hipEvent_t start, stop;
    bool launched;
};
StageTiming*& stage_timing();

// Every kernel of the library is launched through here (errors are left for
// the caller's hipGetLastError).
template <typename F, typename... Args>
inline void launch_kernel(F kernel, dim3 grid, dim3 block, uint32_t lds, hipStream_t s,
                          Args... args) {
    StageTiming* t = stage_timing();
    hipEvent_t start = nullptr, stop = nullptr;
    if (t) {
        start = t->launched ? nullptr : t->start;
        stop = t->stop;
        t->launched = true;
    }
    hipExtLaunchKernelGGL(kernel, grid, block, lds, s, start, stop, 0u, args...);
}

// Tile height (token rows) of the MFMA and of the general grouped GEMM.
constexpr int kMfmaBM = 256;
constexpr int kMfmaBN = 256;
constexpr int kSimtBM = 64;

// The FFN half of a DiT block around the MoE (block.rs:96-101):
//   h   = modulate(norm2(x), shift, scale)   (norm.rs:55-65, modulate.rs:69-79)
//   out = x + moe(h) * gate
// Row r belongs to sequence r / seq; shift, scale, gate are (sequences, D) f32.
// seam_h_kernel writes h (read by the router and the dispatch as their x);
// the combine applies the gated residual in its epilogue.
struct SeamArgs {
    const void* x;        // rows x D, model dtype
    void* h;              // rows x D, model dtype
    int64_t rows;
    int D;
    int64_t seq;          // rows per sequence
    const float* norm_w;  // D (null: no affine gain)
    double eps;
    const float* shift;   // sequences x D
    const float* scale;
    int factor_lds;       // set by the launcher: LDS bytes for the factors
};

struct RouterArgs {
    const void* x;
    const void* wr;
    int64_t rows;
    int D, E, k;
    int k_slots;        // k, or k + 1 with the shared dense slot
    float dense_coef;   // gate of the dense slot
    int32_t* topk_idx;  // rows x k_slots
    float* topk_w;      // rows x k_slots
    float* gap;         // rows
    int32_t* chunk_counts;  // ceil(rows / block_rows) x E_cols: one histogram per router block
    int block_rows;         // rows per router block: router_block_rows() of this launch
};


// K-blocked layout (MFMA path): a matrix of R rows and K columns is stored as
// column blocks of KB = 64 bytes of elements (32 for 16-bit types, 16 for
// f32), each R rows x KB contiguous elements, i.e. element (r, k) at
// ((k / KB) * R + r) * KB + k % KB.  One k step of a GEMM tile (256 rows x
// 64 bytes) is then a single contiguous 16 KB run of memory, fetched as whole
// 128-byte lines.
constexpr int kKBlockBytes = 64;
template <typename T>
__host__ __device__ constexpr int kblock_elems() { return kKBlockBytes / (int)sizeof(T); }

struct DispatchArgs {
    const void* x;
    int64_t rows;
    int D, E_cols, k_slots;
    const int32_t* topk_idx;
    const int32_t* chunk_counts;  // ceil(rows / count_rows) x E_cols, from the router
    int nchunks;            // 64-row chunks
    int count_rows;         // rows per histogram (the router's rows per block: 64 or 32)
    int BM;                 // GEMM tile rows
    int max_tiles;
    int32_t* expert_count;  // E_cols
    int32_t* expert_off;    // E_cols + 1
    TileInfo* tiles;        // max_tiles
    int32_t* tile_total;    // 3: the tile count, then the two GEMMs' tail counters (cleared)
    int32_t* tok_pos;  // rows x k_slots
    void* x_perm;      // a_cap x D, row-major or K-blocked
    int64_t a_cap;     // rows of x_perm (positions must stay below)
    int kblocked;      // 1: write x_perm K-blocked (R = a_cap), 0: row-major
};

struct GemmArgs {
    const void* X;     // token rows (a_cap x K), expert-contiguous
    const void* W;     // expert weights
    const float* bias; // expert biases (f32)
    void* out;
    const TileInfo* tiles;
    const int32_t* tile_total;
    int max_tiles;
    int N;  // output columns of the weight GEMM (2H for gate/up, D for down)
    int K;
    int num_experts;  // experts with weights (tiles naming others are skipped)
    int64_t a_cap;    // rows of X / out (tiles reaching beyond are skipped)
    // MFMA path: f32 partial sums of tiles split along K (kSplitUnits units of
    // kSplitUnitFloats each) and one arrival counter per split tile (zero
    // between launches: the last part to arrive resets it)
    float* split_ws;
    int32_t* split_cnt;
    // MFMA path: the ticket counter of the tail units handed out at run time
    // (zero before the launch: the kernel that writes the tile table clears it)
    int32_t* tail_cnt = nullptr;
    // down GEMM (MFMA path): write `out` with the nontemporal hint.  For
    // outputs larger than the chip's last-level cache, which the combine reads
    // back once: their lines then go to HBM as they are written instead of
    // being evicted dirty while the combine streams them in.
    int out_nt = 0;
};
// MI355X's last-level cache (the Infinity Cache in front of HBM).
constexpr int64_t kLastLevelCacheBytes = (int64_t)256 << 20;
// MI355X's L2 caches together (8 XCDs x 4 MB).
constexpr int64_t kL2TotalBytes = (int64_t)32 << 20;
// One split unit's partial tile: 256 x 256 f32.
constexpr int64_t kSplitUnitFloats = 256 * 256;
constexpr int kSplitUnits = 256;

struct CombineArgs {
    const void* y_perm;
    const int32_t* tok_pos;
    const float* topk_w;
    int64_t rows;
    int D, k_slots;
    void* out;
    int64_t a_cap;  // rows of y_perm
    // gated residual (gate non-null): out = x + out_moe * gate[row / seq]
    const void* resid_x;  // rows x D, model dtype
    const float* gate;    // sequences x D
    int64_t seq;
    // write `out` with the nontemporal hint: when y_perm is larger than the
    // last-level cache, its reads stream through it and would evict the
    // output's dirty lines into the middle of them anyway
    int out_nt = 0;
};

size_t router_lds_bytes(int E);
// Rows per router block (and per histogram it writes) for a launch of
// `rows` rows: 64, or 32 for small launches that 64-row blocks would leave
// short of bytes in flight.
int router_block_rows(DType dt, int64_t rows, int D, int E);
// Smallest rows per router block: the histogram buffer holds
// ceil(rows / kMinRouterBlockRows) histograms.
constexpr int kMinRouterBlockRows = 32;
// Whether the dispatch kernel's LDS holds E_cols experts and k_slots slots per row.
bool dispatch_supported(int E_cols, int k_slots);

hipError_t launch_seam_h(DType dt, const SeamArgs& a, hipStream_t s);
hipError_t launch_gated_residual(DType dt, const void* x, const void* y, const float* gate,
                                 void* out, int64_t rows, int D, int64_t seq, hipStream_t s);
hipError_t launch_router(DType dt, const RouterArgs& a, hipStream_t s);
hipError_t launch_dispatch(DType dt, const DispatchArgs& a, hipStream_t s);
// MFMA grouped GEMMs (bf16 / f16): W packed as described in moe_layer.cpp.
hipError_t launch_gemm_gate_up_mfma(DType dt, const GemmArgs& a, hipStream_t s);
hipError_t launch_gemm_down_mfma(DType dt, const GemmArgs& a, hipStream_t s);
// General grouped GEMMs (any dtype, any shape).
hipError_t launch_gemm_gate_up_simt(DType dt, const GemmArgs& a, hipStream_t s);
hipError_t launch_gemm_down_simt(DType dt, const GemmArgs& a, hipStream_t s);
hipError_t launch_combine(DType dt, const CombineArgs& a, hipStream_t s);
// Dense feed-forward (no routing): the tile table of `rows` rows of one
// expert in BM-row tiles (max_tiles entries written), and x re-laid out
// K-blocked ((col / 32) * a_cap + row) * 32 + col % 32 for the MFMA GEMM.
hipError_t launch_dense_tiles(int64_t rows, int BM, int max_tiles, TileInfo* tiles,
                              int32_t* tile_total, hipStream_t s);
hipError_t launch_kblock(DType dt, const void* x, void* xk, int64_t rows, int D, int64_t a_cap,
                         hipStream_t s);

}  // namespace nomas
