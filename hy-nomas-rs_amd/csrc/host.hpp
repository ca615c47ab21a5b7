// Host-side C++ of the MoE feed-forward block: the layer object behind the C
// ABI, the weight sources (random init, safetensors, host arrays) and the
// error convention.
#pragma once

#include <condition_variable>
#include <cstdint>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/nomas_moe.h"
#include "kernels.hpp"

namespace nomas {

// ---- stage timing -----------------------------------------------------------
// One profiled forward's six stages: stage i's events are ev[2 i] (start) and
// ev[2 i + 1] (stop), stamped by the runtime at the start of the stage's first
// kernel and the end of its last one (launch_kernel).  A stage that launches
// nothing records only its start event (so that later stages still have one to
// synchronise on) and is flagged in `empty`; its time reads zero.  The
// destructor leaves no stage in progress on the thread, whatever path the
// forward returns by.
constexpr int kProfStages = 6;
constexpr int kProfEvents = 2 * kProfStages;
class StageClock {
public:
    StageClock(hipEvent_t* ev, uint8_t* empty, hipStream_t s) : ev_(ev), empty_(empty), s_(s) {}
    ~StageClock() { stage_timing() = nullptr; }
    StageClock(const StageClock&) = delete;
    StageClock& operator=(const StageClock&) = delete;
    // ends stage i - 1 and begins stage i (i == kProfStages: ends the last)
    hipError_t mark(int i) {
        if (!ev_) return hipSuccess;
        stage_timing() = nullptr;
        if (open_) {
            empty_[i - 1] = !cur_.launched;
            if (!cur_.launched) {
                const hipError_t e = hipEventRecord(cur_.start, s_);
                if (e != hipSuccess) return e;
            }
        }
        open_ = i < kProfStages;
        if (open_) {
            cur_ = StageTiming{ev_[2 * i], ev_[2 * i + 1], false};
            stage_timing() = &cur_;
        }
        return hipSuccess;
    }

private:
    hipEvent_t* ev_;
    uint8_t* empty_;
    hipStream_t s_;
    StageTiming cur_{nullptr, nullptr, false};
    bool open_ = false;
};

// ---- errors ---------------------------------------------------------------
// Thread-local last error; functions return a nomas_status code.
int set_error(int code, const char* fmt, ...);
const char* last_error();
void clear_error();

// ---- host <-> device copies for the host-tensor forward (host_copy.cpp) ----
// memcpy split over a few persistent worker threads (the caller takes a part)
class CopyPool {
public:
    explicit CopyPool(int workers);
    ~CopyPool();
    void copy(void* dst, const void* src, size_t n);

private:
    void loop(int part);
    void range(int part, size_t* b, size_t* e) const;
    std::vector<std::thread> threads_;
    std::mutex m_;
    std::condition_variable cv_work_, cv_done_;
    uint64_t gen_ = 0;
    int remaining_ = 0;
    bool stop_ = false;
    const int parts_;
    unsigned char* dst_ = nullptr;
    const unsigned char* src_ = nullptr;
    size_t n_ = 0;
};

// Pageable host memory <-> device through two pinned staging buffers, the
// host copies of one chunk overlapping the DMA of the other.
class HostStager {
public:
    ~HostStager();
    int to_device(void* dst_dev, const void* src_host, size_t bytes, hipStream_t s);
    int to_host(void* dst_host, const void* src_dev, size_t bytes, hipStream_t s);

private:
    int ensure();
    void release();
    void* pin_[2] = {nullptr, nullptr};
    hipEvent_t ev_[2] = {nullptr, nullptr};
    std::unique_ptr<CopyPool> pool_;
};

// ---- generator (generator.cpp) -------------------------------------------
uint64_t path_seed(uint64_t seed, const char* path);
void randn_affine(uint64_t seed, double mean, double std, int64_t n, float* out);
uint16_t f32_to_bf16_bits(float f);
float bf16_bits_to_f32(uint16_t b);
uint16_t f32_to_f16_bits(float f);
float f16_bits_to_f32(uint16_t b);

// ---- safetensors (safetensors.cpp) ---------------------------------------
struct StTensor {
    std::string dtype;           // "F32", "F64", "BF16", "F16", ...
    std::vector<int64_t> shape;
    std::vector<uint8_t> data;   // raw little-endian payload
};

// Reads the named tensors of `files` (later files override earlier ones).
// Tensors not present are left out of `out`.  Returns a nomas_status.
int read_safetensors(const std::vector<std::string>& files, const std::vector<std::string>& names,
                     std::map<std::string, StTensor>* out);

// Converts a safetensors payload to f32 (F32/F64/BF16/F16 sources).
int st_to_f32(const StTensor& t, std::vector<float>* out);

// ---- the layer -----------------------------------------------------------

// Device buffers of one forward.  The handle keeps its own (grown as
// needed); the no-allocation forward lays the same buffers out in the
// device's scratch array.  The split-tile counters and partials come first,
// at offsets that do not depend on the row count, so counters left at zero
// by one forward are where the next one looks for them.
struct Workspace {
    int64_t cap_rows = 0;  // rows the buffers are laid out for (a multiple of 64)
    int32_t* split_cnt = nullptr;    // MFMA path: arrival counters of K-split tiles
    float* split_ws = nullptr;       // MFMA path: their f32 partial tiles
    int32_t* idx = nullptr;          // rows x k_slots
    float* w = nullptr;              // rows x k_slots
    float* gap = nullptr;            // rows
    int32_t* pos = nullptr;          // rows x k_slots
    int32_t* chunk_counts = nullptr; // chunks x E_cols
    int32_t* expert_count = nullptr; // E_cols
    int32_t* expert_off = nullptr;   // E_cols + 1
    TileInfo* tiles = nullptr;       // max_tiles
    int32_t* tile_total = nullptr;   // 3: tile count, the GEMMs' tail counters
    void* xperm = nullptr;           // a_cap x D
    void* h = nullptr;               // a_cap x H
    void* yperm = nullptr;           // a_cap x D (MoE only)
    void* block_h = nullptr;         // forward_block: rows x D
};

// The device scratch array of the no-allocation forward (scratch.hip):
// 512 MiB per GPU, enough for one 4,744-row segment of the 8B preset
// (dim 3072, 8 experts, top-2, hidden 8192: 8,128 rows).
constexpr size_t kScratchBytes = (size_t)512 << 20;
// Its address on `device` (looked up once per device; the first call also
// clears the split-tile counters with a kernel on `s`).  Never allocates.
// Each call counts as one use of the array: *gen receives that use's number
// on this device (1, 2, ...).
int scratch_acquire(int device, hipStream_t s, void** out, uint64_t* gen);
// The number of the last use of the array on `device` (0 before the first).
uint64_t scratch_generation(int device);

// Parameters of one Lin in f32, reference (out, in) layout.
struct LinF32 {
    std::vector<float> w;
    std::vector<float> b;  // empty = no bias / zero bias
};

// Expert and router parameters in f32 before rounding to the model dtype.
struct MoeParamsF32 {
    LinF32 router;
    std::vector<LinF32> gate, up, down;  // per expert
    bool has_dense = false;
    LinF32 dgate, dup, ddown;
};

class MoeLayer {
public:
    MoeLayer(const nomas_moe_config& cfg, int64_t dim, int64_t hidden, DType dt, int device);
    // A dense SwiGLU feed-forward (mlp.rs:39-48): one expert that every row
    // goes to with gate 1, no router; forward skips routing, dispatch and
    // combine.
    struct DenseTag {};
    MoeLayer(DenseTag, int64_t dim, int64_t hidden, DType dt, int device);
    ~MoeLayer();
    MoeLayer(const MoeLayer&) = delete;
    MoeLayer& operator=(const MoeLayer&) = delete;

    // Checks config and shape support before anything touches the GPU.
    static int check_shape(const nomas_moe_config& cfg, int64_t dim, int64_t hidden, int dtype);

    // Uploads parameters given as host arrays in the model dtype (reference
    // layout).  Any bias may be null (zero).  Packs for the GEMM path.
    int upload(const void* router_w, const void* gate_w, const void* gate_b, const void* up_w,
               const void* up_b, const void* down_w, const void* down_b, const void* dg_w,
               const void* dg_b, const void* du_w, const void* du_b, const void* dd_w,
               const void* dd_b);
    // Rounds f32 parameters to the model dtype and uploads them.
    int upload_f32(const MoeParamsF32& p);

    int forward(const void* x, void* y, int64_t rows, hipStream_t s);
    // forward() with every device buffer in the device's scratch array: no
    // allocation, and an error if `rows` needs more than kScratchBytes.
    int forward_noalloc(const void* x, void* y, int64_t rows, hipStream_t s);
    // The FFN half of a DiT block around the MoE (block.rs:96-101):
    // out = x + moe(modulate(norm2(x), shift, scale)) * gate, with (rows / seq,
    // D) f32 shift / scale / gate and an optional f32 norm gain, all device
    // pointers.  out may alias x.
    struct BlockArgs {
        int64_t seq;
        const float* norm_w;
        double eps;
        const float* shift;
        const float* scale;
        const float* gate;
    };
    int forward_block(const void* x, void* out, int64_t rows, const BlockArgs& b, hipStream_t s);
    int forward_host(const void* x, void* y, int64_t rows);
    int forward_host_pieces(const void* x, void* y, int64_t rows, int np, void* dx, void* dy);
    int routing(int32_t* idx, float* w, int32_t* counts, float* gap);
    int set_profiling(bool on);
    int stage_times(float* ms6);

    int64_t n_params() const;
    int64_t dim() const { return D_; }
    int64_t hidden() const { return H_; }
    int64_t experts() const { return E_; }
    int64_t top_k() const { return k_; }
    DType dtype() const { return dt_; }
    bool uses_mfma() const { return mfma_; }
    bool dense_only() const { return dense_only_; }

private:
    int ensure_workspace(int64_t rows);
    void free_workspace();
    int max_tiles(int64_t rows) const;
    // Lays out the buffers of a forward on up to `cap` rows (a multiple of
    // 64) from `base` (nullptr: sizes only) and returns the bytes used.
    size_t layout(int64_t cap, bool block, uint8_t* base, Workspace* w) const;

    int64_t D_, H_, E_, k_;
    int64_t Ecols_, kslots_;  // with the shared dense branch: E + 1, k + 1
    double shared_dense_;
    DType dt_;
    int device_;
    bool mfma_;
    int BM_;
    bool dense_only_ = false;
    int forward_dense(const void* x, void* y, int64_t rows, hipStream_t s);
    int check_forward(const void* x, const void* y, int64_t rows) const;
    int forward_impl(const void* x, void* y, int64_t rows, hipStream_t s, const BlockArgs* blk);
    // the stages of a routed forward on the buffers of `w`
    int run_routed(const void* x, void* y, int64_t rows, hipStream_t s, const BlockArgs* blk,
                   const Workspace& w);
    int finish_forward(int64_t rows, hipStream_t s, const Workspace& w);
    bool want_block_ = false;  // the workspace holds h for forward_block

    // device weights
    void* d_wr_ = nullptr;
    void* d_w1_ = nullptr;    // gate/up: MFMA packed [Ecols][2H][D], else [Ecols][2][H][D]
    float* d_b1_ = nullptr;   // matching layout, f32
    void* d_w2_ = nullptr;    // down [Ecols][D][H]
    float* d_b2_ = nullptr;   // [Ecols][D]

    // the handle's workspace (sized for ws_.cap_rows rows)
    void* d_ws_ = nullptr;
    Workspace ws_;
    // where the last forward's routing lives: ws_, or the scratch array
    Workspace last_ws_;
    uint64_t last_scratch_gen_ = 0;  // scratch use of the last no-allocation forward
    bool last_in_scratch_ = false;
    // forward_host: device copies of x and y, kept between calls (grown as
    // needed), and the pinned staging of the copies
    void* d_hio_ = nullptr;
    size_t hio_bytes_ = 0;  // bytes of each of the two halves
    HostStager stager_;
    // large host-tensor forwards run in row pieces: the copies of one piece
    // overlap the forward of another (two non-blocking streams of the
    // default priority, an input-landed and a forward-done event per piece)
    static constexpr int kHostMaxPieces = 4;
    static constexpr int64_t kHostPieceRows = 4096;  // at least, per piece
    hipStream_t hs_copy_ = nullptr, hs_comp_ = nullptr;
    hipEvent_t hev_in_[kHostMaxPieces] = {}, hev_fw_[kHostMaxPieces] = {};
    int host_pipe_setup();
    // the routing of a pieced forward, gathered per piece: idx and w
    // [rows][k_slots], gap [rows], then each piece's expert counts [E_cols]
    void* d_route_ = nullptr;
    size_t route_bytes_ = 0;
    int host_pieces_ = 0;  // pieces of the last forward when it was pieced, else 0

    int64_t last_rows_ = -1;
    hipStream_t last_stream_ = nullptr;
    // recorded at the end of every forward: a forward on another stream waits
    // for it, since both use the same workspace
    hipEvent_t done_ = nullptr;
    bool done_recorded_ = false;

    // profiling: one set of kProfEvents events per recorded forward
    bool profiling_ = false;
    static constexpr int kRing = 512;
    std::vector<hipEvent_t> events_;
    std::vector<uint8_t> stage_empty_;  // kProfStages flags per event set
    int recorded_ = 0;
};

}  // namespace nomas
