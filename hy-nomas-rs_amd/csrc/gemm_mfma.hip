// Grouped expert GEMMs on CDNA4 matrix cores (bf16 / f16 / f32 in, f32
// accumulate).
//
// Problem per expert e (rows of x_perm / h that belong to e):
//   gate/up:  h[m, :] = silu(x W_gate^T + b_gate) * (x W_up^T + b_up)   K = D, N = 2H
//   down:     y[m, :] = h W_down^T + b_down                              K = H, N = D
// (hy-nomas-rs mlp.rs:42-46 applied to the rows routed to e).
//
// Work unit: a 256 x 256 output tile of one expert.  The dispatch kernel
// lists the experts' 256-row tiles; the grid enumerates (row tile, column
// tile).
//  - Operands: weights are the MFMA "A" operand (rows = output columns),
//    token rows the "B" operand, so each lane's accumulator holds 4
//    consecutive output columns of one token row.
//  - v_mfma_f32_16x16x32_{bf16,f16} (f32: four v_mfma_f32_16x16x4f32 per
//    16-byte fragment): 4 waves in a 2 x 2 grid, each wave a
//    128 x 128 tile of 8 x 8 MFMA blocks (256 f32 accumulators per lane, in
//    AGPRs).  The 16x16x32 form does the same work per cycle as 32x32x16 for
//    less power, which matters because these GEMMs run at the power limit.
//  - K is walked 64 bytes at a time (32 elements, 16 for f32) through a ring
//    of 4 LDS stages filled by direct global->LDS loads
//    (global_load_lds_dwordx4, no VGPR staging), issued 2-3 steps ahead.  Operands are K-blocked in memory
//    (kernels.hpp): one k step of a tile is a single contiguous 16 KB run.
//  - LDS rows (64 bytes) keep their 16-byte chunks XOR-swizzled by row bits
//    1-2, so the 16-row operand reads (ds_read_b128) are free of bank
//    conflicts, and one lane's read offset is the same for every block (the
//    block index folds into the instruction's immediate offset).  The swizzle
//    is applied on the global side: lane l of a load instruction always
//    writes LDS slot l and reads the global chunk that belongs there.
//  - Gate and up rows are interleaved in groups of 32 when the weights are
//    packed (rows 64g..64g+31 = gate 32g.., rows 64g+32.. = up 32g..), so
//    gate block 4p+b and up block 4p+b+2 of a wave hold the same hidden units
//    in the same lanes, and the SwiGLU is applied in the epilogue without an
//    extra pass over HBM.
//  - Block ids are mapped to tiles XCD-aware (tile_map.hpp): the XCDs work on
//    one expert at a time (its weights shared through the MALL), each XCD on
//    an 8 x 4 group of tiles that share panels in its own L2.
#include <type_traits>

#include "kernels.hpp"
#include "lds_dma.hpp"
#include "tile_map.hpp"

namespace nomas {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// A lane's 16-byte operand fragment (one row, 64 bytes of k per stage split
// over the 4 lane groups) feeds kSub MFMAs: one 16x16x32 for 16-bit types,
// four 16x16x4 for f32 (MFMA t takes element t; lane group g then holds
// k = 4 g + t of the stage, the same for both operands).
template <typename T> struct Mfma;
template <> struct Mfma<__bf16> {
    typedef bf16x8_t V;
    static constexpr int kSub = 1;
    static __device__ __forceinline__ f32x4_t run(V a, V b, f32x4_t c, int) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};
template <> struct Mfma<_Float16> {
    typedef f16x8_t V;
    static constexpr int kSub = 1;
    static __device__ __forceinline__ f32x4_t run(V a, V b, f32x4_t c, int) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};
template <> struct Mfma<float> {
    typedef f32x4_t V;
    static constexpr int kSub = 4;
    static __device__ __forceinline__ f32x4_t run(V a, V b, f32x4_t c, int t) {
        return __builtin_amdgcn_mfma_f32_16x16x4f32(a[t], b[t], c, 0, 0, 0);
    }
};

enum { kGateUp = 0, kDown = 1 };

constexpr int kStages = 4;  // LDS ring depth; the main loop is unrolled over one turn
// Waves along the token rows of a tile: 2 (4 waves, one per SIMD, 128 x 128
// outputs each) or 4 (8 waves, two per SIMD, 64 token rows x 128 weight rows
// each: while one wave of a SIMD waits, the other issues MFMAs).
#ifndef NOMAS_GEMM_WAVE_ROWS
#define NOMAS_GEMM_WAVE_ROWS 2
#endif
constexpr int kWaveRows = NOMAS_GEMM_WAVE_ROWS;
static_assert(kWaveRows == 2 || kWaveRows == 4, "2 or 4 waves along the token rows");

// Physical 16-byte chunk of logical chunk c in LDS row r is c ^ swz(r) (4
// chunks per row).  Any 8 consecutive rows read at one logical chunk then hit
// 8 distinct (row parity, chunk) bank groups.
__device__ __forceinline__ int swz(int r) { return (r >> 1) & 3; }

// Word 3 of a raw buffer resource (gfx9 family: 32-bit data format, no
// swizzle); with stride 0 the buffer is a plain byte range [0, num_records).
constexpr int kBufferRsrcWord3 = 0x00020000;

template <typename T, int MODE, int BM, int BN, int BK, int S, int NWM>
__global__ __launch_bounds__(NWM * 2 * kWave, 1) void gemm_mfma_kernel(GemmArgs a) {
    using V = typename Mfma<T>::V;
    constexpr int kThreads = NWM * 2 * kWave;     // NWM x 2 waves
    constexpr int WM = BM / NWM, WN = BN / 2;     // wave tile: token rows x weight rows
    constexpr int SM = WM / 16, SN = WN / 16;     // 16x16 MFMA blocks per wave
    constexpr int EPC = 16 / (int)sizeof(T);      // elements per 16-byte chunk
    constexpr int CH = BK / EPC;                  // 16-byte chunks per LDS row
    constexpr int kSub = Mfma<T>::kSub;
    constexpr int RPI = kWave / CH;               // rows filled by one load instruction
    constexpr int NW = kThreads / kWave;
    constexpr int QW = BN / RPI / NW;             // load instructions per wave per k step
    constexpr int QX = BM / RPI / NW;
    constexpr int Q = QW + QX;
    static_assert(BK * (int)sizeof(T) == kKBlockBytes && CH == 4, "64 bytes of k per stage");
    static_assert(S == 4, "ring of 4 stages, the loop unrolled over one turn");
    static_assert(SN == 8 && SM * NWM == 16 && Q * NWM == 16,
                  "row schedule: 8 rows of SM blocks, Q loads per step");
    constexpr int RPL = SN / Q;  // rows of the schedule per load (1 or 2)
    static_assert(MODE == kDown || SN % 4 == 0, "gate/up pairs are 2 blocks apart in groups of 4");
    static_assert(BK == kblock_elems<T>(), "operands are K-blocked by the k step");

    // The ring: S weight stages, then S token-row stages (offsets compile-time
    // after unrolling).  The down GEMM's epilogue reuses it, extended to hold
    // the rows of one staging round (all 256 for 16-bit types, 128 for f32).
    constexpr int kRingBytes = S * (BN + BM) * BK * (int)sizeof(T);
    constexpr int kRounds = sizeof(T) == 2 ? 1 : 2;          // down epilogue rounds
    constexpr int kOS = BN * (int)sizeof(T) + 16;            // padded staging row, bytes
    constexpr int kStageOut = MODE == kDown ? BM / kRounds * kOS : 0;
    constexpr int kLdsBytes = kRingBytes > kStageOut ? kRingBytes : kStageOut;
    __shared__ __attribute__((aligned(16))) unsigned char sMem[kLdsBytes];
    T* const sRing = reinterpret_cast<T*>(sMem);
    // the tile's BN biases (f32), loaded by one direct-to-LDS instruction
    __shared__ __attribute__((aligned(16))) float sBias[BN];
    static_assert(BN * sizeof(float) == kWave * 16, "one 16-byte chunk per lane");
    auto stW = [&](int s) -> T* { return sRing + s * BN * BK; };
    auto stX = [&](int s) -> T* { return sRing + S * BN * BK + s * BM * BK; };

    const int N = a.N, K = a.K;
    const int KT_tile = K / BK;  // k steps of a whole tile
    // live row tiles (the dispatch never lists more than max_tiles); the
    // block's unit: by its time-order index, or in the tail a ticket's
    const int live = min(*a.tile_total, a.max_tiles);
    const long long units = unit_count(live, N / BN, KT_tile / S), first_tail = tail_start(units);
    long long L = time_order(blockIdx.x);
    if (L >= first_tail) {
        __shared__ int s_ticket;
        if (threadIdx.x == 0)
            s_ticket = __hip_atomic_fetch_add(a.tail_cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        L = first_tail + s_ticket;
        if (L >= units) return;
    }
    WorkUnit wu;
    unit_at(L, N / BN, live, KT_tile / S, &wu);
    const int mt = wu.mt, nt = wu.nt;
    const TileInfo ti = a.tiles[mt];
    const int e = ti.expert, row0 = ti.row0, nrows = ti.rows;
    if (e < 0 || e >= a.num_experts || nrows < 1 || row0 < 0 || row0 + (int64_t)nrows > a.a_cap)
        return;
    const int n0 = nt * BN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;  // wm in [0, NWM)
    const int uwave = __builtin_amdgcn_readfirstlane(wave);  // wave-uniform (SGPR) copy
    const int l16 = lane & 15, lq = lane >> 4;

    // K-blocked operands: step kt of this tile is one contiguous block of
    // 256 rows x BK for the weights (stride N * BK between steps) and for the
    // token rows (stride a_cap * BK).
    // A split unit walks its own 1/parts of the k steps.
    const int KT = KT_tile / wu.parts;
    const int64_t wstep = (int64_t)N * BK, xstep = a.a_cap * BK;
    const T* Wt = static_cast<const T*>(a.W) + ((int64_t)e * KT_tile * N + n0) * BK +
                  (int64_t)wu.part * KT * wstep;
    const T* Xt = static_cast<const T*>(a.X) + (int64_t)row0 * BK + (int64_t)wu.part * KT * xstep;

    // Lane l of load instruction q writes LDS bytes [q*1024 + l*16, +16): tile
    // row r = RPI*q + l/CH, stored chunk l%CH, which holds logical chunk
    // (l%CH) ^ swz(r) of that row.  The token rows are read through a raw
    // buffer resource over the tile's live rows of one K-block: rows past the
    // tile's end fail its range check and arrive as zeros, with no memory
    // traffic (their results are never stored, and matrix-core operands of
    // zero draw much less power than data: an all-CU loop of these MFMAs runs
    // 23% faster with one operand zero at the chip's power limit).
    int woff[QW], xoff[QX];
#pragma unroll
    for (int i = 0; i < QW; ++i) {
        const int r = (wave * QW + i) * RPI + lane / CH;
        woff[i] = (r * BK + (((lane % CH) ^ swz(r)) * EPC)) * (int)sizeof(T);  // bytes
    }
#pragma unroll
    for (int i = 0; i < QX; ++i) {
        const int r = (wave * QX + i) * RPI + lane / CH;
        xoff[i] = (r * BK + (((lane % CH) ^ swz(r)) * EPC)) * (int)sizeof(T);  // bytes
    }

    f32x4_t acc[SN][SM];

    // load q (0..Q-1) of step kt into ring slot `slot`: q < QW are weight
    // rows, the rest token rows
    const int xbytes = nrows * BK * (int)sizeof(T);  // one K-block's live token rows
    // The loads of one operand and step go out as a group (q = 0.. or
    // QW.., in order): load q of a wave fills the 1 KB LDS block after load
    // q - 1's and reads the 1 KB after its global run (woff[q] = woff[0] +
    // 1 KB q, likewise xoff), so the group shares one M0 write and each load
    // carries its 1 KB step in the immediate offset.  16-bit types only: in
    // the f32 down kernel (four times the MFMAs per load) the register
    // allocator then spills 416 bytes per lane instead of 56.
    static_assert(RPI * BK * (int)sizeof(T) == 1024 && QW <= 4 && QX <= 4, "1 KB per load, 4 at most");
    auto dma = [&](int q, int kt, int slot) {
        if constexpr (sizeof(T) == 4) {
            if (q < QW)
                lds_dma16(Wt + kt * wstep, woff[q], lds_addr(stW(slot)) + (uwave * QW + q) * 1024);
            else
                lds_dma16_buf(__builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(Xt + kt * xstep), 0, xbytes,
                                                                kBufferRsrcWord3),
                              xoff[q - QW], lds_addr(stX(slot)) + (uwave * QX + q - QW) * 1024);
        } else if (q < QW) {
            if (q == 0) set_lds_m0(lds_addr(stW(slot)) + uwave * QW * 1024);
            lds_dma16_q(q, Wt + kt * wstep, woff[0]);
        } else {
            if (q == QW) set_lds_m0(lds_addr(stX(slot)) + uwave * QX * 1024);
            lds_dma16_buf_q(q - QW,
                            __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(Xt + kt * xstep), 0, xbytes,
                                                              kBufferRsrcWord3),
                            xoff[0]);
        }
    };
    // operand fragments: lane (l16, lq) holds row l16 of a 16-row block, k chunk lq
    auto rdA = [&](int slot, int i) -> V {
        const int r = wn * WN + i * 16 + l16;
        return *reinterpret_cast<const V*>(&stW(slot)[r * BK + ((lq ^ swz(r)) * EPC)]);
    };
    auto rdB = [&](int slot, int j) -> V {
        const int r = wm * WM + j * 16 + l16;
        return *reinterpret_cast<const V*>(&stX(slot)[r * BK + ((lq ^ swz(r)) * EPC)]);
    };

    // Stage s (ring slot s % 4) runs the 64 MFMAs of k step s as 8 rows
    // (weight block i) of 8 (token block j), with one block barrier B_s in the
    // middle:
    //   rows 0..3  read A block 4+i of stage s (used 4 rows later) and issue
    //              loads 4..7 of step s + 2 (into slot (s + 2) % 4, which
    //              every wave finished reading before B_{s-1});
    //   B_s        this wave's loads of step s + 1 have landed (exactly the 8
    //              loads of step s + 2 may still be in flight); after the
    //              barrier every wave's have, and every wave is done with
    //              stage s - 1;
    //   rows 4..7  read A block i-4 of stage s + 1 into the register that
    //              row i-4 freed, and issue loads 0..3 of step s + 3 (into
    //              slot (s - 1) % 4);
    //   row 7      after MFMA (7, j), read B block j of stage s + 1 into the
    //              register that MFMA was the last to use (8 MFMAs ahead).
    // Every fragment read thus lands well ahead of its MFMA with only 16
    // fragment registers, and each load is pinned right behind an MFMA: a
    // load can stall this wave's in-order issue while the memory pipeline is
    // busy, and behind a fresh MFMA that stall overlaps the MFMA instead of
    // idling the matrix core.  Loads past the end re-load the last step (into
    // slots that are never read again), which keeps the loop branch-free and
    // the wait counts constant.
    auto cl = [&](int kt) { return kt < KT ? kt : KT - 1; };
    // Bias slice first: wave 0's oldest load (zeros for the parts of a split
    // tile after the first).  The accumulators start at it, set while the
    // first steps' loads are in flight, so the epilogue adds no bias.
    if (uwave == 0) {
        if (wu.part == 0)
            lds_dma16(a.bias + (int64_t)e * N + n0, lane * 16, lds_addr(sBias));
        else
            *reinterpret_cast<uint4*>(&sBias[lane * 4]) = make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int q = 0; q < Q; ++q) dma(q, 0, 0);
#pragma unroll
    for (int q = 0; q < Q; ++q) dma(q, cl(1), 1);
#pragma unroll
    for (int q = 0; q < Q / 2; ++q) dma(q, cl(2), 2);
    wait_vmcnt<2 * Q + Q / 2>();   // wave 0: the bias has landed
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();  // ... and is visible to every wave
#pragma unroll
    for (int i = 0; i < SN; ++i) {
        const float4 b = *reinterpret_cast<const float4*>(&sBias[wn * WN + i * 16 + 4 * lq]);
#pragma unroll
        for (int j = 0; j < SM; ++j) acc[i][j] = f32x4_t{b.x, b.y, b.z, b.w};
    }
    wait_vmcnt<Q + Q / 2>();
    __builtin_amdgcn_s_barrier();  // bare: __syncthreads() would add a vmcnt(0) fence
    __builtin_amdgcn_sched_barrier(0);
    V fa[SN], fb[SM];
#pragma unroll
    for (int j = 0; j < SM; ++j) fb[j] = rdB(0, j);
#pragma unroll
    for (int i = 0; i < SN / 2; ++i) fa[i] = rdA(0, i);
    __builtin_amdgcn_sched_barrier(0);
    // Waves whose token rows all lie past the tile's live rows (in a tile
    // of at most WM * wm live rows) hold padding rows only: they skip the
    // MFMAs (their accumulators keep their start values and the epilogue
    // stores no padding row) but keep their share of the loads and every
    // barrier, in the same order as the loop below.  At the chip's power
    // limit the skipped MFMAs are time saved.
    const bool pad_wave = (uwave >> 1) * WM >= nrows;
    if (pad_wave) {
        for (int kt0 = 0; kt0 < KT; kt0 += S) {
#pragma unroll
            for (int u = 0; u < S; ++u) {
                const int s = kt0 + u;
#pragma unroll
                for (int q = 0; q < Q / 2; ++q) dma(Q / 2 + q, cl(s + 2), (u + 2) % S);
                wait_vmcnt<Q>();
                __builtin_amdgcn_s_barrier();
#pragma unroll
                for (int q = 0; q < Q / 2; ++q) dma(q, cl(s + 3), (u + 3) % S);
            }
        }
    } else
    for (int kt0 = 0; kt0 < KT; kt0 += S) {
#pragma unroll
        for (int u = 0; u < S; ++u) {
            const int s = kt0 + u;
#pragma unroll
            for (int i = 0; i < SN; ++i) {
                if (i == SN / 2) {
                    __builtin_amdgcn_sched_barrier(0);
                    wait_vmcnt<Q>();
                    __builtin_amdgcn_s_barrier();
                    __builtin_amdgcn_sched_barrier(0);
                }
                if (i < SN / 2) fa[SN / 2 + i] = rdA(u, SN / 2 + i);
                else fa[i - SN / 2] = rdA((u + 1) % S, i - SN / 2);
#pragma unroll
                for (int t = 0; t < kSub; ++t)
#pragma unroll
                for (int j = 0; j < SM; ++j) {
                    acc[i][j] = Mfma<T>::run(fa[i], fb[j], acc[i][j], t);
                    if (t == kSub - 1 && i == SN - 1) fb[j] = rdB((u + 1) % S, j);
                    if (t == 0 && j == 1 && i % RPL == 0) {
                        // load q of this half of the stage, every RPL-th row
                        const int q = (i % (SN / 2)) / RPL;
                        __builtin_amdgcn_sched_barrier(0);
                        if (i < SN / 2) dma(Q / 2 + q, cl(s + 2), (u + 2) % S);
                        else dma(q, cl(s + 3), (u + 3) % S);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
            }
        }
    }
    // drain the trailing loads before this block's LDS can be handed on
    wait_vmcnt<0>();

    if (wu.parts > 1) {
        // Part of a split tile: publish the partial sums, count arrivals; the
        // last part to arrive adds all parts in part order (the same order
        // whichever part that is, so results do not depend on timing) and
        // runs the epilogue.  The parts of one tile run on different XCDs,
        // whose L2 caches are not coherent with each other.  The hand-off is
        // a release/acquire pair at agent scope: every part's counter
        // increment is a release read-modify-write (its partial stores, done
        // by all threads before the barrier, happen-before it), and the part
        // whose increment completes the count (reading every other part's
        // release) runs an agent-scope acquire fence before any partial load.
        // Only that part pays for the acquire's cache invalidation.  The
        // partials themselves are written and read with the agent-scope cache
        // policy (sc1), so they travel past the XCD's L2 instead of through it.
        // Reads past the tile's `parts` partials return zero (buffer range
        // check).  The counter goes back to zero for the next launch.
        constexpr int NB = SN * SM;
        static_assert(NB * 4 * kThreads == kSplitUnitFloats, "one unit = one 256 x 256 tile");
        constexpr int kUnitBytes = (int)(kSplitUnitFloats * sizeof(float));
        constexpr int kSc1 = 16;  // cache policy: agent scope
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            a.split_ws + (int64_t)wu.slot * wu.parts * kSplitUnitFloats, 0, wu.parts * kUnitBytes,
            kBufferRsrcWord3);
#pragma unroll
        for (int i = 0; i < SN; ++i)
#pragma unroll
            for (int j = 0; j < SM; ++j)
                __builtin_amdgcn_raw_buffer_store_b128(
                    acc[i][j], rs, wu.part * kUnitBytes + ((i * SM + j) * kThreads + tid) * 16, 0, kSc1);
        wait_vmcnt<0>();
        __shared__ int s_last;
        __syncthreads();
        if (tid == 0) {
            s_last = __hip_atomic_fetch_add(&a.split_cnt[wu.slot], 1, __ATOMIC_RELEASE,
                                            __HIP_MEMORY_SCOPE_AGENT) == wu.parts - 1;
            if (s_last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        }
        __syncthreads();
        if (!s_last) return;
        // one weight block at a time: its 8 x kMaxSplit loads all in flight
        // before the first add
#pragma unroll
        for (int i = 0; i < SN; ++i) {
            f32x4_t v[SM][kMaxSplit];
#pragma unroll
            for (int j = 0; j < SM; ++j)
#pragma unroll
                for (int p = 0; p < kMaxSplit; ++p)
                    v[j][p] = __builtin_amdgcn_raw_buffer_load_b128(
                        rs, p * kUnitBytes + ((i * SM + j) * kThreads + tid) * 16, 0, kSc1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < SM; ++j) {
                f32x4_t t = v[j][0];
#pragma unroll
                for (int p = 1; p < kMaxSplit; ++p) t += v[j][p];
                acc[i][j] = t;
            }
        }
        if (tid == 0)
            __hip_atomic_store(&a.split_cnt[wu.slot], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // Epilogue (the accumulators include the bias).  Lane (l16, lq) of block
    // (i, j) holds token row wm*WM + j*16 + l16 and weight rows
    // wn*WN + i*16 + 4*lq + (0..3).
    T* out = static_cast<T*>(a.out);
    // a lane's 4 consecutive output columns as one store
    typedef typename std::conditional<sizeof(T) == 2, uint2, uint4>::type Raw4;
    if constexpr (MODE == kGateUp) {
        // h is written K-blocked for the down GEMM: (row, c) at
        // ((c / BK) * a_cap + row) * BK + c % BK
#pragma unroll
        for (int p = 0; p < SN / 4; ++p) {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                // gate block 4p + b, its up block 4p + b + 2 (32-row interleave)
                const int hc = (n0 + wn * WN + p * 64) / 2 + b * 16 + 4 * lq;
                T* hcol = out + (int64_t)(hc / BK) * a.a_cap * BK + hc % BK;
#pragma unroll
                for (int j = 0; j < SM; ++j) {
                    const int m = wm * WM + j * 16 + l16;
                    if (m >= nrows) continue;
                    T hv[4];
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        const float g = acc[4 * p + b][j][s];
                        const float u = acc[4 * p + b + 2][j][s];
                        // silu(g) * u; the reciprocal (1 ulp) and the exponential
                        // add a few f32 ulps, far inside the output tolerance
                        hv[s] = Elt<T>::from_f32(g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u);
                    }
                    Raw4 raw;
                    __builtin_memcpy(&raw, hv, sizeof(raw));
                    *reinterpret_cast<Raw4*>(hcol + (int64_t)(row0 + m) * BK) = raw;
                }
            }
        }
    } else {
        // y goes out through LDS in kRounds rounds (one for 16-bit types, two
        // for f32): every wave writes its rounded blocks of the round (4 values
        // per lane) into padded LDS rows, then all 256 threads store whole row
        // slices, 16 bytes each (64 scattered 8-byte stores per lane cost 24k
        // cycles a tile).  The barriers are bare s_barriers after lgkmcnt(0):
        // __syncthreads() would also wait for the global stores.
        constexpr int kJR = SM / kRounds;   // a wave's token blocks per round
        constexpr int kWR = kJR * 16;       // a wave's rows per round
        unsigned char* sO = sMem;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();  // every wave is done with the ring
        // lq again, from the lane counter (keeping the first one alive
        // through the loop cost a spill)
        const int lq_e = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)) >> 4;
#pragma unroll
        for (int rd = 0; rd < kRounds; ++rd) {
#pragma unroll
            for (int i = 0; i < SN; ++i) {
                const int nl = wn * WN + i * 16 + 4 * lq_e;
#pragma unroll
                for (int jj = 0; jj < kJR; ++jj) {
                    T ov[4];
#pragma unroll
                    for (int s = 0; s < 4; ++s) ov[s] = Elt<T>::from_f32(acc[i][rd * kJR + jj][s]);
                    Raw4 raw;
                    __builtin_memcpy(&raw, ov, sizeof(raw));
                    *reinterpret_cast<Raw4*>(sO + (wm * kWR + jj * 16 + l16) * kOS + nl * (int)sizeof(T)) = raw;
                }
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            __builtin_amdgcn_s_barrier();
            // staging row sr = (wave row h, row w) holds tile row h * WM + rd * kWR + w;
            // 8 pieces per thread at a time: their LDS reads all in flight before
            // the first store (one read-to-store latency per 8 pieces, not per piece)
            constexpr int kRowChunks = BN * (int)sizeof(T) / 16;
            constexpr int kPieces = NWM * kWR * kRowChunks / kThreads;  // per thread per round
            constexpr int kGrp = 8;
            static_assert(kPieces * kThreads == NWM * kWR * kRowChunks && kPieces % kGrp == 0,
                          "whole groups of pieces per thread");
#pragma unroll
            for (int g0 = 0; g0 < kPieces; g0 += kGrp) {
                uint4 v[kGrp];
#pragma unroll
                for (int u = 0; u < kGrp; ++u) {
                    const int q = tid + (g0 + u) * kThreads;
                    v[u] = *reinterpret_cast<const uint4*>(sO + (q / kRowChunks) * kOS +
                                                           (q % kRowChunks) * 16);
                }
#pragma unroll
                for (int u = 0; u < kGrp; ++u) {
                    const int q = tid + (g0 + u) * kThreads;
                    const int sr = q / kRowChunks, ch = q % kRowChunks;
                    const int tr = (sr / kWR) * WM + rd * kWR + sr % kWR;
                    if (tr < nrows) {
                        T* dst = out + (int64_t)(row0 + tr) * N + n0 + ch * EPC;
                        if (a.out_nt) store16_nt(dst, v[u]);
                        else *reinterpret_cast<uint4*>(dst) = v[u];
                    }
                }
            }
            if (rd < kRounds - 1) {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                __builtin_amdgcn_s_barrier();  // the reads of this round are done
            }
        }
    }
}

template <typename T, int MODE>
hipError_t launch_mfma_t(const GemmArgs& a, hipStream_t s) {
    constexpr int BM = kMfmaBM, BN = kMfmaBN;
    // whole column tiles, and whole turns of the ring in K
    constexpr int BK = kblock_elems<T>();
    if (a.N % BN != 0 || a.K % (BK * kStages) != 0) return hipErrorInvalidValue;
    if (a.split_ws == nullptr || a.split_cnt == nullptr || a.tail_cnt == nullptr)
        return hipErrorInvalidValue;
    // whole tiles, plus one round for the K-split units of a short last round
    static_assert(kSplitUnits == kRound, "the split units fill one round");
    const int64_t grid = tile_grid(a.max_tiles, a.N / BN) + kSplitUnits;
    if (a.max_tiles <= 0) return hipSuccess;
    if (grid > 0x7fffffff) return hipErrorInvalidValue;
    launch_kernel((gemm_mfma_kernel<T, MODE, BM, BN, BK, kStages, kWaveRows>), dim3((unsigned)grid),
                  dim3(kWaveRows * 2 * kWave), 0, s, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_gate_up_mfma(DType dt, const GemmArgs& a, hipStream_t s) {
    if (dt == DType::BF16) return launch_mfma_t<__bf16, kGateUp>(a, s);
    if (dt == DType::F16) return launch_mfma_t<_Float16, kGateUp>(a, s);
    if (dt == DType::F32) return launch_mfma_t<float, kGateUp>(a, s);
    return hipErrorInvalidValue;
}

hipError_t launch_gemm_down_mfma(DType dt, const GemmArgs& a, hipStream_t s) {
    if (dt == DType::BF16) return launch_mfma_t<__bf16, kDown>(a, s);
    if (dt == DType::F16) return launch_mfma_t<_Float16, kDown>(a, s);
    if (dt == DType::F32) return launch_mfma_t<float, kDown>(a, s);
    return hipErrorInvalidValue;
}

}  // namespace nomas
