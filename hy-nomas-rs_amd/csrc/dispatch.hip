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
#include <type_traits>

#include "kernels.hpp"
#include "seam.hpp"

namespace nomas {

namespace {

constexpr int kDispThreads = 1024;
constexpr int kDispWaves = kDispThreads / kWave;
constexpr int kSlabBytes = 512;                // bytes of a row per slab
constexpr int kSlabStride = kSlabBytes + 16;   // LDS row, padded
constexpr int kSlabPieces = kSlabBytes / 16;   // 16-byte pieces per row per slab
constexpr int kProdThreads = kDispThreads / 2; // waves 0-7 load, waves 8-15 store
constexpr int kDispCUs = 256;                  // MI355X compute units
constexpr int kDispMaxParts = 8;               // blocks sharing one chunk, at most
constexpr int kHistInFlight = 16;              // histogram loads in flight per lane
constexpr int kProdLoads = kRouterRows * kSlabPieces / kProdThreads;  // 4
static_assert(kProdLoads * kProdThreads == kRouterRows * kSlabPieces, "whole slabs");

// LDS of dispatch_kernel: two slabs (which first hold the histogram partials
// and the chunk's expert slots), then the int arrays that live to the end.
constexpr size_t kSlabLds = (size_t)2 * kRouterRows * kSlabStride;
__host__ __device__ inline size_t dispatch_lds(int E_cols, int k) {
    return kSlabLds + sizeof(int) * ((size_t)5 * (E_cols + 1) + (size_t)2 * kRouterRows * k);
}
__host__ __device__ inline bool dispatch_fits(int E_cols, int k) {
    return sizeof(int) * ((size_t)2 * kDispWaves * E_cols + (size_t)kRouterRows * k) <= kSlabLds &&
           dispatch_lds(E_cols, k) <= 160 * 1024;
}

// One block per 64-row chunk.  It does the whole bookkeeping of its chunk
// from the router's per-chunk histograms -- no separate scan pass:
//  1. rows of each expert in the chunks before it and in all chunks (each
//     wave sums every 16th chunk, the waves' partials added in LDS);
//  2. expert offsets (exclusive scan over experts, ascending) and the chunk's
//     own per-expert slot offsets; block 0 also publishes the expert counts
//     and offsets and the GEMM tile table (ceil(count / BM) tiles of BM rows
//     per expert);
//  3. the waves rank the chunk's slots, each taking every 16th expert: a
//     ballot over the 64 rows gives every row its rank among the chunk's rows
//     of that expert; base + rank is a stable position.  The slots are listed
//     in position order (expert, then row), positions increasing;
//  4. the copy, 512-byte column slabs of the 64 rows at a time: waves 0-7
//     stream slabs of x into one half of an LDS double buffer, waves 8-15 write
//     the other half to x_perm in position order, so consecutive lanes write
//     consecutive positions: K-blocked, one run of (slots of an expert) x 64
//     bytes per K-block; row-major, whole 512-byte slab rows.  Producers and
//     consumers run separate loops with the same barriers, so neither waits
//     on the other's memory operations.  The first two slabs are loaded into
//     the producers' registers during steps 1-3 (slab 0 with step 1's loads,
//     slab 1 once step 1's values have arrived: steps 2-3 then wait on LDS
//     only), so the bookkeeping overlaps the copy's first memory latencies.
//     x_perm is written with the nontemporal hint: the GEMM reads it much
//     later, from HBM.  Where x is larger than the L2 caches together, its
//     rows are loaded with that hint too (no later kernel of the forward reads
//     them); a smaller x is still in L2 from the router and loads faster
//     without it.
template <typename T, bool kKBlocked, bool kNtX>
__global__ __launch_bounds__(kDispThreads) void dispatch_kernel(DispatchArgs a) {
    extern __shared__ __align__(16) unsigned char s_raw[];
    // parts > 1: blocks b * parts .. b * parts + parts - 1 share chunk b, each
    // doing the bookkeeping and copying its own contiguous range of slabs
    const int Ec = a.E_cols, k = a.k_slots, nch = a.nchunks;
    const int parts = gridDim.x / nch, b = blockIdx.x / parts, part = blockIdx.x % parts;
    unsigned char* slab = s_raw;                   // [2][64][kSlabStride] (step 4)
    int* s_red = reinterpret_cast<int*>(s_raw);    // [2][16][Ec] (steps 1-2)
    int* s_idx = s_red + 2 * kDispWaves * Ec;      // [64 k] the chunk's expert slots (steps 1-3)
    int* s_bef = reinterpret_cast<int*>(s_raw + kSlabLds);  // [Ec + 1]
    int* s_off = s_bef + Ec + 1;               // [Ec + 1]
    int* s_lb = s_off + Ec + 1;                // [Ec + 1] the chunk's slots before expert e
    int* s_ts = s_lb + Ec + 1;                 // [Ec + 1] first tile of expert e
    int* s_prow = s_ts + Ec + 1;               // [64 k] row of the i-th slot in position order
    int* s_ppos = s_prow + kRouterRows * k;    // [64 k] its position
    int* s_lc = s_ppos + kRouterRows * k;      // [Ec] the chunk's own rows per expert
    int* s_tot = s_red;                        // [Ec] after the reduction (s_red is free)
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int64_t row0 = (int64_t)b * kRouterRows;
    const int nvalid = (int)min<int64_t>(kRouterRows, a.rows - row0);

    // the copy's geometry (step 4) and the producers' slab loads
    constexpr int EPC = 16 / sizeof(T);
    const int nck = a.D / EPC;  // 16-byte chunks per row (D % 8 == 0)
    const int nslab_all = (nck + kSlabPieces - 1) / kSlabPieces;
    const int per_part = (nslab_all + parts - 1) / parts;
    const int sl0 = min(part * per_part, nslab_all);        // this block's first slab
    const int nslab = min(per_part, nslab_all - sl0);       // and its count (may be 0)
    const T* __restrict__ x = static_cast<const T*>(a.x);  // x_perm is the layer's own buffer
    const bool producer = tid < kProdThreads;
    static_assert(kProdLoads == 4, "four pieces per producer thread");
    auto fetch = [&](int sl, int u) {  // unconditional: clamped to a valid chunk
        const int q = tid + u * kProdThreads;
        const int r = min(q / kSlabPieces, nvalid - 1);
        const int c = min((sl0 + sl) * kSlabPieces + q % kSlabPieces, nck - 1);
        const T* src = x + (row0 + r) * (int64_t)a.D + (int64_t)c * EPC;
        if constexpr (kNtX) return load16_nt(src);
        else return *reinterpret_cast<const uint4*>(src);
    };
    // slab 0, in flight with step 1's loads
    uint4 f0, f1, f2, f3;
    if (producer) {
        f0 = fetch(0, 0);
        f1 = fetch(0, 1);
        f2 = fetch(0, 2);
        f3 = fetch(0, 3);
    }

    // 1. histograms (one per router block of count_rows rows, sub = 64 /
    // count_rows of them per chunk): each wave sums every 16th histogram, 16
    // histograms' counts in flight per lane (clamped loads, masked values; a
    // chain of single loads would pay one round trip per load): one round trip
    // up to 256 histograms (32 in flight measured 5 us slower, a second round
    // trip about as much).  The chunk's own counts: threads e < Ec add its sub
    // histograms.
    const int sub = kRouterRows / a.count_rows;
    const int nhist = (int)((a.rows + a.count_rows - 1) / a.count_rows);
    if (tid < Ec) {
        int own = 0;
        for (int h = b * sub; h < min(b * sub + sub, nhist); ++h)
            own += a.chunk_counts[(int64_t)h * Ec + tid];
        s_lc[tid] = own;
    }
    for (int e = lane; e < Ec; e += kWave) {
        int bef = 0, tot = 0;
        for (int c0 = wave; c0 < nhist; c0 += kHistInFlight * kDispWaves) {
            int v[kHistInFlight];
#pragma unroll
            for (int u = 0; u < kHistInFlight; ++u)
                v[u] = a.chunk_counts[(int64_t)min(c0 + u * kDispWaves, nhist - 1) * Ec + e];
#pragma unroll
            for (int u = 0; u < kHistInFlight; ++u) {
                const int h = c0 + u * kDispWaves;
                const int n = h < nhist ? v[u] : 0;
                tot += n;
                bef += h < b * sub ? n : 0;
            }
        }
        s_red[wave * Ec + e] = bef;
        s_red[(kDispWaves + wave) * Ec + e] = tot;
    }
    for (int i = tid; i < kRouterRows * k; i += kDispThreads)
        s_idx[i] = (i / k < nvalid) ? a.topk_idx[row0 * k + i] : -1;
    // slab 1, in flight through steps 2-3 (which read LDS only)
    uint4 v0, v1, v2, v3;
    if (producer) {
        v0 = fetch(1, 0);
        v1 = fetch(1, 1);
        v2 = fetch(1, 2);
        v3 = fetch(1, 3);
    }
    __syncthreads();
    int my_tot = 0;
    if (tid < Ec) {
        int bef = 0;
        for (int w = 0; w < kDispWaves; ++w) {
            bef += s_red[w * Ec + tid];
            my_tot += s_red[(kDispWaves + w) * Ec + tid];
        }
        s_bef[tid] = bef;
    }
    __syncthreads();
    if (tid < Ec) s_tot[tid] = my_tot;
    __syncthreads();
    // 2. offsets: wave 0 scans 64 experts at a time with carries
    if (wave == 0) {
        int carry = 0, lcarry = 0, tcarry = 0;
        for (int e0 = 0; e0 < Ec; e0 += kWave) {
            const int e = e0 + lane;
            const int v = e < Ec ? s_tot[e] : 0;
            const int lv = e < Ec ? s_lc[e] : 0;
            const int tv = (v + a.BM - 1) / a.BM;
            int inc = v, linc = lv, tinc = tv;
#pragma unroll
            for (int o = 1; o < kWave; o <<= 1) {
                const int t0 = __shfl_up(inc, o), t1 = __shfl_up(linc, o), t2 = __shfl_up(tinc, o);
                if (lane >= o) {
                    inc += t0;
                    linc += t1;
                    tinc += t2;
                }
            }
            if (e < Ec) {
                s_off[e] = carry + inc - v;
                s_lb[e] = lcarry + linc - lv;
                s_ts[e] = tcarry + tinc - tv;
            }
            carry += __shfl(inc, kWave - 1);
            lcarry += __shfl(linc, kWave - 1);
            tcarry += __shfl(tinc, kWave - 1);
        }
        if (lane == 0) {
            s_off[Ec] = carry;
            s_lb[Ec] = lcarry;
            s_ts[Ec] = tcarry;
        }
    }
    __syncthreads();
    if (b == 0 && part == 0) {
        for (int e = tid; e < Ec; e += kDispThreads) {
            a.expert_count[e] = s_tot[e];
            a.expert_off[e] = s_off[e];
        }
        const int total_tiles = s_ts[Ec];
        if (tid == 0) {
            a.expert_off[Ec] = s_off[Ec];
            a.tile_total[0] = min(total_tiles, a.max_tiles);
            a.tile_total[1] = 0;  // the GEMMs' tail counters
            a.tile_total[2] = 0;
        }
        for (int i = tid; i < total_tiles && i < a.max_tiles; i += kDispThreads) {
            int lo = 0, hi = Ec - 1;  // last expert with s_ts <= i (skipping empty ones)
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (s_ts[mid] <= i) lo = mid; else hi = mid - 1;
            }
            const int j = i - s_ts[lo];
            TileInfo t;
            t.expert = lo;
            t.row0 = s_off[lo] + j * a.BM;
            t.rows = min(a.BM, s_tot[lo] - j * a.BM);
            t.pad = 0;
            a.tiles[i] = t;
        }
    }
    // 3. ranks and positions.  Every wave holds each row's experts as a bit
    // set (lane = row); a row's slots hold distinct experts in ascending
    // order, so the slot of expert e is the number of the row's experts below
    // e.  The waves take the experts in turn (wave w: w, w + 16, ...), and
    // one ballot over the chunk's rows ranks expert e's slots.
    {
        constexpr int kSetWords = (kMaxExperts + 1 + 63) / 64;
        uint64_t eset[kSetWords];
#pragma unroll
        for (int w = 0; w < kSetWords; ++w) eset[w] = 0;
        for (int t = 0; t < k; ++t) {
            const int e = s_idx[lane * k + t];  // -1 past the chunk's rows
#pragma unroll
            for (int w = 0; w < kSetWords; ++w)
                if (e >= 0 && (e >> 6) == w) eset[w] |= 1ull << (e & 63);
        }
        int below[kSetWords];  // the row's experts in the words before word w
        below[0] = 0;
#pragma unroll
        for (int w = 1; w < kSetWords; ++w) below[w] = below[w - 1] + __popcll(eset[w - 1]);
        for (int e = wave; e < Ec; e += kDispWaves) {
            uint64_t word = 0;
            int j = 0;
#pragma unroll
            for (int w = 0; w < kSetWords; ++w)
                if ((e >> 6) == w) {
                    word = eset[w];
                    j = below[w];
                }
            const bool has = (word >> (e & 63)) & 1ull;
            const uint64_t bal = __ballot(has);
            if (has) {
                j += __popcll(word & ((1ull << (e & 63)) - 1ull));
                const int rank = __popcll(bal & ((1ull << lane) - 1ull));
                const int p = s_off[e] + s_bef[e] + rank;
                const int li = s_lb[e] + rank;
                s_prow[li] = lane;
                s_ppos[li] = p;
                if (part == 0) a.tok_pos[(row0 + lane) * k + j] = p;
            }
        }
    }
    __syncthreads();
    // 4. the copy
    constexpr int KB = kblock_elems<T>();
    constexpr int kPPK = kKBlockBytes / 16;  // pieces of one row in one K-block
    static_assert(kSlabPieces % kPPK == 0, "a slab holds whole K-blocks");
    const int npairs = s_lb[Ec];
    T* __restrict__ xp = static_cast<T*>(a.x_perm);
    if (producer) {
        // producers: slab sl + 1 into LDS while the consumers write slab sl;
        // four 16-byte pieces per thread, in named registers
        auto stash = [&](int buf, int u, const uint4& v) {
            const int q = tid + u * kProdThreads;
            *reinterpret_cast<uint4*>(slab + (buf * kRouterRows + q / kSlabPieces) * kSlabStride +
                                      (q % kSlabPieces) * 16) = v;
        };
        stash(0, 0, f0);
        stash(0, 1, f1);
        stash(0, 2, f2);
        stash(0, 3, f3);
        __syncthreads();
        for (int sl = 0; sl < nslab; ++sl) {
            const int buf = (sl + 1) & 1;  // slabs past the end are never read
            stash(buf, 0, v0);
            stash(buf, 1, v1);
            stash(buf, 2, v2);
            stash(buf, 3, v3);
            v0 = fetch(sl + 2, 0);
            v1 = fetch(sl + 2, 1);
            v2 = fetch(sl + 2, 2);
            v3 = fetch(sl + 2, 3);
            __syncthreads();
        }
    } else {
        // consumers
        constexpr int kCons = kDispThreads - kProdThreads;
        const int ct = tid - kProdThreads;
        __syncthreads();
        for (int sl = 0; sl < nslab; ++sl) {
            const unsigned char* sb = slab + (sl & 1) * kRouterRows * kSlabStride;
            if constexpr (kKBlocked) {
                // A thread owns piece ct % kPPK of slots ct / kPPK, + kCons / kPPK,
                // ...: for each, one position and row lookup, then the slab's
                // K-blocks of that piece, their LDS reads all in flight before
                // the stores (a_cap * KB elements apart).  Lanes 4i..4i+3 write
                // slot i's 64 bytes of a K-block: one store instruction covers
                // 16 consecutive positions.  (The slab holds whole K-blocks:
                // the K-blocked layout needs D % KB == 0.)
                constexpr int kKbs = kSlabPieces / kPPK;  // K-blocks per slab
                const int piece = ct % kPPK;
                const int kb0 = (sl0 + sl) * kKbs;
                const int nkb = min(kKbs, nck / kPPK - kb0);
                const int64_t kstep = a.a_cap * KB;
                for (int pr = ct / kPPK; pr < npairs; pr += kCons / kPPK) {
                    const int p = s_ppos[pr];
                    if (p < 0 || p >= a.a_cap) continue;
                    const unsigned char* src = sb + s_prow[pr] * kSlabStride + piece * 16;
                    T* dst = xp + ((int64_t)kb0 * a.a_cap + p) * KB + piece * EPC;
                    if (nkb == kKbs) {
                        uint4 val[kKbs];
#pragma unroll
                        for (int q = 0; q < kKbs; ++q)
                            val[q] = *reinterpret_cast<const uint4*>(src + q * kKBlockBytes);
#pragma unroll
                        for (int q = 0; q < kKbs; ++q) store16_nt(dst + q * kstep, val[q]);
                    } else {
                        for (int q = 0; q < nkb; ++q)
                            store16_nt(dst + q * kstep,
                                       *reinterpret_cast<const uint4*>(src + q * kKBlockBytes));
                    }
                }
            } else {
                // (slot, piece): whole 512-byte slab rows
                const int npieces = npairs * kSlabPieces;
                for (int v = ct; v < npieces; v += kCons) {
                    const int pr = v / kSlabPieces, h = v % kSlabPieces;
                    const int c = (sl0 + sl) * kSlabPieces + h;
                    const int p = s_ppos[pr];
                    if (c >= nck || p < 0 || p >= a.a_cap) continue;
                    const uint4 val =
                        *reinterpret_cast<const uint4*>(sb + s_prow[pr] * kSlabStride + h * 16);
                    store16_nt(xp + (int64_t)p * a.D + (int64_t)c * EPC, val);
                }
            }
            __syncthreads();
        }
    }
}

// One wave per row: out[row] = sum_j w_j * y_perm[pos_j] over the row's slots
// in ascending expert order (then the dense slot), accumulated in f32.  The
// row's positions and gates are read once (lane j holds slot j) and broadcast
// with readlane; each lane has a group of slots' loads of its chunks in
// flight together (8 slots of 2 chunks, or 4 of 6).  kResid: the block's gated residual out = x + y * gate
// (block.rs:101), its x and gate loaded with the first slots' loads.  kNt:
// nontemporal output stores.  kBatch: 16-byte chunks per lane per pass (6: a
// whole 3072-wide 16-bit row per pass, its slots' loads 4 at a time).
template <typename T, bool kResid, bool kNt, int kBatch>
__global__ __launch_bounds__(256) void combine_kernel(CombineArgs a) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + wave;
    if (row >= a.rows) return;
    constexpr int EPC = 16 / sizeof(T);
    const int nchunk = a.D / EPC;
    const int k = a.k_slots;   // slots past 64 are read from memory
    const T* __restrict__ y = static_cast<const T*>(a.y_perm);
    T* out = static_cast<T*>(a.out);
    const int my_p = lane < k ? a.tok_pos[row * k + lane] : -1;
    const float my_w = lane < k ? a.topk_w[row * k + lane] : 0.0f;
    // gated residual: the row's gate and input
    const float* grow = kResid ? a.gate + row / a.seq * a.D : nullptr;
    const T* xrow = kResid ? static_cast<const T*>(a.resid_x) + row * a.D : nullptr;
    for (int c0 = lane; c0 < nchunk; c0 += kWave * kBatch) {
        float acc[kBatch][EPC], xv[kBatch][EPC], gv[kBatch][EPC];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int c = min(c0 + u * kWave, nchunk - 1);  // past the end: not stored
            if constexpr (kResid) {
                load16(xrow + (int64_t)c * EPC, xv[u]);
                load_f32s<EPC>(grow + (int64_t)c * EPC, gv[u]);
            }
#pragma unroll
            for (int i = 0; i < EPC; ++i) acc[u][i] = 0.0f;
        }
        // N slots at a time: their N * kBatch loads are all in flight before
        // the first is added; the adds keep ascending slot order
        // (slots below 64 come from the lanes, later ones from memory)
        auto slots = [&](auto n, auto from_lanes, int j0) {
            constexpr int N = decltype(n)::value;
            int p[N];
            float w[N];
            uint4 raw[N][kBatch];
#pragma unroll
            for (int t = 0; t < N; ++t) {
                const int j = j0 + t;
                if constexpr (decltype(from_lanes)::value) {
                    p[t] = __builtin_amdgcn_readlane(my_p, j);
                    w[t] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_w), j));
                } else {
                    p[t] = a.tok_pos[row * k + j];
                    w[t] = a.topk_w[row * k + j];
                }
                // a slot without a position (none in a valid routing) adds 0 x row 0
                const bool ok = p[t] >= 0 && p[t] < a.a_cap;
                const int64_t pc = ok ? p[t] : 0;
                w[t] = ok ? w[t] : 0.0f;
#pragma unroll
                for (int u = 0; u < kBatch; ++u) {
                    // y_perm is read once: nontemporally, so that it does not
                    // push other data (the next forward's x) out of the caches
                    raw[t][u] = load16_nt(y + pc * a.D + (int64_t)min(c0 + u * kWave, nchunk - 1) * EPC);
                }
            }
#pragma unroll
            for (int t = 0; t < N; ++t) {
#pragma unroll
                for (int u = 0; u < kBatch; ++u) {
                    float v[EPC];
                    unpack16<T>(raw[t][u], v);
#pragma unroll
                    for (int i = 0; i < EPC; ++i) acc[u][i] = acc[u][i] + v[i] * w[t];
                }
            }
        };
        using Lanes = std::true_type;
        const int k1 = min(k, kWave);
        int j0 = 0;
        constexpr int kGroup = kBatch > 2 ? 4 : 8;  // slots per group: kGroup * kBatch loads
        for (; j0 + kGroup <= k1; j0 += kGroup) slots(std::integral_constant<int, kGroup>{}, Lanes{}, j0);
        for (; j0 + 4 <= k1; j0 += 4) slots(std::integral_constant<int, 4>{}, Lanes{}, j0);
        switch (k1 - j0) {
            case 3: slots(std::integral_constant<int, 3>{}, Lanes{}, j0); break;
            case 2: slots(std::integral_constant<int, 2>{}, Lanes{}, j0); break;
            case 1: slots(std::integral_constant<int, 1>{}, Lanes{}, j0); break;
            default: break;
        }
        for (int j = kWave; j < k; ++j) slots(std::integral_constant<int, 1>{}, std::false_type{}, j);
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int c = c0 + u * kWave;
            if (c >= nchunk) continue;
            if constexpr (kResid) {  // y and each step rounded to the model dtype
#pragma unroll
                for (int i = 0; i < EPC; ++i)
                    acc[u][i] = seam_residual<T>(xv[u][i], Elt<T>::to_f32(Elt<T>::from_f32(acc[u][i])),
                                                 gv[u][i]);
            }
            T* dst = out + row * a.D + (int64_t)c * EPC;
            if constexpr (kNt) store16_nt(dst, pack16<T>(acc[u]));
            else store16(dst, acc[u]);
        }
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
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        tile_total[0] = (int32_t)min<int64_t>(ntiles, max_tiles);
        tile_total[1] = 0;  // the GEMMs' tail counters
        tile_total[2] = 0;
    }
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
        constexpr int KB = kblock_elems<T>();
        *reinterpret_cast<uint4*>(xk + ((col / KB) * a_cap + r) * KB + col % KB) = v;
    }
}

template <typename T>
hipError_t launch_dispatch_t(const DispatchArgs& a, hipStream_t s) {
    const int nblk = (int)((a.rows + kRouterRows - 1) / kRouterRows);
    if (nblk == 0) return hipSuccess;
    if (a.nchunks != nblk || a.count_rows < kMinRouterBlockRows || a.count_rows > kRouterRows ||
        kRouterRows % a.count_rows != 0 || a.E_cols < 1 || a.E_cols > kMaxExperts + 1 || a.k_slots < 1 ||
        a.k_slots > a.E_cols || a.BM < 1 || !dispatch_fits(a.E_cols, a.k_slots) ||
        (a.kblocked && (int64_t)a.D * (int64_t)sizeof(T) % kKBlockBytes != 0))
        return hipErrorInvalidValue;
    const size_t lds = dispatch_lds(a.E_cols, a.k_slots);
    // the x_perm layout and the load hint as compile-time choices: no tests in
    // the copy loop.  Nontemporal x loads: headline 14,232 rows (87 MB)
    // 41.9 -> 40.2 us; one 4,680-row segment (29 MB, in L2 after the router)
    // 17.6 -> 19.5 us (A/B on one box, two repeats each).
    const bool nt_x = a.rows * (int64_t)a.D * (int64_t)sizeof(T) > kL2TotalBytes;
    auto kern = a.kblocked ? (nt_x ? dispatch_kernel<T, true, true> : dispatch_kernel<T, true, false>)
                           : (nt_x ? dispatch_kernel<T, false, true> : dispatch_kernel<T, false, false>);
    hipError_t err = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                         (int)lds);
    if (err != hipSuccess) return err;
    // several blocks per chunk when the chunks alone would leave CUs idle
    // (the copy splits by slabs, the bookkeeping is repeated), as long as the
    // grid stays within one block per CU: more blocks than CUs measured slower
    const int nslab = (int)((a.D * sizeof(T) + kSlabBytes - 1) / kSlabBytes);
    const int parts = std::max(1, std::min({kDispCUs / nblk, nslab, kDispMaxParts}));
    launch_kernel(kern, dim3(nblk * parts), dim3(kDispThreads), lds, s, a);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_combine_t(const CombineArgs& a, hipStream_t s) {
    const int nblk = (int)((a.rows + 3) / 4);
    // the residual, the store kind and the pass width as compile-time
    // choices: a run-time store-kind test inside the chunk loop measured 3%
    // slower.  Where the output goes out nontemporally (y_perm exceeds the
    // last-level cache), whole rows per pass: each pass then writes a row's
    // bytes at once (64 experts top-8: 182-184 -> 176-178 us; two chunks per
    // pass measured the same as whole rows at top-2 with cached stores).
    // 16-bit types only, where it was measured.
    const bool whole = sizeof(T) == 2 && a.out_nt && (a.D / (16 / (int)sizeof(T))) % (kWave * 6) == 0;
    auto kern = a.gate ? (a.out_nt ? combine_kernel<T, true, true, 2> : combine_kernel<T, true, false, 2>)
              : a.out_nt ? (whole ? combine_kernel<T, false, true, 6> : combine_kernel<T, false, true, 2>)
                         : combine_kernel<T, false, false, 2>;
    launch_kernel(kern, dim3(nblk), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace

bool dispatch_supported(int E_cols, int k_slots) { return dispatch_fits(E_cols, k_slots); }

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
    launch_kernel(dense_tiles_kernel, dim3(nblk), dim3(256), 0, s, rows, BM, max_tiles, tiles,
                  tile_total);
    return hipGetLastError();
}

hipError_t launch_kblock(DType dt, const void* x, void* xk, int64_t rows, int D, int64_t a_cap,
                         hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if ((int64_t)D * (int64_t)dtype_size(dt) % kKBlockBytes != 0 || a_cap < rows)
        return hipErrorInvalidValue;
    const int64_t chunks = rows * (D / (16 / (int)dtype_size(dt)));
    const unsigned nblk = (unsigned)std::min<int64_t>((chunks + 255) / 256, 65536);
    switch (dt) {
        case DType::BF16:
            launch_kernel(kblock_kernel<__bf16>, dim3(nblk), dim3(256), 0, s,
                          (const __bf16*)x, (__bf16*)xk, rows, D, a_cap);
            break;
        case DType::F16:
            launch_kernel(kblock_kernel<_Float16>, dim3(nblk), dim3(256), 0, s,
                          (const _Float16*)x, (_Float16*)xk, rows, D, a_cap);
            break;
        case DType::F32:
            launch_kernel(kblock_kernel<float>, dim3(nblk), dim3(256), 0, s,
                          (const float*)x, (float*)xk, rows, D, a_cap);
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
