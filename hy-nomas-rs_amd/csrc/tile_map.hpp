// Block-id -> GEMM work mapping of the grouped MFMA GEMMs (host + device, so
// the mapping is checked exhaustively on the CPU).
#pragma once

#include <hip/hip_runtime.h>

namespace nomas {

constexpr int kTileGroupM = 8;   // row tiles per group (row index fastest inside)
constexpr int kXcds = 8;         // MI355X: 8 XCDs
constexpr int kCusPerXcd = 32;   // 32 CUs per XCD
constexpr int kRound = kXcds * kCusPerXcd;  // blocks that run at once (one per CU)
constexpr int kMaxSplit = 4;     // most parts a tail tile is split into along K

// Grid size: the tile count padded to whole rounds of all XCDs.
__host__ __device__ inline long long tile_grid(int max_tiles, int ntn) {
    return ((long long)max_tiles * ntn + kRound - 1) / kRound * kRound;
}

// Blocks are dispatched in id order, block i to XCD i % 8, so one XCD's queue
// is ids x, x+8, ...  Its k-th group of kCusPerXcd consecutive queue entries
// ("round") runs roughly at time k.  Round R = k * 8 + x takes logical
// indices [R * kCusPerXcd, (R + 1) * kCusPerXcd): logical order is time order,
// and at any time the eight XCDs work on eight consecutive rounds.  A
// bijection of [0, n) for every n that is a multiple of kRound.
__host__ __device__ inline int time_order(int pid) {
    const int xcd = pid % kXcds, loc = pid / kXcds;
    const int round = (loc / kCusPerXcd) * kXcds + xcd;
    return round * kCusPerXcd + loc % kCusPerXcd;
}

// Tile (mt, nt) of logical index L < tiles * ntn: groups of kTileGroupM row
// tiles x all column tiles, row index fastest inside a group.  Consecutive
// rounds then share the same expert's weights (through the MALL), and a
// round inside an XCD is an 8 x 4 block of tiles sharing panels in its L2.
__host__ __device__ inline void group_tile(long long L, int ntn, int tiles, int* mt, int* nt) {
    const long long group = L / ((long long)kTileGroupM * ntn);
    const int first_m = (int)group * kTileGroupM;
    const int gm = tiles - first_m < kTileGroupM ? tiles - first_m : kTileGroupM;
    const int within = (int)(L - group * kTileGroupM * ntn);
    *mt = first_m + within % gm;
    *nt = within / gm;
}

// Maps the hardware block id to (row tile mt, column tile nt) of a grid of
// max_tiles x ntn tiles; returns false for padding blocks.
__host__ __device__ inline bool tile_coords(int pid, int ntn, int max_tiles, int* mt, int* nt) {
    const int L = time_order(pid);
    // a partial last group holds only gm * ntn tiles: reject every index at
    // or past max_tiles * ntn, not just whole groups
    if (L >= (long long)max_tiles * ntn) return false;
    group_tile(L, ntn, max_tiles, mt, nt);
    return *nt < ntn;
}

// Parts the tiles of the last, partial round are split into along K, for T
// live tiles and `turns` whole k-loop turns per tile: when that round would
// keep at most half the CUs busy for a whole tile, its r tiles become
// parts * r <= kRound shorter units.  Parts must divide the turns.
__host__ __device__ inline int split_parts(long long T, int turns) {
    const int r = (int)(T % kRound);
    if (r == 0 || 2 * r > kRound) return 1;
    int p = kMaxSplit;
    while (p > 1 && (p * r > kRound || turns % p != 0)) p >>= 1;
    return p;
}

// One block's work: a whole tile (parts == 1), or part `part` of `parts` of
// a tile split along K; `slot` numbers the split tiles (0 .. r - 1).
struct WorkUnit {
    int mt, nt;
    int part, parts;
    int slot;
};

// The work units of `tiles` live row tiles in time order: the whole tiles,
// then the split units of the last r tiles, which fill the final round.
__host__ __device__ inline long long unit_count(int tiles, int ntn, int turns) {
    const long long T = (long long)tiles * ntn;
    const int parts = split_parts(T, turns);
    const long long F = parts > 1 ? T - T % kRound : T;  // whole tiles
    return F + (T - F) * parts;
}

// Unit L (0 <= L < unit_count) of that order.
__host__ __device__ inline void unit_at(long long L, int ntn, int tiles, int turns, WorkUnit* u) {
    const long long T = (long long)tiles * ntn;
    const int parts = split_parts(T, turns);
    const long long F = parts > 1 ? T - T % kRound : T;
    long long tile;
    if (L < F) {
        tile = L;
        u->part = 0;
        u->parts = 1;
        u->slot = -1;
    } else {
        const long long q = L - F;
        tile = F + q / parts;
        u->part = (int)(q % parts);
        u->parts = parts;
        u->slot = (int)(q / parts);
    }
    group_tile(tile, ntn, tiles, &u->mt, &u->nt);
}

// Work of block pid when `tiles` row tiles are live (tiles <= the max_tiles
// the grid was sized for, grid = tile_grid(max_tiles, ntn) + kRound): unit
// time_order(pid).  Returns false for blocks with no work.
__host__ __device__ inline bool unit_coords(int pid, int ntn, int tiles, int turns, WorkUnit* u) {
    const long long L = time_order(pid);
    if (L >= unit_count(tiles, ntn, turns)) return false;
    unit_at(L, ntn, tiles, turns, u);
    return true;
}

// The tail.  The XCDs do not run at the same speed (same work, same kernel:
// the slowest finishes a few percent after the fastest), and with the static
// map each XCD's share is fixed.  So the last units in time order (at least
// kTailUnits of them) are handed out at run time instead: every block whose time-order index is
// at or past tail_start (the grid's padding blocks included) takes a ticket
// from a counter and runs unit tail_start + ticket, or nothing when the
// tickets pass the last unit.  An XCD that is ahead reaches its tail blocks
// sooner and takes more of the tail.  The static part is whole rounds of all
// XCDs, so every XCD has the same static work (otherwise an XCD with one more
// static round reaches the tail after it has been handed out).  No block
// waits for another, and there are at least as many such blocks as tail units
// (the grid has a round of padding beyond the split units), so every unit
// runs exactly once.
constexpr int kTailUnits = 2 * kRound;  // at least; fewer than kTailUnits + kRound
__host__ __device__ inline long long tail_start(long long units) {
    return units > kTailUnits ? (units - kTailUnits) / kRound * kRound : 0;
}

}  // namespace nomas
