// Block-id -> GEMM tile mapping of the grouped MFMA GEMMs (host + device, so
// the mapping is checked exhaustively on the CPU).
#pragma once

#include <hip/hip_runtime.h>

namespace nomas {

constexpr int kTileGroupM = 8;   // row tiles per group (row index fastest inside)
constexpr int kXcds = 8;         // MI355X: 8 XCDs
constexpr int kCusPerXcd = 32;   // 32 CUs per XCD

// Grid size: the tile count padded to whole rounds of all XCDs.
__host__ __device__ inline long long tile_grid(int max_tiles, int ntn) {
    const long long pad = (long long)kXcds * kCusPerXcd;
    return ((long long)max_tiles * ntn + pad - 1) / pad * pad;
}

// Maps the hardware block id to (row tile mt, column tile nt); returns false
// for padding blocks.  Blocks are dispatched in id order, block i to XCD
// i % 8, so one XCD's queue is ids x, x+8, ...  Its k-th group of kCusPerXcd
// consecutive queue entries ("round") runs roughly at time k.  Round
// R = k * 8 + x takes logical tiles [R * kCusPerXcd, (R + 1) * kCusPerXcd):
// at any time the eight XCDs work on eight consecutive rounds (the same
// expert's weights, shared through the MALL), and inside an XCD a round is a
// kTileGroupM x 8 block of tiles sharing panels in that XCD's L2.
__host__ __device__ inline bool tile_coords(int pid, int ntn, int max_tiles, int* mt, int* nt) {
    const int xcd = pid % kXcds, loc = pid / kXcds;
    const int round = (loc / kCusPerXcd) * kXcds + xcd;
    const int L = round * kCusPerXcd + loc % kCusPerXcd;
    // a partial last group holds only gm * ntn tiles: reject every index at
    // or past max_tiles * ntn, not just whole groups
    if (L >= max_tiles * ntn) return false;
    const int group = L / (kTileGroupM * ntn);
    const int first_m = group * kTileGroupM;
    const int gm = max_tiles - first_m < kTileGroupM ? max_tiles - first_m : kTileGroupM;
    const int within = L - group * kTileGroupM * ntn;
    *mt = first_m + within % gm;
    *nt = within / gm;
    return *nt < ntn;
}

}  // namespace nomas
