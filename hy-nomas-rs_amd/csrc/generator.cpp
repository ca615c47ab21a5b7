// Deterministic parameter generator of hy-nomas-rs, for Weights::Random
// (modules/mod.rs:38-45,80-95) and the seeded test/benchmark inputs.
//
//  - path_seed: FNV-1a over the path bytes with the offset basis xor'ed with
//    the base seed (mod.rs:47-55).
//  - randn_affine: SplitMix64 (tensor_utils.rs:76-83) + Box-Muller
//    (tensor_utils.rs:93-106): the pair of draws (2j, 2j+1) gives element 2j =
//    r cos(theta) and element 2j+1 = r sin(theta), each scaled by std, shifted
//    by mean and rounded to f32 (tensor_utils.rs:123-138).
// SplitMix64's state after n draws is seed + n * 0x9E3779B97F4A7C15, so pairs
// are generated independently on host threads with bit-identical results.
// This file is compiled with -ffp-contract=off: a*std + mean stays two
// roundings, as in the reference.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "host.hpp"

namespace nomas {

namespace {

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;

inline uint64_t mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Draw number n (0-based) of the stream seeded with `seed`.
inline double draw_f64(uint64_t seed, uint64_t n) {
    const uint64_t z = mix(seed + (n + 1) * kGamma);
    return (double)(z >> 11) * (1.0 / 9007199254740992.0);
}

void randn_range(uint64_t seed, double mean, double std, int64_t n, float* out, int64_t p0,
                 int64_t p1) {
    for (int64_t p = p0; p < p1; ++p) {
        double u1 = draw_f64(seed, 2 * (uint64_t)p);
        if (u1 < 2.2250738585072014e-308) u1 = 2.2250738585072014e-308;
        const double u2 = draw_f64(seed, 2 * (uint64_t)p + 1);
        const double r = std::sqrt(-2.0 * std::log(u1));
        const double theta = 2.0 * 3.14159265358979323846 * u2;
        const double c = r * std::cos(theta);
        const double s = r * std::sin(theta);
        out[2 * p] = (float)(c * std + mean);
        if (2 * p + 1 < n) out[2 * p + 1] = (float)(s * std + mean);
    }
}

}  // namespace

uint64_t path_seed(uint64_t seed, const char* path) {
    uint64_t h = 0xcbf29ce484222325ull ^ seed;
    for (const unsigned char* p = reinterpret_cast<const unsigned char*>(path); *p; ++p) {
        h ^= (uint64_t)*p;
        h *= 0x100000001b3ull;
    }
    return h;
}

void randn_affine(uint64_t seed, double mean, double std, int64_t n, float* out) {
    if (n <= 0) return;
    const int64_t pairs = (n + 1) / 2;
    unsigned nt = std::thread::hardware_concurrency();
    if (nt == 0) nt = 1;
    if (nt > 16) nt = 16;
    if (pairs < (1 << 16)) nt = 1;
    if (nt == 1) {
        randn_range(seed, mean, std, n, out, 0, pairs);
        return;
    }
    std::vector<std::thread> th;
    const int64_t per = (pairs + nt - 1) / nt;
    int64_t done = 0;  // pairs [0, done) are handed to threads
    try {
        th.reserve(nt);
        for (unsigned t = 0; t < nt; ++t) {
            const int64_t p0 = (int64_t)t * per, p1 = std::min<int64_t>(pairs, p0 + per);
            if (p0 >= p1) break;
            th.emplace_back(randn_range, seed, mean, std, n, out, p0, p1);
            done = p1;
        }
    } catch (...) {
        // no thread (or no memory) for the rest: this thread draws it; the
        // values do not depend on who draws them
    }
    if (done < pairs) randn_range(seed, mean, std, n, out, done, pairs);
    for (auto& x : th) x.join();
}

uint16_t f32_to_bf16_bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float bf16_bits_to_f32(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

uint16_t f32_to_f16_bits(float f) {
    _Float16 h = (_Float16)f;  // IEEE round to nearest even
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}

float f16_bits_to_f32(uint16_t b) {
    _Float16 h;
    std::memcpy(&h, &b, 2);
    return (float)h;
}

}  // namespace nomas
