// Element math of the DiT block seams (norm2 + modulate, the gated residual).
// Every operation is an explicitly rounded f32 (or f64) step in the order the
// reference's tensor ops take (no contraction into fma), so a CPU evaluation
// of the same steps gives the same bits.
#pragma once

#include "common.hpp"

namespace nomas {

// f32 multiply and add, each rounded to f32 on its own.  Contraction is off
// (HIP's __fmul_rn / __fadd_rn are plain operators that may be fused into an
// fma), and the result passes through an empty asm so instruction selection
// cannot fold it into a mixed-precision fma with the next conversion either
// (v_fma_mix* rounds a*b straight to f16, skipping the f32 rounding).
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
    float r = a * b;
    asm("" : "+v"(r));
    return r;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
    float r = a + b;
    asm("" : "+v"(r));
    return r;
}

// f32 add without contraction (for sums whose addends come from memory, where
// no multiply is in reach to fuse with).
__device__ __forceinline__ float add_nc(float a, float b) {
#pragma clang fp contract(off)
    return a + b;
}

// N consecutive f32 (N % 4 == 0) from a 16-byte aligned address, 16 bytes at a time.
template <int N>
__device__ __forceinline__ void load_f32s(const float* p, float* o) {
#pragma unroll
    for (int q = 0; q < N / 4; ++q) {
        const float4 f = reinterpret_cast<const float4*>(p)[q];
        o[4 * q] = f.x;
        o[4 * q + 1] = f.y;
        o[4 * q + 2] = f.z;
        o[4 * q + 3] = f.w;
    }
}

// RmsNorm's scale for a row whose squares sum to ss (norm.rs:55-65, over
// candle-core 0.11.1's f32 ops): var = ss * f32(1/D) (mean_keepdim is a sum
// times 1/D), t = var + f32(eps), inv = t^-1/2, each rounded to f32; t^-1/2 is
// 1/sqrt in f64, rounded once (the reference's powf(t, -0.5) is within an ulp).
__device__ __forceinline__ float seam_inv_rms(float ss, int D, double eps) {
    const float var = mul_rn(ss, (float)(1.0 / (double)D));
    const float t = add_rn(var, (float)eps);
    return (float)(1.0 / sqrt((double)t));
}

// h = modulate(rmsnorm(x) * w, shift, scale) for one element: the norm's f32
// product rounded to the model dtype (norm.rs:64), then x * (1 + scale) + shift
// in f32 rounded to the model dtype (modulate.rs:76-78).
template <typename T>
__device__ __forceinline__ float seam_h(float x, float inv, float w, float sc, float sh) {
    const float n = Elt<T>::to_f32(Elt<T>::from_f32(mul_rn(mul_rn(x, inv), w)));
    const float h = add_rn(mul_rn(n, add_rn(sc, 1.0f)), sh);
    return Elt<T>::to_f32(Elt<T>::from_f32(h));
}

// out = x + y * gate in the model dtype (block.rs:101): y is the MoE output
// (already rounded), the product and the sum each rounded to the model dtype.
template <typename T>
__device__ __forceinline__ float seam_residual(float x, float y, float g) {
    const float t = Elt<T>::to_f32(Elt<T>::from_f32(mul_rn(y, g)));
    return Elt<T>::to_f32(Elt<T>::from_f32(add_rn(x, t)));
}

}  // namespace nomas
