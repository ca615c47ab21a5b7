// Shared device/host definitions for the gfx950 MoE feed-forward kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nomas {

enum class DType : int { F32 = 0, BF16 = 1, F16 = 2 };

inline size_t dtype_size(DType t) { return t == DType::F32 ? 4 : 2; }

// Element conversions.  bf16 <-> f32 use gfx950's native conversions through
// clang's __bf16 type (round to nearest even); f16 likewise through _Float16.
template <typename T> struct Elt;
template <> struct Elt<float> {
    static __device__ __forceinline__ float to_f32(float v) { return v; }
    static __device__ __forceinline__ float from_f32(float v) { return v; }
};
template <> struct Elt<__bf16> {
    static __device__ __forceinline__ float to_f32(__bf16 v) { return (float)v; }
    static __device__ __forceinline__ __bf16 from_f32(float v) { return (__bf16)v; }
};
template <> struct Elt<_Float16> {
    static __device__ __forceinline__ float to_f32(_Float16 v) { return (float)v; }
    static __device__ __forceinline__ _Float16 from_f32(float v) { return (_Float16)v; }
};

// 16-byte vector of elements: 8 x 16-bit or 4 x f32.
template <typename T> struct Vec16 {
    static constexpr int N = 16 / sizeof(T);
    T v[N];
};

template <typename T>
__device__ __forceinline__ void unpack16(const uint4& raw, float* out) {
    Vec16<T> t;
    __builtin_memcpy(&t, &raw, 16);
#pragma unroll
    for (int i = 0; i < Vec16<T>::N; ++i) out[i] = Elt<T>::to_f32(t.v[i]);
}

template <typename T>
__device__ __forceinline__ void load16(const T* p, float* out) {
    unpack16<T>(*reinterpret_cast<const uint4*>(p), out);
}

// A 16-byte store with the nontemporal hint (global_store_dwordx4 ... nt):
// for streams written once and not read again by the same kernel.
__device__ __forceinline__ void store16_nt(void* p, const uint4& v) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 t = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(t, reinterpret_cast<u32x4*>(p));
}

// A 16-byte load with the nontemporal hint (global_load_dwordx4 ... nt), for
// data read exactly once.
__device__ __forceinline__ uint4 load16_nt(const void* p) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return uint4{t.x, t.y, t.z, t.w};
}

// 16 bytes of T from f32 values (rounded to T).
template <typename T>
__device__ __forceinline__ uint4 pack16(const float* in) {
    Vec16<T> t;
#pragma unroll
    for (int i = 0; i < Vec16<T>::N; ++i) t.v[i] = Elt<T>::from_f32(in[i]);
    uint4 raw;
    __builtin_memcpy(&raw, &t, 16);
    return raw;
}

template <typename T>
__device__ __forceinline__ void store16(T* p, const float* in) {
    *reinterpret_cast<uint4*>(p) = pack16<T>(in);
}

// One tile of token rows belonging to one expert: rows [row0, row0 + rows)
// of the expert-contiguous buffers.
struct TileInfo {
    int expert;
    int row0;
    int rows;
    int pad;
};

constexpr int kWave = 64;
constexpr int kNumXcd = 8;        // MI355X: 8 XCDs, 32 CUs each, own L2 per XCD
constexpr int kRouterRows = 64;   // rows per router / dispatch chunk (one block)

}  // namespace nomas
