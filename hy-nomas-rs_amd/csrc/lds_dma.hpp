// Direct global->LDS loads and the waits that go with them (device code).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nomas {

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Direct global->LDS load of 16 bytes per lane from sbase + voff (a uniform
// 64-bit base in SGPRs plus a per-lane 32-bit byte offset): lane l's bytes
// land at LDS address lds_base + 16 * l (global_load_lds_dwordx4, M0 = LDS
// base; one wait state between the M0 write and the load).  Issued as inline
// assembly so the compiler does not track it: completion is waited for
// explicitly with wait_vmcnt, and nothing else in the kernels that use it
// touches M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // M0 is clobbered on purpose, see above
__device__ __forceinline__ void lds_dma16(const void* sbase, uint32_t voff, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(sbase), "s"(lds_base)
                 : "memory", "m0");
}
// The same through a raw buffer resource (buffer_load_dwordx4 ... lds): lanes
// whose byte offset is at or past the resource's num_records fail the range
// check, read no memory and return zeros.
__device__ __forceinline__ void lds_dma16_buf(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff,
                                              uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 :
                 : "v"(voff), "s"(rsrc), "s"(lds_base)
                 : "memory", "m0");
}
// Groups of loads into consecutive 1 KB LDS blocks: M0 is written once per
// group (set_lds_m0) and load q of the group carries q * 1024 in its
// immediate offset, which the hardware adds to both the global (or buffer)
// address and the LDS address.  One M0 write and wait state per group
// instead of per load.
__device__ __forceinline__ void set_lds_m0(uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0" : : "s"(lds_base) : "memory", "m0");
}
template <int OFF>
__device__ __forceinline__ void lds_dma16_at(const void* sbase, uint32_t voff) {
    asm volatile("global_load_lds_dwordx4 %0, %1 offset:%2" : : "v"(voff), "s"(sbase), "n"(OFF)
                 : "memory");
}
template <int OFF>
__device__ __forceinline__ void lds_dma16_buf_at(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff) {
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen offset:%2 lds" : : "v"(voff), "s"(rsrc), "n"(OFF)
                 : "memory");
}
#pragma clang diagnostic pop
// Load q (0-3, a constant after unrolling) of a group.
__device__ __forceinline__ void lds_dma16_q(int q, const void* sbase, uint32_t voff) {
    switch (q) {
        case 0: lds_dma16_at<0>(sbase, voff); break;
        case 1: lds_dma16_at<1024>(sbase, voff); break;
        case 2: lds_dma16_at<2048>(sbase, voff); break;
        default: lds_dma16_at<3072>(sbase, voff); break;
    }
}
__device__ __forceinline__ void lds_dma16_buf_q(int q, __amdgpu_buffer_rsrc_t rsrc, uint32_t voff) {
    switch (q) {
        case 0: lds_dma16_buf_at<0>(rsrc, voff); break;
        case 1: lds_dma16_buf_at<1024>(rsrc, voff); break;
        case 2: lds_dma16_buf_at<2048>(rsrc, voff); break;
        default: lds_dma16_buf_at<3072>(rsrc, voff); break;
    }
}

// The LDS byte address of a __shared__ object (for M0).
template <typename P>
__device__ __forceinline__ uint32_t lds_addr(P* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

}  // namespace nomas
