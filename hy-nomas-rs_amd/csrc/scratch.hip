// The device scratch array of the no-allocation forward
// (nomas_moe_forward_noalloc): a fixed kScratchBytes of device memory per GPU,
// in the library's code object, so that a forward can run without any
// allocation (callers under HIP graph capture or in tight serving loops).
//
// On the host, `scratch` names a host-side stand-in, not device memory: its
// device address is looked up per device with hipGetSymbolAddress (with that
// device current) and only that address is handed to kernels.  Every GPU
// holds its own copy of the array at its own address, until the process
// ends.  All no-allocation forwards on one GPU share it: each keeps the
// previous one's contents, and two that overlap on one GPU race.
#include <mutex>

#include "host.hpp"

namespace nomas {

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
uint64_t g_scratch_gen[kMaxDevices] = {};  // uses of the array per device

// The split-tile arrival counters at the start of the array must start at
// zero; the GEMMs return them to zero.  A kernel, not a memset: the first
// call may be the one a caller captures.
__global__ void clear_counters_kernel(int32_t* p, int n) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0;
}

}  // namespace

int scratch_acquire(int device, hipStream_t s, void** out, uint64_t* gen) {
    if (device < 0 || device >= kMaxDevices)
        return set_error(NOMAS_ERR_INVALID_ARGUMENT, "device %d beyond the %d the scratch array serves",
                         device, kMaxDevices);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        // once per device, with that device current (the caller set it)
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return set_error(NOMAS_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d failed: %s",
                             device, hipGetErrorString(e));
        launch_kernel(clear_counters_kernel, dim3(1), dim3(256), 0, s,
                      static_cast<int32_t*>(p), kSplitUnits);
        const hipError_t le = hipGetLastError();
        if (le != hipSuccess)
            return set_error(NOMAS_ERR_HIP, "clearing the scratch counters failed: %s",
                             hipGetErrorString(le));
        g_scratch_ptr[device] = p;
    }
    *out = g_scratch_ptr[device];
    *gen = ++g_scratch_gen[device];
    return NOMAS_OK;
}

uint64_t scratch_generation(int device) {
    if (device < 0 || device >= kMaxDevices) return 0;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    return g_scratch_gen[device];
}

}  // namespace nomas
