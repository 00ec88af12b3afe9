// kvr_scratch.hip -- the file-scope device scratch of kvr_recall_layer_noalloc.
//
// Callers that may not allocate (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc) score a layer with the
// logits, packed queries and per-lane completion counters in this array
// instead of the context's workspace.  Every GPU the library runs on holds
// its own copy for the life of the process.  Host code never passes the
// array's name to a kernel: the name is a host-side stand-in, not a device
// address.  scratch_init() looks the device address up once per device, with
// that device current, and every later use goes through that address.
#include "kvr_internal.hpp"

#include <hip/hip_runtime.h>

#include <mutex>

namespace kvr {
namespace {

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch[kMaxDevices] = {};

__global__ __launch_bounds__(256) void k_fill_u32(uint32_t *p, uint32_t n, uint32_t v) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = v;
}

}  // namespace

hipError_t scratch_init(int device) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch[device]) return hipSuccess;
    int current = -1;
    if (hipError_t e = hipGetDevice(&current)) return e;
    if (current != device) return hipErrorInvalidDevice;  // the caller makes `device` current
    void *ptr = nullptr;
    if (hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch))) return e;
    g_scratch[device] = ptr;
    return hipSuccess;
}

uint8_t *scratch_address(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    return static_cast<uint8_t *>(g_scratch[device]);
}

hipError_t launch_fill_u32(uint32_t *p, uint32_t n, uint32_t v, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(k_fill_u32, dim3((n + 255) / 256), dim3(256), 0, s, p, n, v);
    return hipGetLastError();
}

}  // namespace kvr
