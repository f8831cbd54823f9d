// The allocation-free sampler entry point: generate's sampler on buffers the
// caller already holds on the device, with the only scratch it needs (each
// row's append counter) in a fixed device array of this file.  For callers
// that cannot allocate: code under HIP graph capture, serving loops.
#include <hip/hip_runtime.h>

#include <mutex>

#include "kernels.hpp"

namespace meshgpt::kern {
namespace {

// One append counter per row; the sampler kernels append each row's token at
// tokens[row + counter] and bump the counter, so every call clears the
// counters it uses first.  Each GPU the library runs on holds its own copy
// until the process ends.
static __device__ __align__(256) int scratch[kNoAllocRows];

constexpr int kMaxDevices = 64;

__global__ void __launch_bounds__(256) fill_int_kernel(int *p, int value, int n) {
    for (int i = int(blockIdx.x * blockDim.x + threadIdx.x); i < n; i += int(gridDim.x * blockDim.x)) p[i] = value;
}

}  // namespace

// The device address of `scratch` on `device` (the current device), looked up
// once per device: in host code the array's name is not a device address.
hipError_t noalloc_scratch(int device, int **out) {
    static std::mutex lock;
    static int *address[kMaxDevices] = {};
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> guard(lock);
    if (!address[device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        address[device] = static_cast<int *>(p);
    }
    *out = address[device];
    return hipSuccess;
}

void fill_int(int *p, int value, int n, hipStream_t stream) {
    if (n <= 0) return;
    const int blocks = (n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024;
    hipLaunchKernelGGL(fill_int_kernel, dim3(blocks), dim3(256), 0, stream, p, value, n);
}

}  // namespace meshgpt::kern
