// Device scratch of the allocation-free forward (moe_layer_forward_device_noalloc): a file-scope
// array that every GPU the library runs on holds for the life of the process, and the fill
// kernel that clears the parts of it a call needs zeroed.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>

#include "kernels.hpp"

namespace {

constexpr size_t kScratchBytes = (size_t)16 << 20;
constexpr int kMaxDevices = 64;

// Each device holds its own copy at its own address. Host code never passes this name to a
// kernel or a copy: it is a host-side stand-in; the address comes from noalloc_scratch_ptr.
__device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_mu;
void *g_ptr[kMaxDevices] = {};

// Zeroes n16 16-byte words, then `tail` bytes after them.
__global__ void k_zero(uint4 *p, size_t n16, size_t tail) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
    p[i] = uint4{0u, 0u, 0u, 0u};
  if (blockIdx.x == 0 && threadIdx.x < tail) reinterpret_cast<uint8_t *>(p + n16)[threadIdx.x] = 0;
}

}  // namespace

namespace moe {

size_t noalloc_scratch_bytes() { return kScratchBytes; }

// The device address of device `dev`'s copy of the scratch array. The first call for a device
// (made by moe_create, with that device current) resolves it with hipGetSymbolAddress; later
// calls return the kept address.
hipError_t noalloc_scratch_ptr(int dev, void **ptr) {
  *ptr = nullptr;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_ptr[dev]) {
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    if (cur != dev) return hipErrorInvalidDevice;
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_ptr[dev] = p;
  }
  *ptr = g_ptr[dev];
  return hipSuccess;
}

// Clears `bytes` bytes at the 16-byte aligned device address p with a kernel (not a memset node,
// so the call stays correct inside a captured graph).
hipError_t launch_zero(void *p, size_t bytes, hipStream_t s) {
  if (!bytes) return hipSuccess;
  const size_t n16 = bytes / 16, tail = bytes % 16;
  const unsigned blocks = (unsigned)std::min<size_t>((n16 + 255) / 256 + 1, 1024);
  k_zero<<<blocks, 256, 0, s>>>(reinterpret_cast<uint4 *>(p), n16, tail);
  return hipGetLastError();
}

}  // namespace moe
