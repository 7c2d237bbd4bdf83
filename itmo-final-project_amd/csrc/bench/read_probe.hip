// Measurement helper for bench.py, not part of the W4A16 library: a kernel
// that only reads a buffer (16-byte loads, grid-stride, results folded into a
// value that is stored only if it matches a constant), giving the rate that
// plain HBM reads reach on this device -- for one long stream and for one
// launch of a given size -- next to the datasheet peak the roofline uses.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

__global__ void read_kernel(const uint4* __restrict__ p, size_t n16, unsigned* sink) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  unsigned acc = 0;
#pragma unroll 8
  for (; i < n16; i += stride) {
    const uint4 v = p[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;  // keeps the loads alive
}

}  // namespace

// Reads bytes (a multiple of 16) at p with grid x block threads on stream.
// sink: a device word the kernel may write.  Returns 0, or the HIP error code.
extern "C" int w4bench_read(const void* p, size_t bytes, int grid, int block, unsigned* sink, void* stream) {
  if (p == nullptr || sink == nullptr || bytes % 16 != 0 || grid < 1 || block < 64 || block > 1024) return -1;
  hipLaunchKernelGGL(read_kernel, dim3((unsigned)grid), dim3((unsigned)block), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint4*>(p), bytes / 16, sink);
  return (int)hipGetLastError();
}
