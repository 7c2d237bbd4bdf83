// Measurement helper for bench.py, not part of the W4A16 library: kernels
// that only read a buffer (16-byte loads, results folded into a value that is
// stored only if it matches a constant), giving the rate that plain HBM reads
// reach on this device next to the datasheet peak the roofline uses:
//  - read_kernel: grid-stride over the buffer (one long stream);
//  - read_slices_kernel<U>: one workgroup per contiguous slice of the buffer,
//    every thread issuing its U loads before using any of them, so that one
//    launch of ~one workgroup per CU has all its bytes in flight at once --
//    the best pattern for a single launch that moves a fixed number of bytes.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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

// Workgroup b reads elements [b * per_wg, min((b + 1) * per_wg, n16)); thread
// t loads elements base + j * blockDim + t for j < U (U * blockDim >= per_wg).
template <int U, bool NT>
__global__ void read_slices_kernel(const u32x4* __restrict__ p, size_t n16, size_t per_wg, unsigned* sink) {
  const size_t base = blockIdx.x * per_wg;
  size_t end = base + per_wg;
  if (end > n16) end = n16;
  u32x4 v[U];
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const size_t i = base + (size_t)j * blockDim.x + threadIdx.x;
    if (i < end) {
      if constexpr (NT)
        v[j] = __builtin_nontemporal_load(p + i);
      else
        v[j] = p[i];
    } else {
      v[j] = u32x4{0, 0, 0, 0};
    }
  }
  unsigned acc = 0;
#pragma unroll
  for (int j = 0; j < U; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
  if (acc == 0x9E3779B9u) sink[0] = acc;
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

// Reads bytes (a multiple of 16) at p as `grid` contiguous slices, one
// 1024-thread workgroup each, every load of a thread in flight at once
// (at most 16 loads of 16 bytes per thread: bytes <= grid * 256 KiB).
// nontemporal != 0 uses non-temporal loads.  Returns 0, -1 for bad
// arguments, or the HIP error code.
extern "C" int w4bench_read_slices(const void* p, size_t bytes, int grid, int nontemporal, unsigned* sink,
                                   void* stream) {
  if (p == nullptr || sink == nullptr || bytes % 16 != 0 || grid < 1) return -1;
  const size_t n16 = bytes / 16;
  const size_t per_wg = (n16 + grid - 1) / grid;
  const int block = 1024;
  const size_t u = (per_wg + block - 1) / block;
  if (u > 16) return -1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const u32x4* q = static_cast<const u32x4*>(p);
#define W4B_SLICES(U)                                                                                  \
  do {                                                                                                 \
    if (nontemporal)                                                                                   \
      hipLaunchKernelGGL((read_slices_kernel<U, true>), dim3((unsigned)grid), dim3(block), 0, st, q, n16, \
                         per_wg, sink);                                                                \
    else                                                                                               \
      hipLaunchKernelGGL((read_slices_kernel<U, false>), dim3((unsigned)grid), dim3(block), 0, st, q, n16, \
                         per_wg, sink);                                                                \
  } while (0)
  if (u <= 4)
    W4B_SLICES(4);
  else if (u <= 8)
    W4B_SLICES(8);
  else
    W4B_SLICES(16);
#undef W4B_SLICES
  return (int)hipGetLastError();
}
