// HBM read ceiling probe: the rate a streaming read reaches on this part, the ceiling the decode kernels (HBM-bound)
// are measured against next to the published 8 TB/s. Not part of the reference's path.
#include "bb_common.h"
#include "bb_internal.h"

namespace bb {
namespace {

// Each workgroup reads one contiguous range with non-temporal 16-byte loads, eight in flight per thread, so that every
// load instruction covers 1 KB of whole 128-byte lines (measured over 4 GiB: 7.0-7.1 TB/s; plain loads reach 6.2-6.3
// TB/s in the same pattern and 6.0-6.2 TB/s in a grid-stride loop). Every loaded word enters an XOR that the
// workgroup writes out, so no load can be dropped. Buffer bytes are a multiple of 16.
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4_t* __restrict__ buf, int64_t n16,
                                                          uint32_t* __restrict__ sink) {
  __shared__ uint32_t red[4];
  const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const int64_t b0 = (int64_t)blockIdx.x * per, b1 = b0 + per < n16 ? b0 + per : n16;
  u32x4_t a = {0, 0, 0, 0};
  int64_t i = b0 + threadIdx.x;
  for (; i + 7 * 256 < b1; i += 8 * 256) {
    u32x4_t v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = __builtin_nontemporal_load(buf + i + u * 256);
#pragma unroll
    for (int u = 0; u < 8; ++u) a ^= v[u];
  }
  for (; i < b1; i += 256) a ^= __builtin_nontemporal_load(buf + i);
  uint32_t x = a[0] ^ a[1] ^ a[2] ^ a[3];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x ^= __shfl_xor(x, off);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  if (threadIdx.x == 0) sink[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

}  // namespace

hipError_t launch_stream_read(const void* buf, int64_t bytes, uint32_t* sink, int workgroups, hipStream_t stream) {
  if (bytes < 16 || workgroups <= 0) return hipSuccess;
  hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)workgroups), dim3(256), 0, stream,
                     static_cast<const u32x4_t*>(buf), bytes / 16, sink);
  return hipGetLastError();
}

}  // namespace bb
