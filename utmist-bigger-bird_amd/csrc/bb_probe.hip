// HBM read ceiling probe: the rate a plain 16-byte streaming read reaches on this part, the ceiling the decode
// kernels (HBM-bound) are measured against next to the published 8 TB/s. Not part of the reference's path.
#include "bb_common.h"
#include "bb_internal.h"

namespace bb {
namespace {

// Grid-stride 16-byte loads, four in flight per thread; every loaded word enters an XOR that the workgroup writes
// out, so no load can be dropped. Buffer bytes are a multiple of 16.
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4_t* __restrict__ buf, int64_t n16,
                                                          uint32_t* __restrict__ sink) {
  __shared__ uint32_t red[4];
  const int64_t stride = (int64_t)gridDim.x * 256;
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  u32x4_t a = {0, 0, 0, 0};
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4_t v0 = buf[i], v1 = buf[i + stride], v2 = buf[i + 2 * stride], v3 = buf[i + 3 * stride];
    a ^= v0 ^ v1 ^ v2 ^ v3;
  }
  for (; i < n16; i += stride) a ^= buf[i];
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
