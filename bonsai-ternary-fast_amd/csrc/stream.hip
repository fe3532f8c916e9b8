// stream.hip -- a plain streaming read of device memory: the practical HBM
// read ceiling that the GEMV and step figures are read against (MI355X's
// 8 TB/s is the published peak; a streaming read reaches less). Every lane
// reads 16-byte words with the non-temporal policy, as the GEMV kernels read
// their weights, eight loads in flight per lane, grid-stride over the buffer;
// the words are folded with XOR and the result is stored only if it equals a
// value the caller passes (it never does in practice), so the loads are kept
// and nothing is written. Measurement hook: no reference counterpart.
#include <hip/hip_runtime.h>

#include "../../include/btf/hip_abi.h"
#include "common.h"

namespace btfhip {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(256) stream_read_kernel(const u32x4* __restrict__ src, uint64_t n16,
                                                          uint32_t never, uint32_t* sink) {
  const uint64_t stride = (uint64_t)gridDim.x * 256u;
  uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (; i + 7 * stride < n16; i += 8 * stride) {
    u32x4 w[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) w[k] = __builtin_nontemporal_load(src + i + k * stride);
#pragma unroll
    for (int k = 0; k < 8; ++k) acc ^= w[k];
  }
  for (; i < n16; i += stride) acc ^= __builtin_nontemporal_load(src + i);
  const uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (x == never) sink[0] = x;
}

}  // namespace

int stream_read(const void* src, uint64_t bytes, uint32_t never, uint32_t* sink, hipStream_t st,
                const DevState& ds) {
  const int blocks = (ds.cu_count > 0 ? ds.cu_count : 256) * 8;
  hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(256), 0, st, static_cast<const u32x4*>(src), bytes / 16,
                     never, sink);
  return launch_status("stream_read_kernel");
}

}  // namespace btfhip
