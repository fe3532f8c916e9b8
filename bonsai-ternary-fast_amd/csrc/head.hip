// head.hip -- the kernels either side of a decode step's GEMV chain (gfx950):
// the embedding lookup from the packed table with its inverse transform, the
// greedy pick over the logits, and the position counter.
//
//  * embed_slices_kernel: behaviour of the reference's launch_embed
//    (src/cuda/kernels.cuh:82-85) and of its CPU twin, the embedding step of
//    EmuDecoder::chunk (src/emu_decoder.cpp:171-180) with bd::hadamard_inverse
//    (ref/bonsai-decoder/src/cpu_ops.cpp:113-118). One wave per 1024 columns
//    of a token row, 16 columns per lane: in the T2 layout columns 16 h ..
//    16 h + 15 of a 128-block are exactly code word h of the block
//    (include/btf/packed.hpp:35-38), so lane l reads ONE aligned 32-bit word
//    (the table may be mapped host memory) and the fp16 scale of its block,
//    decodes 16 values (code - 1) * scale, runs the blockwise FWHT in
//    registers (slice.h, the CPU's stage order), times 1/sqrt(block), times
//    the signs. Bit-exact with the CPU. As on the CPU, the signs belong to the
//    transform (block 0: neither).
//  * argmax: the greedy pick (src/cuda/kernels.cuh:87-90; CPU:
//    ref/bonsai-decoder/src/sampler.cpp:20-25). Every logit becomes a 64-bit
//    key that orders (value, -index) totally: the value's bits in an
//    order-preserving form in the high word (-0 folded onto +0, a NaN key 0,
//    below every number), the complement of the index in the low word. The
//    largest key is the largest value at its smallest index, so the result
//    does not depend on the order of the reductions. Stage 1: contiguous
//    2048-value parts, one workgroup each, a max over keys (DPP and
//    v_permlane16/32_swap in the wave, LDS across waves) into `part`; stage 2:
//    one wave over the parts. A NaN never wins; all-NaN gives 0.
//  * pos_add: *d_pos += M, as a vector atomic (src/cuda/kernels.cuh:92).
#include <cmath>
#include <string>

#include "../../include/btf/hip_abi.h"
#include "common.h"
#include "slice.h"

#pragma clang fp contract(off)

namespace btfhip {
namespace {

// ---- embedding ----
constexpr int kEmbedWaves = 4;

template <bool VEC>
__global__ void __launch_bounds__(64 * kEmbedWaves)
    embed_slices_kernel(const uint8_t* __restrict__ codes, const uint16_t* __restrict__ scales,
                        const int* __restrict__ d_tok, int E, int nslices, int block, float hs,
                        const float* __restrict__ signs, float* __restrict__ x) {
  const int lane = threadIdx.x & 63;
  const int sl = blockIdx.x * kEmbedWaves + (threadIdx.x >> 6);
  if (sl >= nslices) return;  // a whole wave: the butterflies below stay in step
  const int m = blockIdx.y;
  const size_t tok = (size_t)d_tok[m];
  const int c0 = sl * kSliceVals + 16 * lane;
  const bool live = c0 < E;  // E % 128 == 0: whole 128-blocks are live
  uint32_t w = 0;
  float sc = 0.f;
  if (live) {
    w = reinterpret_cast<const uint32_t*>(codes + tok * (size_t)(E / 4))[c0 >> 4];
    sc = h2f(scales[tok * (size_t)(E / 128) + (c0 >> 7)]);
  }
  float v[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {  // column j of the word: byte j % 4, 2-bit field j / 4
    const int c = (int)((w >> (8 * (j & 3) + 2 * (j >> 2))) & 3u);
    v[j] = (float)(c - 1) * sc;
  }
  if (block > 0) {
    slice_fwht(v, lane, block);
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = v[j] * hs;
    if (signs && live)
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = v[j] * signs[c0 + j];
  }
  if (!live) return;
  float* xo = x + (size_t)m * E + c0;
  if (VEC) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int k = 0; k < 4; ++k)
      reinterpret_cast<f32x4*>(xo)[k] = f32x4{v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) xo[j] = v[j];
  }
}

// ---- greedy pick ----
constexpr int kArgThreads = 256;

__global__ void __launch_bounds__(kArgThreads) argmax_parts_kernel(const float* __restrict__ x, int V, int per,
                                                                   uint64_t* __restrict__ part) {
  __shared__ uint64_t wk[kArgThreads / 64];
  const int i0 = blockIdx.x * per, i1 = min(V, i0 + per);
  uint64_t best = 0;
  for (int i = i0 + (int)threadIdx.x; i < i1; i += kArgThreads) best = key_max(best, argmax_key(x[i], i));
  best = wave_max_key(best);
  if ((threadIdx.x & 63) == 0) wk[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = wk[0];
    for (int w = 1; w < kArgThreads / 64; ++w) b = key_max(b, wk[w]);
    part[blockIdx.x] = b;
  }
}
__global__ void __launch_bounds__(64) argmax_pick_kernel(const uint64_t* __restrict__ part, int nparts,
                                                         int* __restrict__ out) {
  uint64_t best = 0;
  for (int i = threadIdx.x; i < nparts; i += 64) best = key_max(best, part[i]);
  best = wave_max_key(best);
  if (threadIdx.x == 0) *out = argmax_key_index(best);
}

__global__ void __launch_bounds__(64) pos_add_kernel(int* d_pos, int M) {
  if (threadIdx.x == 0) (void)atomicAdd(d_pos, M);
}

}  // namespace

int embed(const uint8_t* codes, const uint16_t* scales, const int* d_tok, int M, int E, int block, const float* signs,
          float* x, hipStream_t st) {
  int span = 1024;  // the largest power of two <= 1024 dividing E
  while (E % span) span >>= 1;
  if (span < 128) return fail(BTF_ERR_ARGS, "embed: width must be a multiple of 128");
  if (block > 0 && span % block) return fail(BTF_ERR_ARGS, "embed: hadamard block does not divide the span");
  const int nslices = (E + kSliceVals - 1) / kSliceVals;
  const float hs = block > 0 ? 1.0f / std::sqrt((float)block) : 1.0f;
  const dim3 grid((nslices + kEmbedWaves - 1) / kEmbedWaves, M), blk(64 * kEmbedWaves);
  if ((reinterpret_cast<uintptr_t>(x) & 15) == 0)
    hipLaunchKernelGGL(embed_slices_kernel<true>, grid, blk, 0, st, codes, scales, d_tok, E, nslices, block, hs,
                       block > 0 ? signs : nullptr, x);
  else
    hipLaunchKernelGGL(embed_slices_kernel<false>, grid, blk, 0, st, codes, scales, d_tok, E, nslices, block, hs,
                       block > 0 ? signs : nullptr, x);
  return launch_status("embed_slices_kernel");
}

namespace {
constexpr int kArgPer = 2048;    // logits per part
constexpr int kArgMaxParts = 256;
int argmax_parts_of(int V, int* per) {
  int n = (V + kArgPer - 1) / kArgPer;
  if (n > kArgMaxParts) n = kArgMaxParts;
  if (n < 1) n = 1;
  *per = (V + n - 1) / n;
  return n;
}
}  // namespace

// The no-allocation greedy pick's scratch: one key per part, at most
// kArgMaxParts parts whatever V. Each GPU holds its own copy until the
// process ends; host code uses the address hipGetSymbolAddress gave for the
// device (set up by kernels_init), never this name.
static __device__ __align__(256) uint64_t scratch[kArgMaxParts];

int argmax_scratch_setup(DevState& ds) {
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p)
    return fail(BTF_ERR_DEVICE, std::string("argmax scratch: hipGetSymbolAddress: ") + hipGetErrorString(e));
  ds.argmax_scratch = p;
  return BTF_OK;
}

int argmax_noalloc(const float* logits, int V, int* out, hipStream_t st, const DevState& ds) {
  int per;
  const int n = argmax_parts_of(V, &per);
  if (n > kArgMaxParts) return fail(BTF_ERR_ARGS, "argmax_noalloc: more parts than the static scratch holds");
  if (!ds.argmax_scratch) return fail(BTF_ERR_NOT_INIT, "argmax_noalloc: scratch not set up for this device");
  return argmax(logits, V, ds.argmax_scratch, out, st);
}

int64_t argmax_part_bytes(int V) {
  int per;
  return (int64_t)argmax_parts_of(V > 0 ? V : 1, &per) * (int64_t)sizeof(uint64_t);
}

int argmax(const float* logits, int V, void* part, int* out, hipStream_t st) {
  int per;
  const int n = argmax_parts_of(V, &per);
  hipLaunchKernelGGL(argmax_parts_kernel, dim3(n), dim3(kArgThreads), 0, st, logits, V, per,
                     static_cast<uint64_t*>(part));
  const int rc = launch_status("argmax_parts_kernel");
  if (rc != BTF_OK) return rc;
  hipLaunchKernelGGL(argmax_pick_kernel, dim3(1), dim3(64), 0, st, static_cast<const uint64_t*>(part), n, out);
  return launch_status("argmax_pick_kernel");
}

int pos_add(int* d_pos, int M, hipStream_t st) {
  hipLaunchKernelGGL(pos_add_kernel, dim3(1), dim3(64), 0, st, d_pos, M);
  return launch_status("pos_add_kernel");
}

}  // namespace btfhip
