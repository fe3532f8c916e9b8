// head.hip -- the kernels either side of a decode step's GEMV chain (gfx950):
// the embedding lookup from the packed table with its inverse transform, the
// greedy pick over the logits, and the position counter.
//
//  * embed_kernel: behaviour of the reference's embed_kernel / launch_embed
//    (src/cuda/kernels.cu:632-662, 886-895) and of its CPU twin, the embedding
//    step of EmuDecoder::chunk (src/emu_decoder.cpp:171-180) with
//    bd::hadamard_inverse (ref/bonsai-decoder/src/cpu_ops.cpp:113-118). One
//    workgroup per (span of S <= 1024 columns, row): the span's code words are
//    staged in LDS with 4-byte reads (the table may live in mapped host
//    memory), decoded to (code - 1) * fp16 scale, then the blockwise FWHT runs
//    in LDS in the CPU's stage order (len = 1, 2, 4, ...), times 1/sqrt(block),
//    times the signs: bit-exact with the CPU.
//  * argmax: the greedy pick, smallest index on ties (src/cuda/kernels.cu:
//    664-704, 897-904; CPU: ref/bonsai-decoder/src/sampler.cpp:20-25). Stage 1:
//    kArgParts workgroups scan interleaved slices and reduce (value, index)
//    pairs in the wave with DPP and v_permlane16/32_swap, then across waves in
//    LDS; stage 2: one workgroup reduces the parts. A NaN logit never wins.
//  * pos_add: *d_pos += M (src/cuda/kernels.cu:706-708), as a vector atomic.
#include <cmath>

#include "../../include/btf/hip_abi.h"
#include "common.h"

#pragma clang fp contract(off)

namespace btfhip {
namespace {

constexpr int kEmbedThreads = 256;

__global__ void __launch_bounds__(kEmbedThreads) embed_kernel(const uint8_t* __restrict__ codes,
                                                               const uint16_t* __restrict__ scales,
                                                               const int* __restrict__ d_tok, int E, int S, int block,
                                                               const float* __restrict__ signs, float* __restrict__ x) {
  extern __shared__ float buf[];                     // S floats
  __shared__ uint32_t cw[1024 / 16];                 // the span's code words (S / 16)
  const int m = blockIdx.y, base = blockIdx.x * S;  // E % S == 0, S % 128 == 0
  const size_t tok = (size_t)d_tok[m];
  const uint32_t* rowc = reinterpret_cast<const uint32_t*>(codes + tok * (size_t)(E / 4) + base / 4);
  for (int i = threadIdx.x; i < S / 16; i += blockDim.x) cw[i] = rowc[i];
  __syncthreads();
  const uint16_t* rows = scales + tok * (size_t)(E / 128);
  for (int o = threadIdx.x; o < S; o += blockDim.x) {
    const int e = base + o, eb = e & 127;
    // T2 address of column eb of a 128-block (include/btf/packed.hpp:35-38)
    const int byte = (e >> 7) * 32 + (eb >> 5) * 8 + ((eb >> 4) & 1) * 4 + (eb & 3) - base / 4;
    const int shift = ((eb >> 2) & 3) * 2;
    const uint32_t c = (cw[byte >> 2] >> ((byte & 3) * 8 + shift)) & 3u;
    buf[o] = (float)((int)c - 1) * h2f(rows[e >> 7]);
  }
  __syncthreads();
  float hs = 1.0f;
  if (block > 0) {
    for (int len = 1; len < block; len <<= 1) {
      for (int p = threadIdx.x; p < (S >> 1); p += blockDim.x) {
        const int j = (p / len) * (len << 1) + (p % len);
        const float u = buf[j], w = buf[j + len];
        buf[j] = u + w;
        buf[j + len] = u - w;
      }
      __syncthreads();
    }
    hs = 1.0f / sqrtf((float)block);
  }
  for (int o = threadIdx.x; o < S; o += blockDim.x) {
    float v = buf[o];
    if (block > 0) v = v * hs;
    if (signs) v = v * signs[base + o];
    x[(size_t)m * E + base + o] = v;
  }
}

// ---- argmax ----
constexpr int kArgParts = 128;
constexpr int kArgThreads = 256;

__device__ __forceinline__ void arg_better(float& bv, int& bi, float v, int i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}
// (value, index) reduction over the 64 lanes; every lane gets the winner.
__device__ __forceinline__ void wave_arg(float& bv, int& bi) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float v;
    int i;
    switch (k) {  // butterfly inside each 16-lane row
      case 0: v = dpp_f<0xB1>(bv), i = dpp_i<0xB1>(bi); break;    // quad_perm(1,0,3,2)
      case 1: v = dpp_f<0x4E>(bv), i = dpp_i<0x4E>(bi); break;    // quad_perm(2,3,0,1)
      case 2: v = dpp_f<0x141>(bv), i = dpp_i<0x141>(bi); break;  // row_half_mirror
      default: v = dpp_f<0x140>(bv), i = dpp_i<0x140>(bi); break; // row_mirror
    }
    arg_better(bv, bi, v, i);
  }
  {  // rows 0 <-> 1, 2 <-> 3
    const auto rv = __builtin_amdgcn_permlane16_swap(__float_as_uint(bv), __float_as_uint(bv), false, false);
    const auto ri = __builtin_amdgcn_permlane16_swap((uint32_t)bi, (uint32_t)bi, false, false);
    arg_better(bv, bi, __uint_as_float(rv[0]), (int)ri[0]);
    arg_better(bv, bi, __uint_as_float(rv[1]), (int)ri[1]);
  }
  {  // halves 0 <-> 1
    const auto rv = __builtin_amdgcn_permlane32_swap(__float_as_uint(bv), __float_as_uint(bv), false, false);
    const auto ri = __builtin_amdgcn_permlane32_swap((uint32_t)bi, (uint32_t)bi, false, false);
    arg_better(bv, bi, __uint_as_float(rv[0]), (int)ri[0]);
    arg_better(bv, bi, __uint_as_float(rv[1]), (int)ri[1]);
  }
}
__device__ __forceinline__ void block_arg(float& bv, int& bi) {
  __shared__ float rv[kArgThreads / 64];
  __shared__ int ri[kArgThreads / 64];
  wave_arg(bv, bi);
  if ((threadIdx.x & 63) == 0) {
    rv[threadIdx.x >> 6] = bv;
    ri[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  bv = -INFINITY;
  bi = 0x7fffffff;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) arg_better(bv, bi, rv[w], ri[w]);
}

__global__ void __launch_bounds__(kArgThreads) argmax_parts(const float* __restrict__ x, int V,
                                                            float2* __restrict__ part) {
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < V; i += gridDim.x * blockDim.x) arg_better(bv, bi, x[i], i);
  block_arg(bv, bi);
  if (threadIdx.x == 0) part[blockIdx.x] = make_float2(bv, __int_as_float(bi));
}
__global__ void __launch_bounds__(kArgThreads) argmax_final(const float2* __restrict__ part, int n,
                                                            int* __restrict__ out) {
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = threadIdx.x; i < n; i += blockDim.x) arg_better(bv, bi, part[i].x, __float_as_int(part[i].y));
  block_arg(bv, bi);
  if (threadIdx.x == 0) *out = bi == 0x7fffffff ? 0 : bi;
}

__global__ void __launch_bounds__(64) pos_add_kernel(int* d_pos, int M) {
  if (threadIdx.x == 0) (void)atomicAdd(d_pos, M);
}

int span_of(int n) {
  int s = 1;
  while (s < 1024 && n % (s * 2) == 0) s *= 2;
  return s;
}

}  // namespace

int embed(const uint8_t* codes, const uint16_t* scales, const int* d_tok, int M, int E, int block, const float* signs,
          float* x, hipStream_t st) {
  const int S = span_of(E);
  if (S < 128) return fail(BTF_ERR_ARGS, "embed: width must be a multiple of 128");
  if (block > 0 && S % block) return fail(BTF_ERR_ARGS, "embed: hadamard block does not divide the span");
  hipLaunchKernelGGL(embed_kernel, dim3(E / S, M), dim3(kEmbedThreads), (size_t)S * sizeof(float), st, codes, scales,
                     d_tok, E, S, block, signs, x);
  return launch_status("embed_kernel");
}

int64_t argmax_part_bytes() { return (int64_t)kArgParts * (int64_t)sizeof(float2); }

int argmax(const float* logits, int V, void* part, int* out, hipStream_t st) {
  hipLaunchKernelGGL(argmax_parts, dim3(kArgParts), dim3(kArgThreads), 0, st, logits, V, static_cast<float2*>(part));
  int rc = launch_status("argmax_parts");
  if (rc != BTF_OK) return rc;
  hipLaunchKernelGGL(argmax_final, dim3(1), dim3(kArgThreads), 0, st, static_cast<const float2*>(part), kArgParts,
                     out);
  return launch_status("argmax_final");
}

int pos_add(int* d_pos, int M, hipStream_t st) {
  hipLaunchKernelGGL(pos_add_kernel, dim3(1), dim3(64), 0, st, d_pos, M);
  return launch_status("pos_add_kernel");
}

}  // namespace btfhip
