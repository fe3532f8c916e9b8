// prep.hip -- activation prep for the ternary matmul (gfx950).
//
// Behaviour of the reference's launch_prep / prep_kernel
// (src/cuda/kernels.cu:147-202, 745-774) and of its CPU twin
// EmuDecoder::prep (src/emu_decoder.cpp:122-140):
//   x [M][ldx] -> [RMSNorm * w] -> tiled->grouped perm -> signs ->
//   blockwise WHT (x 1/sqrt(block)) -> Q8_0 (q, d, s) per 32 values.
//
// Two kernels:
//  * q8_kernel: no norm and no transform (every quantize feeding a GEMV in the
//    synthetic workloads). Four lanes own one 32-value block, 8 values each;
//    amax and sum(q) are 2-step DPP quad reductions. Bit-exact with
//    include/btf/packed.hpp:117-134: d = fp16_rn(amax/127) (IEEE division),
//    q = rint(x * (127/amax)) with ties to even, s = sum q. An all-zero block
//    gets d = +-0 with the sign of its last element, as the CPU loop does.
//  * prep_kernel<NORM>: the full transform. One workgroup per (span, row),
//    span S = the largest power of two <= 1024 dividing n; the WHT runs in LDS
//    with the CPU's stage order (len = 1, 2, 4, ...), so it is bit-exact; the
//    RMSNorm sum of squares is a fixed-order double tree, so its last bit can
//    differ from the CPU's sequential double sum (the reference's own GPU
//    kernel has the same property).
#include "../../include/btf/hip_abi.h"
#include "common.h"

#pragma clang fp contract(off)

namespace btfhip {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Quantize 8 consecutive values of one Q8 block held by this lane; the 4
// lanes of a DPP quad hold the block. Returns the two packed q words; d and s
// are valid in every lane of the quad.
__device__ __forceinline__ void q8_quad(const float (&v)[8], uint32_t& q0, uint32_t& q1, float& d, int& s) {
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = quad_max_f(amax);
  // sign of the block's last value, for the all-zero case
  const float last = dpp_f<0xFF>(v[7]);  // quad_perm(3,3,3,3)
  float dd = h2f(f2h_bits(amax / 127.0f));
  if (amax == 0.f) dd = copysignf(0.f, last);
  d = dd;
  const float id = amax != 0.f ? 127.0f / amax : 0.f;
  int qi[8];
  int sum = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    qi[i] = (int)__builtin_rintf(v[i] * id);
    sum += qi[i];
  }
  q0 = (uint32_t)(qi[0] & 0xff) | ((uint32_t)(qi[1] & 0xff) << 8) | ((uint32_t)(qi[2] & 0xff) << 16) |
       ((uint32_t)(qi[3] & 0xff) << 24);
  q1 = (uint32_t)(qi[4] & 0xff) | ((uint32_t)(qi[5] & 0xff) << 8) | ((uint32_t)(qi[6] & 0xff) << 16) |
       ((uint32_t)(qi[7] & 0xff) << 24);
  s = quad_sum_i(sum);
}

// One lane per 8 values. Grid covers M * n / 8 lanes exactly (multiple of 4).
template <bool VEC>
__global__ void __launch_bounds__(256) q8_kernel(const float* __restrict__ x, int ldx, int n, int64_t total_lanes,
                                                  int8_t* __restrict__ q, float* __restrict__ d,
                                                  int32_t* __restrict__ s) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  // Out-of-range lanes still run the quad reductions (on zeros) but store nothing.
  const bool live = gid < total_lanes;
  const int64_t g = live ? gid : 0;
  const int lanes_per_row = n >> 3;
  const int64_t m = g / lanes_per_row;
  const int c8 = (int)(g - m * lanes_per_row);  // 8-value chunk within the row
  const float* xp = x + m * (int64_t)ldx + 8 * c8;
  float v[8];
  if (VEC) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(xp);
    const f32x4 b = *reinterpret_cast<const f32x4*>(xp + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = xp[i];
  }
  uint32_t q0, q1;
  float dd;
  int ss;
  q8_quad(v, q0, q1, dd, ss);
  if (!live) return;
  uint32_t* qp = reinterpret_cast<uint32_t*>(q + m * (int64_t)n + 8 * c8);
  qp[0] = q0;
  qp[1] = q1;
  if ((c8 & 3) == 0) {
    const int64_t bi = m * (int64_t)(n >> 5) + (c8 >> 2);
    d[bi] = dd;
    s[bi] = ss;
  }
}

// ---- full prep ----
struct PrepArgs {
  const float* x;
  int ldx, n, S;
  const float* normw;
  float eps;
  int block, perm_hd, perm_nk, perm_rep;
  const float* signs;
  float* xn_out;
  int ldxn;
  int8_t* q;
  float* d;
  int32_t* s;
};

constexpr int kPrepThreads = 256;

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <bool NORM>
__global__ void __launch_bounds__(kPrepThreads) prep_kernel(PrepArgs a) {
  extern __shared__ float buf[];  // S floats
  __shared__ double red[kPrepThreads / 64];
  const int m = blockIdx.y;
  const int base = blockIdx.x * a.S;
  const float* xr = a.x + (size_t)m * a.ldx;
  float scale = 1.0f;
  if (NORM) {
    double acc = 0.0;
    for (int i = threadIdx.x; i < a.n; i += blockDim.x) acc += (double)xr[i] * (double)xr[i];
    acc = wave_sum_d(acc);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    double sum = 0.0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) sum += red[w];
    const float mean = (float)(sum / (double)a.n);
    scale = 1.0f / sqrtf(mean + a.eps);
  }
  for (int o = threadIdx.x; o < a.S; o += blockDim.x) {
    const int og = base + o;
    int src = og;
    if (a.block > 0 && a.perm_rep > 1) {
      const int dd = og % a.perm_hd, t = og / a.perm_hd;
      const int r = t % a.perm_rep, k = t / a.perm_rep;
      src = dd + a.perm_hd * (k + a.perm_nk * r);
    }
    float v = xr[src];
    if (NORM) v = (v * scale) * a.normw[src];
    if (a.block > 0 && a.signs) v = v * a.signs[og];
    buf[o] = v;
    if (a.xn_out) {
      float u = xr[og];
      if (NORM) u = (u * scale) * a.normw[og];
      a.xn_out[(size_t)m * a.ldxn + og] = u;
    }
  }
  __syncthreads();
  float hs = 1.0f;
  if (a.block > 0) {
    for (int len = 1; len < a.block; len <<= 1) {
      for (int p = threadIdx.x; p < (a.S >> 1); p += blockDim.x) {
        const int j = (p / len) * (len << 1) + (p % len);
        const float u = buf[j], w = buf[j + len];
        buf[j] = u + w;
        buf[j + len] = u - w;
      }
      __syncthreads();
    }
    hs = 1.0f / sqrtf((float)a.block);
  }
  // Q8: 4 lanes per 32-value block, 8 values each.
  const int nlanes = a.S >> 3;
  for (int l0 = 0; l0 < nlanes; l0 += blockDim.x) {
    const int l = l0 + threadIdx.x;
    const bool live = l < nlanes;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float u = live ? buf[8 * l + i] : 0.f;
      v[i] = a.block > 0 ? u * hs : u;
    }
    uint32_t q0, q1;
    float dd;
    int ss;
    q8_quad(v, q0, q1, dd, ss);
    if (live) {
      const size_t col = (size_t)base + 8 * l;
      uint32_t* qp = reinterpret_cast<uint32_t*>(a.q + (size_t)m * a.n + col);
      qp[0] = q0;
      qp[1] = q1;
      if ((l & 3) == 0) {
        const size_t bi = (size_t)m * (a.n >> 5) + (col >> 5);
        a.d[bi] = dd;
        a.s[bi] = ss;
      }
    }
  }
}

int span_of(int n) {
  int s = 1;
  while (s < 1024 && n % (s * 2) == 0) s *= 2;
  return s;
}

}  // namespace

int prep(const float* x, int ldx, int M, int n, const float* normw, float eps, int block, int perm_hd, int perm_nk,
         int perm_rep, const float* signs, float* xn_out, int ldxn, int8_t* q, float* d, int32_t* s, hipStream_t st,
         const DevState& ds) {
  (void)ds;
  if (!normw && block <= 0 && !xn_out) {
    const int64_t lanes = (int64_t)M * (n / 8);
    const int64_t grid = (lanes + 255) / 256;
    const bool vec = ((reinterpret_cast<uintptr_t>(x) & 15) == 0) && (ldx % 4 == 0);
    if (vec)
      hipLaunchKernelGGL(q8_kernel<true>, dim3((unsigned)grid), dim3(256), 0, st, x, ldx, n, lanes, q, d, s);
    else
      hipLaunchKernelGGL(q8_kernel<false>, dim3((unsigned)grid), dim3(256), 0, st, x, ldx, n, lanes, q, d, s);
    return launch_status("q8_kernel");
  }
  PrepArgs p{};
  p.x = x;
  p.ldx = ldx;
  p.n = n;
  p.S = span_of(n);
  p.normw = normw;
  p.eps = eps;
  p.block = block;
  p.perm_hd = perm_hd;
  p.perm_nk = perm_nk;
  p.perm_rep = perm_rep;
  p.signs = signs;
  p.xn_out = xn_out;
  p.ldxn = ldxn;
  p.q = q;
  p.d = d;
  p.s = s;
  if (block > 0 && (p.S % block)) return fail(BTF_ERR_ARGS, "prep: hadamard block does not divide the span");
  const dim3 grid(n / p.S, M);
  const size_t smem = (size_t)p.S * sizeof(float);
  if (normw)
    hipLaunchKernelGGL(prep_kernel<true>, grid, dim3(kPrepThreads), smem, st, p);
  else
    hipLaunchKernelGGL(prep_kernel<false>, grid, dim3(kPrepThreads), smem, st, p);
  return launch_status("prep_kernel");
}

}  // namespace btfhip
