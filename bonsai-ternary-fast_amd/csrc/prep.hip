// prep.hip -- activation prep for the ternary matmul (gfx950).
//
// Behaviour of the reference's launch_prep (src/cuda/kernels.cuh:40-43) and
// of its CPU twin EmuDecoder::prep (src/emu_decoder.cpp:122-140) with
// bd::rmsnorm and bd::hadamard_input (ref/bonsai-decoder/src/cpu_ops.cpp:
// 90-127):
//   x [M][ldx] -> [RMSNorm * w] -> tiled->grouped perm -> signs ->
//   blockwise WHT (x 1/sqrt(block)) -> Q8_0 (q, d, s) per 32 values.
// As on the CPU, the perm and the signs belong to the transform: with
// block == 0 neither is applied.
//
// Two kernels:
//  * q8_kernel: no norm and no transform (every quantize feeding a GEMV in the
//    synthetic workloads). Four lanes own one 32-value block, 8 values each;
//    amax and sum(q) are 2-step DPP quad reductions. Bit-exact with
//    include/btf/packed.hpp:117-134: d = fp16_rn(amax/127) (IEEE division),
//    q = rint(x * (127/amax)) with ties to even, s = sum q. An all-zero block
//    gets d = +-0 with the sign of its last element, as the CPU loop does.
//  * prep_slice_kernel<NORM, PERM, VEC>: the full transform, a wave per
//    (1024-value slice, row) in registers (slice.h): the FWHT runs in the
//    CPU's stage order, so without the norm the result is bit-exact; the
//    RMSNorm's double sum of squares is taken in a fixed canonical order (per
//    32-value block, then over the blocks), so its last bit can differ from
//    the CPU's sequential sum (the reference's own GPU kernel differs
//    likewise).
#include <cmath>

#include "../../include/btf/hip_abi.h"
#include "common.h"
#include "slice.h"

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
// One wave per (1024-value slice, row), every one independent: with the
// norm, the wave first forms the row's RMSNorm scale itself -- lane l sums
// the canonical sums of squares of 32-value blocks l, l + 64, ... (128
// contiguous bytes per lane and block), then the wave sum (slice.h), the
// order in which the step program sums its producers' block sums, so both
// get the same scale bit for bit. Then its slice in registers (lane l holds
// values 16 l .. 16 l + 15): gather through the perm, (x * scale) * w, the
// normed values to xn_out, * signs, the blockwise FWHT, * 1/sqrt(block), the
// Q8 of each lane pair's block.
struct PrepArgs {
  const float* x;
  int ldx, n;
  const float* normw;
  float eps;
  int block, hd, nk, rep;  // rep > 1: tiled -> grouped gather
  float hs;                // 1/sqrtf(block) (block > 0)
  const float* signs;
  float* xn;
  int ldxn;
  int8_t* q;
  float* d;
  int32_t* s;
};

// 16 consecutive values of row xr from index c0 (16-byte loads when VEC).
template <bool VEC>
__device__ __forceinline__ void load16(const float* xr, int c0, float (&v)[16]) {
  if (VEC) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const f32x4 t = reinterpret_cast<const f32x4*>(xr + c0)[k];
      v[4 * k] = t.x;
      v[4 * k + 1] = t.y;
      v[4 * k + 2] = t.z;
      v[4 * k + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = xr[c0 + i];
  }
}

template <bool NORM, bool PERM, bool VEC>
__global__ void __launch_bounds__(64) prep_slice_kernel(PrepArgs a) {
  const int lane = threadIdx.x, m = blockIdx.y;
  const float* xr = a.x + (size_t)m * a.ldx;
  float scale = 1.0f;
  if (NORM) {
    double acc = 0.0;
    for (int b = lane; b < (a.n >> 5); b += 64) {
      float lo[16], hi[16];
      load16<VEC>(xr, 32 * b, lo);
      load16<VEC>(xr, 32 * b + 16, hi);
      acc += block_sumsq(lo, hi);
    }
    scale = norm_scale_of(acc, a.n, a.eps);
  }
  const int c0 = blockIdx.x * kSliceVals + 16 * lane;
  const bool live = c0 < a.n;  // a.n % 32 == 0: a lane pair is all in or all out
  float v[16];
  if (live) {
    if (PERM) {
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] = xr[perm_src(c0 + i, a.hd, a.nk, a.rep)];
    } else {
      load16<VEC>(xr, c0, v);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = 0.f;
  }
  if (NORM && live)
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = (v[i] * scale) * a.normw[PERM ? perm_src(c0 + i, a.hd, a.nk, a.rep) : c0 + i];
  if (a.xn && live) {
    float* xo = a.xn + (size_t)m * a.ldxn + c0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float u = xr[c0 + i];
      if (NORM) u = (u * scale) * a.normw[c0 + i];
      xo[i] = u;
    }
  }
  if (a.block > 0) {
    if (a.signs && live)
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] = v[i] * a.signs[c0 + i];
    slice_fwht(v, lane, a.block);
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = v[i] * a.hs;
  }
  uint32_t qw[4];
  float dd;
  int ss;
  q8_pair(v, qw, dd, ss);
  if (live) {
    uint32_t* qp = reinterpret_cast<uint32_t*>(a.q + (size_t)m * a.n + c0);
    qp[0] = qw[0];
    qp[1] = qw[1];
    qp[2] = qw[2];
    qp[3] = qw[3];
    if (!(lane & 1)) {
      const size_t bi = (size_t)m * (a.n >> 5) + (c0 >> 5);
      a.d[bi] = dd;
      a.s[bi] = ss;
    }
  }
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
  // The transform acts in blocks of `block` values (a power of two) that
  // must divide the span: the largest power of two <= 1024 dividing n.
  int span = 1024;
  while (n % span) span >>= 1;
  if (block > 0 && span % block) return fail(BTF_ERR_ARGS, "prep: hadamard block does not divide the span");
  PrepArgs p{};
  p.x = x;
  p.ldx = ldx;
  p.n = n;
  p.normw = normw;
  p.eps = eps;
  p.block = block > 0 ? block : 0;
  const bool perm = block > 0 && perm_rep > 1;
  p.hd = perm_hd;
  p.nk = perm_nk;
  p.rep = perm_rep;
  p.hs = block > 0 ? 1.0f / std::sqrt((float)block) : 1.0f;
  p.signs = block > 0 ? signs : nullptr;
  p.xn = xn_out;
  p.ldxn = ldxn;
  p.q = q;
  p.d = d;
  p.s = s;
  const bool vec = ((reinterpret_cast<uintptr_t>(x) & 15) == 0) && (ldx % 4 == 0);
  const dim3 grid((n + kSliceVals - 1) / kSliceVals, M), blk(64);
#define BTF_PREP_LAUNCH(NORM, PERM, VEC) \
  hipLaunchKernelGGL((prep_slice_kernel<NORM, PERM, VEC>), grid, blk, 0, st, p)
  if (normw) {
    if (perm) {
      if (vec) BTF_PREP_LAUNCH(true, true, true); else BTF_PREP_LAUNCH(true, true, false);
    } else {
      if (vec) BTF_PREP_LAUNCH(true, false, true); else BTF_PREP_LAUNCH(true, false, false);
    }
  } else {
    if (perm) {
      if (vec) BTF_PREP_LAUNCH(false, true, true); else BTF_PREP_LAUNCH(false, true, false);
    } else {
      if (vec) BTF_PREP_LAUNCH(false, false, true); else BTF_PREP_LAUNCH(false, false, false);
    }
  }
#undef BTF_PREP_LAUNCH
  return launch_status("prep_slice_kernel");
}

}  // namespace btfhip
