// slice.h -- a 1024-value slice of a vector held by one wave64 in registers,
// 16 consecutive values per lane (lane l holds values 16 l .. 16 l + 15), and
// what the activation prep, the embedding lookup and the step program do to
// it without LDS: the blockwise fast Walsh-Hadamard transform, the Q8_0 of
// each 32-value block (one lane pair) and the canonical sum of squares of the
// RMSNorm.
//
// The FWHT follows the CPU's stage order (ref/bonsai-decoder/src/cpu_ops.cpp:
// 76-88: len = 1, 2, 4, ...; x[j] = a + b, x[j + len] = a - b), so it is
// bit-exact: stages len = 1..8 pair values inside a lane, stages len = 16 ..
// 512 pair lane l with lane l ^ (len / 16), exchanged by DPP within a row
// (xor 1, 2 and 8 directly; xor 4 as two moves) and by v_permlane16_swap /
// v_permlane32_swap across rows.
#pragma once
#include "common.h"

namespace btfhip {

constexpr int kSliceVals = 1024;  // values per wave

// Value of lane l ^ X within the 16-lane DPP row (X = 1, 2, 4, 8). A
// composition dpp<B>(dpp<A>(v)) reads lane srcA(srcB(l)): row_half_mirror is
// l ^ 7, quad_perm(3,2,1,0) l ^ 3; a rotation of the row by 8 is l ^ 8.
template <int X>
__device__ __forceinline__ float lane_xor(float v) {
  static_assert(X == 1 || X == 2 || X == 4 || X == 8, "DPP exchange within a row");
  if constexpr (X == 1) return dpp_f<0xB1>(v);                // quad_perm(1,0,3,2)
  if constexpr (X == 2) return dpp_f<0x4E>(v);                // quad_perm(2,3,0,1)
  if constexpr (X == 4) return dpp_f<0x1B>(dpp_f<0x141>(v));  // (l ^ 3) ^ 7
  return dpp_f<0x128>(v);                                     // row_ror:8 = l ^ 8
}
template <int X>
__device__ __forceinline__ int lane_xor_i(int v) {
  return __float_as_int(lane_xor<X>(__int_as_float(v)));
}
template <int X>
__device__ __forceinline__ double lane_xor_d(double v) {
  const uint64_t u = __double_as_longlong(v);
  const uint32_t lo = (uint32_t)__float_as_uint(lane_xor<X>(__uint_as_float((uint32_t)u)));
  const uint32_t hi = (uint32_t)__float_as_uint(lane_xor<X>(__uint_as_float((uint32_t)(u >> 32))));
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
// The values of the lane pair (l & ~16, l | 16) -- lo, hi -- in both lanes
// (v_permlane16_swap of a register with itself), and of (l & ~32, l | 32).
__device__ __forceinline__ void pair16(float v, float& lo, float& hi) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  lo = __uint_as_float(r[0]);
  hi = __uint_as_float(r[1]);
}
__device__ __forceinline__ void pair32(float v, float& lo, float& hi) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  lo = __uint_as_float(r[0]);
  hi = __uint_as_float(r[1]);
}

// One cross-lane butterfly stage: the lower lane of each pair keeps a + b,
// the upper a - b (a = the lower lane's value, b the upper's).
//  * X <= 8 (DPP): without a lane select, each lane adds its partner's value
//    to its own with the sign bit flipped in the upper lane, p + (-v) ==
//    p - v exactly in IEEE (so no lane mask is held in scalar registers).
//  * X = 16, 32: two entries at a time through the swaps of two different
//    registers. v_permlane16_swap(a, b) leaves rows (a0 b0 a2 b2) and
//    (a1 b1 a3 b3) (row = 16 lanes); v_permlane32_swap(a, b) halves (a_lo
//    b_lo) and (a_hi b_hi). Their sum and difference hold a + b and a - b of
//    every pair of both entries, and swapping those two back puts each
//    entry's sums in its lower lanes and differences in its upper lanes: two
//    swaps, an add and a subtract per two entries.
template <int X>
__device__ __forceinline__ void xstage(float (&v)[16], int lane) {
  // Four values (two pairs) at a time: each value a DPP or permlane
  // instruction reads is written two or more instructions before it, so no
  // wait states go between them (one value at a time, the compiler reused one
  // register for every flip and put an s_nop before each read of it; whole
  // token 2.766 -> 2.717 ms). The l ^ 4 stage issues its four mirror moves
  // before the quad permutes that read them, and the cross-row stages swap two
  // pairs before adding either, for the same reason (2.716 -> 2.711 ms).
  if constexpr (X <= 8) {
    constexpr int kBit = X == 1 ? 0 : X == 2 ? 1 : X == 4 ? 2 : 3;
    const uint32_t flip = ((uint32_t)lane >> kBit & 1u) << 31;  // the upper lane negates its own value
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      float t[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) t[k] = __uint_as_float(__float_as_uint(v[i + k]) ^ flip);
      if constexpr (X == 4) {  // l ^ 4 = (l ^ 7) ^ 3: the mirror of all four first
        float m[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) m[k] = dpp_f<0x141>(v[i + k]);
#pragma unroll
        for (int k = 0; k < 4; ++k) v[i + k] = dpp_f<0x1B>(m[k]) + t[k];
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) v[i + k] = lane_xor<X>(v[i + k]) + t[k];
      }
    }
  } else {
    static_assert(X == 16 || X == 32, "cross-row stages");
    auto swap = [](float a, float b, float& lo, float& hi) {
      const auto r = X == 16 ? __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false)
                             : __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
      lo = __uint_as_float(r[0]);
      hi = __uint_as_float(r[1]);
    };
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      float lo[2], hi[2], sm[2], df[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) swap(v[i + 2 * k], v[i + 2 * k + 1], lo[k], hi[k]);
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        sm[k] = lo[k] + hi[k];
        df[k] = lo[k] - hi[k];
      }
#pragma unroll
      for (int k = 0; k < 2; ++k) swap(sm[k], df[k], v[i + 2 * k], v[i + 2 * k + 1]);
    }
  }
}

// Blockwise FWHT butterflies (no scaling) of the wave's slice: every
// `block`-sized run of consecutive values (block a power of two, 1..1024;
// block <= 1 is no transform). Uniform control flow: `block` is the same in
// every lane.
template <int LEN>
__device__ __forceinline__ void istage(float (&v)[16]) {  // an in-lane stage
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    if (j & LEN) continue;
    const float a = v[j], b = v[j + LEN];
    v[j] = a + b;
    v[j + LEN] = a - b;
  }
}
__device__ __forceinline__ void slice_fwht(float (&v)[16], int lane, int block) {
  // (`block` passes an empty asm: its comparisons are made here, per call,
  // not hoisted out of a caller's loop into scalar registers held through it)
  asm volatile("" : "+s"(block));
  if (block > 1) istage<1>(v);
  if (block > 2) istage<2>(v);
  if (block > 4) istage<4>(v);
  if (block > 8) istage<8>(v);
  if (block > 16) xstage<1>(v, lane);
  if (block > 32) xstage<2>(v, lane);
  if (block > 64) xstage<4>(v, lane);
  if (block > 128) xstage<8>(v, lane);
  if (block > 256) xstage<16>(v, lane);
  if (block > 512) xstage<32>(v, lane);
}

// The same butterflies for a slice held strided: lane l holds values
// l + 64 i (i = 0..15), so loads of consecutive values are coalesced across
// the wave. Stages len = 1..32 pair lane l with lane l ^ len, stages
// len = 64..512 pair entries i and i ^ (len / 64) inside the lane; the order
// of the stages and the arithmetic of each butterfly are the CPU's.
__device__ __forceinline__ void slice_fwht_strided(float (&v)[16], int lane, int block) {
  asm volatile("" : "+s"(block));
  if (block > 1) xstage<1>(v, lane);
  if (block > 2) xstage<2>(v, lane);
  if (block > 4) xstage<4>(v, lane);
  if (block > 8) xstage<8>(v, lane);
  if (block > 16) xstage<16>(v, lane);
  if (block > 32) xstage<32>(v, lane);
  if (block > 64) istage<1>(v);
  if (block > 128) istage<2>(v);
  if (block > 256) istage<4>(v);
  if (block > 512) istage<8>(v);
}

// Q8_0 of the 32-value block held by a lane pair (l, l ^ 1): the q bytes of
// this lane's 16 values as 4 little-endian words (word k = values 4k..4k+3),
// and the block's d and s in both lanes. Arithmetic of the q8 kernel
// (include/btf/packed.hpp:117-134): d = fp16_rn(amax / 127) widened, an
// all-zero block's d carries the sign of its last value (the CPU's running
// amax keeps the last zero it compared), q = rint(x * (127 / amax)), s = sum q.
__device__ __forceinline__ void q8_pair(const float (&v)[16], uint32_t (&qw)[4], float& d, int& s) {
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = fmaxf(amax, lane_xor<1>(amax));
  const float last = dpp_f<0xF5>(v[15]);  // quad_perm(1,1,3,3): the odd lane's v[15], value 31 of the block
  float dd = h2f(f2h_bits(amax / 127.0f));
  if (amax == 0.f) dd = copysignf(0.f, last);
  const float id = amax != 0.f ? 127.0f / amax : 0.f;
  int sum = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint32_t w = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int q = (int)__builtin_rintf(v[4 * k + b] * id);
      sum += q;
      w |= (uint32_t)(q & 0xff) << (8 * b);
    }
    qw[k] = w;
  }
  s = sum + lane_xor_i<1>(sum);
  d = dd;
}

// Q8_0 of the 32-value block held by an aligned group of 8 lanes, 4
// consecutive values per lane (lane l: values 4 (l & 7) .. 4 (l & 7) + 3 of
// the block): this lane's q word (word l & 7 of the block) and the block's s
// in every lane of the group, d in its first lane (the one that stores it:
// the all-zero case reads the sign of value 31, lane 7's v[3], through the
// half-row mirror). Arithmetic of q8_pair.
__device__ __forceinline__ uint32_t q8_oct(const float (&v)[4], float& d, int& s) {
  float amax = 0.f;  // (from 0, as q8_pair: a NaN value never becomes the amax)
#pragma unroll
  for (int b = 0; b < 4; ++b) amax = fmaxf(amax, fabsf(v[b]));
  amax = fmaxf(amax, lane_xor<1>(amax));
  amax = fmaxf(amax, lane_xor<2>(amax));
  amax = fmaxf(amax, dpp_f<0x141>(amax));  // row_half_mirror: the other quad of the 8
  const float last = dpp_f<0x141>(v[3]);   // lane 0 of the group <- lane 7
  float dd = h2f(f2h_bits(amax / 127.0f));
  if (amax == 0.f) dd = copysignf(0.f, last);
  const float id = amax != 0.f ? 127.0f / amax : 0.f;
  int sum = 0;
  uint32_t w = 0;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int q = (int)__builtin_rintf(v[b] * id);
    sum += q;
    w |= (uint32_t)(q & 0xff) << (8 * b);
  }
  sum += lane_xor_i<1>(sum);
  sum += lane_xor_i<2>(sum);
  sum += dpp_i<0x141>(sum);
  s = sum;
  d = dd;
  return w;
}

// Canonical sum of squares of a 32-value block, in double: the pairwise tree
// over the value index bits 0, 1, 2, 3, 4 (squares of floats are exact in
// double). Here the lane pair holds the block (levels 1-4 in the lane, level
// 5 across the pair); the step program's producers compute the same tree with
// one value per lane. Both lanes get the sum.
__device__ __forceinline__ double pair_sumsq(const float (&v)[16]) {
  double t[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const double a = (double)v[2 * i], b = (double)v[2 * i + 1];
    const double sa = a * a, sb = b * b;
    t[i] = sa + sb;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) t[i] = t[2 * i] + t[2 * i + 1];
  t[0] = t[0] + t[1];
  t[1] = t[2] + t[3];
  t[0] = t[0] + t[1];
  return t[0] + lane_xor_d<1>(t[0]);
}

// The same canonical sum of squares of a 32-value block held in one lane
// (lo = values 0..15, hi = values 16..31).
__device__ __forceinline__ double block_sumsq(const float (&lo)[16], const float (&hi)[16]) {
  double t[16];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const double a = (double)lo[2 * i], b = (double)lo[2 * i + 1];
    const double c = (double)hi[2 * i], d = (double)hi[2 * i + 1];
    const double sa = a * a, sb = b * b, sc = c * c, sd = d * d;
    t[i] = sa + sb;
    t[8 + i] = sc + sd;
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int i = 0; i < 4; ++i) t[8 * h + i] = t[8 * h + 2 * i] + t[8 * h + 2 * i + 1];
    t[8 * h] = t[8 * h] + t[8 * h + 1];
    t[8 * h + 1] = t[8 * h + 2] + t[8 * h + 3];
    t[8 * h] = t[8 * h] + t[8 * h + 1];
  }
  return t[0] + t[8];
}

// Sum over the wave of one double per lane, every lane getting the total:
// a butterfly over lane bits 0..5 (each pair adds the same two values, so all
// lanes agree bit for bit).
__device__ __forceinline__ double wave_sum_d(double v) {
  v += lane_xor_d<1>(v);
  v += lane_xor_d<2>(v);
  v += lane_xor_d<4>(v);
  v += lane_xor_d<8>(v);
  {
    const uint64_t u = __double_as_longlong(v);
    float llo, lhi, hlo, hhi;
    pair16(__uint_as_float((uint32_t)u), llo, lhi);
    pair16(__uint_as_float((uint32_t)(u >> 32)), hlo, hhi);
    const double a = __longlong_as_double((long long)(((uint64_t)__float_as_uint(hlo) << 32) | __float_as_uint(llo)));
    const double b = __longlong_as_double((long long)(((uint64_t)__float_as_uint(hhi) << 32) | __float_as_uint(lhi)));
    v = a + b;
  }
  {
    const uint64_t u = __double_as_longlong(v);
    float llo, lhi, hlo, hhi;
    pair32(__uint_as_float((uint32_t)u), llo, lhi);
    pair32(__uint_as_float((uint32_t)(u >> 32)), hlo, hhi);
    const double a = __longlong_as_double((long long)(((uint64_t)__float_as_uint(hlo) << 32) | __float_as_uint(llo)));
    const double b = __longlong_as_double((long long)(((uint64_t)__float_as_uint(hhi) << 32) | __float_as_uint(lhi)));
    v = a + b;
  }
  return v;
}

// The RMSNorm scale from the canonical total of a row's block sums of
// squares: lane l adds block sums l, l + 64, ... in order, from 0 (acc);
// then wave_sum_d; mean = f32(total / n), scale = 1 / sqrtf(mean + eps)
// (ref/bonsai-decoder/src/cpu_ops.cpp:121-127).
__device__ __forceinline__ float norm_scale_of(double acc, int n, float eps) {
  const double total = wave_sum_d(acc);
  const float mean = (float)(total / (double)n);
  return 1.0f / sqrtf(mean + eps);
}

// ---- greedy-pick keys ----
// A total order on (value, index) as one 64-bit key: the value's bits made
// order-preserving in the high word (negative: all bits flipped; otherwise
// the sign bit set; -0 is first folded onto +0, as -0 == +0), the complement
// of the index in the low word (the smaller index wins a tie). A NaN gets key
// 0, below every number's key (-inf maps to 0x007FFFFF...), so it never wins
// and an all-NaN input keeps key 0.
__device__ __forceinline__ uint64_t argmax_key(float v, int i) {
  if (v != v) return 0;
  const uint32_t b = __float_as_uint(v + 0.0f);
  const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)o << 32) | (uint32_t)~(uint32_t)i;
}
__device__ __forceinline__ uint64_t key_max(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ __forceinline__ int argmax_key_index(uint64_t k) { return k ? (int)~(uint32_t)k : 0; }
// Max over the wave's 64 keys, in every lane.
__device__ __forceinline__ uint64_t wave_max_key(uint64_t k) {
  auto xchg = [](uint64_t v, auto f) {
    const uint32_t lo = __float_as_uint(f(__uint_as_float((uint32_t)v)));
    const uint32_t hi = __float_as_uint(f(__uint_as_float((uint32_t)(v >> 32))));
    return ((uint64_t)hi << 32) | lo;
  };
  k = key_max(k, xchg(k, [](float x) { return lane_xor<1>(x); }));
  k = key_max(k, xchg(k, [](float x) { return lane_xor<2>(x); }));
  k = key_max(k, xchg(k, [](float x) { return lane_xor<4>(x); }));
  k = key_max(k, xchg(k, [](float x) { return lane_xor<8>(x); }));
  {
    float llo, lhi, hlo, hhi;
    pair16(__uint_as_float((uint32_t)k), llo, lhi);
    pair16(__uint_as_float((uint32_t)(k >> 32)), hlo, hhi);
    k = key_max(((uint64_t)__float_as_uint(hlo) << 32) | __float_as_uint(llo),
                ((uint64_t)__float_as_uint(hhi) << 32) | __float_as_uint(lhi));
  }
  {
    float llo, lhi, hlo, hhi;
    pair32(__uint_as_float((uint32_t)k), llo, lhi);
    pair32(__uint_as_float((uint32_t)(k >> 32)), hlo, hhi);
    k = key_max(((uint64_t)__float_as_uint(hlo) << 32) | __float_as_uint(llo),
                ((uint64_t)__float_as_uint(hhi) << 32) | __float_as_uint(lhi));
  }
  return k;
}

// Source index of destination og under the tiled -> grouped gather
// (ref/bonsai-decoder/src/cpu_ops.cpp:96-104: out[d + hd (r + rep k)] =
// x[d + hd (k + nk r)]).
__device__ __forceinline__ int perm_src(int og, int hd, int nk, int rep) {
  const int dd = og % hd, t = og / hd;
  const int r = t % rep, k = t / rep;
  return dd + hd * (k + nk * r);
}

}  // namespace btfhip
