// gemv_b3.hip -- ternary GEMV reading PTQ1_0 blocks directly (1.75 bits per
// weight), without the T2 repack: y = W x, y += W x or silu(W_g x) * (W_u x)
// on 28-byte blocks (26 bytes of base-3 digits + an fp16 scale per 128
// weights), 18 % fewer weight bytes per row than T2's 34.
//
// The digit layout is the reference's ptq1_0_trit (src/types.hpp:70-78;
// dequantize_row_ptq1_0, src/types.cpp:86-111): element e < 80 is digit e>>4
// of byte e&15, 80 <= e < 120 digit (e-80)>>3 of byte 16+(e&7), 120 <= e
// digit (e-120)>>1 of byte 24+(e&1), where digit n of byte b is
// ((u8)(b*3^n) * 3) >> 8 and the weight is digit - 1. So digit n of four
// consecutive bytes j..j+3 are four consecutive elements, and their dot4
// operand is one activation word as stored.
//
// Decode (two bytes per 16-bit lane): t = q*3 (v_pk_mul_lo_u16) puts the
// digit in each lane's high byte and the next q in its low byte; one
// v_perm_b32 gathers the high bytes of the two lanes of two words (bytes
// j, j+2 and j+1, j+3) into the dot4 operand of bytes j..j+3. Per 4 weights:
// 2 multiplies, 1 permute, 1 dot4, 2 masks.
//
// Work decomposition: one lane owns one 128-weight block of a row; an
// 8-lane group owns one 1024-column slice; a workgroup covers R rows per
// step (R * slices groups, 8 per wave) and T steps. The sums are formed in
// the same floating-point order as the T2 kernel (gemv_dot4.hip): per
// 64-column chunk p = d0*I0, p = fma(d1, I1, p), scaled by the block's
// scale; the two chunks of a block added as the T2 kernel's first butterfly
// level does; an 8-lane butterfly; a fixed-order sum over the slices. So the
// outputs equal the T2 kernel's on the repacked matrix, bit for bit.
#include <climits>

#include "../../include/btf/hip_abi.h"
#include "common.h"

#pragma clang fp contract(off)

namespace btfhip {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));  // blocks are 4-byte aligned
typedef uint32_t u32x3a __attribute__((ext_vector_type(3), aligned(4)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

constexpr int kMaxSlices = 32;  // K <= 32768

struct B3Args {
  const uint8_t* codes[3];  // PTQ1_0 rows (nblk * 28 bytes each)
  float* y[3];
  int N[3];
  int ldy[3];
  int wg_start[3];  // first workgroup of each segment; INT_MAX when absent
  const uint8_t* up_codes;  // swiglu: the up matrix (segment 0 is gate)
  int K, nblk, nsl, nsl_t2, nsub;
  const int8_t* q;
  const float* d;
  const int32_t* s;
  int m0, nb;
};

// k*v in each 16-bit lane
__device__ __forceinline__ uint32_t mulk(uint32_t v, uint16_t k) {
  u16x2 x = __builtin_bit_cast(u16x2, v);
  x = x * k;
  return __builtin_bit_cast(uint32_t, x);
}
// t = 3*v in each 16-bit lane
__device__ __forceinline__ uint32_t mul3(uint32_t v) {
  u16x2 x = __builtin_bit_cast(u16x2, v);
  x = x * (uint16_t)3;
  return __builtin_bit_cast(uint32_t, x);
}

// bytes 0, 2 / 1, 3 of a word into the low bytes of two 16-bit lanes
__device__ __forceinline__ uint32_t spread_lo(uint32_t w) { return __builtin_amdgcn_perm(0u, w, 0x0c020c00u); }
__device__ __forceinline__ uint32_t spread_hi(uint32_t w) { return __builtin_amdgcn_perm(0u, w, 0x0c030c01u); }

// Digit n of a byte b is H(n+1) - 3*H(n), H(n) = floor(b * 3^n / 256) (the
// high byte of b * 3^n, b * 3^5 < 2^16; H(0) = 0): the reference's
// ((u8)(b*3^n) * 3) >> 8 is the carry out of the base-3 shift, and b * 3^n =
// 256 * H(n) + (u8)(b*3^n). So for four bytes, with H(n) gathered into one
// word (the high bytes of b * 3^n in two 16-bit-lane words, v_perm_b32),
// sum_n digit_n . a_n = sum_n [H(n+1) . a_n - 3 * H(n) . a_n]: the products
// are independent (no mask-and-multiply chain) and the -3 * H(n) terms go to
// a second accumulator per sub-block. H(n) <= 80 for n <= 4 (a signed dot4
// operand); H(5) <= 242 is not, so digit 4 is formed as bytes H(5) - 3*H(4)
// (no carry: 3*H(4) <= 240, the difference is 0..2).
struct Acc {
  int a[4];  // sum of H(n+1) . a_n (and digit-4 / tail terms), starting at -s
  int b[4];  // sum of H(n) . a_n, taken 3 times at the end
};
// Bytes of one word w (elements e(n, i) for digit n of byte i): the five
// digit words dot the activation words act[n] (n = 0..4), into sub-blocks sb[n].
__device__ __forceinline__ void word_dot(uint32_t w, const uint32_t (&act)[5], const int (&sb)[5], Acc& c) {
  const uint32_t lo = spread_lo(w), hi = spread_hi(w);  // bytes 0, 2 / 1, 3 in 16-bit lanes
  uint32_t H[6];
#pragma unroll
  for (int n = 1; n <= 5; ++n) {
    constexpr uint16_t p3[6] = {1, 3, 9, 27, 81, 243};
    const uint32_t pl = mulk(lo, p3[n]), ph = mulk(hi, p3[n]);  // b * 3^n, independent of each other
    H[n] = __builtin_amdgcn_perm(ph, pl, 0x07030501u);           // high bytes: bytes 0, 1, 2, 3
  }
  // digits 0..3: H(n+1) . a_n - 3 H(n) . a_n
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    c.a[sb[n]] = sdot4(H[n + 1], act[n], c.a[sb[n]]);
    if (n > 0) c.b[sb[n]] = sdot4(H[n], act[n], c.b[sb[n]]);
  }
  // digit 4 as bytes
  const uint32_t d4 = H[5] - (H[4] + (H[4] << 1));
  c.a[sb[4]] = sdot4(d4, act[4], c.a[sb[4]]);
}

// Sub-block sums I[k] = sum over the block's sub-block k of (digit - 1) * q,
// from the block's 7 words w and its activation words a[0..31] (element 4i..
// 4i+3 in a[i]); I[k] starts at -s[k].
__device__ __forceinline__ void block_dot(const uint32_t (&w)[7], const uint32_t* a, int (&I)[4]) {
  Acc c;
#pragma unroll
  for (int k = 0; k < 4; ++k) c.a[k] = I[k], c.b[k] = 0;
  // bytes 0..15: digit n of bytes 4g..4g+3 = elements 16n+4g.. -> word 4n+g, sub-block n/2
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint32_t act[5] = {a[g], a[4 + g], a[8 + g], a[12 + g], a[16 + g]};
    const int sb[5] = {0, 0, 1, 1, 2};
    word_dot(w[g], act, sb, c);
  }
  // bytes 16..23: digit n of bytes 16+4g.. = elements 80+8n+4g.. -> word 20+2n+g, sub-block (80+8n)/32
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const uint32_t act[5] = {a[20 + g], a[22 + g], a[24 + g], a[26 + g], a[28 + g]};
    const int sb[5] = {2, 2, 3, 3, 3};
    word_dot(w[4 + g], act, sb, c);
  }
  // bytes 24, 25: digits 0..3, elements 120+2n, 121+2n -> words 30, 31, sub-block 3
  uint32_t x = __builtin_amdgcn_perm(0u, w[6], 0x0c010c00u);  // byte 24 | byte 25 << 16
  uint32_t t[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    t[n] = mul3(x);
    x = t[n] & 0x00ff00ffu;
  }
  c.a[3] = sdot4(__builtin_amdgcn_perm(t[1], t[0], 0x07050301u), a[30], c.a[3]);
  c.a[3] = sdot4(__builtin_amdgcn_perm(t[3], t[2], 0x07050301u), a[31], c.a[3]);
#pragma unroll
  for (int k = 0; k < 4; ++k) I[k] = c.a[k] - 3 * c.b[k];
}

template <int NB, int T, int R, int MODE>
__global__ void __launch_bounds__(1024) gemv_b3_kernel(B3Args a) {
  constexpr int RB = R * T;  // virtual rows per workgroup
  __shared__ float red[NB][kMaxSlices + 1][RB];

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int l8 = lane & 7;
  const int grp = w * 8 + (lane >> 3);
  const int nsl = a.nsl;
  const int r = grp / nsl;  // row within a step (r >= R: idle group)
  const int sl = grp - r * nsl;
  const bool glive = r < R;
  const int blk = sl * 8 + l8;
  const bool live = glive && blk < a.nblk;

  const int bid = blockIdx.x;
  const int seg = (bid >= a.wg_start[1]) + (bid >= a.wg_start[2]);
  const uint8_t* codes = seg == 0 ? a.codes[0] : seg == 1 ? a.codes[1] : a.codes[2];
  float* y = seg == 0 ? a.y[0] : seg == 1 ? a.y[1] : a.y[2];
  const int N = seg == 0 ? a.N[0] : seg == 1 ? a.N[1] : a.N[2];
  const int ldy = seg == 0 ? a.ldy[0] : seg == 1 ? a.ldy[1] : a.ldy[2];
  const int wg0 = seg == 0 ? 0 : seg == 1 ? a.wg_start[1] : a.wg_start[2];
  const int r0 = (bid - wg0) * (MODE == BTF_GEMV_SWIGLU ? RB / 2 : RB);
  const uint8_t* base = (MODE == BTF_GEMV_SWIGLU && (r & 1)) ? a.up_codes : codes;
  const size_t rowb = (size_t)a.nblk * 28;
  const int K = a.K;

  // ---- loads: the activation (L2-resident) first, then the weight stream ----
  // Loads return in order, so the blocks of step t are dotted as soon as they
  // are in while the later steps stream. Lanes past the row end or batch load
  // valid addresses (block 0, activation row m0) and are zeroed afterwards.
  u32x4 rq[NB][8];
  float2 rd[NB][2];
  int2 rs[NB][2];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const size_t m = (size_t)(a.m0 + (b < a.nb ? b : 0));
    const int c = live ? blk : 0;
    const u32x4* qp = reinterpret_cast<const u32x4*>(a.q + m * K + (size_t)c * 128);
#pragma unroll
    for (int i = 0; i < 8; ++i) rq[b][i] = qp[i];
    const float2* dp = reinterpret_cast<const float2*>(a.d + m * a.nsub + 4 * c);  // 8-byte aligned
    const int2* sp = reinterpret_cast<const int2*>(a.s + m * a.nsub + 4 * c);
    rd[b][0] = dp[0], rd[b][1] = dp[1];
    rs[b][0] = sp[0], rs[b][1] = sp[1];
  }
  __builtin_amdgcn_sched_barrier(0);

  uint32_t wv[T][7];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int vr = t * R + (glive ? r : 0);
    const int row = MODE == BTF_GEMV_SWIGLU ? r0 + (vr >> 1) : r0 + vr;
    const int rowc = row < N ? row : N - 1;  // clamp: loads stay in bounds
    const uint8_t* p = base + (size_t)rowc * rowb + (size_t)(live ? blk : 0) * 28;
    const u32x4a v0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4a*>(p));
    const u32x3a v1 = __builtin_nontemporal_load(reinterpret_cast<const u32x3a*>(p + 16));
    wv[t][0] = v0.x, wv[t][1] = v0.y, wv[t][2] = v0.z, wv[t][3] = v0.w;
    wv[t][4] = v1.x, wv[t][5] = v1.y, wv[t][6] = v1.z;
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- activation registers: the block's 128 q, d and -s of its 4 sub-blocks ----
  uint32_t aq[NB][32];
  float ad[NB][4];
  int an[NB][4];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const bool on = live && b < a.nb;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      aq[b][4 * i] = on ? rq[b][i].x : 0u;
      aq[b][4 * i + 1] = on ? rq[b][i].y : 0u;
      aq[b][4 * i + 2] = on ? rq[b][i].z : 0u;
      aq[b][4 * i + 3] = on ? rq[b][i].w : 0u;
    }
    ad[b][0] = on ? rd[b][0].x : 0.f, ad[b][1] = on ? rd[b][0].y : 0.f;
    ad[b][2] = on ? rd[b][1].x : 0.f, ad[b][3] = on ? rd[b][1].y : 0.f;
    an[b][0] = on ? -rs[b][0].x : 0, an[b][1] = on ? -rs[b][0].y : 0;
    an[b][2] = on ? -rs[b][1].x : 0, an[b][3] = on ? -rs[b][1].y : 0;
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- per block: 4 exact sub-block sums -> 2 chunk partials -> block partial ----
  float acc[T][NB];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const float f = h2f((uint16_t)(wv[t][6] >> 16));
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      int I[4] = {an[b][0], an[b][1], an[b][2], an[b][3]};
      block_dot(wv[t], aq[b], I);
      float pe = ad[b][0] * (float)I[0];
      pe = fmaf(ad[b][1], (float)I[1], pe);
      float po = ad[b][2] * (float)I[2];
      po = fmaf(ad[b][3], (float)I[3], po);
      acc[t][b] = f * pe + f * po;
    }
  }

  // ---- reduce: 8 lanes -> one value per (row, activation row) and slice ----
  // (the T2 kernel's butterfly levels 2..4 over pairs of its lanes)
  float z[T];  // the T2 kernel's value for a slice with no live column
#pragma unroll
  for (int t = 0; t < T; ++t) {
    z[t] = h2f((uint16_t)(wv[t][6] >> 16)) * 0.0f;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      float v = acc[t][b];
      v += dpp_f<0xB1>(v);   // quad_perm(1,0,3,2)
      v += dpp_f<0x4E>(v);   // quad_perm(2,3,0,1)
      v += dpp_f<0x141>(v);  // row_half_mirror: the other quad of the 8
      if (glive && l8 == 0) red[b][sl][t * R + r] = v;
    }
  }
  if (a.nsl_t2 > nsl && glive && sl == 0 && l8 == 0) {
    // The T2 kernel sums one slice past the row end (its waves cover two
    // slices each); that slice holds 16 copies of block 0's scale * +0.
#pragma unroll
    for (int t = 0; t < T; ++t) {
      float v = z[t];
      v += v;
      v += v;
      v += v;
      v += v;
#pragma unroll
      for (int b = 0; b < NB; ++b) red[b][nsl][t * R + r] = v;
    }
  }
  __syncthreads();
  const int nsum = a.nsl_t2;

  // ---- epilogue: fixed-order sum over the slices ----
  for (int i = threadIdx.x; i < NB * RB; i += blockDim.x) {
    const int b = i / RB;
    const int v = i - b * RB;
    if (b >= a.nb) continue;
    const size_t m = (size_t)(a.m0 + b);
    if constexpr (MODE == BTF_GEMV_SWIGLU) {
      if (v & 1) continue;
      float g = 0.f, u = 0.f;
      for (int k = 0; k < nsum; ++k) {
        g += red[b][k][v];
        u += red[b][k][v + 1];
      }
      const int row = r0 + (v >> 1);
      if (row < N) y[m * ldy + row] = g / (1.0f + expf(-g)) * u;
    } else {
      float sum = 0.f;
      for (int k = 0; k < nsum; ++k) sum += red[b][k][v];
      const int row = r0 + v;
      if (row < N) {
        if constexpr (MODE == BTF_GEMV_ADD)
          y[m * ldy + row] += sum;
        else
          y[m * ldy + row] = sum;
      }
    }
  }
}

template <int NB, int T, int R>
void by_mode(int mode, const B3Args& a, int grid, int threads, hipStream_t st) {
  if (mode == BTF_GEMV_STORE)
    hipLaunchKernelGGL((gemv_b3_kernel<NB, T, R, BTF_GEMV_STORE>), dim3(grid), dim3(threads), 0, st, a);
  else if (mode == BTF_GEMV_ADD)
    hipLaunchKernelGGL((gemv_b3_kernel<NB, T, R, BTF_GEMV_ADD>), dim3(grid), dim3(threads), 0, st, a);
  else
    hipLaunchKernelGGL((gemv_b3_kernel<NB, T, R, BTF_GEMV_SWIGLU>), dim3(grid), dim3(threads), 0, st, a);
}

template <int NB, int R>
void by_t(int T, int mode, const B3Args& a, int grid, int threads, hipStream_t st) {
  if (T == 1)
    by_mode<NB, 1, R>(mode, a, grid, threads, st);
  else if (T == 2)
    by_mode<NB, 2, R>(mode, a, grid, threads, st);
  else
    by_mode<NB, 4, R>(mode, a, grid, threads, st);
}

}  // namespace

int gemv_b3(const GemvSeg* segs, int nseg, int K, int m0, int nb, const Q8& act, int mode, hipStream_t st,
            const DevState& ds) {
  const int nblk = K / 128;
  const int nsl = (K + 1023) / 1024;
  if (nsl > kMaxSlices) return fail(BTF_ERR_ARGS, "gemv_ptq1_0: K must be at most 32768");
  if (nb < 1 || nb > 2) return fail(BTF_ERR_ARGS, "gemv_ptq1_0: 1 or 2 activation rows per pass");
  // rows per step: 8 up to K = 16384 (one wave per slice), else 4
  const int R = nsl <= 16 ? 8 : 4;
  const int nw = (R * nsl + 7) / 8;
  // keep >= 2 workgroups per CU
  long rows = 0;
  for (int i = 0; i < nseg; ++i) rows += (mode == BTF_GEMV_SWIGLU && i > 0) ? 0 : segs[i].N;
  const int unit = mode == BTF_GEMV_SWIGLU ? R / 2 : R;
  int T = 4;
  while (T > 1 && rows / (unit * T) < 2L * ds.cu_count) T /= 2;
  if (nb == 2) T = 1;  // register budget (two activation blocks per lane)

  B3Args a{};
  int wg = 0;
  const int nuse = mode == BTF_GEMV_SWIGLU ? 1 : nseg;
  for (int i = 0; i < 3; ++i) {
    if (i < nuse) {
      a.codes[i] = segs[i].codes;
      a.y[i] = segs[i].y;
      a.N[i] = segs[i].N;
      a.ldy[i] = segs[i].ldy;
      a.wg_start[i] = wg;
      wg += (segs[i].N + unit * T - 1) / (unit * T);
    } else {
      a.wg_start[i] = INT_MAX;
    }
  }
  if (mode == BTF_GEMV_SWIGLU) a.up_codes = segs[1].codes;
  a.K = K;
  a.nblk = nblk;
  a.nsl = nsl;
  // slices the T2 kernel sums: one per 1024 columns up to K = 16384, else
  // two per wave of 32 chunks
  const int cpr = K / 64;
  a.nsl_t2 = cpr <= 256 ? nsl : 2 * ((cpr + 31) / 32);
  a.nsub = K / 32;
  a.q = act.q;
  a.d = act.d;
  a.s = act.s;
  a.m0 = m0;
  a.nb = nb;
  if (wg == 0) return BTF_OK;
  const int threads = 64 * nw;
  if (nb == 1) {
    if (R == 8)
      by_t<1, 8>(T, mode, a, wg, threads, st);
    else
      by_t<1, 4>(T, mode, a, wg, threads, st);
  } else {
    if (R == 8)
      by_mode<2, 1, 8>(mode, a, wg, threads, st);
    else
      by_mode<2, 1, 4>(mode, a, wg, threads, st);
  }
  return launch_status("gemv_b3_kernel");
}

}  // namespace btfhip
