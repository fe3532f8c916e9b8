// gemv_dot4.hip -- ternary GEMV / small-batch GEMM on T2 codes with
// v_dot4_i32_i8 (gfx950). Behaviour of the reference's gemv_kernel
// (src/cuda/kernels.cu:238-334): y = W x, y += W x, or silu(W_g x) * (W_u x),
// with y[m][n] = sum_s fp16(scale[n][s/4]) * d[m][s] * I[m][n][s] and the
// exact integer I[m][n][s] = code . q - s[m][s] per 32-column sub-block.
//
// Work decomposition (designed for wave64 and 16-lane DPP rows):
//  * chunk = 16 B of codes = 64 columns = 2 sub-blocks; a row has CPR = K/64.
//  * A workgroup owns RB = 4*T consecutive output rows of one segment (swiglu:
//    2*T gate rows interleaved with the matching 2*T up rows) and all K.
//  * Its NW waves split K: wave w, lane l owns chunk (w*CL + j)*16 + (l & 15)
//    for j < CL, so every load instruction of a 16-lane group reads 256
//    contiguous bytes of one row, and the lane's activation (64 q bytes,
//    d/16 and -s of its 2 sub-blocks) is loaded once into registers and
//    reused for all T row steps.
//  * The 4 groups of a wave (l >> 4) take 4 different rows per step.
//  * Per row and 1024-column slice (16 lanes x 64 columns): lane partial ->
//    16-lane DPP butterfly -> LDS [slice][row] -> fixed-order sum over the
//    slices -> epilogue. The float order is fixed (deterministic run to run)
//    and does not depend on how slices are spread over waves, so the
//    persistent step kernel, which walks the same slices, gives identical
//    results.
//  * QOUT (fused output quantize, one activation row): a workgroup owns one
//    32-row block of the output (T = 8; swiglu T = 16), and its epilogue
//    also writes the Q8 of that block (a half-wave per block, DPP
//    reductions), so the next GEMV of a chain reads it without a quantize
//    launch in between.
//  * QIN (fused input quantize, one activation row): instead of reading Q8
//    rows, each wave quantizes the fp32 input over its own K range (lane t:
//    16*CL consecutive values, a 32-value block per lane pair or per lane)
//    into LDS with the arithmetic of the q8 kernel, while the weight loads
//    are in flight; the q/d/s it reads back are those a separate quantize
//    launch would have written.
#include <climits>

#include "../../include/btf/hip_abi.h"
#include "common.h"

// Floating-point expressions are evaluated as written (no fused multiply-add
// unless fmaf is spelled out), so the per-slice row sums have one defined
// rounding order, shared by every kernel that produces them.
#pragma clang fp contract(off)

namespace btfhip {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct Dot4Args {
  const uint8_t* codes[3];
  const uint16_t* scales[3];
  float* y[3];
  int N[3];
  int ldy[3];
  int wg_start[3];  // first workgroup of each segment; INT_MAX when absent
  const uint8_t* up_codes;  // swiglu: the up matrix (segment 0 is gate)
  const uint16_t* up_scales;
  int K, cpr, nsub;
  const int8_t* q;
  const float* d;
  const int32_t* s;
  int m0, nb;
  int32_t* dump;
  const float* x;  // QIN: fp32 input rows
  int ldx;
  int8_t* oq;  // QOUT: Q8 rows of the output (q [.][N], d and s [.][N/32])
  float* od;
  int32_t* os;
};

constexpr int kMaxWaves = 16;

// QIN: the Q8 of values [v0, v0 + 16*CL) of row x (0 past K) into this
// wave's LDS region xw: words q, then d and s per 32-value block. CL == 1: a
// block spans lanes 2u, 2u+1 (DPP quad_perm exchanges of amax, sum, last).
// Same arithmetic as the q8 kernel: d = fp16_rn(amax/127), q = rint(x *
// (127/amax)), s = sum q, all-zero block: d = +-0 with its last value's sign.
// The lane's values, loaded before the weight stream is issued (loads return
// in order: issued after it, they would arrive after the last weight).
// A lane past K loads the row's first values (in bounds) and zeroes them in
// quantize_lane.
template <int CL>
__device__ __forceinline__ void load_lane_x(const float* __restrict__ xrow, int v0, int K, float4 (&v)[4 * CL]) {
  const float* p = xrow + (v0 < K ? v0 : 0);  // K % 128 == 0: the lane's range is all in or all out
#pragma unroll
  for (int i = 0; i < 4 * CL; ++i) v[i] = *reinterpret_cast<const float4*>(p + 4 * i);
}
template <int CL>
__device__ __forceinline__ void quantize_lane(const float4 (&xv)[4 * CL], bool live, int lane, uint32_t* xw) {
  constexpr int NV = 16 * CL;
  float v[NV];
#pragma unroll
  for (int i = 0; i < 4 * CL; ++i) {
    v[4 * i] = live ? xv[i].x : 0.f;
    v[4 * i + 1] = live ? xv[i].y : 0.f;
    v[4 * i + 2] = live ? xv[i].z : 0.f;
    v[4 * i + 3] = live ? xv[i].w : 0.f;
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) amax = fmaxf(amax, fabsf(v[i]));
  float last = v[NV - 1];
  if constexpr (CL == 1) {
    amax = fmaxf(amax, dpp_f<0xB1>(amax));  // quad_perm(1,0,3,2): the pair's other half
    last = dpp_f<0xF5>(last);               // quad_perm(1,1,3,3): the odd lane holds the block's end
  }
  float d = h2f(f2h_bits(amax / 127.0f));
  if (amax == 0.f) d = copysignf(0.f, last);
  const float id = amax != 0.f ? 127.0f / amax : 0.f;
  int sum = 0;
  uint32_t wq[NV / 4];
#pragma unroll
  for (int k = 0; k < NV / 4; ++k) {
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = (int)__builtin_rintf(v[4 * k + i] * id);
      sum += q;
      word |= (uint32_t)(q & 0xff) << (8 * i);
    }
    wq[k] = word;
  }
  if constexpr (CL == 1) sum += dpp_i<0xB1>(sum);
#pragma unroll
  for (int k = 0; k < NV / 4; k += 4)
    *reinterpret_cast<u32x4*>(xw + lane * (NV / 4) + k) = u32x4{wq[k], wq[k + 1], wq[k + 2], wq[k + 3]};
  const int blk = CL == 1 ? lane >> 1 : lane;
  if (CL == 2 || (lane & 1) == 0) {
    xw[CL * 256 + blk] = __float_as_uint(d);
    xw[CL * 288 + blk] = (uint32_t)sum;
  }
}

template <int CL, int NB, int T, int MODE, bool DUMP, bool QIN, bool QOUT>
__global__ void __launch_bounds__(QOUT ? 640 : 1024) gemv_dot4_kernel(Dot4Args a) {
  constexpr int RB = 4 * T;  // virtual rows per workgroup (4 per step)
  __shared__ float red[NB][kMaxWaves * CL][RB];
  constexpr int kXW = CL * 320;  // QIN: LDS words per wave (q, d, s of its K range)
  __shared__ uint32_t xq[QIN ? kMaxWaves * kXW : 1];

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const int l16 = lane & 15;
  const int grp = lane >> 4;

  const int bid = blockIdx.x;
  const int seg = (bid >= a.wg_start[1]) + (bid >= a.wg_start[2]);
  const uint8_t* codes = seg == 0 ? a.codes[0] : seg == 1 ? a.codes[1] : a.codes[2];
  const uint16_t* scales = seg == 0 ? a.scales[0] : seg == 1 ? a.scales[1] : a.scales[2];
  float* y = seg == 0 ? a.y[0] : seg == 1 ? a.y[1] : a.y[2];
  const int N = seg == 0 ? a.N[0] : seg == 1 ? a.N[1] : a.N[2];
  const int ldy = seg == 0 ? a.ldy[0] : seg == 1 ? a.ldy[1] : a.ldy[2];
  const int wg0 = seg == 0 ? 0 : seg == 1 ? a.wg_start[1] : a.wg_start[2];

  const int K = a.K;
  const int rowb = K >> 2;     // code bytes per row
  const int nsc = K >> 7;      // scales per row
  const int nsub = a.nsub;     // sub-blocks per row

  // First real row of this workgroup, and this lane's matrix / row stride.
  int r0;
  const uint8_t* cbase = codes;
  const uint16_t* sbase = scales;
  if constexpr (MODE == BTF_GEMV_SWIGLU) {
    r0 = (bid - wg0) * (2 * T);
    if (grp & 1) {
      cbase = a.up_codes;
      sbase = a.up_scales;
    }
  } else {
    r0 = (bid - wg0) * RB;
  }

  // ---- this lane's chunks ----
  int chunk[CL];
  bool cval[CL];
#pragma unroll
  for (int j = 0; j < CL; ++j) {
    chunk[j] = (w * CL + j) * 16 + l16;
    cval[j] = chunk[j] < a.cpr;
  }
  // ---- stream the rows ----
  float acc[T][NB][CL];  // one partial per 1024-column slice

  // The activation (L2-resident) is loaded first, then every code and scale
  // load of the workgroup's rows (the HBM stream): loads return in order, so
  // the dot products of row step t start as soon as its codes are in, while
  // the later steps stream. The scheduling barriers keep the compiler from
  // hoisting consumers of early loads above later issues, which would
  // serialise the round trips. Lanes past the row end or batch load valid
  // addresses and are zeroed after the barrier.
  float4 xv[QIN ? 4 * CL : 1];
  uint4 rq[QIN ? 1 : NB][CL][4];
  float2 rd[QIN ? 1 : NB][CL];
  int2 rs[QIN ? 1 : NB][CL];
  if constexpr (QIN) {
    load_lane_x<CL>(a.x + (size_t)a.m0 * a.ldx, w * CL * 1024 + lane * 16 * CL, K, xv);
  } else {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int j = 0; j < CL; ++j) {
        const size_t m = (size_t)(a.m0 + (b < a.nb ? b : 0));
        const int c = cval[j] ? chunk[j] : 0;
        const uint4* qp = reinterpret_cast<const uint4*>(a.q + m * K + (size_t)c * 64);
#pragma unroll
        for (int i = 0; i < 4; ++i) rq[b][j][i] = qp[i];
        rd[b][j] = *reinterpret_cast<const float2*>(a.d + m * nsub + 2 * c);
        rs[b][j] = *reinterpret_cast<const int2*>(a.s + m * nsub + 2 * c);
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  u32x4 wv[T][CL];
  uint32_t sc[T][CL];  // 32-bit: keeps every scale load in its own register
  int rowv[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int row = MODE == BTF_GEMV_SWIGLU ? r0 + 2 * t + (grp >> 1) : r0 + 4 * t + grp;
    rowv[t] = row;
    const int rowc = row < N ? row : N - 1;  // clamp: loads stay in bounds
    const uint8_t* crow = cbase + (size_t)rowc * rowb;
    const uint16_t* srow = sbase + (size_t)rowc * nsc;
#pragma unroll
    for (int j = 0; j < CL; ++j) {
      // Unconditional (branch-free) loads: a lane past the row's last chunk
      // reads chunk 0 again; its activation registers are zero, so it adds 0.
      const int c = cval[j] ? chunk[j] : 0;
      wv[t][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(crow + (size_t)c * 16));
      sc[t][j] = __builtin_nontemporal_load(srow + (c >> 1));
    }
  }

  __builtin_amdgcn_sched_barrier(0);

  if constexpr (QIN) {
    quantize_lane<CL>(xv, w * CL * 1024 + lane * 16 * CL < K, lane, &xq[w * kXW]);
    // LDS only: the weight loads stay in flight
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }

  // ---- activation registers ----
  uint32_t aq[NB][CL][16];
  float ad[NB][CL][2];
  int an[NB][CL][2];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
#pragma unroll
    for (int j = 0; j < CL; ++j) {
      if (cval[j] && b < a.nb) {
        const int lc = j * 16 + l16;  // QIN: chunk within the wave's LDS region
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint4 v = QIN ? reinterpret_cast<const uint4*>(&xq[w * kXW + lc * 16])[i] : rq[QIN ? 0 : b][j][i];
          aq[b][j][4 * i + 0] = v.x;
          aq[b][j][4 * i + 1] = v.y;
          aq[b][j][4 * i + 2] = v.z;
          aq[b][j][4 * i + 3] = v.w;
        }
        const float2 dv = QIN ? *reinterpret_cast<const float2*>(&xq[w * kXW + CL * 256 + 2 * lc]) : rd[QIN ? 0 : b][j];
        const int2 sv = QIN ? *reinterpret_cast<const int2*>(&xq[w * kXW + CL * 288 + 2 * lc]) : rs[QIN ? 0 : b][j];
        ad[b][j][0] = dv.x * 0.0625f;  // exact: the dot returns 16 * I
        ad[b][j][1] = dv.y * 0.0625f;
        an[b][j][0] = -sv.x;
        an[b][j][1] = -sv.y;
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) aq[b][j][i] = 0u;
        ad[b][j][0] = ad[b][j][1] = 0.f;
        an[b][j][0] = an[b][j][1] = 0;
      }
    }
  }

  __builtin_amdgcn_sched_barrier(0);

#pragma unroll
  for (int t = 0; t < T; ++t) {
#pragma unroll
    for (int j = 0; j < CL; ++j) {
      const float f = h2f((uint16_t)sc[t][j]);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int y0 = subblock_dot16(wv[t][j].x, wv[t][j].y, &aq[b][j][0], an[b][j][0]);
        const int y1 = subblock_dot16(wv[t][j].z, wv[t][j].w, &aq[b][j][8], an[b][j][1]);
        if constexpr (DUMP) {
          if (cval[j] && b < a.nb && rowv[t] < N) {
            int32_t* o = a.dump + ((size_t)(a.m0 + b) * N + rowv[t]) * nsub + 2 * chunk[j];
            o[0] = y0 >> 4;
            o[1] = y1 >> 4;
          }
        } else {
          float p = ad[b][j][0] * (float)y0;
          p = fmaf(ad[b][j][1], (float)y1, p);
          acc[t][b][j] = f * p;
        }
      }
    }
  }
  if constexpr (DUMP) return;

  // ---- reduce: 16 lanes -> one value per (row, activation row) and slice ----
#pragma unroll
  for (int t = 0; t < T; ++t) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int j = 0; j < CL; ++j) {
        const float v = row16_sum(acc[t][b][j]);
        if (l16 == 0) red[b][w * CL + j][4 * t + grp] = v;
      }
    }
  }
  __syncthreads();
  const int nsl = nw * CL;  // slices; those past the row end hold +0

  // ---- epilogue: fixed-order sum over waves ----
  if constexpr (QOUT) {
    // One 32-row block per activation row: lane r of half-wave b computes
    // row r0 + r, then the half-wave quantizes the block (every lane takes
    // part in the DPP reductions; dead halves work on zeros).
    static_assert(MODE == BTF_GEMV_SWIGLU ? 2 * T == 32 : RB == 32, "QOUT: one 32-row block per workgroup");
    for (int i0 = 0; i0 < NB * 32; i0 += blockDim.x) {
      const int t = i0 + threadIdx.x;
      const int b = t >> 5, r = t & 31;
      const bool live = t < NB * 32 && b < a.nb;  // uniform over the half-wave
      const size_t m = (size_t)(a.m0 + (live ? b : 0));
      const int row = r0 + r;  // N % 32 == 0: the block is inside the output
      float v = 0.f;
      if (live) {
        if constexpr (MODE == BTF_GEMV_SWIGLU) {
          float g = 0.f, u = 0.f;
          for (int k = 0; k < nsl; ++k) {
            g += red[b][k][2 * r];
            u += red[b][k][2 * r + 1];
          }
          v = g / (1.0f + expf(-g)) * u;
        } else {
          float sum = 0.f;
          for (int k = 0; k < nsl; ++k) sum += red[b][k][r];
          v = MODE == BTF_GEMV_ADD ? y[m * ldy + row] + sum : sum;
        }
        y[m * ldy + row] = v;
      }
      float dq;
      int sq;
      const int q = q8_half(v, dq, sq);
      uint32_t wq = (uint32_t)(q & 0xff) << (8 * (r & 3));
      wq |= (uint32_t)dpp_i<0xB1>((int)wq);  // quad_perm(1,0,3,2)
      wq |= (uint32_t)dpp_i<0x4E>((int)wq);  // quad_perm(2,3,0,1)
      if (live) {
        if ((r & 3) == 0) *reinterpret_cast<uint32_t*>(a.oq + m * N + row) = wq;
        if (r == 0) {
          a.od[m * (N / 32) + r0 / 32] = dq;
          a.os[m * (N / 32) + r0 / 32] = sq;
        }
      }
    }
    return;
  }
  for (int i = threadIdx.x; i < NB * RB; i += blockDim.x) {
    const int b = i / RB;
    const int v = i - b * RB;
    if (b >= a.nb) continue;
    const size_t m = (size_t)(a.m0 + b);
    if constexpr (MODE == BTF_GEMV_SWIGLU) {
      if (v & 1) continue;
      float g = 0.f, u = 0.f;
      for (int k = 0; k < nsl; ++k) {
        g += red[b][k][v];
        u += red[b][k][v + 1];
      }
      const int row = r0 + (v >> 1);
      if (row < N) y[m * ldy + row] = g / (1.0f + expf(-g)) * u;
    } else {
      float sum = 0.f;
      for (int k = 0; k < nsl; ++k) sum += red[b][k][v];
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

template <int CL, int NB, int T, int MODE, bool DUMP, bool QIN = false, bool QOUT = false>
void launch_one(const Dot4Args& a, int grid, int threads, hipStream_t st) {
  hipLaunchKernelGGL((gemv_dot4_kernel<CL, NB, T, MODE, DUMP, QIN, QOUT>), dim3(grid), dim3(threads), 0, st, a);
}

template <int CL, int NB, int T, bool DUMP, bool QIN = false>
void by_mode(int mode, const Dot4Args& a, int grid, int threads, hipStream_t st) {
  if (mode == BTF_GEMV_STORE)
    launch_one<CL, NB, T, BTF_GEMV_STORE, DUMP, QIN>(a, grid, threads, st);
  else if (mode == BTF_GEMV_ADD)
    launch_one<CL, NB, T, BTF_GEMV_ADD, DUMP, QIN>(a, grid, threads, st);
  else
    launch_one<CL, NB, T, BTF_GEMV_SWIGLU, DUMP, QIN>(a, grid, threads, st);
}

// QIN (one activation row): CL 1 with T 2/4/8, CL 2 with T 2/4.
template <int CL>
void qin_by_t(int T, int mode, const Dot4Args& a, int grid, int threads, hipStream_t st) {
  if (T == 2) {
    by_mode<CL, 1, 2, false, true>(mode, a, grid, threads, st);
  } else if constexpr (CL == 2) {
    by_mode<CL, 1, 4, false, true>(mode, a, grid, threads, st);
  } else {
    if (T == 4)
      by_mode<CL, 1, 4, false, true>(mode, a, grid, threads, st);
    else
      by_mode<CL, 1, 8, false, true>(mode, a, grid, threads, st);
  }
}

// QOUT (one activation row, with or without QIN): T = 8 (swiglu 16, CL 1
// only: with 2 chunks per lane it would not fit the register file).
template <int CL, bool QIN>
void qout_by_mode(int mode, const Dot4Args& a, int grid, int threads, hipStream_t st) {
  if (mode == BTF_GEMV_STORE)
    launch_one<CL, 1, 8, BTF_GEMV_STORE, false, QIN, true>(a, grid, threads, st);
  else if (mode == BTF_GEMV_ADD)
    launch_one<CL, 1, 8, BTF_GEMV_ADD, false, QIN, true>(a, grid, threads, st);
  else if constexpr (CL == 1)
    launch_one<CL, 1, 16, BTF_GEMV_SWIGLU, false, QIN, true>(a, grid, threads, st);
}

// Instantiated shapes: CL=1 with NB 1/2 (T 2/4/8) and NB 4 (T 2); CL=2 with
// NB 1 (T 2/4). Every one of them fits 128 VGPRs without scratch.
template <int CL, int NB>
void by_t(int T, int mode, bool dump, const Dot4Args& a, int grid, int threads, hipStream_t st) {
  if (dump) {
    by_mode<CL, NB, 2, true>(mode, a, grid, threads, st);
    return;
  }
  if constexpr (CL * NB >= 4) {
    by_mode<CL, NB, 2, false>(mode, a, grid, threads, st);
  } else if constexpr (CL == 2) {
    if (T == 2)
      by_mode<CL, NB, 2, false>(mode, a, grid, threads, st);
    else
      by_mode<CL, NB, 4, false>(mode, a, grid, threads, st);
  } else {
    switch (T) {
      case 2: by_mode<CL, NB, 2, false>(mode, a, grid, threads, st); break;
      case 4: by_mode<CL, NB, 4, false>(mode, a, grid, threads, st); break;
      default: by_mode<CL, NB, 8, false>(mode, a, grid, threads, st); break;
    }
  }
}

}  // namespace

int gemv_dot4(const GemvSeg* segs, int nseg, int K, int m0, int nb, const Q8& act, int mode, int32_t* dump,
              hipStream_t st, const DevState& ds, const float* x, int ldx, const Q8* qout) {
  const int cpr = K / 64;
  // chunks per lane: 1 up to K = 16384 (16 waves x 16 lanes x 64 columns), else 2
  // (the fused output quantize runs at most 10 waves: 2 chunks per lane past K = 10240)
  const int CL = cpr <= (qout ? 160 : 16 * kMaxWaves) ? 1 : 2;
  const int nw = (cpr + 16 * CL - 1) / (16 * CL);
  if (nw > kMaxWaves) return fail(BTF_ERR_ARGS, "gemv: K too large for the dot4 path");
  const int NB = nb <= 1 ? 1 : nb <= 2 ? 2 : 4;
  if (CL * NB > 4 || (CL == 2 && NB > 1)) return fail(BTF_ERR_ARGS, "gemv: batch too large for the dot4 path");
  if ((x || qout) && (nb != 1 || dump)) return fail(BTF_ERR_ARGS, "gemv: the fused quantizes take one row");
  if (qout && nw > 10) return fail(BTF_ERR_ARGS, "gemv: the fused output quantize takes K <= 20480");
  if (qout && CL == 2 && mode == BTF_GEMV_SWIGLU)
    return fail(BTF_ERR_ARGS, "gemv: the fused output quantize takes swiglu with K <= 10240");

  // rows per workgroup: 4*T (swiglu: 2*T output rows); keep >= 2 workgroups per CU
  const int unit = mode == BTF_GEMV_SWIGLU ? 2 : 4;
  long rows = 0;
  for (int i = 0; i < nseg; ++i) rows += (mode == BTF_GEMV_SWIGLU && i > 0) ? 0 : segs[i].N;
  int T = 8;
  while (T > 2 && rows / (unit * T) < 2L * ds.cu_count) T /= 2;
  if (NB * CL >= 4 && T > 2) T = 2;  // register budget
  if (CL == 2 && T > 4) T = 4;
  if (dump) T = 2;
  if (qout) T = mode == BTF_GEMV_SWIGLU ? 16 : 8;  // one 32-row output block per workgroup

  Dot4Args a{};
  int wg = 0;
  const int nuse = mode == BTF_GEMV_SWIGLU ? 1 : nseg;
  for (int i = 0; i < 3; ++i) {
    if (i < nuse) {
      a.codes[i] = segs[i].codes;
      a.scales[i] = segs[i].scales;
      a.y[i] = segs[i].y;
      a.N[i] = segs[i].N;
      a.ldy[i] = segs[i].ldy;
      a.wg_start[i] = wg;
      wg += (segs[i].N + unit * T - 1) / (unit * T);
    } else {
      a.wg_start[i] = INT_MAX;
    }
  }
  if (mode == BTF_GEMV_SWIGLU) {
    a.up_codes = segs[1].codes;
    a.up_scales = segs[1].scales;
  }
  a.K = K;
  a.cpr = cpr;
  a.nsub = K / 32;
  a.q = act.q;
  a.d = act.d;
  a.s = act.s;
  a.m0 = m0;
  a.nb = nb;
  a.dump = dump;
  a.x = x;
  a.ldx = ldx;
  if (qout) {
    a.oq = const_cast<int8_t*>(qout->q);
    a.od = const_cast<float*>(qout->d);
    a.os = const_cast<int32_t*>(qout->s);
  }
  if (wg == 0) return BTF_OK;
  const int threads = 64 * nw;
  const bool dmp = dump != nullptr;
  if (qout) {
    if (CL == 1)
      x ? qout_by_mode<1, true>(mode, a, wg, threads, st) : qout_by_mode<1, false>(mode, a, wg, threads, st);
    else
      x ? qout_by_mode<2, true>(mode, a, wg, threads, st) : qout_by_mode<2, false>(mode, a, wg, threads, st);
    return launch_status("gemv_dot4_kernel");
  }
  if (x) {
    if (CL == 1)
      qin_by_t<1>(T, mode, a, wg, threads, st);
    else
      qin_by_t<2>(T, mode, a, wg, threads, st);
    return launch_status("gemv_dot4_kernel");
  }
  if (CL == 1) {
    if (NB == 1) by_t<1, 1>(T, mode, dmp, a, wg, threads, st);
    else if (NB == 2) by_t<1, 2>(T, mode, dmp, a, wg, threads, st);
    else by_t<1, 4>(T, mode, dmp, a, wg, threads, st);
  } else {
    by_t<2, 1>(T, mode, dmp, a, wg, threads, st);
  }
  return launch_status("gemv_dot4_kernel");
}

}  // namespace btfhip
