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
#include <climits>

#include "../../include/btf/hip_abi.h"
#include "common.h"

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
};

constexpr int kMaxWaves = 16;

template <int CL, int NB, int T, int MODE, bool DUMP>
__global__ void __launch_bounds__(1024) gemv_dot4_kernel(Dot4Args a) {
  constexpr int RB = 4 * T;  // virtual rows per workgroup (4 per step)
  __shared__ float red[NB][kMaxWaves * CL][RB];

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

  // Issue every code and scale load of the workgroup's rows first (the HBM
  // stream), then the activation (L2-resident). The scheduling barriers keep
  // the compiler from hoisting consumers of early loads above later issues,
  // which would serialise the round trips.
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

  // ---- activation registers ----
  uint32_t aq[NB][CL][16];
  float ad[NB][CL][2];
  int an[NB][CL][2];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
#pragma unroll
    for (int j = 0; j < CL; ++j) {
      if (cval[j] && b < a.nb) {
        const size_t m = (size_t)(a.m0 + b);
        const uint4* qp = reinterpret_cast<const uint4*>(a.q + m * K + (size_t)chunk[j] * 64);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint4 v = qp[i];
          aq[b][j][4 * i + 0] = v.x;
          aq[b][j][4 * i + 1] = v.y;
          aq[b][j][4 * i + 2] = v.z;
          aq[b][j][4 * i + 3] = v.w;
        }
        const float2 dv = *reinterpret_cast<const float2*>(a.d + m * nsub + 2 * chunk[j]);
        const int2 sv = *reinterpret_cast<const int2*>(a.s + m * nsub + 2 * chunk[j]);
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

template <int CL, int NB, int T, int MODE, bool DUMP>
void launch_one(const Dot4Args& a, int grid, int threads, hipStream_t st) {
  hipLaunchKernelGGL((gemv_dot4_kernel<CL, NB, T, MODE, DUMP>), dim3(grid), dim3(threads), 0, st, a);
}

template <int CL, int NB, int T, bool DUMP>
void by_mode(int mode, const Dot4Args& a, int grid, int threads, hipStream_t st) {
  if (mode == BTF_GEMV_STORE)
    launch_one<CL, NB, T, BTF_GEMV_STORE, DUMP>(a, grid, threads, st);
  else if (mode == BTF_GEMV_ADD)
    launch_one<CL, NB, T, BTF_GEMV_ADD, DUMP>(a, grid, threads, st);
  else
    launch_one<CL, NB, T, BTF_GEMV_SWIGLU, DUMP>(a, grid, threads, st);
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
              hipStream_t st, const DevState& ds) {
  const int cpr = K / 64;
  // chunks per lane: 1 up to K = 16384 (16 waves x 16 lanes x 64 columns), else 2
  const int CL = cpr <= 16 * kMaxWaves ? 1 : 2;
  const int nw = (cpr + 16 * CL - 1) / (16 * CL);
  if (nw > kMaxWaves) return fail(BTF_ERR_ARGS, "gemv: K too large for the dot4 path");
  const int NB = nb <= 1 ? 1 : nb <= 2 ? 2 : 4;
  if (CL * NB > 4 || (CL == 2 && NB > 1)) return fail(BTF_ERR_ARGS, "gemv: batch too large for the dot4 path");

  // rows per workgroup: 4*T (swiglu: 2*T output rows); keep >= 2 workgroups per CU
  const int unit = mode == BTF_GEMV_SWIGLU ? 2 : 4;
  long rows = 0;
  for (int i = 0; i < nseg; ++i) rows += (mode == BTF_GEMV_SWIGLU && i > 0) ? 0 : segs[i].N;
  int T = 8;
  while (T > 2 && rows / (unit * T) < 2L * ds.cu_count) T /= 2;
  if (NB * CL >= 4 && T > 2) T = 2;  // register budget
  if (CL == 2 && T > 4) T = 4;
  if (dump) T = 2;

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
  if (wg == 0) return BTF_OK;
  const int threads = 64 * nw;
  const bool dmp = dump != nullptr;
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
