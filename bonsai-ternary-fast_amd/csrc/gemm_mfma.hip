// gemm_mfma.hip -- ternary GEMM on T2 codes with int8 MFMA (gfx950), for
// batched decode and prefill. Same contract as the reference's gemv_kernel
// (src/cuda/kernels.cu:238-334) for M activation rows.
//
// Tile: a workgroup of 4 waves owns 64 weight rows (wave w: rows 16w..16w+15;
// swiglu: waves 0-1 gate rows, waves 2-3 the matching up rows) and
// BM = 16*MT activation rows. The K loop walks 128-column blocks (one fp16
// weight scale): codes (64 x 32 B), the block's scales, q (BM x 128 B) and the
// activation d / -s (BM x 4) are staged in LDS, then every wave runs, per
// 32-column sub-block,
//     I = mfma_i32_16x16x32_i8(A = q, B = codes, C = -s)     (exact int32)
//     blk += d[m][s] * (float)I
// and per block acc += fp16(scale[n]) * blk.
// Lane l of a 16x16x32 MFMA holds A row (l%16) and B column (l%16) bytes for
// k = 8*(l/16) .. +7; the codes for columns 8t..8t+7 of a sub-block are the
// 2-bit fields {2(t%2), 2(t%2)+1} of its word t/2, so each lane unpacks its
// B fragment with two shift+mask ops. C row 4*(l/16)+r, column l%16 lands in
// accumulator r of lane l.
#include <climits>

#include "../../include/btf/hip_abi.h"
#include "common.h"

// Floating-point expressions are evaluated as written (no fused multiply-add
// unless fmaf is spelled out), so the per-slice row sums have one defined
// rounding order, shared by every kernel that produces them.
#pragma clang fp contract(off)

namespace btfhip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct MfmaArgs {
  const uint8_t* codes[3];
  const uint16_t* scales[3];
  float* y[3];
  int N[3];
  int ldy[3];
  int tile_start[3];  // first n-tile of each segment; INT_MAX when absent
  const uint8_t* up_codes;
  const uint16_t* up_scales;
  int K, nsub;
  const int8_t* q;
  const float* d;
  const int32_t* s;
  int m0, nb;
  int32_t* dump;
};

// KB 128-column blocks are staged per iteration (one round of loads per KB
// blocks instead of per block: the loop is bound by load latency, not by
// the MFMA work of a block).
template <int MT, int KB, int MODE, bool DUMP>
__global__ void __launch_bounds__(256) gemm_mfma_kernel(MfmaArgs a) {
  constexpr int BM = 16 * MT;
  constexpr int CS = 8 * KB + 1;   // words per staged code row (KB x 32 B + 4 B pad)
  constexpr int QS = 32 * KB + 2;  // words per staged q row (KB x 128 B + 8 B pad)
  __shared__ uint32_t cs[64 * CS];
  __shared__ uint16_t scs[64 * KB];
  __shared__ uint32_t qsm[BM * QS];
  __shared__ float dsm[4 * KB][BM];
  __shared__ int32_t nsm[4 * KB][BM];
  __shared__ float upx[(MODE == BTF_GEMV_SWIGLU) ? 32 * BM : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int li = lane & 15;
  const int t = lane >> 4;

  const int bx = blockIdx.x;
  const int seg = (bx >= a.tile_start[1]) + (bx >= a.tile_start[2]);
  const uint8_t* codes = seg == 0 ? a.codes[0] : seg == 1 ? a.codes[1] : a.codes[2];
  const uint16_t* scales = seg == 0 ? a.scales[0] : seg == 1 ? a.scales[1] : a.scales[2];
  float* y = seg == 0 ? a.y[0] : seg == 1 ? a.y[1] : a.y[2];
  const int N = seg == 0 ? a.N[0] : seg == 1 ? a.N[1] : a.N[2];
  const int ldy = seg == 0 ? a.ldy[0] : seg == 1 ? a.ldy[1] : a.ldy[2];
  const int tile0 = seg == 0 ? 0 : seg == 1 ? a.tile_start[1] : a.tile_start[2];
  const int K = a.K;
  const int rowb = K >> 2, nsc = K >> 7, nsub = a.nsub;

  // staged row r (0..63) -> matrix row and source
  constexpr int ROWS_REAL = MODE == BTF_GEMV_SWIGLU ? 32 : 64;
  const int n0 = (bx - tile0) * ROWS_REAL;
  const int mb = blockIdx.y * BM;  // first activation row of the tile (relative to m0)

  float acc[MT][4], blk[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[mt][r] = 0.f;

  for (int kb0 = 0; kb0 < nsc; kb0 += KB) {
    const int nkb = nsc - kb0 < KB ? nsc - kb0 : KB;  // blocks this iteration
    // ---- stage nkb blocks: codes (64 rows x 32 B each), scales, q, d / -s ----
    for (int i = tid; i < 64 * 2 * KB; i += 256) {
      const int r = i / (2 * KB), part = i - r * (2 * KB);  // part: 16-byte half of block part / 2
      if (part >= 2 * nkb) continue;
      const bool up = MODE == BTF_GEMV_SWIGLU && r >= 32;
      const int nr = n0 + (MODE == BTF_GEMV_SWIGLU ? (r & 31) : r);
      const int nc = nr < N ? nr : N - 1;
      const uint8_t* cb = up ? a.up_codes : codes;
      const u32x4 v = *reinterpret_cast<const u32x4*>(cb + (size_t)nc * rowb + kb0 * 32 + 16 * part);
      uint32_t* o = &cs[r * CS + 4 * part];
      o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    }
    for (int i = tid; i < 64 * KB; i += 256) {
      const int r = i / KB, j = i - r * KB;
      if (j >= nkb) continue;
      const bool up = MODE == BTF_GEMV_SWIGLU && r >= 32;
      const int nr = n0 + (MODE == BTF_GEMV_SWIGLU ? (r & 31) : r);
      const int nc = nr < N ? nr : N - 1;
      const uint16_t* sb = up ? a.up_scales : scales;
      scs[r * KB + j] = sb[(size_t)nc * nsc + kb0 + j];
    }
    for (int i = tid; i < BM * 8 * KB; i += 256) {
      const int r = i / (8 * KB), part = i - r * (8 * KB);
      if (part >= 8 * nkb) continue;
      const int m = mb + r;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (m < a.nb) v = *reinterpret_cast<const u32x4*>(a.q + (size_t)(a.m0 + m) * K + kb0 * 128 + 16 * part);
      uint32_t* o = &qsm[r * QS + 4 * part];
      o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    }
    for (int i = tid; i < BM * 4 * KB; i += 256) {
      const int r = i / (4 * KB), sb = i - r * (4 * KB);
      if (sb >= 4 * nkb) continue;
      const int m = mb + r;
      float dv = 0.f;
      int sv = 0;
      if (m < a.nb) {
        const size_t o = (size_t)(a.m0 + m) * nsub + kb0 * 4 + sb;
        dv = a.d[o];
        sv = a.s[o];
      }
      dsm[sb][r] = dv;
      nsm[sb][r] = -sv;
    }
    __syncthreads();

    for (int kbi = 0; kbi < nkb; ++kbi) {
    const int kb = kb0 + kbi;
    // ---- 4 sub-blocks of MFMA ----
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      const int sbx = 4 * kbi + sb;  // staged sub-block
      const uint32_t word = cs[(16 * w + li) * CS + 2 * sbx + (t >> 1)];
      const int sh = 4 * (t & 1);
      const uint32_t lo = (word >> sh) & 0x03030303u;
      const uint32_t hi = (word >> (sh + 2)) & 0x03030303u;
      const long bfrag = (long)(((uint64_t)hi << 32) | lo);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const uint32_t* ap = &qsm[(16 * mt + li) * QS + 8 * sbx + 2 * t];
        const long afrag = (long)(((uint64_t)ap[1] << 32) | ap[0]);
        v4i cin;
        cin[0] = nsm[sbx][16 * mt + 4 * t + 0];
        cin[1] = nsm[sbx][16 * mt + 4 * t + 1];
        cin[2] = nsm[sbx][16 * mt + 4 * t + 2];
        cin[3] = nsm[sbx][16 * mt + 4 * t + 3];
        const v4i I = __builtin_amdgcn_mfma_i32_16x16x32_i8(afrag, bfrag, cin, 0, 0, 0);
        if constexpr (DUMP) {
          const int n = n0 + 16 * w + li;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = mb + 16 * mt + 4 * t + r;
            if (m < a.nb && n < N) a.dump[((size_t)(a.m0 + m) * N + n) * nsub + kb * 4 + sb] = I[r];
          }
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float dv = dsm[sbx][16 * mt + 4 * t + r];
            blk[mt][r] = sb == 0 ? dv * (float)I[r] : fmaf(dv, (float)I[r], blk[mt][r]);
          }
        }
      }
    }
    if constexpr (!DUMP) {
      const float sc = h2f(scs[(16 * w + li) * KB + kbi]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[mt][r] = fmaf(sc, blk[mt][r], acc[mt][r]);
    }
    }  // kbi
    __syncthreads();
  }
  if constexpr (DUMP) return;

  // ---- epilogue ----
  if constexpr (MODE == BTF_GEMV_SWIGLU) {
    if (w >= 2) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) upx[(16 * (w - 2) + li) * BM + 16 * mt + 4 * t + r] = acc[mt][r];
    }
    __syncthreads();
    if (w < 2) {
      const int n = n0 + 16 * w + li;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = mb + 16 * mt + 4 * t + r;
          if (m < a.nb && n < N) {
            const float g = acc[mt][r];
            const float u = upx[(16 * w + li) * BM + 16 * mt + 4 * t + r];
            y[(size_t)(a.m0 + m) * ldy + n] = g / (1.0f + expf(-g)) * u;
          }
        }
    }
  } else {
    const int n = n0 + 16 * w + li;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = mb + 16 * mt + 4 * t + r;
        if (m < a.nb && n < N) {
          float* o = &y[(size_t)(a.m0 + m) * ldy + n];
          if constexpr (MODE == BTF_GEMV_ADD)
            *o += acc[mt][r];
          else
            *o = acc[mt][r];
        }
      }
  }
}

template <int MT, bool DUMP>
void by_mode(int mode, const MfmaArgs& a, dim3 grid, hipStream_t st) {
  constexpr int KB = MT >= 4 ? 1 : 8;
  if (mode == BTF_GEMV_STORE)
    hipLaunchKernelGGL((gemm_mfma_kernel<MT, KB, BTF_GEMV_STORE, DUMP>), grid, dim3(256), 0, st, a);
  else if (mode == BTF_GEMV_ADD)
    hipLaunchKernelGGL((gemm_mfma_kernel<MT, KB, BTF_GEMV_ADD, DUMP>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((gemm_mfma_kernel<MT, KB, BTF_GEMV_SWIGLU, DUMP>), grid, dim3(256), 0, st, a);
}

}  // namespace

int mfma_rows_per_pass() { return 64; }

int gemm_mfma(const GemvSeg* segs, int nseg, int K, int m0, int nb, const Q8& act, int mode, int32_t* dump,
              hipStream_t st, const DevState& ds) {
  (void)ds;
  MfmaArgs a{};
  const int rows_real = mode == BTF_GEMV_SWIGLU ? 32 : 64;
  const int nuse = mode == BTF_GEMV_SWIGLU ? 1 : nseg;
  int tiles = 0;
  for (int i = 0; i < 3; ++i) {
    if (i < nuse) {
      a.codes[i] = segs[i].codes;
      a.scales[i] = segs[i].scales;
      a.y[i] = segs[i].y;
      a.N[i] = segs[i].N;
      a.ldy[i] = segs[i].ldy;
      a.tile_start[i] = tiles;
      tiles += (segs[i].N + rows_real - 1) / rows_real;
    } else {
      a.tile_start[i] = INT_MAX;
    }
  }
  if (mode == BTF_GEMV_SWIGLU) {
    a.up_codes = segs[1].codes;
    a.up_scales = segs[1].scales;
  }
  a.K = K;
  a.nsub = K / 32;
  a.q = act.q;
  a.d = act.d;
  a.s = act.s;
  a.m0 = m0;
  a.nb = nb;
  a.dump = dump;
  if (tiles == 0) return BTF_OK;
  const int MT = nb <= 16 ? 1 : nb <= 32 ? 2 : 4;
  const int BM = 16 * MT;
  const dim3 grid(tiles, (nb + BM - 1) / BM);
  const bool dmp = dump != nullptr;
  if (MT == 1)
    dmp ? by_mode<1, true>(mode, a, grid, st) : by_mode<1, false>(mode, a, grid, st);
  else if (MT == 2)
    dmp ? by_mode<2, true>(mode, a, grid, st) : by_mode<2, false>(mode, a, grid, st);
  else
    dmp ? by_mode<4, true>(mode, a, grid, st) : by_mode<4, false>(mode, a, grid, st);
  return launch_status("gemm_mfma_kernel");
}

}  // namespace btfhip
