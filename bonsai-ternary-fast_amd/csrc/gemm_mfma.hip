// gemm_mfma.hip -- ternary GEMM on T2 codes with int8 MFMA (gfx950), for
// batched decode and prefill. Same contract as the reference's gemv_kernel
// (src/cuda/kernels.cu:238-334) for M activation rows. Kernels:
//   gemm_kp_kernel   up to 16 rows (batched decode): 16 weight rows per
//                    workgroup, K split over its waves, two 32-column
//                    sub-blocks of 8 rows per 16x16x64 MFMA, an LDS-direct
//                    ring per wave;
//   gemm_ks_kernel   17 to 32 rows (and up to 16 when d or s are not 16-byte
//                    aligned): the same workgroup, one sub-block per
//                    16x16x32 MFMA, staged through registers;
//   gemm_pf2_kernel  more rows (prefill): 64 weight rows x 64 or 128
//                    activation rows, fed by an LDS-direct ring;
//   gemm_pf_kernel   the same tile staged through registers (activation
//                    scales not 16-byte aligned).
// Each has a DUMP instance (btf_hip_gemv_i32_dump) that writes the exact
// int32 I of every (row, output, sub-block) from the same tile.
//
// The prefill tile: a workgroup of 4 waves owns 64 weight rows (swiglu: 32
// gate rows and the same 32 up rows) and BM = 32 * MW activation rows; the
// K loop walks 128-column blocks (one fp16 weight scale): codes (64 x 32 B),
// the block's scales, q (BM x 128 B) and the activation d (BM x 4) are staged
// in LDS, then every wave runs, per 32-column sub-block,
//     I = mfma_i32_16x16x32_i8(A = q, B = codes)              (exact int32)
//     blk += d[m][s] * (float)I
// and per block acc += fp16(scale[n]) * blk.
// Lane l of a 16x16x32 MFMA holds A row (l%16) and B column (l%16) bytes for
// k = 8*(l/16) .. +7; the codes for columns 8t..8t+7 of a sub-block are the
// 2-bit fields {2(t%2), 2(t%2)+1} of its word t/2, so each lane unpacks its
// B fragment with two shift+mask ops. C row 4*(l/16)+r, column l%16 lands in
// accumulator r of lane l. gemm_pf_kernel starts the accumulator at -s (the
// codes 0 / 1 / 2 as they are); gemm_pf2_kernel and gemm_ks_kernel map the
// codes to int8 -1 / 0 / +1 (one byte permute per word) and start it at 0.
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
  // optional Q8 of the outputs (segment 0 after the mode), for the next GEMM:
  // q [.][N], d and s [.][N / 32] at activation row m0 + m (gemm_ks_kernel, TR = 2)
  int8_t* oq;
  float* od;
  int32_t* os;
};

// ---- LDS-direct loads (the packed K-split tile and the prefill tile) ----
// vmcnt(N) alone (expcnt, lgkmcnt not waited on).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | 0x0F70);
}
// One wave-wide load into LDS: lane l's 16 bytes from g land at LDS byte
// address lds + 16 l; a 2-byte load fills the low half of the 4-byte slot at
// lds + 4 l (sub-dword loads keep 4-byte lane slots). Issued as inline assembly so that the compiler's
// wait insertion does not order every later LDS read behind it; the kernel
// waits with wait_vm itself. The LDS base is an input bound to M0 (the
// "{m0}" constraint): the compiler writes M0 itself and knows what it holds;
// the statement adds the one wait state an LDS-direct load needs after an
// SALU write of M0.
__device__ __forceinline__ void lds_dma16(const void* g, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}
__device__ __forceinline__ void lds_dma2(const void* g, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_ushort %0, off" : : "v"(g), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}
__device__ __forceinline__ void lds_dma4(const void* g, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" : : "v"(g), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}

// K-split tile for batched decode (up to 32 activation rows): a workgroup of
// NW waves owns 16 weight rows (swiglu: 16 gate rows and the same 16 up rows)
// and BM activation rows, and wave w walks its 1/NW of the 128-column blocks,
// staging its own codes, scales, q and d in a private LDS region (the codes
// are permuted to int8 -1 / 0 / +1, so the MFMA yields I with accumulator 0
// and s is not read), KB blocks per round. The activation is re-read from L2
// by each tile. Per wave the row sums follow the prefill tile's order over
// its blocks (blk = d * I over a block's sub-blocks, acc += scale * blk per
// block), and the NW wave partials are added in wave order: ((p0 + p1) + p2) + ...
// TR = 2: the workgroup owns 32 weight rows (two 16-row tiles, each with its
// gate and up rows), one Q8 block of the output for every activation row, so
// it also writes the Q8 of its outputs (a.oq) with the q8 kernel's
// arithmetic. The per-output sums do not depend on TR.
template <int NW, int MT, int KB, int MODE, bool DUMP, int TR = 1>
__global__ void __launch_bounds__(64 * NW) gemm_ks_kernel(MfmaArgs a) {
  constexpr int BM = 16 * MT;
  constexpr int G1 = MODE == BTF_GEMV_SWIGLU ? 2 : 1;  // 16-row groups of a tile: gate (and up)
  constexpr int G = G1 * TR;                           // 16-row groups: tile t, matrix g1 at t * G1 + g1
  constexpr int RW = 16 * G;                           // staged rows per wave
  constexpr int CS = 8 * KB + 1;
  constexpr int QS = 32 * KB + 2;
  constexpr int NCV = (RW * 2 * KB + 63) / 64;  // per-lane 16-byte code loads
  constexpr int NSV = (RW * KB + 63) / 64;      // scale loads
  constexpr int NQV = (BM * 8 * KB + 63) / 64;  // 16-byte q loads
  constexpr int NDV = (BM * 4 * KB + 63) / 64;  // d / s loads
  __shared__ uint32_t cs[NW][RW * CS];
  __shared__ uint16_t scs[NW][RW * KB];
  constexpr int QSM = BM * QS > G * 16 * BM ? BM * QS : G * 16 * BM;  // (also holds the partials)
  __shared__ uint32_t qsm[NW][QSM];
  __shared__ float dsm[NW][4 * KB][BM];
  static_assert(sizeof(qsm) >= NW * G * 16 * BM * sizeof(float), "partials alias the q stage");

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
  const int n0 = (bx - tile0) * 16 * TR;
  const int mb = blockIdx.y * BM;

  // this wave's blocks [kw0, kw1); every wave runs niter iterations so the
  // workgroup barriers match
  const int kw0 = nsc * w / NW, kw1 = nsc * (w + 1) / NW;
  const int niter = ((nsc + NW - 1) / NW + KB - 1) / KB;

  float acc[G][MT][4], blk[G][MT][4];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[g][mt][r] = 0.f;

  u32x4 rc[NCV], rq[NQV];
  uint16_t rsc[NSV];
  float rd[NDV];
  auto fetch = [&](int it) {
    const int kb0 = kw0 + it * KB;
    const int nkb = kw1 - kb0 < KB ? kw1 - kb0 : KB;  // may be <= 0 on the last iteration
#pragma unroll
    for (int j = 0; j < NCV; ++j) {
      const int i = lane + 64 * j;
      const int r = i / (2 * KB), part = i - r * (2 * KB);
      rc[j] = u32x4{0u, 0u, 0u, 0u};
      if (i < RW * 2 * KB && part < 2 * nkb) {
        const int nr = n0 + 16 * ((r >> 4) / G1) + (r & 15);
        const int nc = nr < N ? nr : N - 1;
        const uint8_t* cb = (r >> 4) % G1 ? a.up_codes : codes;
        rc[j] = *reinterpret_cast<const u32x4*>(cb + (size_t)nc * rowb + kb0 * 32 + 16 * part);
      }
    }
#pragma unroll
    for (int j = 0; j < NSV; ++j) {
      const int i = lane + 64 * j;
      const int r = i / KB, jj = i - r * KB;
      rsc[j] = 0;
      if (i < RW * KB && jj < nkb) {
        const int nr = n0 + 16 * ((r >> 4) / G1) + (r & 15);
        const int nc = nr < N ? nr : N - 1;
        const uint16_t* sb = (r >> 4) % G1 ? a.up_scales : scales;
        rsc[j] = sb[(size_t)nc * nsc + kb0 + jj];
      }
    }
#pragma unroll
    for (int j = 0; j < NQV; ++j) {
      const int i = lane + 64 * j;
      const int r = i / (8 * KB), part = i - r * (8 * KB);
      const int m = mb + r;
      rq[j] = u32x4{0u, 0u, 0u, 0u};
      if (i < BM * 8 * KB && part < 8 * nkb && m < a.nb)
        rq[j] = *reinterpret_cast<const u32x4*>(a.q + (size_t)(a.m0 + m) * K + kb0 * 128 + 16 * part);
    }
#pragma unroll
    for (int j = 0; j < NDV; ++j) {
      const int i = lane + 64 * j;
      const int r = i / (4 * KB), sb = i - r * (4 * KB);
      const int m = mb + r;
      rd[j] = 0.f;
      if (i < BM * 4 * KB && sb < 4 * nkb && m < a.nb) rd[j] = a.d[(size_t)(a.m0 + m) * nsub + kb0 * 4 + sb];
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int j = 0; j < NCV; ++j) {
      const int i = lane + 64 * j;
      if (i < RW * 2 * KB) {
        const int r = i / (2 * KB), part = i - r * (2 * KB);
        uint32_t* o = &cs[w][r * CS + 4 * part];
        o[0] = rc[j].x; o[1] = rc[j].y; o[2] = rc[j].z; o[3] = rc[j].w;
      }
    }
#pragma unroll
    for (int j = 0; j < NSV; ++j) {
      const int i = lane + 64 * j;
      if (i < RW * KB) scs[w][i] = rsc[j];
    }
#pragma unroll
    for (int j = 0; j < NQV; ++j) {
      const int i = lane + 64 * j;
      if (i < BM * 8 * KB) {
        const int r = i / (8 * KB), part = i - r * (8 * KB);
        uint32_t* o = &qsm[w][r * QS + 4 * part];
        o[0] = rq[j].x; o[1] = rq[j].y; o[2] = rq[j].z; o[3] = rq[j].w;
      }
    }
#pragma unroll
    for (int j = 0; j < NDV; ++j) {
      const int i = lane + 64 * j;
      if (i < BM * 4 * KB) {
        const int r = i / (4 * KB), sb = i - r * (4 * KB);
        dsm[w][sb][r] = rd[j];
      }
    }
  };

  fetch(0);
  for (int it = 0; it < niter; ++it) {
    const int kb0 = kw0 + it * KB;
    const int nkb = kw1 - kb0 < KB ? kw1 - kb0 : KB;
    stage();
    __syncthreads();
    if (it + 1 < niter) fetch(it + 1);  // in flight while this stage is dotted

    for (int kbi = 0; kbi < nkb; ++kbi) {
      const int kb = kb0 + kbi;
#pragma unroll
      for (int sb = 0; sb < 4; ++sb) {
        const int sbx = 4 * kbi + sb;
        long bfrag[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const uint32_t word = cs[w][(16 * g + li) * CS + 2 * sbx + (t >> 1)];
          const int sh = 4 * (t & 1);
          // codes 0 / 1 / 2 -> int8 -1 / 0 / +1: the MFMA gives I = sum q * w with accumulator 0
          const uint32_t lo = __builtin_amdgcn_perm(0u, 0x000100FFu, (word >> sh) & 0x03030303u);
          const uint32_t hi = __builtin_amdgcn_perm(0u, 0x000100FFu, (word >> (sh + 2)) & 0x03030303u);
          bfrag[g] = (long)(((uint64_t)hi << 32) | lo);
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const uint32_t* ap = &qsm[w][(16 * mt + li) * QS + 8 * sbx + 2 * t];
          const long afrag = (long)(((uint64_t)ap[1] << 32) | ap[0]);
          const v4i cin = {0, 0, 0, 0};
#pragma unroll
          for (int g = 0; g < G; ++g) {
            const v4i I = __builtin_amdgcn_mfma_i32_16x16x32_i8(afrag, bfrag[g], cin, 0, 0, 0);
            if constexpr (DUMP) {
              const int n = n0 + 16 * (g / G1) + li;
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int m = mb + 16 * mt + 4 * t + r;
                if (g % G1 == 0 && m < a.nb && n < N) a.dump[((size_t)(a.m0 + m) * N + n) * nsub + kb * 4 + sb] = I[r];
              }
            } else {
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const float dv = dsm[w][sbx][16 * mt + 4 * t + r];
                blk[g][mt][r] = sb == 0 ? dv * (float)I[r] : fmaf(dv, (float)I[r], blk[g][mt][r]);
              }
            }
          }
        }
      }
      if constexpr (!DUMP) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float sc = h2f(scs[w][(16 * g + li) * KB + kbi]);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[g][mt][r] = fmaf(sc, blk[g][mt][r], acc[g][mt][r]);
        }
      }
    }  // kbi
    __syncthreads();
  }
  if constexpr (DUMP) return;

  // ---- wave partials -> LDS (over the q stage), summed in wave order ----
  float* red = reinterpret_cast<float*>(&qsm[0][0]);  // [NW][G][16][BM]
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[((w * G + g) * 16 + li) * BM + 16 * mt + 4 * t + r] = acc[g][mt][r];
  __syncthreads();
  // thread idx: output row rr = idx % RT of the tile, activation row mm = idx / RT
  // (with TR = 2 a half-wave holds the 32 outputs of one activation row: one Q8 block)
  constexpr int RT = 16 * TR;
  for (int idx = tid; idx < RT * BM; idx += 64 * NW) {
    const int rr = idx & (RT - 1), mm = idx / RT;
    const int n = n0 + rr, m = mb + mm;
    const bool live = m < a.nb && n < N;
    if (TR == 1 && !live) continue;
    const int gb = (rr >> 4) * G1;  // first group of the row's tile
    float v[G1];
#pragma unroll
    for (int g = 0; g < G1; ++g) {
      float sacc = red[((0 * G + gb + g) * 16 + (rr & 15)) * BM + mm];
#pragma unroll
      for (int ww = 1; ww < NW; ++ww) sacc = sacc + red[((ww * G + gb + g) * 16 + (rr & 15)) * BM + mm];
      v[g] = sacc;
    }
    float* o = &y[(size_t)(a.m0 + m) * ldy + n];
    float out = 0.f;
    if (live) {
      if constexpr (MODE == BTF_GEMV_SWIGLU)
        out = v[0] / (1.0f + expf(-v[0])) * v[G1 - 1];
      else if constexpr (MODE == BTF_GEMV_ADD)
        out = *o + v[0];
      else
        out = v[0];
      *o = out;
    }
    if constexpr (TR == 2) {
      if (a.oq) {  // (uniform) the Q8 block of rows n0 .. n0 + 31 of activation row m
        float dq;
        int sq;
        const int q = q8_half(out, dq, sq);
        uint32_t wq = (uint32_t)(q & 0xff) << (8 * (rr & 3));
        wq |= (uint32_t)dpp_i<0xB1>((int)wq);  // quad_perm(1,0,3,2)
        wq |= (uint32_t)dpp_i<0x4E>((int)wq);  // quad_perm(2,3,0,1)
        if (live) {
          const size_t mr = (size_t)(a.m0 + m);
          if ((rr & 3) == 0) *reinterpret_cast<uint32_t*>(a.oq + mr * N + n) = wq;
          if (rr == 0) {
            a.od[mr * (N / 32) + n0 / 32] = dq;
            a.os[mr * (N / 32) + n0 / 32] = sq;
          }
        }
      }
    }
  }
}

template <int NW, int MT, bool DUMP, int TR>
void by_mode_ks(int mode, const MfmaArgs& a, dim3 grid, hipStream_t st) {
  constexpr int KB = MT >= 2 ? 1 : 2;  // small stages: occupancy (4-5 waves per SIMD) beats bytes per round
  if (mode == BTF_GEMV_STORE)
    hipLaunchKernelGGL((gemm_ks_kernel<NW, MT, KB, BTF_GEMV_STORE, DUMP, TR>), grid, dim3(64 * NW), 0, st, a);
  else if (mode == BTF_GEMV_ADD)
    hipLaunchKernelGGL((gemm_ks_kernel<NW, MT, KB, BTF_GEMV_ADD, DUMP, TR>), grid, dim3(64 * NW), 0, st, a);
  else
    hipLaunchKernelGGL((gemm_ks_kernel<NW, MT, KB, BTF_GEMV_SWIGLU, DUMP, TR>), grid, dim3(64 * NW), 0, st, a);
}

template <int MT, bool DUMP, int TR = 1>
void by_waves_ks(int nw, int mode, const MfmaArgs& a, dim3 grid, hipStream_t st) {
  if (nw == 8)
    by_mode_ks<8, MT, DUMP, TR>(mode, a, grid, st);
  else
    by_mode_ks<4, MT, DUMP, TR>(mode, a, grid, st);
}

// The longest wave range (128-column blocks) the packed tile's preloads hold:
// the host picks the waves per workgroup so that ceil(nsc / NW) fits.
__host__ __device__ constexpr int kp_max_blocks(int nw) { return nw == 4 ? 16 : 20; }

// Packed K-split tile for batched decode (up to 16 activation rows). The
// workgroup and the K split are gemm_ks_kernel's (16 * TR weight rows, for
// swiglu with their up rows; wave w walks its contiguous 1/NW of the
// 128-column blocks), but one v_mfma_i32_16x16x64_i8 covers two 32-column
// sub-blocks of 8 activation rows: A rows 0-7 hold q of rows 8mg .. 8mg + 7
// over sub-block 2P (k 0-31: lane groups 0 and 1) and A rows 8-15 the same
// rows over sub-block 2P + 1 (k 32-63: lane groups 2 and 3), zero elsewhere,
// so every MFMA output is a real I (no padding rows). The codes enter as
// stored (0 / 1 / 2; a lane group's 16 columns are one code word, whose four
// 2-bit fields are its four int8 words after shift and mask) and the
// accumulator starts at -s, so the MFMA gives I = sum (code - 1) * q exactly.
// Lane groups 0-1 hold the even sub-blocks and 2-3 the odd ones of the same
// 16 x 8 outputs; each keeps its own sums (blk = d * I over the block's two
// sub-blocks of its parity, acc += scale * blk per block), and per output
//     y = sum over waves w, in order, of (accE_w + accO_w).
// Each wave streams its blocks two at a time through a private S-stage ring
// of LDS-direct loads (no registers held by loads in flight): each code load
// reads 64 contiguous bytes (two blocks) of each of 16 rows. Where the LDS
// allows (all but two swiglu instances, below) the weight scales of the
// wave's whole range are loaded once,
// before the first stage, into [R][SR] 4-byte slots after the ring: a stage
// of 2 blocks then carries no scale loads (their HBM lines, apart from the
// code rows, cost ~2.5 us of gate+up at M = 8 when every stage fetched its
// own). Stages past the wave's range reload its last block (L2 hits, never
// read back) to keep the per-stage load count. Stage layout (bytes): codes
// [R][4 x 16 B] with chunk c of row n at slot c ^ ((n >> 2) & 3) (the 64
// lanes' words then fall in 64 banks), scales [2][R] in 4-byte slots (without the preload), q
// [2][BQ][8 x 16 B] with chunk c of row r at slot c ^ (r & 7), then 256 zero
// bytes (the A lanes that carry no data read one 16-byte chunk of them, on
// banks that the data lanes of the same pass leave free), d
// [MG][2][4][8] and s [MG][2][4][8] (row group, block, sub-block, row: a
// lane's four rows are one 16-byte read).
template <int NW, int MG, int S, int MODE, bool DUMP, int TR = 1>
__global__ void __launch_bounds__(64 * NW) gemm_kp_kernel(MfmaArgs a) {
  constexpr int G1 = MODE == BTF_GEMV_SWIGLU ? 2 : 1;
  constexpr int G = G1 * TR;  // 16-row groups: tile t, matrix g1 at t * G1 + g1
  constexpr int R = 16 * G;   // staged weight rows per wave
  constexpr int BQ = 8 * MG;  // activation rows
  // PS: the wave's weight scales are loaded once, before the ring starts,
  // instead of with every stage. Not for swiglu with two row groups on 2
  // waves of 16-row tiles (the preload would cost the fifth resident
  // workgroup per CU that gate+up's 1088 need) or on 8 waves of 32-row tiles
  // (past the 160 KB of LDS).
  constexpr bool PS = MG == 1 || !(MODE == BTF_GEMV_SWIGLU && (TR == 1 ? NW == 2 : NW == 8));
  constexpr int NB = kp_max_blocks(NW);  // blocks of the longest wave range
  constexpr int SR = NB == 16 ? 17 : NB;  // scale row stride in 4-byte slots (rows on distinct banks)
  constexpr int CB = R * 64, SB = PS ? 0 : 2 * R * 4, QB = 2 * BQ * 128 + 256, DB = BQ * 32;
  constexpr int OQ = CB + SB, OD = OQ + QB;  // stage offsets of q and d
  constexpr int STG = OD + 2 * DB;
  constexpr int PSB = PS ? R * SR * 4 : 0;  // the preloaded scales
  constexpr int WB = S * STG + PSB;         // LDS bytes per wave
  constexpr int NCI = R / 16;               // code loads per stage (16 rows x 64 B each)
  constexpr int L = NCI + (PS ? 0 : 2) + 2 * MG + 2 * MG;  // loads per stage: codes, scales, q, d + s
  static_assert(STG % 16 == 0 && WB % 16 == 0 && S >= 2 && L * (S - 2) < 64 && R <= 64, "stage layout");
  constexpr int RING = NW * WB, RED = NW * G * 2 * 16 * BQ * 4;
  __shared__ __attribute__((aligned(16))) uint8_t ring[RING > RED ? RING : RED];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: ring base and K range
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
  const int n0 = (bx - tile0) * 16 * TR;
  const int mb = blockIdx.y * BQ;
  const int kw0 = nsc * w / NW, kw1 = nsc * (w + 1) / NW;
  const int niter = ((nsc + NW - 1) / NW + 1) / 2;  // every wave runs the longest range's stage count

  uint8_t* rw = ring + w * WB;
  const uint32_t ring0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)rw;  // LDS byte address
  uint8_t* pre = rw + S * STG;  // the preloaded scales [R][SR] (4-byte slots)
  const uint32_t pre0 = ring0 + S * STG;
  // the wave's last block (a wave with none: block 0); stages past its range reload it
  const int klast = kw1 > kw0 ? kw1 - 1 : 0;
  const int bmax = kw1 > kw0 ? kw1 - kw0 - 1 : 0;  // last preloaded block, relative to kw0

  // ---- the scale preload (issued before the first stage) ----
  if constexpr (PS) {
    // slot e: row e / SR, block kw0 + e % SR (past the range: its last block)
#pragma unroll
    for (int j = 0; j < (R * SR + 63) / 64; ++j) {
      const int e = 64 * j + lane;
      const int n = e / SR < R ? e / SR : R - 1;
      const int b = e % SR < bmax ? e % SR : bmax;
      const int nr = n0 + 16 * ((n >> 4) / G1) + (n & 15);
      const int nc = nr < N ? nr : N - 1;
      if (e < R * SR) lds_dma2(((n >> 4) % G1 ? a.up_scales : scales) + (size_t)nc * nsc + kw0 + b, pre0 + 256 * j);
    }
  }
  // ---- this lane's load sources (block offsets added per stage, clamped to the row) ----
  const uint8_t* csrc[NCI];  // codes: load j -> row 16 j + lane / 4, slot lane % 4
  int cblk[NCI];             // which of the stage's two blocks that slot holds
#pragma unroll
  for (int j = 0; j < NCI; ++j) {
    const int n = 16 * j + (lane >> 2);
    const int h = (lane & 3) ^ ((n >> 2) & 3);
    const int nr = n0 + 16 * ((n >> 4) / G1) + (n & 15);
    const int nc = nr < N ? nr : N - 1;
    csrc[j] = ((n >> 4) % G1 ? a.up_codes : codes) + (size_t)nc * rowb + 16 * (h & 1);
    cblk[j] = h >> 1;
  }
  const uint16_t* ssrc;  // scales: lane < R -> row lane
  {
    const int n = lane < R ? lane : R - 1;
    const int nr = n0 + 16 * ((n >> 4) / G1) + (n & 15);
    const int nc = nr < N ? nr : N - 1;
    ssrc = ((n >> 4) % G1 ? a.up_scales : scales) + (size_t)nc * nsc;
  }
  const int8_t* qsrc[MG];  // q: load (block, mg) -> row 8 mg + lane / 8, slot lane % 8 holds chunk (lane % 8) ^ (lane / 8)
#pragma unroll
  for (int mg = 0; mg < MG; ++mg) {
    const int r = 8 * mg + (lane >> 3);
    const int m = mb + r < a.nb ? mb + r : a.nb - 1;
    qsrc[mg] = a.q + (size_t)(a.m0 + m) * K + 16 * ((lane & 7) ^ (lane >> 3));
  }
  const float* dsrc[MG];  // d and s: load mg -> slot lane of group mg: [block lane / 32][sub-block][row 8 mg + lane % 8]
  const int32_t* s_src[MG];
  const int dblk = lane >> 5;  // which of the stage's two blocks
#pragma unroll
  for (int mg = 0; mg < MG; ++mg) {
    const int r = 8 * mg + (lane & 7);
    const int m = mb + r < a.nb ? mb + r : a.nb - 1;
    dsrc[mg] = a.d + (size_t)(a.m0 + m) * nsub + ((lane >> 3) & 3);
    s_src[mg] = a.s + (size_t)(a.m0 + m) * nsub + ((lane >> 3) & 3);
  }
  auto issue = [&](int it) {
    const int kb = kw0 + 2 * it;
    const uint32_t st = ring0 + (uint32_t)((it % S) * STG);
    auto blk_of = [&](int i) { return kb + i < klast ? kb + i : klast; };
#pragma unroll
    for (int j = 0; j < NCI; ++j) lds_dma16(csrc[j] + (size_t)blk_of(cblk[j]) * 32, st + 1024 * j);
    if constexpr (!PS)
#pragma unroll
      for (int i = 0; i < 2; ++i)
        if (lane < R) lds_dma2(ssrc + blk_of(i), st + CB + i * R * 4);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int mg = 0; mg < MG; ++mg) lds_dma16(qsrc[mg] + (size_t)blk_of(i) * 128, st + OQ + (i * BQ + 8 * mg) * 128);
#pragma unroll
    for (int mg = 0; mg < MG; ++mg) {
      lds_dma4(dsrc[mg] + 4 * blk_of(dblk), st + OD + 256 * mg);
      lds_dma4(s_src[mg] + 4 * blk_of(dblk), st + OD + DB + 256 * mg);
    }
  };

  // the zero bytes after the q rows of every stage (no load writes them)
#pragma unroll
  for (int s = 0; s < S; ++s)
    if (lane < 16) *reinterpret_cast<u32x4*>(rw + s * STG + OQ + 2 * BQ * 128 + 16 * lane) = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
  for (int it = 0; it < S - 1; ++it) issue(it);

  // ---- this lane's LDS read offsets within a stage ----
  const int x = li & 7;
  const bool holds = (li < 8) == (t < 2);  // A lane with data (else the zero row)
  int aoff[2][MG][2];  // block i, group mg, pair P (the data-less lanes: the zero bytes, for every block)
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int mg = 0; mg < MG; ++mg)
#pragma unroll
      for (int P = 0; P < 2; ++P)
        aoff[i][mg][P] = OQ + (holds ? (i * BQ + 8 * mg + x) * 128 + 16 * ((4 * P) ^ t ^ x)
                                     : 2 * BQ * 128 + 16 * ((t & 1) ^ 1));
  int boff[2][2];  // code word 4P + t of block i of row li (group g adds 1024)
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int P = 0; P < 2; ++P) boff[i][P] = li * 64 + 16 * ((2 * i + P) ^ ((li >> 2) & 3)) + 4 * t;
  // d / s of output rows 4 (t & 1) .. + 3 of group mg, block i, sub-block 2P + (t >> 1): one 16-byte read
  const int dl = 4 * (8 * (t >> 1) + 4 * (t & 1));

  float acc[G][MG][4];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int mg = 0; mg < MG; ++mg)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[g][mg][r] = 0.f;

  for (int it = 0; it < niter; ++it) {
    wait_vm<L * (S - 2)>();  // this wave's loads of stage it have landed
    issue(it + S - 1);       // into the stage read in iteration it - 1
    const int kb = kw0 + 2 * it;
    if (kb >= kw1) continue;        // (wave-uniform; later iterations only wait and issue)
    const bool two = kb + 1 < kw1;  // (wave-uniform) the stage's second block is in the wave's range
    const uint8_t* st = rw + (it % S) * STG;
    auto rel = [&](int i) { return (kb + i < klast ? kb + i : klast) - kw0; };  // preloaded block index
    // Per block: every LDS read first, then every MFMA into its own
    // registers, then the scaling, so that LDS and MFMA latencies overlap
    // instead of each product waiting for its own operands. A second block
    // past the wave's range is multiplied on its (valid) staged data but not
    // accumulated.
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      v4i A[2][MG], C[2][MG];
      u32x4 D[2][MG];
      uint32_t W[2][G];
      uint16_t SC[G];
#pragma unroll
      for (int P = 0; P < 2; ++P) {
#pragma unroll
        for (int mg = 0; mg < MG; ++mg) {
          A[P][mg] = *reinterpret_cast<const v4i*>(st + aoff[i][mg][P]);
          const uint8_t* o = st + OD + 256 * mg + 128 * i + 64 * P + dl;
          D[P][mg] = *reinterpret_cast<const u32x4*>(o);
          C[P][mg] = *reinterpret_cast<const v4i*>(o + DB);
        }
#pragma unroll
        for (int g = 0; g < G; ++g) W[P][g] = *reinterpret_cast<const uint32_t*>(st + boff[i][P] + 1024 * g);
      }
#pragma unroll
      for (int g = 0; g < G; ++g)
        SC[g] = PS ? *reinterpret_cast<const uint16_t*>(pre + 4 * ((16 * g + li) * SR + rel(i)))
                   : *reinterpret_cast<const uint16_t*>(st + CB + i * R * 4 + 4 * (16 * g + li));
      v4i I[2][G][MG];
#pragma unroll
      for (int P = 0; P < 2; ++P) {
#pragma unroll
        for (int mg = 0; mg < MG; ++mg) C[P][mg] = -C[P][mg];  // the accumulator starts at -s
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const uint32_t wd = W[P][g];
          const v4i B = {(int)(wd & 0x03030303u), (int)((wd >> 2) & 0x03030303u), (int)((wd >> 4) & 0x03030303u),
                         (int)((wd >> 6) & 0x03030303u)};
#pragma unroll
          for (int mg = 0; mg < MG; ++mg) I[P][g][mg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[P][mg], B, C[P][mg], 0, 0, 0);
        }
      }
      if (i == 1 && !two) break;  // (wave-uniform)
      if constexpr (DUMP) {  // the exact I of every (row, output, sub-block)
#pragma unroll
        for (int P = 0; P < 2; ++P)
#pragma unroll
          for (int g = 0; g < G; g += G1) {
            const int n = n0 + 16 * (g / G1) + li;
#pragma unroll
            for (int mg = 0; mg < MG; ++mg)
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int m = mb + 8 * mg + 4 * (t & 1) + r;
                if (m < a.nb && n < N)
                  a.dump[((size_t)(a.m0 + m) * N + n) * nsub + (kb + i) * 4 + 2 * P + (t >> 1)] = I[P][g][mg][r];
              }
          }
      } else {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float sc = h2f(SC[g]);
#pragma unroll
          for (int mg = 0; mg < MG; ++mg)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float b0 = __uint_as_float(D[0][mg][r]) * (float)I[0][g][mg][r];
              const float b1 = fmaf(__uint_as_float(D[1][mg][r]), (float)I[1][g][mg][r], b0);
              acc[g][mg][r] = fmaf(sc, b1, acc[g][mg][r]);
            }
        }
      }
    }
  }
  wait_vm<0>();  // the trailing loads land before the ring is reused or released
  if constexpr (DUMP) return;

  // ---- per-parity wave partials -> LDS (over the ring), summed per wave, then in wave order ----
  __syncthreads();
  float* red = reinterpret_cast<float*>(ring);  // [NW][G][2][16][BQ]
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int mg = 0; mg < MG; ++mg)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        red[(((w * G + g) * 2 + (t >> 1)) * 16 + li) * BQ + 8 * mg + 4 * (t & 1) + r] = acc[g][mg][r];
  __syncthreads();
  // thread idx: output row rr = idx % RT of the tile, activation row mm = idx / RT
  // (with TR = 2 a half-wave holds the 32 outputs of one activation row: one Q8 block)
  constexpr int RT = 16 * TR;
  for (int idx = tid; idx < RT * BQ; idx += 64 * NW) {
    const int rr = idx & (RT - 1), mm = idx / RT;
    const int n = n0 + rr, m = mb + mm;
    const bool live = m < a.nb && n < N;
    if (TR == 1 && !live) continue;
    const int gb = (rr >> 4) * G1;  // first group of the row's tile
    float v[G1];
#pragma unroll
    for (int g = 0; g < G1; ++g) {
      const int base = ((gb + g) * 2 * 16 + (rr & 15)) * BQ + mm;  // wave 0, even parity
      float sacc = red[base] + red[base + 16 * BQ];
#pragma unroll
      for (int ww = 1; ww < NW; ++ww) {
        const int o = base + ww * G * 2 * 16 * BQ;
        sacc = sacc + (red[o] + red[o + 16 * BQ]);
      }
      v[g] = sacc;
    }
    float* o = &y[(size_t)(a.m0 + m) * ldy + n];
    float out = 0.f;
    if (live) {
      if constexpr (MODE == BTF_GEMV_SWIGLU)
        out = v[0] / (1.0f + expf(-v[0])) * v[G1 - 1];
      else if constexpr (MODE == BTF_GEMV_ADD)
        out = *o + v[0];
      else
        out = v[0];
      *o = out;
    }
    if constexpr (TR == 2) {
      if (a.oq) {  // (uniform) the Q8 block of rows n0 .. n0 + 31 of activation row m
        float dq;
        int sq;
        const int q = q8_half(out, dq, sq);
        uint32_t wq = (uint32_t)(q & 0xff) << (8 * (rr & 3));
        wq |= (uint32_t)dpp_i<0xB1>((int)wq);  // quad_perm(1,0,3,2)
        wq |= (uint32_t)dpp_i<0x4E>((int)wq);  // quad_perm(2,3,0,1)
        if (live) {
          const size_t mr = (size_t)(a.m0 + m);
          if ((rr & 3) == 0) *reinterpret_cast<uint32_t*>(a.oq + mr * N + n) = wq;
          if (rr == 0) {
            a.od[mr * (N / 32) + n0 / 32] = dq;
            a.os[mr * (N / 32) + n0 / 32] = sq;
          }
        }
      }
    }
  }
}

// Two stages per wave (deeper rings measured no faster at M = 4, 8 and 16:
// their LDS cost resident workgroups, and one wave per gate+up workgroup with
// 2 to 8 stages took the same time for every depth).
template <int NW, int MG, bool DUMP, int TR>
void by_mode_kp(int mode, const MfmaArgs& a, dim3 grid, hipStream_t st) {
  constexpr int S = 2;
  if (mode == BTF_GEMV_STORE)
    hipLaunchKernelGGL((gemm_kp_kernel<NW, MG, S, BTF_GEMV_STORE, DUMP, TR>), grid, dim3(64 * NW), 0, st, a);
  else if (mode == BTF_GEMV_ADD)
    hipLaunchKernelGGL((gemm_kp_kernel<NW, MG, S, BTF_GEMV_ADD, DUMP, TR>), grid, dim3(64 * NW), 0, st, a);
  else
    hipLaunchKernelGGL((gemm_kp_kernel<NW, MG, S, BTF_GEMV_SWIGLU, DUMP, TR>), grid, dim3(64 * NW), 0, st, a);
}

// Waves per workgroup (the K split, so the outputs' summation order depends
// on it; every caller of a shape gets the same): gate+up 2, K >= 8192 8,
// else 4 (measured best of 2 / 4 / 8 at M = 4, 8, 16 on the 27B shapes),
// and more where a wave's share would pass kp_max_blocks; 0: the shape is
// longer than the packed tile takes.
int kp_waves(int K, int mode) {
  const int nsc = K / 128;
  const int nw = mode == BTF_GEMV_SWIGLU ? (nsc <= 40 ? 2 : nsc <= 64 ? 4 : 8) : K >= 8192 ? 8 : 4;
  return (nsc + nw - 1) / nw <= kp_max_blocks(nw) ? nw : 0;
}

template <int MG, bool DUMP, int TR = 1>
void by_waves_kp(int nw, int mode, const MfmaArgs& a, dim3 grid, hipStream_t st) {
  if (nw == 2)
    by_mode_kp<2, MG, DUMP, TR>(mode, a, grid, st);
  else if (nw == 8)
    by_mode_kp<8, MG, DUMP, TR>(mode, a, grid, st);
  else
    by_mode_kp<4, MG, DUMP, TR>(mode, a, grid, st);
}

// Prefill tile (more than 32 activation rows): a workgroup owns 64 staged
// weight rows (swiglu: 32 gate rows and the same 32 up rows) and BM = 32 * MW
// activation rows; wave (wn, wm) = (w & 1, w >> 1) computes 32 staged rows x
// 16 * MW activation rows, 2 x MW MFMA tiles per 32-column sub-block from 2 B
// and MW A fragments (swiglu: its two B tiles are the gate and up rows of the same
// 16 outputs, so the epilogue stays in the lane). Per output the sums follow
// this order: blk = d * I over the block's sub-blocks, then
// acc += scale * blk per block.
template <int MW, int KB, int MODE, bool DUMP = false>
__global__ void __launch_bounds__(256) gemm_pf_kernel(MfmaArgs a) {
  constexpr int BM = 32 * MW;
  constexpr int CS = 8 * KB + 1;
  constexpr int QS = 32 * KB + 2;
  constexpr int NCV = (64 * 2 * KB + 255) / 256;
  constexpr int NSV = (64 * KB + 255) / 256;
  constexpr int NQV = (BM * 8 * KB + 255) / 256;
  constexpr int NDV = (BM * 4 * KB + 255) / 256;
  constexpr bool SW = MODE == BTF_GEMV_SWIGLU;
  __shared__ uint32_t cs[64 * CS];
  __shared__ uint16_t scs[64 * KB];
  __shared__ uint32_t qsm[BM * QS];
  __shared__ float dsm[4 * KB][BM];
  __shared__ int32_t nsm[4 * KB][BM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int wn = w & 1, wm = w >> 1;
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
  constexpr int ROWS_REAL = SW ? 32 : 64;
  const int n0 = (bx - tile0) * ROWS_REAL;
  const int mb = blockIdx.y * BM;

  // staged row of this wave's B tile j (lane row li added at use)
  int srow[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) srow[j] = SW ? 32 * j + 16 * wn : 32 * wn + 16 * j;

  float acc[2][MW][4], blk[2][MW][4];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int mt = 0; mt < MW; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[j][mt][r] = 0.f;

  u32x4 rc[NCV], rq[NQV];
  uint16_t rsc[NSV];
  float rd[NDV];
  int rs[NDV];
  auto fetch = [&](int kb0) {
    const int nkb = nsc - kb0 < KB ? nsc - kb0 : KB;
#pragma unroll
    for (int j = 0; j < NCV; ++j) {
      const int i = tid + 256 * j;
      const int r = i / (2 * KB), part = i - r * (2 * KB);
      rc[j] = u32x4{0u, 0u, 0u, 0u};
      if (i < 64 * 2 * KB && part < 2 * nkb) {
        const bool up = SW && r >= 32;
        const int nr = n0 + (SW ? (r & 31) : r);
        const int nc = nr < N ? nr : N - 1;
        const uint8_t* cb = up ? a.up_codes : codes;
        rc[j] = *reinterpret_cast<const u32x4*>(cb + (size_t)nc * rowb + kb0 * 32 + 16 * part);
      }
    }
#pragma unroll
    for (int j = 0; j < NSV; ++j) {
      const int i = tid + 256 * j;
      const int r = i / KB, jj = i - r * KB;
      rsc[j] = 0;
      if (i < 64 * KB && jj < nkb) {
        const bool up = SW && r >= 32;
        const int nr = n0 + (SW ? (r & 31) : r);
        const int nc = nr < N ? nr : N - 1;
        const uint16_t* sb = up ? a.up_scales : scales;
        rsc[j] = sb[(size_t)nc * nsc + kb0 + jj];
      }
    }
#pragma unroll
    for (int j = 0; j < NQV; ++j) {
      const int i = tid + 256 * j;
      const int r = i / (8 * KB), part = i - r * (8 * KB);
      const int m = mb + r;
      rq[j] = u32x4{0u, 0u, 0u, 0u};
      if (i < BM * 8 * KB && part < 8 * nkb && m < a.nb)
        rq[j] = *reinterpret_cast<const u32x4*>(a.q + (size_t)(a.m0 + m) * K + kb0 * 128 + 16 * part);
    }
#pragma unroll
    for (int j = 0; j < NDV; ++j) {
      const int i = tid + 256 * j;
      const int r = i / (4 * KB), sb = i - r * (4 * KB);
      const int m = mb + r;
      rd[j] = 0.f;
      rs[j] = 0;
      if (i < BM * 4 * KB && sb < 4 * nkb && m < a.nb) {
        const size_t o = (size_t)(a.m0 + m) * nsub + kb0 * 4 + sb;
        rd[j] = a.d[o];
        rs[j] = a.s[o];
      }
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int j = 0; j < NCV; ++j) {
      const int i = tid + 256 * j;
      if (i < 64 * 2 * KB) {
        const int r = i / (2 * KB), part = i - r * (2 * KB);
        uint32_t* o = &cs[r * CS + 4 * part];
        o[0] = rc[j].x; o[1] = rc[j].y; o[2] = rc[j].z; o[3] = rc[j].w;
      }
    }
#pragma unroll
    for (int j = 0; j < NSV; ++j) {
      const int i = tid + 256 * j;
      if (i < 64 * KB) scs[i] = rsc[j];
    }
#pragma unroll
    for (int j = 0; j < NQV; ++j) {
      const int i = tid + 256 * j;
      if (i < BM * 8 * KB) {
        const int r = i / (8 * KB), part = i - r * (8 * KB);
        uint32_t* o = &qsm[r * QS + 4 * part];
        o[0] = rq[j].x; o[1] = rq[j].y; o[2] = rq[j].z; o[3] = rq[j].w;
      }
    }
#pragma unroll
    for (int j = 0; j < NDV; ++j) {
      const int i = tid + 256 * j;
      if (i < BM * 4 * KB) {
        const int r = i / (4 * KB), sb = i - r * (4 * KB);
        dsm[sb][r] = rd[j];
        nsm[sb][r] = -rs[j];
      }
    }
  };

  fetch(0);
  for (int kb0 = 0; kb0 < nsc; kb0 += KB) {
    const int nkb = nsc - kb0 < KB ? nsc - kb0 : KB;
    stage();
    __syncthreads();
    if (kb0 + KB < nsc) fetch(kb0 + KB);  // in flight while this stage is dotted

    for (int kbi = 0; kbi < nkb; ++kbi) {
#pragma unroll
      for (int sb = 0; sb < 4; ++sb) {
        const int sbx = 4 * kbi + sb;
        long bfrag[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const uint32_t word = cs[(srow[j] + li) * CS + 2 * sbx + (t >> 1)];
          const int sh = 4 * (t & 1);
          const uint32_t lo = (word >> sh) & 0x03030303u;
          const uint32_t hi = (word >> (sh + 2)) & 0x03030303u;
          bfrag[j] = (long)(((uint64_t)hi << 32) | lo);
        }
#pragma unroll
        for (int mt = 0; mt < MW; ++mt) {
          const int mr = 16 * MW * wm + 16 * mt;
          const uint32_t* ap = &qsm[(mr + li) * QS + 8 * sbx + 2 * t];
          const long afrag = (long)(((uint64_t)ap[1] << 32) | ap[0]);
          v4i cin;
          float dv[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            cin[r] = nsm[sbx][mr + 4 * t + r];
            dv[r] = dsm[sbx][mr + 4 * t + r];
          }
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const v4i I = __builtin_amdgcn_mfma_i32_16x16x32_i8(afrag, bfrag[j], cin, 0, 0, 0);
            if constexpr (DUMP) {  // the exact I of every (row, output, sub-block), as launched
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int m = mb + mr + 4 * t + r, n = n0 + srow[j] + li;
                if (m < a.nb && n < N) a.dump[((size_t)(a.m0 + m) * N + n) * nsub + (kb0 + kbi) * 4 + sb] = I[r];
              }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)
              blk[j][mt][r] = sb == 0 ? dv[r] * (float)I[r] : fmaf(dv[r], (float)I[r], blk[j][mt][r]);
          }
        }
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float sc = h2f(scs[(srow[j] + li) * KB + kbi]);
#pragma unroll
        for (int mt = 0; mt < MW; ++mt)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[j][mt][r] = fmaf(sc, blk[j][mt][r], acc[j][mt][r]);
      }
    }
    __syncthreads();
  }
  if constexpr (DUMP) return;

#pragma unroll
  for (int mt = 0; mt < MW; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = mb + 16 * MW * wm + 16 * mt + 4 * t + r;
      if (m >= a.nb) continue;
      if constexpr (SW) {
        const int n = n0 + 16 * wn + li;
        if (n < N) {
          const float g = acc[0][mt][r], u = acc[1][mt][r];
          y[(size_t)(a.m0 + m) * ldy + n] = g / (1.0f + expf(-g)) * u;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int n = n0 + srow[j] + li;
          if (n < N) {
            float* o = &y[(size_t)(a.m0 + m) * ldy + n];
            if constexpr (MODE == BTF_GEMV_ADD)
              *o += acc[j][mt][r];
            else
              *o = acc[j][mt][r];
          }
        }
      }
    }
}

template <int MW>
void by_mode_pf(int mode, const MfmaArgs& a, dim3 grid, hipStream_t st) {
  constexpr int KB = 1;
  if (mode == BTF_GEMV_STORE)
    hipLaunchKernelGGL((gemm_pf_kernel<MW, KB, BTF_GEMV_STORE>), grid, dim3(256), 0, st, a);
  else if (mode == BTF_GEMV_ADD)
    hipLaunchKernelGGL((gemm_pf_kernel<MW, KB, BTF_GEMV_ADD>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((gemm_pf_kernel<MW, KB, BTF_GEMV_SWIGLU>), grid, dim3(256), 0, st, a);
}

// The prefill tile of gemm_pf_kernel (64 staged weight rows x BM = 32 * MW
// activation rows, wave (w & 1, w >> 1) computes 32 x 16 * MW) fed by an
// S-stage ring of LDS-direct loads: after the barrier of block k each wave
// issues its share of block k + S - 1, so a load has S - 1 blocks of compute
// to arrive in and no staging registers. The 2-bit codes are mapped to int8
// {-1, 0, +1} with one byte permute per word, so the MFMA yields
// I = sum q * w directly (accumulator 0) and s is not read. Stage layout:
// q [BM][128 B] with the 16-byte chunk c of row r at slot c ^ (r & 7) (the A
// fragments of 16 rows fall in 8 bank groups), codes [64][2 x 16 B] with the
// halves of row r swapped when bit 3 of r is set (rows r and r + 8 of a
// fragment read then fall in different banks), d [BM][4], scales [64] in
// 4-byte slots. Same sums, in the same order, as gemm_pf_kernel.
template <int MW, int S, int MODE, bool DUMP = false>
__global__ void __launch_bounds__(256) gemm_pf2_kernel(MfmaArgs a) {
  constexpr int BM = 32 * MW;
  constexpr bool SW = MODE == BTF_GEMV_SWIGLU;
  constexpr int QB = BM * 128, CB = 64 * 32, DB = BM * 16, SCB = 64 * 4;
  constexpr int STG = QB + CB + DB + SCB;
  constexpr int NQ = BM / 32;  // q loads per wave per block
  static_assert(STG % 16 == 0, "stage alignment");
  __shared__ __attribute__((aligned(16))) uint8_t ring[S * STG];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: LDS bases and roles
  const int wn = w & 1, wm = w >> 1;
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
  constexpr int ROWS_REAL = SW ? 32 : 64;
  const int n0 = (bx - tile0) * ROWS_REAL;
  const int mb = blockIdx.y * BM;
  const uint32_t ring0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)ring;  // LDS byte address

  // ---- this lane's load sources (block 0; block kb adds kb * step) ----
  // q: load i covers slots (w * NQ + i) * 64 + lane -> row P / 8, slot P % 8
  const int8_t* qsrc[NQ];
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int P = (w * NQ + i) * 64 + lane;
    const int r = P >> 3, c = (P & 7) ^ (r & 7);
    const int m = mb + r < a.nb ? mb + r : a.nb - 1;
    qsrc[i] = a.q + (size_t)(a.m0 + m) * K + 16 * c;
  }
  // codes (waves 0, 1): slot P = w * 64 + lane -> staged row P / 2, slot P % 2
  // holding half (P % 2) ^ (bit 3 of the row)
  const uint8_t* csrc;
  {
    const int P = (w & 1) * 64 + lane;
    const int r = P >> 1;
    const int nr = n0 + (SW ? (r & 31) : r);
    const int nc = nr < N ? nr : N - 1;
    csrc = (SW && r >= 32 ? a.up_codes : codes) + (size_t)nc * rowb + 16 * ((P & 1) ^ ((r >> 3) & 1));
  }
  // d (waves 2, 3): row (w - 2) * 64 + lane; scales (wave 3): staged row lane
  const float* dsrc;
  {
    const int r = ((w - 2) & 1) * 64 + lane;
    const int m = mb + r < a.nb ? mb + r : a.nb - 1;
    dsrc = a.d + (size_t)(a.m0 + m) * nsub;
  }
  const uint16_t* ssrc;
  {
    const int nr = n0 + (SW ? (lane & 31) : lane);
    const int nc = nr < N ? nr : N - 1;
    ssrc = (SW && lane >= 32 ? a.up_scales : scales) + (size_t)nc * nsc;
  }
  // Loads per wave per block: NQ q + (waves 0, 1: codes; waves 2, 3: d when
  // BM covers them) + (wave 3: scales).
  const bool do_d = w >= 2 && (w - 2) * 64 < BM;
  auto issue = [&](int kb) {
    const int kc = kb < nsc ? kb : nsc - 1;  // blocks past the end reload the last (never read)
    const uint32_t st = ring0 + (uint32_t)((kb % S) * STG);
#pragma unroll
    for (int i = 0; i < NQ; ++i) lds_dma16(qsrc[i] + (size_t)kc * 128, st + (uint32_t)((w * NQ + i) * 1024));
    if (w < 2) lds_dma16(csrc + (size_t)kc * 32, st + QB + (uint32_t)(w * 1024));
    if (do_d) lds_dma16(dsrc + (size_t)kc * 4, st + QB + CB + (uint32_t)((w - 2) * 1024));
    if (w == 3) lds_dma2(ssrc + kc, st + QB + CB + DB);
  };

  int srow[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) srow[j] = SW ? 32 * j + 16 * wn : 32 * wn + 16 * j;

  float acc[2][MW][4], blk[2][MW][4];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int mt = 0; mt < MW; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[j][mt][r] = 0.f;

#pragma unroll
  for (int kb = 0; kb < S - 1; ++kb) issue(kb);
  const v4i zero = {0, 0, 0, 0};
  for (int kb = 0; kb < nsc; ++kb) {
    // this wave's loads of block kb have landed once at most (S - 2) blocks of
    // its loads are outstanding
    constexpr int L012 = NQ + 1, L3 = NQ + (BM > 64 ? 1 : 0) + 1;
    if (w == 3)
      wait_vm<L3 * (S - 2)>();
    else
      wait_vm<L012 * (S - 2)>();
    __syncthreads();  // every wave's loads of kb landed; every wave is done with block kb - 1
    issue(kb + S - 1);  // into the stage of block kb - 1
    const uint8_t* stg = ring + (kb % S) * STG;
    const uint8_t* cst = stg + QB;
    const float* dst = reinterpret_cast<const float*>(stg + QB + CB);
    const uint8_t* sst = stg + QB + CB + DB;
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      long bfrag[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int wi = 2 * sb + (t >> 1);  // word of the staged row (half wi / 4, stored swapped for rows 8-15 of 16)
        const uint32_t word =
            *reinterpret_cast<const uint32_t*>(cst + (srow[j] + li) * 32 + 16 * ((wi >> 2) ^ (li >> 3)) + 4 * (wi & 3));
        const int sh = 4 * (t & 1);
        const uint32_t lo = __builtin_amdgcn_perm(0u, 0x000100FFu, (word >> sh) & 0x03030303u);
        const uint32_t hi = __builtin_amdgcn_perm(0u, 0x000100FFu, (word >> (sh + 2)) & 0x03030303u);
        bfrag[j] = (long)(((uint64_t)hi << 32) | lo);
      }
      // every MFMA of the sub-block first, into its own registers, then the
      // scaling: the matrix core runs the next products while the vector ALU
      // converts the earlier ones (one result register set, reused, would
      // make each MFMA wait for the conversions of the one before)
      v4i I[MW][2];
#pragma unroll
      for (int mt = 0; mt < MW; ++mt) {
        const int r = 16 * MW * wm + 16 * mt + li;
        const long afrag = *reinterpret_cast<const long*>(stg + r * 128 + 16 * ((2 * sb + (t >> 1)) ^ (r & 7)) +
                                                          8 * (t & 1));
#pragma unroll
        for (int j = 0; j < 2; ++j) I[mt][j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(afrag, bfrag[j], zero, 0, 0, 0);
      }
      if constexpr (DUMP) {  // the exact I of every (row, output, sub-block), as launched
#pragma unroll
        for (int mt = 0; mt < MW; ++mt)
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
              const int m = mb + 16 * MW * wm + 16 * mt + 4 * t + rr, n = n0 + srow[j] + li;
              if (m < a.nb && n < N) a.dump[((size_t)(a.m0 + m) * N + n) * nsub + kb * 4 + sb] = I[mt][j][rr];
            }
      }
#pragma unroll
      for (int mt = 0; mt < MW; ++mt) {
        const int mr = 16 * MW * wm + 16 * mt;
        float dv[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) dv[rr] = dst[(mr + 4 * t + rr) * 4 + sb];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr)
            blk[j][mt][rr] =
                sb == 0 ? dv[rr] * (float)I[mt][j][rr] : fmaf(dv[rr], (float)I[mt][j][rr], blk[j][mt][rr]);
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float sc = h2f(*reinterpret_cast<const uint16_t*>(sst + 4 * (srow[j] + li)));
#pragma unroll
      for (int mt = 0; mt < MW; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[j][mt][r] = fmaf(sc, blk[j][mt][r], acc[j][mt][r]);
    }
  }
  wait_vm<0>();  // the trailing loads land before the workgroup's LDS is released
  if constexpr (DUMP) return;

#pragma unroll
  for (int mt = 0; mt < MW; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = mb + 16 * MW * wm + 16 * mt + 4 * t + r;
      if (m >= a.nb) continue;
      if constexpr (SW) {
        const int n = n0 + 16 * wn + li;
        if (n < N) {
          const float g = acc[0][mt][r], u = acc[1][mt][r];
          y[(size_t)(a.m0 + m) * ldy + n] = g / (1.0f + expf(-g)) * u;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int n = n0 + srow[j] + li;
          if (n < N) {
            float* o = &y[(size_t)(a.m0 + m) * ldy + n];
            if constexpr (MODE == BTF_GEMV_ADD)
              *o += acc[j][mt][r];
            else
              *o = acc[j][mt][r];
          }
        }
      }
    }
}

template <int MW, int S>
void by_mode_pf2(int mode, const MfmaArgs& a, dim3 grid, hipStream_t st) {
  if (mode == BTF_GEMV_STORE)
    hipLaunchKernelGGL((gemm_pf2_kernel<MW, S, BTF_GEMV_STORE>), grid, dim3(256), 0, st, a);
  else if (mode == BTF_GEMV_ADD)
    hipLaunchKernelGGL((gemm_pf2_kernel<MW, S, BTF_GEMV_ADD>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((gemm_pf2_kernel<MW, S, BTF_GEMV_SWIGLU>), grid, dim3(256), 0, st, a);
}

}  // namespace

int mfma_rows_per_pass() { return 64; }

int gemm_mfma(const GemvSeg* segs, int nseg, int K, int m0, int nb, const Q8& act, int mode, int32_t* dump,
              hipStream_t st, const DevState& ds, const Q8* qout) {
  MfmaArgs a{};
  // up to 32 activation rows: the K-split 16-row tile (32 rows with a Q8
  // output); more: the prefill tile
  const bool ks = nb <= 32;
  if (qout && (!ks || dump)) return fail(BTF_ERR_ARGS, "gemm: a Q8 output needs at most 32 rows");
  const int rows_real = ks ? (qout ? 32 : 16) : mode == BTF_GEMV_SWIGLU ? 32 : 64;
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
  if (qout) {
    a.oq = const_cast<int8_t*>(qout->q);  // (Q8 holds read-only views; this one is written)
    a.od = const_cast<float*>(qout->d);
    a.os = const_cast<int32_t*>(qout->s);
  }
  if (tiles == 0) return BTF_OK;
  const int MT = nb <= 16 ? 1 : nb <= 32 ? 2 : 4;
  const int BM = 16 * MT;
  const dim3 grid(tiles, (nb + BM - 1) / BM);
  const bool dmp = dump != nullptr;
  if (ks) {
    // up to 16 rows with d and s 16-byte aligned (the LDS-direct loads of the
    // packed tile read them in 16-byte pieces): the packed tile
    const int kw = kp_waves(K, mode);
    if (nb <= 16 && kw && ((reinterpret_cast<uintptr_t>(act.d) | reinterpret_cast<uintptr_t>(act.s)) & 15) == 0) {
      const dim3 gk(tiles, 1);
      if (qout) {
        if (nb <= 8)
          by_waves_kp<1, false, 2>(kw, mode, a, gk, st);
        else
          by_waves_kp<2, false, 2>(kw, mode, a, gk, st);
      } else if (nb <= 8) {
        dmp ? by_waves_kp<1, true>(kw, mode, a, gk, st) : by_waves_kp<1, false>(kw, mode, a, gk, st);
      } else {
        dmp ? by_waves_kp<2, true>(kw, mode, a, gk, st) : by_waves_kp<2, false>(kw, mode, a, gk, st);
      }
      return launch_status("gemm_kp_kernel");
    }
    // 8 waves split K for one activation tile (measured: down 29.6 -> 25.2 us and
    // QKV 11.0 -> 10.1 us at M = 8), except gate+up at K = 5120 (27 -> 31 us);
    // with two activation tiles 8 waves were slower on every shape
    const int nw = MT == 1 && (K >= 8192 || mode != BTF_GEMV_SWIGLU) ? 8 : 4;
    // (the K split depends on nw only: the outputs do not depend on the tile height)
    if (qout) {
      if (MT == 1)
        by_waves_ks<1, false, 2>(nw, mode, a, grid, st);
      else
        by_waves_ks<2, false, 2>(nw, mode, a, grid, st);
      return launch_status("gemm_ks_kernel");
    }
    if (MT == 1)
      dmp ? by_waves_ks<1, true>(nw, mode, a, grid, st) : by_waves_ks<1, false>(nw, mode, a, grid, st);
    else
      dmp ? by_waves_ks<2, true>(nw, mode, a, grid, st) : by_waves_ks<2, false>(nw, mode, a, grid, st);
    return launch_status("gemm_ks_kernel");
  }
  // 128 activation rows per tile while that still gives two workgroups per CU, else 64
  const int cus = ds.cu_count > 0 ? ds.cu_count : 256;
  const bool wide = (int64_t)tiles * ((nb + 127) / 128) >= 2 * cus;
  const dim3 gw(tiles, (nb + 127) / 128), gn(tiles, (nb + 63) / 64);
  // the LDS-direct ring loads d in 16-byte pieces
  if ((reinterpret_cast<uintptr_t>(act.d) & 15) == 0) {
    if (dmp) {  // the exact-I dump (btf_hip_gemv_i32_dump, one matrix): the same tile, writing I
      if (wide)
        hipLaunchKernelGGL((gemm_pf2_kernel<4, 2, BTF_GEMV_STORE, true>), gw, dim3(256), 0, st, a);
      else
        hipLaunchKernelGGL((gemm_pf2_kernel<2, 3, BTF_GEMV_STORE, true>), gn, dim3(256), 0, st, a);
    } else if (wide) {
      by_mode_pf2<4, 2>(mode, a, gw, st);  // 41 KB; 190 VGPRs: 2 workgroups per CU
    } else {
      by_mode_pf2<2, 3>(mode, a, gn, st);  // 34 KB: 4 workgroups per CU
    }
    return launch_status("gemm_pf2_kernel");
  }
  if (dmp) {
    if (wide)
      hipLaunchKernelGGL((gemm_pf_kernel<4, 1, BTF_GEMV_STORE, true>), gw, dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((gemm_pf_kernel<2, 1, BTF_GEMV_STORE, true>), gn, dim3(256), 0, st, a);
  } else if (wide) {
    by_mode_pf<4>(mode, a, gw, st);
  } else {
    by_mode_pf<2>(mode, a, gn, st);
  }
  return launch_status("gemm_pf_kernel");
}

}  // namespace btfhip
