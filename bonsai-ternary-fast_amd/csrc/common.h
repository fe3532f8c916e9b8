// common.h -- device helpers and internal launcher declarations shared by the
// HIP translation units of libbtf_hip.so (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "../../include/btf/hip_abi.h"

namespace btfhip {

// ---- T2 / Q8 geometry (the reference's include/btf/packed.hpp:29-32) ----
constexpr int kBlock = 128;        // weights per PTQ1_0 block and per fp16 scale
constexpr int kBlockBytes = 28;    // PTQ1_0 block
constexpr int kSub = 32;           // weights per Q8 activation block (sub-block)
constexpr int kPackedBytes = 32;   // T2 code bytes per 128-weight block

// ---- per-device state filled by kernels_init ----
struct DevState {
  bool init = false;
  int cu_count = 0;
  int lds_per_block = 0;
  int max_threads = 0;
};
DevState* dev_state(int device);  // nullptr if device id out of range
// State of the current device, or nullptr (with the error set) if
// kernels_init has not run for it.
const DevState* current_state();

// ---- error plumbing (thread-local last error) ----
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int launch_status(const char* what);  // hipGetLastError -> BTF_ERR_LAUNCH

// ---- wave64 reductions with DPP (no LDS) ----
// dpp_ctrl encodings (GCN3+/CDNA): quad_perm(a,b,c,d) = a | b<<2 | c<<4 | d<<6,
// row_half_mirror = 0x141, row_mirror = 0x140. Every pattern used here is a
// permutation within each 16-lane row with all rows and banks enabled, so no
// lane reads an invalid source; bound_ctrl lets the compiler fuse the move
// into the consuming add (v_add_f32_dpp).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, true);
}
// Sum over each 16-lane DPP row; every lane of the row gets the total.
// Butterfly: swap neighbours, swap pairs, mirror halves of 8, mirror halves of 16.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<0xB1>(v);   // quad_perm(1,0,3,2)
  v += dpp_f<0x4E>(v);   // quad_perm(2,3,0,1)
  v += dpp_f<0x141>(v);  // row_half_mirror
  v += dpp_f<0x140>(v);  // row_mirror
  return v;
}
// Sum / max over each aligned group of 4 lanes (every lane gets the result).
__device__ __forceinline__ int quad_sum_i(int v) {
  v += dpp_i<0xB1>(v);
  v += dpp_i<0x4E>(v);
  return v;
}
__device__ __forceinline__ float quad_max_f(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  return v;
}

// fp16 bits -> f32 (exact) and f32 -> fp16 (round to nearest even) -> f32.
__device__ __forceinline__ float h2f(uint16_t h) {
  _Float16 x;
  __builtin_memcpy(&x, &h, 2);
  return (float)x;
}
__device__ __forceinline__ uint16_t f2h_bits(float f) {
  _Float16 x = (_Float16)f;
  uint16_t h;
  __builtin_memcpy(&h, &x, 2);
  return h;
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// 16 * (code . q - s) over one 32-column sub-block. w0/w1 are the sub-block's
// two code words (columns 0..15 / 16..31; 2-bit field k of byte j is column
// 16h + 4k + j), a[0..7] the activation words (word 4h + k holds columns
// 16h+4k .. +3) and ns = -s. The four 2-bit fields are masked in place
// (values c, 4c, 16c, and 16c for the top field after >>2), dotted into three
// partial sums, and recombined as 16*c0 + 4*c1 + c23 with two shift-adds, so
// the result is exact (|result| < 2^18) and the caller scales by d/16.
__device__ __forceinline__ int subblock_dot16(uint32_t w0, uint32_t w1, const uint32_t* a, int ns) {
  int c0 = sdot4(w0 & 0x03030303u, a[0], ns);
  c0 = sdot4(w1 & 0x03030303u, a[4], c0);
  int c1 = sdot4(w0 & 0x0C0C0C0Cu, a[1], 0);
  c1 = sdot4(w1 & 0x0C0C0C0Cu, a[5], c1);
  int c2 = sdot4(w0 & 0x30303030u, a[2], 0);
  c2 = sdot4((w0 >> 2) & 0x30303030u, a[3], c2);
  c2 = sdot4(w1 & 0x30303030u, a[6], c2);
  c2 = sdot4((w1 >> 2) & 0x30303030u, a[7], c2);
  return (((c0 << 2) + c1) << 2) + c2;
}

// ---- internal launchers (host) ----
struct GemvSeg {
  const uint8_t* codes;
  const uint16_t* scales;
  int N;
  float* y;
  int ldy;
};
struct Q8 {
  const int8_t* q;
  const float* d;
  const int32_t* s;
};

// v_dot4 path: rows m0 .. m0+nb-1 (nb <= 4) of the activation.
int gemv_dot4(const GemvSeg* segs, int nseg, int K, int m0, int nb, const Q8& a, int mode, int32_t* dump,
              hipStream_t st, const DevState& ds);
// int8 MFMA path: rows m0 .. m0+nb-1.
int gemm_mfma(const GemvSeg* segs, int nseg, int K, int m0, int nb, const Q8& a, int mode, int32_t* dump,
              hipStream_t st, const DevState& ds);
int mfma_rows_per_pass();

int repack(const uint8_t* src, int64_t nblocks, uint8_t* codes, uint16_t* scales, hipStream_t st,
           const DevState& ds);
int prep(const float* x, int ldx, int M, int n, const float* normw, float eps, int block, int perm_hd, int perm_nk,
         int perm_rep, const float* signs, float* xn_out, int ldxn, int8_t* q, float* d, int32_t* s, hipStream_t st,
         const DevState& ds);
struct StepProgram;
int step_validate(const btf_step_vec* vecs, int nvec, const btf_step_gemv* ops, int nops);  // host only
int step_create(const btf_step_vec* vecs, int nvec, const btf_step_gemv* ops, int nops, StepProgram** out,
                const DevState& ds);
int step_check_residency(const DevState& ds);
int step_launch(StepProgram* P, hipStream_t st);
int step_error(StepProgram* P, int* err);
int step_set_spin_limit(StepProgram* P, uint32_t polls);
void step_destroy(StepProgram* P);

int gen_ptq1_0(uint64_t seed, uint64_t mat, int64_t first_block, int64_t nblocks, uint8_t* dst, hipStream_t st,
               const DevState& ds);

}  // namespace btfhip
