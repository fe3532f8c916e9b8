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
  void* argmax_scratch = nullptr;  // this device's copy of the no-allocation pick's static scratch
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

// Q8 of 32 values held by a 32-lane half-wave (lane j holds value j), identical
// to the q8 kernel / include/btf/packed.hpp:117-134. Returns q of this lane;
// d and s valid in every lane of the half.
// The reductions run in DPP within 16-lane rows, then v_permlane16_swap
// combines rows 0/1 and 2/3 (no LDS traffic).
__device__ __forceinline__ float half32_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ int half32_sum(int v) {
  v += dpp_i<0xB1>(v);
  v += dpp_i<0x4E>(v);
  v += dpp_i<0x141>(v);
  v += dpp_i<0x140>(v);
  const auto r = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
  return (int)r[0] + (int)r[1];
}
__device__ __forceinline__ int q8_half(float v, float& d, int& s) {
  // (the running max starts at 0, as the q8 kernel's and the CPU's: a NaN
  // value never becomes the block's amax)
  const float amax = half32_max(fmaxf(0.f, fabsf(v)));
  float dd = h2f(f2h_bits(amax / 127.0f));
  if (amax == 0.f) dd = copysignf(0.f, __shfl(v, 31, 32));  // all 32 lanes of the half take this branch
  d = dd;
  const float id = amax != 0.f ? 127.0f / amax : 0.f;
  const int q = (int)__builtin_rintf(v * id);
  s = half32_sum(q);
  return q;
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
// x != nullptr (nb == 1, no dump): the activation row m0 is quantized from
// fp32 x [.][ldx] inside the kernel instead of read from `a`. qout != nullptr
// (nb == 1, one output segment, N % 32 == 0): the kernel also writes the Q8
// of the output rows into qout (row stride N).
int gemv_dot4(const GemvSeg* segs, int nseg, int K, int m0, int nb, const Q8& a, int mode, int32_t* dump,
              hipStream_t st, const DevState& ds, const float* x = nullptr, int ldx = 0,
              const Q8* qout = nullptr);
// int8 MFMA path: rows m0 .. m0+nb-1.
// PTQ1_0 path (codes = PTQ1_0 rows, scales unused): rows m0 .. m0+nb-1 (nb <= 2), K <= 32768.
int gemv_b3(const GemvSeg* segs, int nseg, int K, int m0, int nb, const Q8& a, int mode, hipStream_t st,
            const DevState& ds);
// qout: also the Q8 of the output rows (nb <= 32, N % 32 == 0), for the next GEMM.
int gemm_mfma(const GemvSeg* segs, int nseg, int K, int m0, int nb, const Q8& a, int mode, int32_t* dump,
              hipStream_t st, const DevState& ds, const Q8* qout = nullptr);
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
int step_validate_ops(const btf_step_vec* vecs, int nvec, const btf_step_op* ops, int nops);  // host only
int step_create_ops(const btf_step_vec* vecs, int nvec, const btf_step_op* ops, int nops, StepProgram** out,
                    const DevState& ds);
int step_check_residency(const DevState& ds);
int step_launch(StepProgram* P, hipStream_t st);
int step_error(StepProgram* P, int* err);
int step_set_spin_limit(StepProgram* P, uint32_t polls);
int step_guards(StepProgram* P, int* guards);
int step_audit(const btf_step_vec* vecs, int nvec, const btf_step_op* ops, int nops, int G, btf_step_audit* res);  // host only
void step_destroy(StepProgram* P);

int stream_read(const void* src, uint64_t bytes, uint32_t never, uint32_t* sink, hipStream_t st, const DevState& ds);
int gen_ptq1_0(uint64_t seed, uint64_t mat, int64_t first_block, int64_t nblocks, uint8_t* dst, hipStream_t st,
               const DevState& ds);
int embed(const uint8_t* codes, const uint16_t* scales, const int* d_tok, int M, int E, int block, const float* signs,
          float* x, hipStream_t st);
int64_t argmax_part_bytes(int V);
int argmax(const float* logits, int V, void* part, int* out, hipStream_t st);
int argmax_scratch_setup(DevState& ds);  // with the device current
int argmax_noalloc(const float* logits, int V, int* out, hipStream_t st, const DevState& ds);
int pos_add(int* d_pos, int M, hipStream_t st);

}  // namespace btfhip
