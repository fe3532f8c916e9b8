/*
 * btf_oracle.h -- CPU restatement of the reference's fused ternary matmul
 * math, used ONLY as test infrastructure.
 *
 * Who may use it: tests/, __graft_entry__.smoke() and the cpu_baseline leg of
 * bench.py. The product library (libbtf_hip.so) never links, loads or calls
 * anything in this directory; it fails loudly when its HIP build is missing.
 *
 * Every function names the reference file:line it restates (paths relative to
 * the reference repository root). The restatement is written from the
 * reference's documented behaviour, not copied from it.
 */
#ifndef BTF_ORACLE_H
#define BTF_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- layout constants: include/btf/packed.hpp:29-32 -------------------- */
#define BTF_OR_BLOCK 128       /* weights per PTQ1_0 block / per fp16 scale   */
#define BTF_OR_BLOCK_BYTES 28  /* PTQ1_0 block in the GGUF                    */
#define BTF_OR_SUB 32          /* weights per Q8 activation block             */
#define BTF_OR_PACKED_BYTES 32 /* T2 code bytes of one 128-weight block       */

/* ---- fp16 <-> f32 ------------------------------------------------------ */
/* ref/bonsai-decoder/include/bd/types.hpp:37-57 (exact widening). */
float btf_or_fp16_to_f32(uint16_t h);
/* ref/bonsai-decoder/src/types.cpp:42-62 (round to nearest even, subnormals,
 * overflow to inf, NaN -> quiet NaN 0x7e00 with the input's sign). */
uint16_t btf_or_f32_to_fp16(float f);

/* ---- PTQ1_0 source format ---------------------------------------------- */
/* Trit (-1/0/+1) of element e (0..127) of one 28-byte block:
 * ref/bonsai-decoder/include/bd/types.hpp:70-78. */
int btf_or_ptq1_0_trit(const uint8_t* blk, int e);
/* PTQ1_0 encoder (test-input synthesis), n % 128 == 0:
 * ref/bonsai-decoder/src/types.cpp:289-320. */
void btf_or_quant_ptq1_0(const float* x, uint8_t* dst, int64_t n);
/* Encodes 128 trits (-1/0/+1, element order) + fp16 scale bits into one
 * 28-byte block with the same digit layout as the encoder above. */
void btf_or_encode_trits(const int8_t* trits, uint16_t scale_bits, uint8_t* blk);

/* ---- T2 resident layout ------------------------------------------------ */
/* include/btf/packed.hpp:35-38 */
int btf_or_code_byte(int e);
int btf_or_code_shift(int e);
/* include/btf/packed.hpp:94-98: code (0..2) of column e of a packed row. */
int btf_or_packed_code(const uint8_t* row_codes, int64_t e);
/* include/btf/packed.hpp:49-91: one PTQ1_0 block -> 8 code words + scale. */
void btf_or_pack_block(const uint8_t* blk, uint32_t words[8], uint16_t* scale);
/* src/repack.cpp:16-27: rows x K (K % 128 == 0) -> codes [rows][K/4],
 * scales [rows][K/128]. */
void btf_or_repack_rows(const uint8_t* src, int64_t rows, int64_t K, uint8_t* codes, uint16_t* scales);
/* Same transform on a flat run of nblocks blocks (the launch_repack contract,
 * src/cuda/kernels.cuh:22-24). */
void btf_or_repack_blocks(const uint8_t* src, int64_t nblocks, uint8_t* codes, uint16_t* scales);

/* ---- Q8_0 activations -------------------------------------------------- */
/* include/btf/packed.hpp:117-134: one block of 32 floats; returns sum(q). */
int btf_or_q8_block(const float* x, int8_t* q, float* d);
/* ref/bonsai-decoder/src/cpu_ops.cpp:189-197: q * d in place of x. */
void btf_or_round_q8_0(const float* x, int64_t n, float* out);
/* Q8 stage of src/emu_decoder.cpp:122-140 over M dense rows of width K read
 * with row stride ldx: q [M][K], d [M][K/32], s [M][K/32]. */
void btf_or_quantize_rows(const float* x, int ldx, int M, int K, int8_t* q, float* d, int32_t* s);

/* ---- full fused prep: src/emu_decoder.cpp:122-140 ---------------------- */
/* rmsnorm: ref/bonsai-decoder/src/cpu_ops.cpp:121-127 (w may be NULL). */
void btf_or_rmsnorm(const float* x, const float* w, int64_t n, float eps, float* y);
/* fwht: ref/bonsai-decoder/src/cpu_ops.cpp:76-88 (normalised, in place). */
void btf_or_fwht(float* x, int n);
/* hadamard_input: ref/bonsai-decoder/src/cpu_ops.cpp:90-111.
 * block == 0 means the transform is inactive (copy). signs may be NULL. */
void btf_or_hadamard_input(int block, int perm_hd, int perm_nk, int perm_rep, const float* signs, const float* x,
                           int64_t n, float* out);
/* x [M][ldx] -> optional rmsnorm -> hadamard_input -> Q8. xn_out (optional,
 * [M][ldxn]) receives the normed, untransformed rows. Returns 0, or -1 on a
 * geometry error (perm sizes or n % 32). */
int btf_or_prep(const float* x, int ldx, int M, int n, const float* normw, float eps, int block, int perm_hd,
                int perm_nk, int perm_rep, const float* signs, float* xn_out, int ldxn, int8_t* q, float* d,
                int32_t* s);

/* ---- ternary dot / GEMV ----------------------------------------------- */
/* include/btf/packed.hpp:101-104 */
int btf_or_dp4a(uint32_t a, uint32_t b, int c);
/* include/btf/packed.hpp:108-113: code . q over one 32-column sub-block. */
int btf_or_sub_dot(uint32_t w0, uint32_t w1, const uint32_t* aw);
/* The exact integer anchor I[m][n][s] = code_dot - s[m][s]
 * (src/emu_decoder.cpp:153-158), written as int32 [M][N][K/32]. */
void btf_or_gemv_i32(const uint8_t* codes, int64_t N, int64_t K, const int8_t* q, const int32_t* s, int M,
                     int32_t* I_out);
/* EmuDecoder::gemv, src/emu_decoder.cpp:143-165: per row r and activation row m,
 * acc += fp16(scale[s/4]) * d[m][s] * (float)I, s ascending, fp32, no FMA;
 * y[m*ldy + r] = add ? y + acc : acc. Rows are split over nthreads workers in
 * contiguous chunks (ThreadPool::parallel_for, ref/bonsai-decoder/src/cpu_ops.cpp:57-73);
 * nthreads <= 0 means all hardware threads. */
void btf_or_gemv(const uint8_t* codes, const uint16_t* scales, int64_t N, int64_t K, const int8_t* q, const float* d,
                 const int32_t* s, int M, float* y, int64_t ldy, int add, int nthreads);
/* bd::silu (ref/bonsai-decoder/include/bd/cpu_ops.hpp:49) applied as
 * g = silu(g) * u (src/emu_decoder.cpp:195-197). */
void btf_or_swiglu(float* g, const float* u, int64_t n);

/* ---- either side of the GEMV chain -------------------------------------- */
/* Embedding lookup: src/emu_decoder.cpp:171-180 (row decode of the packed
 * table: (code - 1) * fp16 scale) then bd::hadamard_inverse
 * (ref/bonsai-decoder/src/cpu_ops.cpp:113-118: normalised FWHT per block, then
 * the signs). block == 0: no transform. toks [M] in [0, V), else -1 (the
 * emulator throws); x [M][E]. */
int btf_or_embed(const uint8_t* codes, const uint16_t* scales, const int32_t* toks, int M, int E, int V, int block,
                 const float* signs, float* x);
/* Greedy pick: ref/bonsai-decoder/src/sampler.cpp:20-25 (and the emulator's
 * own loop, src/emu_decoder.cpp:205-207): the first index of the maximum. */
int btf_or_argmax(const float* logits, int n);

/* ---- seeded synthetic weights (the benchmark's generator) ------------- */
/* nblocks PTQ1_0 blocks of matrix `mat`: trits i.i.d. with
 * P(-1,0,+1) = (0.3,0.4,0.3), fp16 scale = RNE(U[0.01,0.05]). Block b's
 * content depends only on (seed, mat, first_block + b). */
void btf_or_gen_ptq1_0(uint64_t seed, uint64_t mat, int64_t first_block, int64_t nblocks, uint8_t* dst);

int btf_or_hw_threads(void);

#ifdef __cplusplus
}
#endif
#endif
