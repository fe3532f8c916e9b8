/*
 * btf_oracle.c -- CPU restatement of the reference's fused ternary matmul
 * path (T2 repack, Q8_0 quantize, ternary GEMV with the fp16 block-scale
 * epilogue). TEST INFRASTRUCTURE ONLY: see btf_oracle.h for who may use it.
 *
 * Build: oracle/Makefile (gcc -O3 -std=c11 -ffp-contract=off). The float
 * epilogue must be evaluated exactly as written (no FMA contraction), because
 * the reference emulator is built for baseline x86-64, which has no FMA.
 */
#define _GNU_SOURCE
#include "btf_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ======================================================================
 * fp16 <-> f32
 * ====================================================================== */

/* ref/bonsai-decoder/include/bd/types.hpp:37-57. Every half is exactly
 * representable in f32: subnormals are man * 2^-24. */
float btf_or_fp16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31;
  const uint32_t ex = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  uint32_t bits;
  float f;
  if (ex == 0x1fu) {
    bits = sign | 0x7f800000u | (man << 13);
  } else if (ex == 0) {
    f = ldexpf((float)man, -24);
    return sign ? -f : f;
  } else {
    bits = sign | ((ex + 112u) << 23) | (man << 13);
  }
  memcpy(&f, &bits, 4);
  return f;
}

/* ref/bonsai-decoder/src/types.cpp:42-62: IEEE binary16 with round to
 * nearest, ties to even. Written from the definition: the result is the
 * significand rounded at the bit that has weight 2^(e-10) (normal) or 2^-24
 * (subnormal); a carry out of the significand bumps the exponent, and a carry
 * into exponent 31 gives inf. */
uint16_t btf_or_f32_to_fp16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return sign | 0x7e00u; /* NaN -> quiet NaN */
  if (ax == 0x7f800000u) return sign | 0x7c00u;
  const int e = (int)(ax >> 23) - 127;
  if (e >= 16) return sign | 0x7c00u; /* >= 65536 */
  if (e < -26) return sign;           /* < 2^-26 rounds to zero (incl. f32 subnormals) */
  const uint32_t sig = (ax & 0x7fffffu) | 0x800000u; /* 24-bit significand, value sig * 2^(e-23) */
  uint32_t r, rem, half;
  int sh;
  if (e >= -14) {
    sh = 13; /* keep 11 significant bits */
    r = (uint32_t)((e + 15) << 10) + ((sig >> 13) & 0x3ffu);
  } else {
    sh = -e - 1; /* units of 2^-24: sig * 2^(e+1) -> shift right by -(e+1) = 14..25 */
    r = sig >> sh;
  }
  rem = sig & ((1u << sh) - 1u);
  half = 1u << (sh - 1);
  if (rem > half || (rem == half && (r & 1u))) ++r;
  return (uint16_t)(sign | r);
}

/* ======================================================================
 * PTQ1_0 source format
 * ====================================================================== */

/* Byte index and base-3 place of element e inside a 28-byte block.
 * Elements 0..79 are digit e/16 of byte e%16, 80..119 digit (e-80)/8 of byte
 * 16+(e-80)%8, 120..127 digit (e-120)/2 of byte 24+(e-120)%2
 * (ref/bonsai-decoder/include/bd/types.hpp:66-78, docs/packed-layout.md:10-17). */
static void ptq_place(int e, int* byte, int* digit) {
  if (e < 80) {
    *byte = e % 16;
    *digit = e / 16;
  } else if (e < 120) {
    *byte = 16 + (e - 80) % 8;
    *digit = (e - 80) / 8;
  } else {
    *byte = 24 + (e - 120) % 2;
    *digit = (e - 120) / 2;
  }
}

static const uint32_t kPow3[6] = {1u, 3u, 9u, 27u, 81u, 243u};

/* Digit `digit` (0 = most significant) of a fractional base-3 byte, +1 offset
 * removed: ((uint8)(b * 3^digit) * 3) >> 8 is the code (trit + 1).
 * ref/bonsai-decoder/include/bd/types.hpp:76-77. */
static int ptq_digit(uint32_t b, int digit) {
  const uint32_t frac = (uint32_t)(uint8_t)(b * kPow3[digit]);
  return (int)((frac * 3u) >> 8);
}

int btf_or_ptq1_0_trit(const uint8_t* blk, int e) {
  int bi, dg;
  ptq_place(e, &bi, &dg);
  return ptq_digit(blk[bi], dg) - 1;
}

/* A byte holding base-3 digits c0..c4 (c0 most significant) is
 * ceil(q * 256 / 243) with q = sum c_n 3^(4-n)
 * (ref/bonsai-decoder/src/types.cpp:301-316). */
static uint8_t ptq_byte(const int* codes, int ndigits) {
  uint32_t q = 0;
  for (int n = 0; n < 5; ++n) q = q * 3u + (uint32_t)(n < ndigits ? codes[n] : 0);
  return (uint8_t)((q * 256u + 242u) / 243u);
}

void btf_or_encode_trits(const int8_t* trits, uint16_t scale_bits, uint8_t* blk) {
  int codes[26][5];
  memset(codes, 0, sizeof codes);
  for (int e = 0; e < 128; ++e) {
    int bi, dg;
    ptq_place(e, &bi, &dg);
    codes[bi][dg] = trits[e] + 1;
  }
  for (int b = 0; b < 24; ++b) blk[b] = ptq_byte(codes[b], 5);
  for (int b = 24; b < 26; ++b) blk[b] = ptq_byte(codes[b], 4);
  blk[26] = (uint8_t)(scale_bits & 0xffu);
  blk[27] = (uint8_t)(scale_bits >> 8);
}

/* ref/bonsai-decoder/src/types.cpp:289-320 (quantize_row_ptq1_0_ref port):
 * d = amax over the 128-block, stored as fp16; trit = lround(x / d)
 * computed as x * (1/d), rounding half away from zero. */
void btf_or_quant_ptq1_0(const float* x, uint8_t* dst, int64_t n) {
  for (int64_t i = 0; i < n / 128; ++i) {
    const float* xb = x + i * 128;
    float amax = 0.0f;
    for (int j = 0; j < 128; ++j) amax = fmaxf(amax, fabsf(xb[j]));
    const float id = amax != 0.0f ? 1.0f / amax : 0.0f;
    int8_t t[128];
    for (int j = 0; j < 128; ++j) t[j] = (int8_t)lroundf(xb[j] * id);
    btf_or_encode_trits(t, btf_or_f32_to_fp16(amax), dst + i * 28);
  }
}

/* ======================================================================
 * T2 layout (include/btf/packed.hpp, docs/packed-layout.md:27-46)
 * ====================================================================== */

int btf_or_code_byte(int e) { return (e / 32) * 8 + ((e / 16) % 2) * 4 + (e % 4); }
int btf_or_code_shift(int e) { return ((e / 4) % 4) * 2; }

int btf_or_packed_code(const uint8_t* row_codes, int64_t e) {
  const uint8_t* blk = row_codes + (e / BTF_OR_BLOCK) * BTF_OR_PACKED_BYTES;
  const int c = (int)(e % BTF_OR_BLOCK);
  return (blk[btf_or_code_byte(c)] >> btf_or_code_shift(c)) & 3;
}

/* Element-wise statement of pack_block (include/btf/packed.hpp:49-91): the
 * code of element e (trit + 1) lands at byte code_byte(e), bit code_shift(e);
 * the scale is bytes 26..27 unchanged. */
void btf_or_pack_block(const uint8_t* blk, uint32_t words[8], uint16_t* scale) {
  uint8_t bytes[32];
  memset(bytes, 0, sizeof bytes);
  for (int e = 0; e < 128; ++e) {
    const int c = btf_or_ptq1_0_trit(blk, e) + 1;
    bytes[btf_or_code_byte(e)] |= (uint8_t)(c << btf_or_code_shift(e));
  }
  for (int w = 0; w < 8; ++w)
    words[w] = (uint32_t)bytes[4 * w] | ((uint32_t)bytes[4 * w + 1] << 8) | ((uint32_t)bytes[4 * w + 2] << 16) |
               ((uint32_t)bytes[4 * w + 3] << 24);
  *scale = (uint16_t)(blk[26] | (blk[27] << 8));
}

void btf_or_repack_blocks(const uint8_t* src, int64_t nblocks, uint8_t* codes, uint16_t* scales) {
  for (int64_t b = 0; b < nblocks; ++b) {
    uint32_t w[8];
    btf_or_pack_block(src + b * BTF_OR_BLOCK_BYTES, w, &scales[b]);
    for (int i = 0; i < 8; ++i) {
      uint8_t* o = codes + b * BTF_OR_PACKED_BYTES + 4 * i;
      o[0] = (uint8_t)w[i];
      o[1] = (uint8_t)(w[i] >> 8);
      o[2] = (uint8_t)(w[i] >> 16);
      o[3] = (uint8_t)(w[i] >> 24);
    }
  }
}

/* src/repack.cpp:16-27: the rows of a matrix are consecutive runs of K/128
 * blocks, so a row-wise repack is the flat repack of rows * K/128 blocks. */
void btf_or_repack_rows(const uint8_t* src, int64_t rows, int64_t K, uint8_t* codes, uint16_t* scales) {
  btf_or_repack_blocks(src, rows * (K / BTF_OR_BLOCK), codes, scales);
}

/* ======================================================================
 * Q8_0 activations
 * ====================================================================== */

/* include/btf/packed.hpp:117-134. amax is the running
 * `amax = amax > a ? amax : a` with a = (x < 0 ? -x : x), so an all-zero
 * block keeps the sign of its last element's zero (only d's sign bit sees
 * it). d = fp16(amax / 127) widened back to f32; q = nearbyint(x * 127/amax)
 * in round-half-even; returns sum(q). */
int btf_or_q8_block(const float* x, int8_t* q, float* d) {
  float amax = 0.0f;
  for (int i = 0; i < 32; ++i) {
    const float a = x[i] < 0 ? -x[i] : x[i];
    amax = amax > a ? amax : a;
  }
  *d = btf_or_fp16_to_f32(btf_or_f32_to_fp16(amax / 127.0f));
  const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
  int s = 0;
  for (int i = 0; i < 32; ++i) {
    const float r = nearbyintf(x[i] * id);
    q[i] = (int8_t)(int)r;
    s += (int)r;
  }
  return s;
}

/* ref/bonsai-decoder/src/cpu_ops.cpp:189-197 */
void btf_or_round_q8_0(const float* x, int64_t n, float* out) {
  for (int64_t b = 0; b < n; b += 32) {
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(x[b + i]));
    const float d = btf_or_fp16_to_f32(btf_or_f32_to_fp16(amax / 127.0f));
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    for (int i = 0; i < 32; ++i) out[b + i] = nearbyintf(x[b + i] * id) * d;
  }
}

void btf_or_quantize_rows(const float* x, int ldx, int M, int K, int8_t* q, float* d, int32_t* s) {
  for (int m = 0; m < M; ++m)
    for (int b = 0; b < K / 32; ++b) {
      const size_t o = (size_t)m * (K / 32) + b;
      s[o] = btf_or_q8_block(x + (size_t)m * ldx + b * 32, q + (size_t)m * K + b * 32, &d[o]);
    }
}

/* ======================================================================
 * fused prep (rmsnorm -> perm -> signs -> WHT -> Q8)
 * ====================================================================== */

/* ref/bonsai-decoder/src/cpu_ops.cpp:121-127: sum of squares in double,
 * mean rounded to float, scale = 1/sqrtf(mean + eps), y = x * scale * w. */
void btf_or_rmsnorm(const float* x, const float* w, int64_t n, float eps, float* y) {
  double sum = 0.0;
  for (int64_t i = 0; i < n; ++i) sum += (double)x[i] * (double)x[i];
  const float mean = (float)(sum / (double)n);
  const float scale = 1.0f / sqrtf(mean + eps);
  for (int64_t i = 0; i < n; ++i) y[i] = x[i] * scale * (w ? w[i] : 1.0f);
}

/* ref/bonsai-decoder/src/cpu_ops.cpp:76-88: butterflies with stage length
 * 1, 2, 4, ... (a+b, a-b), then every value times 1/sqrtf(n). */
void btf_or_fwht(float* x, int n) {
  for (int len = 1; len < n; len *= 2)
    for (int i = 0; i < n; i += 2 * len)
      for (int j = i; j < i + len; ++j) {
        const float a = x[j], b = x[j + len];
        x[j] = a + b;
        x[j + len] = a - b;
      }
  const float sc = 1.0f / sqrtf((float)n);
  for (int i = 0; i < n; ++i) x[i] *= sc;
}

/* ref/bonsai-decoder/src/cpu_ops.cpp:90-111. The tiled -> grouped gather
 * puts source index d + hd*(k + nk*r) at destination d + hd*(r + rep*k). */
void btf_or_hadamard_input(int block, int perm_hd, int perm_nk, int perm_rep, const float* signs, const float* x,
                           int64_t n, float* out) {
  if (block <= 0) {
    if (out != x) memmove(out, x, (size_t)n * sizeof(float));
    return;
  }
  if (perm_rep > 1) {
    float* tmp = (float*)malloc((size_t)n * sizeof(float));
    memcpy(tmp, x, (size_t)n * sizeof(float));
    for (int k = 0; k < perm_nk; ++k)
      for (int r = 0; r < perm_rep; ++r)
        for (int dd = 0; dd < perm_hd; ++dd)
          out[dd + (int64_t)perm_hd * (r + perm_rep * k)] = tmp[dd + (int64_t)perm_hd * (k + perm_nk * r)];
    free(tmp);
  } else if (out != x) {
    memmove(out, x, (size_t)n * sizeof(float));
  }
  if (signs)
    for (int64_t i = 0; i < n; ++i) out[i] *= signs[i];
  for (int64_t b = 0; b < n; b += block) btf_or_fwht(out + b, block);
}

int btf_or_prep(const float* x, int ldx, int M, int n, const float* normw, float eps, int block, int perm_hd,
                int perm_nk, int perm_rep, const float* signs, float* xn_out, int ldxn, int8_t* q, float* d,
                int32_t* s) {
  if (n % 32) return -1;
  if (block > 0 && perm_rep > 1 && (int64_t)perm_hd * perm_nk * perm_rep != n) return -1;
  if (block > 0 && n % block) return -1;
  float* xn = (float*)malloc((size_t)n * sizeof(float));
  float* t = (float*)malloc((size_t)n * sizeof(float));
  for (int m = 0; m < M; ++m) {
    const float* xr = x + (size_t)m * ldx;
    if (normw)
      btf_or_rmsnorm(xr, normw, n, eps, xn);
    else
      memcpy(xn, xr, (size_t)n * sizeof(float));
    if (xn_out) memcpy(xn_out + (size_t)m * ldxn, xn, (size_t)n * sizeof(float));
    btf_or_hadamard_input(block, perm_hd, perm_nk, perm_rep, signs, xn, n, t);
    btf_or_quantize_rows(t, n, 1, n, q + (size_t)m * n, d + (size_t)m * (n / 32), s + (size_t)m * (n / 32));
  }
  free(xn);
  free(t);
  return 0;
}

/* ======================================================================
 * ternary dot and GEMV
 * ====================================================================== */

/* include/btf/packed.hpp:101-104: signed int8x4 dot, accumulated into c. */
int btf_or_dp4a(uint32_t a, uint32_t b, int c) {
  for (int i = 0; i < 4; ++i) c += (int)(int8_t)(uint8_t)(a >> (8 * i)) * (int)(int8_t)(uint8_t)(b >> (8 * i));
  return c;
}

/* include/btf/packed.hpp:108-113: word h of a sub-block holds columns
 * 16h..16h+15; its 2-bit field k (bits 2k..2k+1 of every byte) lines up with
 * activation word 4h+k. */
int btf_or_sub_dot(uint32_t w0, uint32_t w1, const uint32_t* aw) {
  int acc = 0;
  for (int k = 0; k < 4; ++k) acc = btf_or_dp4a((w0 >> (2 * k)) & 0x03030303u, aw[k], acc);
  for (int k = 0; k < 4; ++k) acc = btf_or_dp4a((w1 >> (2 * k)) & 0x03030303u, aw[4 + k], acc);
  return acc;
}

static uint32_t ld32(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

void btf_or_gemv_i32(const uint8_t* codes, int64_t N, int64_t K, const int8_t* q, const int32_t* s, int M,
                     int32_t* I_out) {
  const int64_t nsub = K / 32;
  for (int m = 0; m < M; ++m) {
    uint32_t* aw = (uint32_t*)malloc((size_t)K);
    memcpy(aw, q + (size_t)m * K, (size_t)K);
    for (int64_t r = 0; r < N; ++r) {
      const uint8_t* cr = codes + r * (K / 4);
      for (int64_t sb = 0; sb < nsub; ++sb)
        I_out[((size_t)m * N + r) * nsub + sb] =
            btf_or_sub_dot(ld32(cr + sb * 8), ld32(cr + sb * 8 + 4), aw + sb * 8) - s[(size_t)m * nsub + sb];
    }
    free(aw);
  }
}

/* ---- a small persistent pool with ThreadPool::parallel_for semantics:
 * worker i (0 = the caller) runs [n*i/T, n*(i+1)/T); runs inline when T == 1
 * or n < 2T (ref/bonsai-decoder/src/cpu_ops.cpp:19-73). */
typedef void (*range_fn)(void* ctx, int64_t b, int64_t e);

typedef struct {
  pthread_mutex_t mu;
  pthread_cond_t cv, done;
  pthread_t th[256];
  int n;
  uint64_t gen;
  int pending, stop;
  range_fn fn;
  void* ctx;
  int64_t total;
} pool_t;

static pool_t* g_pool = NULL;

typedef struct {
  pool_t* p;
  int id;
} worker_arg;

static void* pool_worker(void* a) {
  pool_t* p = ((worker_arg*)a)->p;
  const int id = ((worker_arg*)a)->id;
  free(a);
  uint64_t seen = 0;
  for (;;) {
    pthread_mutex_lock(&p->mu);
    while (!p->stop && p->gen == seen) pthread_cond_wait(&p->cv, &p->mu);
    if (p->stop) {
      pthread_mutex_unlock(&p->mu);
      return NULL;
    }
    seen = p->gen;
    range_fn fn = p->fn;
    void* ctx = p->ctx;
    const int64_t total = p->total;
    pthread_mutex_unlock(&p->mu);
    const int64_t b = total * id / p->n, e = total * (id + 1) / p->n;
    if (b < e) fn(ctx, b, e);
    pthread_mutex_lock(&p->mu);
    if (--p->pending == 0) pthread_cond_signal(&p->done);
    pthread_mutex_unlock(&p->mu);
  }
}

int btf_or_hw_threads(void) {
  const long n = sysconf(_SC_NPROCESSORS_ONLN);
  return n > 0 ? (int)n : 1;
}

static pool_t* pool_get(int n) {
  if (n <= 0) n = btf_or_hw_threads();
  if (n > 256) n = 256;
  if (g_pool && g_pool->n == n) return g_pool;
  if (g_pool) {
    pthread_mutex_lock(&g_pool->mu);
    g_pool->stop = 1;
    pthread_cond_broadcast(&g_pool->cv);
    pthread_mutex_unlock(&g_pool->mu);
    for (int i = 1; i < g_pool->n; ++i) pthread_join(g_pool->th[i], NULL);
    free(g_pool);
    g_pool = NULL;
  }
  pool_t* p = (pool_t*)calloc(1, sizeof(pool_t));
  pthread_mutex_init(&p->mu, NULL);
  pthread_cond_init(&p->cv, NULL);
  pthread_cond_init(&p->done, NULL);
  p->n = n;
  for (int i = 1; i < n; ++i) {
    worker_arg* a = (worker_arg*)malloc(sizeof(worker_arg));
    a->p = p;
    a->id = i;
    pthread_create(&p->th[i], NULL, pool_worker, a);
  }
  g_pool = p;
  return p;
}

static void parallel_for(int nthreads, int64_t n, range_fn fn, void* ctx) {
  pool_t* p = pool_get(nthreads);
  if (p->n == 1 || n < 2 * p->n) {
    fn(ctx, 0, n);
    return;
  }
  pthread_mutex_lock(&p->mu);
  p->fn = fn;
  p->ctx = ctx;
  p->total = n;
  p->pending = p->n - 1;
  p->gen++;
  pthread_cond_broadcast(&p->cv);
  pthread_mutex_unlock(&p->mu);
  fn(ctx, 0, n / p->n);
  pthread_mutex_lock(&p->mu);
  while (p->pending != 0) pthread_cond_wait(&p->done, &p->mu);
  pthread_mutex_unlock(&p->mu);
}

typedef struct {
  const uint8_t* codes;
  const uint16_t* scales;
  int64_t K;
  const int8_t* q;
  const float* d;
  const int32_t* s;
  int M;
  float* y;
  int64_t ldy;
  int add;
} gemv_ctx;

/* src/emu_decoder.cpp:147-163, rows [b, e). */
static void gemv_rows(void* vctx, int64_t b, int64_t e) {
  const gemv_ctx* c = (const gemv_ctx*)vctx;
  const int64_t nsub = c->K / 32;
  for (int64_t r = b; r < e; ++r) {
    const uint8_t* cr = c->codes + r * (c->K / 4);
    const uint16_t* sr = c->scales + r * (c->K / 128);
    for (int m = 0; m < c->M; ++m) {
      const uint32_t* aw = (const uint32_t*)(c->q + (size_t)m * c->K);
      float acc = 0.0f;
      for (int64_t sb = 0; sb < nsub; ++sb) {
        const int idot = btf_or_sub_dot(ld32(cr + sb * 8), ld32(cr + sb * 8 + 4), aw + sb * 8) -
                         c->s[(size_t)m * nsub + sb];
        const float f = btf_or_fp16_to_f32(sr[sb / 4]);
        const float fd = f * c->d[(size_t)m * nsub + sb];
        const float t = fd * (float)idot;
        acc = acc + t;
      }
      float* out = &c->y[(size_t)m * c->ldy + r];
      *out = c->add ? *out + acc : acc;
    }
  }
}

void btf_or_gemv(const uint8_t* codes, const uint16_t* scales, int64_t N, int64_t K, const int8_t* q, const float* d,
                 const int32_t* s, int M, float* y, int64_t ldy, int add, int nthreads) {
  gemv_ctx c = {codes, scales, K, q, d, s, M, y, ldy, add};
  parallel_for(nthreads, N, gemv_rows, &c);
}

void btf_or_swiglu(float* g, const float* u, int64_t n) {
  for (int64_t i = 0; i < n; ++i) g[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
}

/* ======================================================================
 * either side of the GEMV chain
 * ====================================================================== */

/* src/emu_decoder.cpp:171-180 with ref/bonsai-decoder/src/cpu_ops.cpp:113-118.
 * The emulator applies hadamard_inverse only when the transform is active
 * (block > 0): then each block gets the normalised FWHT and, if present, the
 * whole row is multiplied by the signs. */
int btf_or_embed(const uint8_t* codes, const uint16_t* scales, const int32_t* toks, int M, int E, int V, int block,
                 const float* signs, float* x) {
  for (int m = 0; m < M; ++m) {
    const int tok = toks[m];
    if (tok < 0 || tok >= V) return -1;
    const uint8_t* cr = codes + (int64_t)tok * (E / 4);
    const uint16_t* sr = scales + (int64_t)tok * (E / 128);
    float* xr = x + (int64_t)m * E;
    for (int i = 0; i < E; ++i) xr[i] = (float)(btf_or_packed_code(cr, i) - 1) * btf_or_fp16_to_f32(sr[i / 128]);
    if (block > 0) {
      for (int b = 0; b < E; b += block) btf_or_fwht(xr + b, block);
      if (signs)
        for (int i = 0; i < E; ++i) xr[i] *= signs[i];
    }
  }
  return 0;
}

/* ref/bonsai-decoder/src/sampler.cpp:20-25: keep the first maximum (strict >). */
int btf_or_argmax(const float* logits, int n) {
  int best = 0;
  for (int i = 1; i < n; ++i)
    if (logits[i] > logits[best]) best = i;
  return best;
}

/* ======================================================================
 * seeded synthetic weights
 * ====================================================================== */

static uint64_t splitmix64(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/* Thresholds on the top 32 bits of a hash: P(u < T1) = 0.3, P(u < T2) = 0.7. */
#define GEN_T1 1288490189u
#define GEN_T2 3006477107u

void btf_or_gen_ptq1_0(uint64_t seed, uint64_t mat, int64_t first_block, int64_t nblocks, uint8_t* dst) {
  const uint64_t key = splitmix64(splitmix64(seed) ^ (mat * 0xD1B54A32D192ED03ull));
  for (int64_t i = 0; i < nblocks; ++i) {
    const uint64_t base = key + (uint64_t)(first_block + i) * 129u;
    int8_t t[128];
    for (int e = 0; e < 128; ++e) {
      const uint32_t u = (uint32_t)(splitmix64(base + (uint64_t)e) >> 32);
      t[e] = (int8_t)(u < GEN_T1 ? -1 : (u < GEN_T2 ? 0 : 1));
    }
    const uint64_t hs = splitmix64(base + 128u);
    const float uf = (float)(uint32_t)(hs >> 40) * 0x1p-24f;
    const float prod = 0.04f * uf;
    const float v = 0.01f + prod;
    btf_or_encode_trits(t, btf_or_f32_to_fp16(v), dst + i * BTF_OR_BLOCK_BYTES);
  }
}
