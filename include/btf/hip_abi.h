/*
 * hip_abi.h -- C ABI of the MI355X (gfx950) fused ternary matmul path.
 *
 * This is the drop-in boundary for the reference's kernel-launch API
 * (src/cuda/kernels.cuh, namespace btf::cuda). Every entry point below names
 * the reference declaration it replaces. The signatures use plain pointers,
 * sizes and an opaque stream handle; no HIP, CUDA or torch types appear, so a
 * host written in C, C++ (include/btf/kernels.hpp), Python (ctypes) or any
 * FFI can bind it.
 *
 * Conventions (as in the reference, src/cuda/kernels.cuh:3-7):
 *  - Every pointer is caller-owned DEVICE memory unless a comment says host.
 *    launch_repack's src may also be pinned, mapped host memory.
 *  - Launches are asynchronous on `stream` (NULL = the device's null stream).
 *    They allocate nothing and never synchronise, so they are legal inside
 *    stream (graph) capture once btf_hip_kernels_init has run for the device.
 *  - Every function returns BTF_OK (0) or an error code; the message of the
 *    last failure on the calling thread is btf_hip_last_error(). Argument
 *    checks run on the host before anything touches the GPU.
 *  - M <= 0 (or nblocks <= 0) is a no-op that returns BTF_OK.
 */
#ifndef BTF_HIP_ABI_H
#define BTF_HIP_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define BTF_OK 0
#define BTF_ERR_ARGS 1      /* invalid arguments (checked on the host)       */
#define BTF_ERR_DEVICE 2    /* no usable device / device query failed        */
#define BTF_ERR_LAUNCH 3    /* the HIP runtime rejected a launch or call     */
#define BTF_ERR_NOT_INIT 4  /* btf_hip_kernels_init was not run for device   */

typedef void* btf_stream_t; /* a hipStream_t */

/* ---- structs, field for field as the reference --------------------------- */
/* Q8_0 activations of M rows of width K: src/cuda/kernels.cuh:26-31. */
typedef struct btf_q8act {
  int8_t* q;  /* [M][K]                                        */
  float* d;   /* [M][K/32]  fp16 value of amax/127, held as f32 */
  int32_t* s; /* [M][K/32]  sum of q over the block            */
} btf_q8act;

/* Input transform of a folded weight (block 0: none): src/cuda/kernels.cuh:33-38. */
typedef struct btf_hx {
  int block;
  int perm_hd, perm_nk, perm_rep; /* rep > 1: tiled -> grouped gather */
  const float* signs;             /* [n] or NULL                       */
} btf_hx;

/* One packed matrix and its output: src/cuda/kernels.cuh:45-51. */
typedef struct btf_gemv_seg {
  const uint8_t* codes;   /* [N][K/4]   T2 codes                  */
  const uint16_t* scales; /* [N][K/128] fp16 bits                 */
  int N;
  float* y;               /* [M][ldy]                             */
  int ldy;
} btf_gemv_seg;

/* src/cuda/kernels.cuh:52 */
enum { BTF_GEMV_STORE = 0, BTF_GEMV_ADD = 1, BTF_GEMV_SWIGLU = 2 };

/* ---- kernel-launch API (src/cuda/kernels.cuh:16-56) ---------------------- */

/* Replaces btf::cuda::kernels_init (kernels.cuh:17). Queries the device's CU
 * count and LDS size and caches them per device. Idempotent; not thread-safe
 * against concurrent launches; call it before any capture. */
int btf_hip_kernels_init(int device);

/* Replaces btf::cuda::gemv_max_nb (kernels.cuh:20). The number of activation
 * rows one launch serves with a single pass over the weights for width K
 * (launch_gemv itself accepts any M). 0 if K is not a positive multiple of 128. */
int btf_hip_gemv_max_nb(int K);

/* Replaces btf::cuda::launch_repack (kernels.cuh:22-24): nblocks PTQ1_0 blocks
 * (28 B each, 4-byte aligned, device or pinned mapped host memory) ->
 * codes [nblocks][32 B] + scales [nblocks] (fp16 bits). */
int btf_hip_launch_repack(const uint8_t* src, int64_t nblocks, uint8_t* codes, uint16_t* scales,
                          btf_stream_t stream);

/* Replaces btf::cuda::launch_prep (kernels.cuh:40-43): x [M][ldx] ->
 * [RMSNorm * normw] -> tiled->grouped perm -> signs -> blockwise WHT -> Q8_0
 * into a (dense rows of width n). normw NULL: no norm; hx NULL or
 * hx->block == 0: no transform; xn_out (optional, [M][ldxn]) receives the
 * normed rows. n % 32 == 0 is required. */
int btf_hip_launch_prep(const float* x, int ldx, int M, int n, const float* normw, float eps, const btf_hx* hx,
                        float* xn_out, int ldxn, const btf_q8act* a, btf_stream_t stream);

/* Replaces btf::cuda::launch_gemv (kernels.cuh:53-56). STORE / ADD:
 * y = W x or y += W x for each of the 1..3 segments (all share K and x).
 * SWIGLU: segs[0] = gate, segs[1] = up (same N); segs[0].y = silu(g) * u and
 * segs[1].y is unused. Requires K % 128 == 0. Any M >= 1. */
int btf_hip_launch_gemv(const btf_gemv_seg* segs, int nseg, int K, int M, const btf_q8act* a, int mode,
                        btf_stream_t stream);

/* Replaces btf::cuda::launch_embed (kernels.cuh:82-85): rows d_tok[0..M) of
 * the packed embedding table (codes [V][E/4], scales [V][E/128] in the T2
 * layout; device or mapped host memory) -> x [M][E] fp32, then the inverse
 * transform: inv NULL or inv->block == 0 for none, else a blockwise
 * normalised FWHT (x 1/sqrt(block)) and, if inv->signs is set, the signs.
 * E % 128 == 0. Token ids must lie in [0, V): as in the reference, V is not a
 * parameter and the ids are device data, so the launch cannot check them. */
int btf_hip_launch_embed(const uint8_t* codes, const uint16_t* scales, const int* d_tok, int M, int E,
                         const btf_hx* inv, float* x, btf_stream_t stream);

/* Replaces btf::cuda::argmax_part_bytes (kernels.cuh:89): scratch bytes
 * launch_argmax needs in `part`. */
int64_t btf_hip_argmax_part_bytes(int V);

/* Replaces btf::cuda::launch_argmax (kernels.cuh:87-90): greedy pick over
 * logits[0..V) (the smallest index on ties; NaN never wins) -> *d_tok_out.
 * part: btf_hip_argmax_part_bytes(V) bytes of device scratch, 8-byte
 * aligned. */
int btf_hip_launch_argmax(const float* logits, int V, void* part, int* d_tok_out, btf_stream_t stream);

/* No counterpart in the reference: launch_argmax without the `part`
 * workspace, for callers that cannot allocate (tight serving loops,
 * harnesses that forbid hipMalloc). Its scratch is a file-scope static
 * device array of 256 8-byte keys (2 KiB per GPU, held until the process
 * ends), enough for any V; the library takes its address per device in
 * btf_hip_kernels_init. Allocates nothing. Every call on a GPU shares that
 * GPU's scratch, so calls must be serialized on that GPU: two calls that may
 * overlap (on different streams, from several threads, or a captured graph
 * replayed while another call or replay runs) race and can return a wrong
 * token. Issue every call -- and replay every graph that holds one -- on one
 * stream. Same result as btf_hip_launch_argmax. */
int btf_hip_launch_argmax_noalloc(const float* logits, int V, int* d_tok_out, btf_stream_t stream);

/* Replaces btf::cuda::launch_pos_add (kernels.cuh:92): *d_pos += M. */
int btf_hip_launch_pos_add(int* d_pos, int M, btf_stream_t stream);

/* Message of the last failure on this thread ("" if none). */
const char* btf_hip_last_error(void);

/* ---- additions without a reference counterpart --------------------------- */

/* Test hook: runs the same GEMV kernels as btf_hip_launch_gemv (path chosen
 * the same way, or forced by btf_hip_gemv_set_policy) but writes the exact
 * integer sub-block accumulators I[m][n][s] = code.q - s[m][s] as int32
 * [M][N][K/32] instead of y. */
int btf_hip_gemv_i32_dump(const uint8_t* codes, int N, int K, int M, const btf_q8act* a, int32_t* I_out,
                          btf_stream_t stream);

/* launch_gemv with the Q8_0 quantizes of a GEMV chain fused in (the v_dot4
 * kernel, one launch per activation row; with Q8 rows in, a Q8 output and a
 * batch of 3..32 rows on the int8-MFMA path (btf_hip_gemv_set_policy), one
 * launch of the MFMA kernel with 32-row output tiles):
 *  - input: exactly one of `a` (Q8 rows, as launch_gemv) or `x` (fp32 rows
 *    [M][ldx], quantized inside the launch with launch_prep's arithmetic, no
 *    norm or transform; x 16-byte aligned, ldx >= K, ldx % 4 == 0);
 *  - out (optional): the Q8 of the output rows (segment 0's y after the
 *    add / swiglu), written as launch_prep would write them for the next
 *    GEMV (q [M][N], d and s [M][N/32]); one output segment, N % 32 == 0,
 *    K <= 20480 (swiglu K <= 10240).
 * The results (y, and the Q8 rows) are bit-identical to launch_prep +
 * launch_gemv on the same path (v_dot4 or MFMA) followed by launch_prep of
 * the output. No reference counterpart: the reference
 * decoder launches the quantize and the GEMV separately
 * (src/cuda/gpu_decoder.cu:411-418). */
int btf_hip_launch_gemv_ex(const btf_gemv_seg* segs, int nseg, int K, int M, const btf_q8act* a, const float* x,
                           int ldx, int mode, const btf_q8act* out, btf_stream_t stream);

/* launch_gemv on PTQ1_0 matrices read directly (1.75 bits per weight, no T2
 * repack): segs[i].codes points at N rows of K/128 PTQ1_0 blocks (28 bytes
 * each: 26 bytes of base-3 digits, fp16 scale; 4-byte aligned) and
 * segs[i].scales must be NULL. Modes, segments, y/ldy and the Q8 activation
 * as in launch_gemv; K <= 32768. The outputs are bit-identical to
 * launch_gemv (v_dot4 path) on the repacked matrices. The reference plans
 * this kernel (docs/kernel-design.md:53; block decode src/types.cpp:86-111)
 * without building it. */
int btf_hip_launch_gemv_ptq1_0(const btf_gemv_seg* segs, int nseg, int K, int M, const btf_q8act* a, int mode,
                               btf_stream_t stream);

/* GEMV path policy: batches of M >= mfma_min_m rows run on the int8-MFMA
 * kernels, smaller ones on the v_dot4 kernel (default 3; K > 32768 always
 * takes the MFMA kernel). 0 restores the default.
 * Process-global; for tests and benchmarks. Returns the previous value. */
int btf_hip_gemv_set_policy(int mfma_min_m);

/* Measurement hook, no reference counterpart: a plain streaming read of
 * `bytes` of device memory at src (16-byte words, non-temporal loads as the
 * GEMV kernels read their weights), the practical HBM read ceiling the GEMV
 * figures are read against. The words are folded and *sink is written only
 * if the fold equals `never`. src 16-byte aligned, bytes % 16 == 0. */
int btf_hip_stream_read(const void* src, uint64_t bytes, uint32_t never, uint32_t* sink, btf_stream_t stream);

/* Seeded synthetic PTQ1_0 blocks (the benchmark's weight generator): blocks
 * [first_block, first_block + nblocks) of matrix `mat`, trits i.i.d. with
 * P(-1,0,+1) = (0.3,0.4,0.3) and fp16 scales RNE(U[0.01,0.05]). dst is
 * device memory [nblocks][28]. */
int btf_hip_gen_ptq1_0(uint64_t seed, uint64_t mat, int64_t first_block, int64_t nblocks, uint8_t* dst,
                       btf_stream_t stream);

/* ---- decode-step program: a chain of GEMVs in one launch ----------------
 * No counterpart in the reference's launch API: it replaces the reference
 * decoder's per-step graph of launches (src/cuda/gpu_decoder.cu:452-486) for
 * the GEMV chain. A program has vector slots and GEMV ops in order; each op
 * reads the first K values of its input vector, quantizes them (Q8_0, as
 * launch_prep without norm or transform) and writes its output vector
 * (STORE: y = W q; ADD: y += W q; SWIGLU: y = silu(W_g q) * (W_u q)), all
 * with the same arithmetic as btf_hip_launch_gemv. Vectors read before any
 * op writes them take their values from `data` at launch; the final value of
 * a vector (the result of the last op that writes it) is written to its
 * `data` when that is non-NULL. Vectors must not overlap in memory.
 * Creation allocates the program's device buffers and needs every workgroup
 * of the launch co-resident (one per CU); launches allocate nothing. One
 * launch at a time per program (launches on one stream serialise). */
typedef struct btf_step_vec {
  int n;       /* length (multiple of 32 when it is quantized) */
  float* data; /* device fp32 [n], or NULL for a vector internal to the step */
} btf_step_vec;
typedef struct btf_step_gemv {
  int mode; /* BTF_GEMV_STORE / ADD / SWIGLU */
  int K;    /* input width, multiple of 128, <= 20480 */
  int N;    /* output rows == length of the output vector */
  const uint8_t* codes;      /* [N][K/4]   (swiglu: gate) */
  const uint16_t* scales;    /* [N][K/128] */
  const uint8_t* up_codes;   /* swiglu: up matrix, else NULL */
  const uint16_t* up_scales;
  int in_vec, out_vec; /* vector slot indices (must differ) */
} btf_step_gemv;
typedef void* btf_step_t;
int btf_hip_step_create(const btf_step_vec* vecs, int nvec, const btf_step_gemv* ops, int nops, btf_step_t* out);
/* One cooperative launch running every op of the program. */
int btf_hip_step_launch(btf_step_t prog, btf_stream_t stream);
/* Synchronous read of the program's device error flag (0 = ok; 1 = a launch
 * timed out waiting for data, its outputs are invalid), then clears it. Call
 * after the launch's stream has been synchronised. */
int btf_hip_step_error(btf_step_t prog, int* error);
int btf_hip_step_destroy(btf_step_t prog);
/* Test hook: bound on the number of polls of every wait in the program's
 * later launches (0 restores the default, about one second). A tiny bound
 * makes a launch give up waiting and set the error flag instead of hanging. */
int btf_hip_step_set_spin_limit(btf_step_t prog, uint32_t polls);
/* Test hook: the number of the program's ops that keep a write-after-read
 * wait (an op overwriting a buffer version that a workgroup may still have to
 * read, where the data flow does not already order every read before it). */
int btf_hip_step_guards(btf_step_t prog, int* guards);

/* A whole batch-1 decode step in one launch: the step program with the ops
 * either side of the GEMV chain and each GEMV's full input prep. It replaces
 * the reference decoder's per-token graph (src/cuda/gpu_decoder.cu:401-421,
 * 452-486: launch_embed, then per GEMV launch_prep + launch_gemv, then
 * launch_argmax and launch_pos_add) for the parts of the step on this path.
 *  - BTF_STEP_GEMV: `gemv` as in btf_hip_step_create, its input first put
 *    through launch_prep's pipeline (src/cuda/kernels.cuh:40-43): RMSNorm *
 *    normw (NULL: none, eps its epsilon), then the transform hx (block 0:
 *    none; a power of two <= 1024; perm_hd * perm_nk * perm_rep == K and
 *    perm_hd % 64 == 0 when perm_rep > 1; signs NULL or [K]), then Q8_0.
 *    With a norm or transform the input vector's length must equal K.
 *    Bit-identical to launch_prep + launch_gemv.
 *  - BTF_STEP_EMBED: vector `vec` (length E, a multiple of 1024) = row
 *    *d_tok of the packed table (table_codes [V][E/4], table_scales
 *    [V][E/128], device or mapped host memory) with the inverse transform hx
 *    (launch_embed, src/cuda/kernels.cuh:82-85). Embed ops come before every
 *    GEMV. d_tok is read when the launch starts.
 *  - BTF_STEP_ARGMAX: *d_tok_out = the greedy pick over vector `vec`
 *    (launch_argmax: the smallest index on ties, a NaN never wins), then, if
 *    d_pos is set, *d_pos += 1 (launch_pos_add). It must directly follow the
 *    GEMV that writes `vec`; at most one per program. d_tok_out may be the
 *    embed op's d_tok: each launch then decodes the token the previous one
 *    picked.
 * Unused fields are ignored. */
enum { BTF_STEP_GEMV = 0, BTF_STEP_EMBED = 1, BTF_STEP_ARGMAX = 2 };
typedef struct btf_step_op {
  int kind;
  btf_step_gemv gemv;           /* GEMV */
  const float* normw;           /* GEMV: RMSNorm weight [K] or NULL */
  float eps;                    /* GEMV: RMSNorm epsilon */
  btf_hx hx;                    /* GEMV: input transform; EMBED: inverse transform */
  int vec;                      /* EMBED: output vector; ARGMAX: logits vector */
  const uint8_t* table_codes;   /* EMBED */
  const uint16_t* table_scales; /* EMBED */
  const int* d_tok;             /* EMBED: token id (device) */
  int* d_tok_out;               /* ARGMAX: picked token (device) */
  int* d_pos;                   /* ARGMAX: position counter (device) or NULL */
} btf_step_op;
int btf_hip_step_create_ops(const btf_step_vec* vecs, int nvec, const btf_step_op* ops, int nops, btf_step_t* out);

/* Test hook, host only (no device is touched): builds the program of
 * btf_hip_step_create_ops for a grid of G workgroups (1..256), its own
 * buffers in host memory, and replays every global store a launch of it
 * makes -- each workgroup's published units (fp32 and Q8 LL words, block
 * sums of squares, plain outputs), progress words, pick keys, the token,
 * the position and the control block -- with the kernel's own placement and
 * address functions, checking that each lies inside a buffer the program
 * owns or was given (a vector's data, d_tok_out, d_pos). No counterpart in
 * the reference; it plays the part of its build-time kernel resource check
 * (cmake/check_kernel_resources.cmake:15-61) for the step kernel's stores. */
typedef struct btf_step_audit {
  int64_t stores;           /* stores checked */
  int64_t outside;          /* stores outside every such buffer (0: none) */
  int ops;                  /* device ops (prologue + embeddings + GEMVs) */
  int guards;               /* as btf_hip_step_guards */
  int full;                 /* 1: the kernel instance with preps, embedding and pick */
  char first_outside[160];  /* the first stray store, described */
} btf_step_audit;
int btf_hip_step_audit(const btf_step_vec* vecs, int nvec, const btf_step_op* ops, int nops, int G,
                       btf_step_audit* out);

/* ---- load path: GGUF reader -> pinned double-buffered staging -> repack --
 * The reference decoder reads its model with bd::Gguf
 * (ref/bonsai-decoder/include/bd/gguf.hpp:49-85, src/gguf.cpp:73-147),
 * uploads each PTQ1_0 matrix with GpuDecoder::upload_mat / upload
 * (src/cuda/gpu_decoder.cu:284-393: slices of rows through two pinned
 * staging slots, launch_repack on each) and sizes the resident layout with
 * plan_memory (src/repack.cpp:142-204). These entry points provide the same
 * three steps; a decoder keeps its own model binding on top.
 *
 * The reader memory-maps the file read-only and parses GGUF v2/v3 in one
 * pass, with the reference's checks (a bad or truncated file fails with
 * BTF_ERR_ARGS and the reason). Tensor data stay in the mapping: `data`
 * points into it (NULL for a tensor past the end of a header-only read) and
 * stays valid until btf_hip_gguf_close. Strings and names are owned by the
 * reader. ne[] is ggml order: ne[0] is contiguous (for a matrix, K), unused
 * dimensions are 1. Numeric metadata keep an integer and a double form
 * (integers convert exactly, floats truncate to the integer form, booleans
 * are 0 or 1); a key present twice resolves to its last entry. */
typedef void* btf_gguf_t;
typedef struct btf_gguf_header {
  uint32_t version;     /* 2 or 3 */
  uint64_t alignment;   /* general.alignment, default 32 */
  uint64_t data_offset; /* start of the data section in the file */
  uint64_t file_bytes;
  int64_t n_tensors, n_kv;
} btf_gguf_header;
typedef struct btf_gguf_tensor {
  const char* name;
  int n_dims;
  int64_t ne[4];
  uint32_t type;   /* ggml type id (PTQ1_0 = 143, F32 = 0, F16 = 1, ...) */
  uint64_t offset; /* in the data section */
  uint64_t bytes;
  const uint8_t* data;
} btf_gguf_tensor;
typedef struct btf_gguf_kv {
  const char* key; /* key_len bytes (may hold NUL bytes) */
  uint64_t key_len;
  uint32_t type;     /* GGUF value type: 0 U8 ... 8 STRING, 9 ARRAY, 10 U64, 11 I64, 12 F64 */
  uint32_t arr_type; /* element type of an array */
  uint64_t len;      /* elements (1 for a scalar) */
} btf_gguf_kv;
int btf_hip_gguf_open(const char* path, int header_only, btf_gguf_t* out);
int btf_hip_gguf_close(btf_gguf_t g);
int btf_hip_gguf_info(btf_gguf_t g, btf_gguf_header* out);
int btf_hip_gguf_tensor(btf_gguf_t g, int64_t index, btf_gguf_tensor* out);
int64_t btf_hip_gguf_find_tensor(btf_gguf_t g, const char* name); /* -1: absent */
int btf_hip_gguf_kv(btf_gguf_t g, int64_t index, btf_gguf_kv* out);
int64_t btf_hip_gguf_find_kv(btf_gguf_t g, const char* key);      /* -1: absent */
/* Element `elem` (0 for a scalar) of a numeric value / of a string value. */
int btf_hip_gguf_kv_num(btf_gguf_t g, int64_t index, uint64_t elem, int64_t* i, double* f);
int btf_hip_gguf_kv_str(btf_gguf_t g, int64_t index, uint64_t elem, const char** s, uint64_t* len);
/* Bytes of n elements of a ggml type (-1: unknown type or n not whole
 * blocks), as bd::row_bytes (ref/bonsai-decoder/src/types.cpp:36-40). */
int64_t btf_hip_ggml_row_bytes(uint32_t type, int64_t n);

/* Resident bytes of the file's PTQ1_0 matrices (2-D tensors of type 143,
 * K = ne[0], N = ne[1]) in the T2 layout, and the staging of a load with
 * slots of staging_bytes. arena_bytes rounds every codes and scales array
 * up to 256 B (one allocation holding them all). */
typedef struct btf_pack_plan {
  int64_t n_matrices;
  uint64_t codes_bytes, scales_bytes, arena_bytes;
  uint64_t source_bytes; /* their PTQ1_0 bytes in the file */
  uint64_t other_bytes;  /* every other tensor's bytes */
  uint64_t staging_host_bytes, staging_device_bytes; /* 2 slots each, freed after the load */
} btf_pack_plan;
int btf_hip_gguf_plan(btf_gguf_t g, uint64_t staging_bytes, btf_pack_plan* out);

/* Staged upload of PTQ1_0 rows src [N][K/128][28] (host memory: a GGUF
 * mapping, or any buffer) into the T2 layout codes [N][K/4], scales
 * [N][K/128] (device). Slices of whole rows go through two pinned host slots
 * of staging_bytes in turn: the host copies a slice into a slot (on up to 8
 * threads) once the slot's previous slice is done, the copy engine moves it
 * into a device slot
 * and the repack kernel writes the packed rows, all on `stream`, so the host
 * copy of one slice overlaps the device's work on the other. Uploads return
 * once their last slice is queued (src may then be reused); finish waits for
 * every queued slice. A loader belongs to the device current at creation
 * (btf_hip_kernels_init must have run for it) and allocates its slots once;
 * uploads allocate nothing. */
typedef void* btf_loader_t;
int btf_hip_loader_create(uint64_t staging_bytes, btf_loader_t* out);
int btf_hip_loader_upload_ptq1_0(btf_loader_t L, const uint8_t* src, int64_t N, int64_t K, uint8_t* codes,
                                 uint16_t* scales, btf_stream_t stream);
int btf_hip_loader_finish(btf_loader_t L, uint64_t* source_bytes); /* total PTQ1_0 bytes uploaded */
int btf_hip_loader_destroy(btf_loader_t L);

/* Device description for reports. name must hold name_len bytes. */
typedef struct btf_device_info {
  int cu_count;
  int lds_bytes_per_block;
  int max_clock_khz;
  int mem_clock_khz;
  int mem_bus_width_bits;
  int l2_bytes;
  int wavefront_size;
  int arch_major, arch_minor;
  int64_t total_mem_bytes;
  char name[256];
  char gcn_arch[64];
} btf_device_info;
int btf_hip_device_info(int device, btf_device_info* out);

/* Minimal runtime helpers so host code never includes HIP headers. */
int btf_hip_device_count(int* n);
int btf_hip_set_device(int device);
int btf_hip_malloc(void** p, size_t bytes);
int btf_hip_free(void* p);
int btf_hip_host_alloc_mapped(void** host, void** dev, size_t bytes); /* pinned, mapped */
int btf_hip_host_free(void* host);
int btf_hip_memcpy_h2d(void* dst, const void* src, size_t bytes);
int btf_hip_memcpy_d2h(void* dst, const void* src, size_t bytes);
int btf_hip_memset(void* dst, int value, size_t bytes);
int btf_hip_device_synchronize(void);
int btf_hip_stream_create(btf_stream_t* s);
int btf_hip_stream_destroy(btf_stream_t s);
int btf_hip_stream_synchronize(btf_stream_t s);
typedef void* btf_event_t;
int btf_hip_event_create(btf_event_t* e);
int btf_hip_event_destroy(btf_event_t e);
int btf_hip_event_record(btf_event_t e, btf_stream_t s);
int btf_hip_event_elapsed_ms(float* ms, btf_event_t start, btf_event_t stop);
typedef void* btf_graph_exec_t;
int btf_hip_graph_begin(btf_stream_t s);                      /* starts stream capture */
int btf_hip_graph_end(btf_stream_t s, btf_graph_exec_t* out); /* ends capture, instantiates */
int btf_hip_graph_launch(btf_graph_exec_t g, btf_stream_t s);
int btf_hip_graph_destroy(btf_graph_exec_t g);

#ifdef __cplusplus
}
#endif
#endif
