// step.hip -- a whole batch-1 decode step's chain of ternary GEMVs in ONE
// persistent kernel launch (gfx950).
//
// Why: in a stream or hipGraph a dependent kernel costs ~2 us of launch plus
// its ramp and drain on MI355X, while a 27B-layer GEMV moves 7-47 MB (1-7 us
// at HBM speed). The reference decoder captures a step
// as one CUDA graph of ~514 launches (src/cuda/gpu_decoder.cu:452-486); here
// the same GEMV chain (with the Q8 quantize of every GEMV input) is one launch.
//
// Execution model (one workgroup per CU, all co-resident: cooperative launch):
//  * Ops run in program order. Output rows of every op are owned in 32-row
//    units (one Q8 block of the output), spread round-robin over workgroups
//    with a rotation chosen op by op to keep each workgroup's total work over
//    the step balanced.
//  * Cross-workgroup data moves through "LL" words: 8 bytes = 4 data bytes +
//    a 32-bit version tag, written and read with agent-scope relaxed atomics
//    (write-through / read-through the per-XCD L2s). A consumer polls the
//    words it needs until every tag equals the producing op's tag, so the data
//    carries its own readiness: no fences, no grid barriers. Producers write
//    (a) the fp32 outputs as LL words (read by later add-mode ops) and (b) the
//    Q8_0 of each output unit (8 q words + d + s = 10 LL words per 32 values),
//    computed in the producer's epilogue, bit-identical to the q8 kernel.
//  * Inside a workgroup: 10 compute waves stream the weights. Each keeps
//    kRing items (16-byte code chunks per lane) in flight in registers, and
//    the refills of an op's last batch load the NEXT op's first items, so
//    the ring never drains between ops. Items run unit by unit; each compute
//    wave fetches (polls) only the input slices its own items read, so it
//    starts as soon as those are published. The 2 I/O waves publish each unit
//    as soon as the compute waves' per-unit counts say it is complete, and
//    fetch the input of an "early" op (one whose producers are two or more
//    ops back) while the previous op computes. One s_barrier per op (without
//    a memory fence: LDS only) separates ops, so the weight stream stays in
//    flight across it.
//  * Op descriptors are staged in LDS at launch.
//  * The dot products, the 16-lane DPP reduction and the fixed-order sum over
//    1024-column slices are those of gemv_dot4_kernel, so outputs are
//    bit-identical to launching the same ops one by one.
//  * Every poll is bounded; a timeout (or the abort flag set by another
//    workgroup) records an error and lets every wave run to completion.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <type_traits>
#include <vector>

#include "../../include/btf/hip_abi.h"
#include "common.h"
#include "slice.h"

// Floating-point expressions are evaluated as written (no fused multiply-add
// unless fmaf is spelled out), so the per-slice row sums have one defined
// rounding order, shared by every kernel that produces them.
#pragma clang fp contract(off)

namespace btfhip {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Compute waves per workgroup, per kernel instance: three waves per SIMD
// (the full kernel needs 164 VGPRs). The plain instance also fits 14 compute
// waves at 128 VGPRs (four per SIMD, 40 % more weight bytes in flight), but
// the step then takes 5 % longer: the I/O waves, which publish each op's
// units on the chain's critical path, share their SIMDs with three compute
// waves instead of two.
constexpr int kCWFull = 10, kCWPlain = 10;
constexpr int kIW = 2;  // I/O waves
template <bool kFull>
constexpr int cw_of() {
  return kFull ? kCWFull : kCWPlain;
}
template <bool kFull>
constexpr int threads_of() {
  return 64 * (cw_of<kFull>() + kIW);
}
constexpr int kRing = 8;                    // weight items (16 B per lane) in flight per compute wave
constexpr int kMaxK = 20480;                // widest GEMV input
constexpr int kMaxPart = 8192;              // partial sums per op per workgroup
constexpr int kMaxOps = 300;                // ops per program (descriptors live in LDS)
constexpr int kMaxOld = 1024;               // rows per workgroup of an add-mode op (the LDS carry)
constexpr int kMaxUnits = 256;              // units of one op per workgroup (kMaxPart / 32)
constexpr int kWordsPerBlock = 10;          // LL words per 32-value Q8 block
constexpr int kSlots = 3;                   // LL buffers of each kind per vector (versions in turn)
constexpr uint32_t kSpinMax = 1u << 20;     // poll bound (each poll is a memory round trip: ~1 s)

// 176 bytes (a multiple of 16: copied into LDS in 16-byte words).
struct OpDev {
  int kind;  // 0 = quantize a user vector (prologue), 1 = GEMV, 2 = embedding lookup (prologue)
  int mode;
  int K, N;
  int cpr;
  int units, rot, qpu_log2;  // units (32 rows; embedding: 1024 values), unit rotation, log2 row quads per unit
  int next;                  // index of the next GEMV op (nops: none)
  int war_op;                // >= 0: wait until every workgroup has fetched that op's input
                             // (the last reader of the version this op overwrites)
  int prep;                  // >= 0: index of the op's PrepDev (GEMV: its input's norm / transform,
                             // read from the fp32 words; embedding: the inverse transform)
  uint32_t in_tag;           // relative tag of the input's producer
  uint32_t old_tag;          // add mode: relative tag of the output's previous version
  uint32_t my_tag;
  uint8_t early;        // 1: the I/O waves fetch this op's input during the previous op
  uint8_t carry_in;     // 1: add-mode old values come from the previous op's epilogue (LDS carry)
  uint8_t carry_out;    // 1: the epilogue keeps its outputs in the LDS carry for the next op
  uint8_t count_reads;  // 1: record the workgroup's progress after the op (a later write-after-read guard waits for it)
  uint8_t out_sq;       // 1: also publish each 32-value block's sum of squares (a later op normalizes it)
  uint8_t argmax;       // 1: the program's greedy pick reads this op's output
  uint8_t prep_flags;   // with a prep: bit 0 RMSNorm, bit 1 the tiled -> grouped gather
  uint8_t pad1;
  const uint8_t* codes;     // GEMV: weights (swiglu: gate); embedding: table codes
  const uint16_t* scales;   // embedding: table scales
  const uint8_t* up_codes;
  const uint16_t* up_scales;
  const uint64_t* in_ll;    // LL words of the input: Q8 words, or with a prep its fp32 words
  float* out_plain;         // user output (nullable)
  uint64_t* out_f32;        // LL fp32 of the output vector [N], then 2 LL words (low, high half of
                            // a double) per 32-value block: the block sums of squares (nullable)
  uint64_t* out_q8;         // LL Q8 of the output vector (nullable)
  const uint64_t* old_f32;  // add mode: previous value of the output vector
  const void* src;          // quantize: user vector (float); embedding: token id (int)
  // the prep's fields (copies of its PrepDev, here in LDS with the rest)
  const float* normw;       // RMSNorm weights (NULL: none)
  const float* signs;       // transform signs (NULL: none)
  float eps, hs;            // RMSNorm epsilon; 1 / sqrtf(block)
  int block;                // transform block (0: none)
  int pad2;
};
static_assert(sizeof(OpDev) == 176, "descriptor layout");

// An op's activation prep: launch_prep's pipeline for a GEMV input, or the
// inverse transform of an embedding lookup (normw = NULL). The host copies
// every field but `runs` into the op's descriptor (LDS); the kernel reads
// only the gather's run table from here (global memory, scalar loads).
struct PrepDev {
  const float* normw;  // NULL: no RMSNorm
  const float* signs;  // NULL: none
  const int* runs;     // the tiled -> grouped gather: first source of each 64-value run (NULL: none)
  float eps;
  float hs;            // 1 / sqrtf(block)
  int block;           // 0: no transform
  int pad;
};

// The program's greedy pick: every workgroup publishes the largest key of
// the rows it produced of the picked vector (2 LL words: the key's low and
// high halves) into parts[2 wg ..]; workgroup 0 reduces them at the end.
struct HeadDev {
  int present;
  uint32_t tag;    // relative tag of the op that publishes the parts
  int* tok_out;
  int* pos;        // += 1 after the pick (nullable)
  uint64_t* parts; // [G][2]
};

struct Ctl {
  uint32_t epoch;
  uint32_t error;
  uint32_t done;
  uint32_t spin_max;  // poll bound of every wait; 0 = kSpinMax
};

// Through global (not flat) instructions: flat ones also count in lgkmcnt,
// so every LDS barrier would wait for the LL round trips in flight.
typedef __attribute__((address_space(1))) uint64_t gu64;
__device__ __forceinline__ uint64_t ll_load(const uint64_t* p) {
  return __hip_atomic_load((const gu64*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_store(uint64_t* p, uint64_t v) {
  __hip_atomic_store((gu64*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ctl_load(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Workgroup barrier for LDS hand-offs only: waits for this wave's LDS ops,
// never for its global loads (the weight stream stays in flight).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// A compute wave's share of a GEMV op (its OpWork, below), computed by an
// I/O wave one op ahead with one lane per compute wave and staged here: the
// ten compute waves would otherwise each run the same scalar code at every
// op boundary, on the one scalar issue slot of each SIMD.
struct WorkRec {
  int t0, n, P, uq;  // uq = u0 | s0 << 8 | q0 << 16
};
struct OpRec {
  int first, R, next, sq;  // sq = S | qlog << 8 | il << 16
};
constexpr int kRecSlots = 3;  // records of ops i, i + 1, i + 2 (slot = op index % 3)

template <bool kFull>
struct Lds {
  static constexpr bool kPrepped = kFull;
  static constexpr int kCW = cw_of<kFull>();
  OpDev opd[kMaxOps];        // the program
  // An op's Q8 input (by op parity) as the image of its LL words: per
  // 32-value block 8 words of q bytes, d (f32 bits), s.
  uint32_t act[2][kMaxK / 32 * kWordsPerBlock];
  float part[kMaxPart];       // [1024-column slice][local row]
  float carry[kMaxOld];       // outputs of the workgroup's rows kept for the next (add-mode) op
  uint32_t ucnt[kCW][kMaxUnits];  // per compute wave: items of each local unit of the current op it has done
  uint32_t early_seq[kIW];    // per I/O wave: op index + 1 of the last input it fetched early
  uint64_t argk[kIW];         // per I/O wave: the largest pick key of the rows it published
  uint32_t sready[2][kMaxK / kSliceVals];  // prep inputs: op index + 1 once slice sl of buffer ob is in LDS
  float stg[kFull ? kCW : 1][256];  // per compute wave: the prep's Q8 transposition
  WorkRec wrec[kRecSlots][kCW];
  OpRec orec[kRecSlots];
  const PrepDev* preps;  // kernel arguments read where needed (not held in
  const HeadDev* head;   // scalar registers through the kernel)
  uint32_t epoch;
  uint32_t abort_;
  uint32_t spin_max;
};

template <class LT>
__device__ __forceinline__ bool aborted(LT& L) {
  return __hip_atomic_load(&L.abort_, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0;
}
// Has another workgroup of this launch failed?
template <class LT>
__device__ __forceinline__ bool grid_failed(const Ctl* ctl, const LT& L) {
  return __hip_atomic_load(&ctl->error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == L.epoch;
}
// The error word holds the epoch of the failing launch, so a failure that the
// host has not cleared yet does not abort later launches.
template <class LT>
__device__ __forceinline__ void set_abort(LT& L, Ctl* ctl) {
  __hip_atomic_store(&ctl->error, L.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(&L.abort_, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Address-space views of pointers. A pointer staged in LDS comes back
// generic, and a load through a generic pointer is a flat instruction, which
// counts in both vmcnt and lgkmcnt: a wait for its result waits for every
// global load issued before it (the weight stream in flight). Descriptors are
// read through the constant space (scalar loads), data through the global
// space.
template <class T>
using cptr = const __attribute__((address_space(4))) T*;
template <class T>
using gptr = const __attribute__((address_space(1))) T*;
template <class T>
__device__ __forceinline__ cptr<T> as_const(const T* p) {
  return (cptr<T>)p;
}
template <class T>
__device__ __forceinline__ gptr<T> as_global(const T* p) {
  return (gptr<T>)p;
}

__device__ __forceinline__ int sgpr(int v) { return __builtin_amdgcn_readfirstlane(v); }
// Is this lane 0 of its wave? Re-derived at each use (the empty asm hides
// that the lane index never changes), so the compiler does not keep a lane
// mask in scalar registers from the kernel's start.
__device__ __forceinline__ bool first_lane(int lane) {
  int t = lane & 63;
  asm volatile("" : "+v"(t));
  return t == 0;
}
template <class T>
__device__ __forceinline__ T* sgpr_ptr(T* p) {
  const uint64_t u = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

// Unit placement and the word offsets of every global store the kernel
// makes. Host code uses the same functions (btf_hip_step_audit replays the
// stores of a program over every workgroup and checks each against the
// buffers the program owns or was given).
// First workgroup-local unit of an op: units u with u % G == (wg - rot) mod G.
__host__ __device__ __forceinline__ int first_unit(int rot, int wg, int G) {
  const int f = wg - rot;
  return f < 0 ? f + G : f;
}
__host__ __device__ __forceinline__ int units_of(int units, int first, int G) {
  return first < units ? (units - 1 - first) / G + 1 : 0;
}
// Output row (fp32 word) of value j of a 32-value unit.
__host__ __device__ __forceinline__ int unit_row(int unit, int j) { return unit * 32 + j; }
// First Q8 LL word of 32-value block `blk` (8 q words, d, s).
__host__ __device__ __forceinline__ size_t q8_block_word(int blk) { return (size_t)blk * kWordsPerBlock; }
// LL words of block `blk`'s sum of squares (low, high half of the double):
// after the vector's N fp32 words.
__host__ __device__ __forceinline__ size_t sq_word(int N, int blk) { return (size_t)N + 2 * (size_t)blk; }
// First value of lane `lane`'s 16 of 1024-value unit `unit` (an embedding's output).
__host__ __device__ __forceinline__ int slice_col(int unit, int lane) { return unit * kSliceVals + 16 * lane; }
// A workgroup's greedy-pick key: 2 LL words.
__host__ __device__ __forceinline__ size_t pick_word(int wg) { return 2 * (size_t)wg; }

// ---------------------------------------------------------------- input fetch
template <class LT>
__device__ __forceinline__ bool poll_step(uint32_t& spins, LT& L, Ctl* ctl) {
  if (aborted(L)) return false;
  if (++spins > L.spin_max || ((spins & 255) == 0 && grid_failed(ctl, L))) {
    set_abort(L, ctl);
    return false;
  }
  return true;  // (no sleep: a poll round is paced by its own loads' round trip)
}

// Fetch LL words [a0, a1) and [b0, b1) of an op's input (its Q8 words, tag = the input
// producer's) into LDS buffer `ob`, by the 64 lanes of one compute wave in
// rounds of kFB words per lane, polling until every tag matches. A slice
// whose items two waves share is fetched by both: the same values land twice.
constexpr int kFB = 10;
template <class LT>
__device__ __forceinline__ void fetch_words(const OpDev& op, LT& L, int lane, Ctl* ctl, uint32_t base_tag, int ob,
                                            int a0, int a1, int b0, int b1) {
  const uint64_t* in = sgpr_ptr(op.in_ll);
  const uint32_t tin = base_tag + sgpr(op.in_tag);
  const int na = a1 - a0, nw = na + (b1 - b0);  // word k < nw: a0 + k, or b0 + k - na
  for (int k0 = 0; k0 < nw; k0 += kFB * 64) {
    uint64_t v[kFB];
    int at[kFB];
#pragma unroll
    for (int b = 0; b < kFB; ++b) {
      const int k = k0 + b * 64 + lane;
      at[b] = k < nw ? (k < na ? a0 + k : b0 + k - na) : -1;
      v[b] = at[b] >= 0 ? ll_load(in + at[b]) : ((uint64_t)tin << 32);
    }
    uint32_t spins = 0;
    for (;;) {
      uint32_t pending = 0;
#pragma unroll
      for (int b = 0; b < kFB; ++b) pending |= ((uint32_t)(v[b] >> 32) != tin) ? (1u << b) : 0u;
      if (__builtin_amdgcn_ballot_w64(pending != 0) == 0) break;
      if (!poll_step(spins, L, ctl)) break;
#pragma unroll
      for (int b = 0; b < kFB; ++b)
        if (pending & (1u << b)) v[b] = ll_load(in + at[b]);
    }
#pragma unroll
    for (int b = 0; b < kFB; ++b)
      if (at[b] >= 0) L.act[ob][at[b]] = (uint32_t)v[b];
  }
}

// The input fetch of an "early" op by the I/O waves (kIW waves, one round):
// its producers all come before the previous op, so the loads are issued
// while the previous op computes and finished (poll what was stale, write
// LDS) once that op's partial sums are in; each I/O wave then records the op
// in L.early_seq, which the compute waves wait for instead of fetching.
constexpr int kIL = 64 * kIW;
constexpr int kEIn = 13;  // input words per lane: K <= 5324
struct EarlyFetch {
  uint64_t v[kEIn];
};
__device__ __forceinline__ void early_issue(const OpDev& op, int lid, uint32_t base_tag, EarlyFetch& f) {
  const uint64_t* in = sgpr_ptr(op.in_ll);
  const uint32_t tin = base_tag + sgpr(op.in_tag);
  const int nin = (sgpr(op.K) / 32) * kWordsPerBlock;
#pragma unroll
  for (int b = 0; b < kEIn; ++b) {
    const int idx = lid + b * kIL;
    f.v[b] = idx < nin ? ll_load(in + idx) : ((uint64_t)tin << 32);
  }
}
// Polls what was stale, writes the input into LDS buffer `ob`, then this
// wave's L.early_seq = seq. Returns false (and writes nothing) if `wait` is
// false and some word of this wave is not yet published.
template <class LT>
__device__ __forceinline__ bool early_finish(const OpDev& op, int lid, uint32_t base_tag, EarlyFetch& f, LT& L, int ob,
                                             Ctl* ctl, bool wait, uint32_t seq) {
  const uint64_t* in = sgpr_ptr(op.in_ll);
  const uint32_t tin = base_tag + sgpr(op.in_tag);
  const int nin = (sgpr(op.K) / 32) * kWordsPerBlock;
  uint32_t spins = 0;
  for (;;) {
    uint32_t pending = 0;
#pragma unroll
    for (int b = 0; b < kEIn; ++b) pending |= ((uint32_t)(f.v[b] >> 32) != tin) ? (1u << b) : 0u;
    if (__builtin_amdgcn_ballot_w64(pending != 0) == 0) break;
    if (!wait) return false;
    if (!poll_step(spins, L, ctl)) break;
    for (int b = 0; b < kEIn; ++b) {
      const int idx = lid + b * kIL;
      if ((pending & (1u << b)) && idx < nin) f.v[b] = ll_load(in + idx);
    }
  }
#pragma unroll
  for (int b = 0; b < kEIn; ++b) {
    const int idx = lid + b * kIL;
    if (idx < nin) L.act[ob][idx] = (uint32_t)f.v[b];
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the input words are in LDS
  // (every lane of the wave stores the same value)
  __hip_atomic_store(&L.early_seq[lid >> 6], seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  return true;
}

// ---------------------------------------------------------------- prep input
// With a prep (norm and/or transform), a GEMV reads its input's fp32 LL words
// and runs launch_prep's pipeline itself: each compute wave, for every
// 1024-value slice its items read, gathers the slice (through the perm),
// normalizes it, applies the signs and the FWHT in registers (slice.h) and
// writes the slice's Q8 into the LDS image, where the plain fetch would have
// copied the producer's Q8 words. Bit-identical to launch_prep on the same
// fp32 vector: the same per-slice arithmetic, and the RMSNorm scale from the
// producers' block sums of squares summed in prep_slices_kernel's order.
struct PrepRegs {  // an op's prep fields in scalar registers
  const float* normw;
  const float* signs;
  float eps, hs;
  int block;
};
__device__ __forceinline__ PrepRegs prep_regs(const OpDev& op) {  // (from the LDS copy of the op)
  PrepRegs r;
  r.normw = sgpr_ptr(op.normw);
  r.signs = sgpr_ptr(op.signs);
  r.eps = __int_as_float(sgpr(__float_as_int(op.eps)));
  r.hs = __int_as_float(sgpr(__float_as_int(op.hs)));
  r.block = sgpr(op.block);
  return r;
}

constexpr int kSQ = 4;  // block sums of squares per lane per poll round
// The RMSNorm scale of a GEMV's input: lane l adds the producers' block sums
// l, l + 64, ... in order, then the wave sum (norm_scale_of). `again` runs
// in every poll round before the stale words are loaded again: the caller
// re-loads its own stale input words there, so they travel with the sums
// (a producer publishes a unit's values before its sum of squares), and
// once the sums are in, the values usually are too -- no further round trip.
template <class LT, class F>
__device__ __forceinline__ float prep_scale(const OpDev& op, const PrepRegs& pd, LT& L, int lane, Ctl* ctl,
                                            uint32_t base_tag, F&& again) {
  const int K = sgpr(op.K), nb = K >> 5;
  const uint64_t* sq = sgpr_ptr(op.in_ll) + K;
  const uint32_t tin = base_tag + sgpr(op.in_tag);
  double acc = 0.0;
  for (int r0 = 0; r0 < nb; r0 += kSQ * 64) {
    uint64_t lo[kSQ], hi[kSQ];
#pragma unroll
    for (int b = 0; b < kSQ; ++b) {
      const int i = r0 + b * 64 + lane;
      lo[b] = i < nb ? ll_load(sq + 2 * i) : ((uint64_t)tin << 32);
      hi[b] = i < nb ? ll_load(sq + 2 * i + 1) : ((uint64_t)tin << 32);
    }
    uint32_t spins = 0;
    for (;;) {
      uint32_t pending = 0;
#pragma unroll
      for (int b = 0; b < kSQ; ++b)
        pending |= ((uint32_t)(lo[b] >> 32) != tin || (uint32_t)(hi[b] >> 32) != tin) ? (1u << b) : 0u;
      if (__builtin_amdgcn_ballot_w64(pending != 0) == 0) break;
      if (!poll_step(spins, L, ctl)) break;
      again();
#pragma unroll
      for (int b = 0; b < kSQ; ++b)
        if (pending & (1u << b)) {
          const int i = r0 + b * 64 + lane;
          lo[b] = ll_load(sq + 2 * i);
          hi[b] = ll_load(sq + 2 * i + 1);
        }
    }
#pragma unroll
    for (int b = 0; b < kSQ; ++b)
      if (r0 + b * 64 + lane < nb)
        acc += __longlong_as_double((long long)(((uint64_t)(uint32_t)hi[b] << 32) | (uint32_t)lo[b]));
  }
  return norm_scale_of(acc, K, pd.eps);
}

// Slice sl of a prep GEMV's input into LDS buffer `ob` (Q8 image). The wave
// holds the slice strided (slice.h): lane l takes values sl * 1024 + l + 64 i,
// so every LL load instruction reads 64 consecutive words (512 contiguous
// bytes). The slice's loads, and those of its norm weights and signs, are
// all issued before the first wait: with `scale_due`, the wait for the
// RMSNorm scale (every producer of the vector) runs while they are in
// flight. After the transform, the Q8 runs in four rounds of 256 values:
// the round's four entries are transposed through the wave's 1 KB of LDS
// staging, so that lane l holds values 4 l .. 4 l + 3 of the round and each
// 32-value block is an aligned group of 8 lanes (q8_oct: one reduction per
// round instead of one per entry). With the perm, each 64-value run comes
// from 64 consecutive sources (the step program takes perm_hd % 64 == 0), so
// the gather costs one uniform source index per run, recomputed at each use
// (an empty asm keeps the compiler from holding 16 of them in registers).
template <bool PERM, class LT>
__device__ __forceinline__ void fetch_prep_slice(const OpDev& op, const PrepDev* preps, int pi, float& scale,
                                                 bool scale_due, LT& L, int wave, int lane, Ctl* ctl,
                                                 uint32_t base_tag, int ob, int sl) {
  // Each field of the prep is loaded (a scalar load) where it is used: the
  // pointer passes an empty asm before every use, so no field is held in
  // scalar registers across the polls.
  auto P = [&]() {
    cptr<PrepDev> p = as_const(preps) + pi;
    asm volatile("" : "+s"(p));
    return p;
  };
  const uint64_t* in = sgpr_ptr(op.in_ll);
  const int c = sl * kSliceVals;
  // word index of entry i of this lane: with the perm, run i's first source
  // from the program's table (a scalar load at each use), plus the lane
  auto src = [&](int i) {
    if constexpr (PERM)
      return as_const(P()->runs)[(c >> 6) + i] + lane;  // (no readfirstlane: the reload below is under a lane mask)
    else
      return c + 64 * i + lane;
  };
  uint64_t w[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) w[i] = ll_load(in + src(i));
  // one factor per entry loaded before the waits: the norm weight, or
  // without a norm the sign (with both, the signs are loaded after the wait:
  // registers are short)
  float pre[16];
  const PrepRegs pd = prep_regs(op);
  const gptr<float> normw = as_global(pd.normw);
  const gptr<float> signs = as_global(pd.block > 0 ? pd.signs : nullptr);
  if (normw) {
#pragma unroll
    for (int i = 0; i < 16; ++i) pre[i] = normw[src(i)];
  } else if (signs) {
#pragma unroll
    for (int i = 0; i < 16; ++i) pre[i] = signs[c + 64 * i + lane];
  }
  const uint32_t tin = base_tag + sgpr(op.in_tag);
  if (scale_due)
    scale = prep_scale(op, pd, L, lane, ctl, base_tag, [&]() {
#pragma unroll
      for (int i = 0; i < 16; ++i) w[i] = ll_load(in + src(i));  // (all of them: no mask to hold)
    });
  uint32_t spins = 0;
  for (;;) {
    uint32_t pending = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) pending |= ((uint32_t)(w[i] >> 32) != tin) ? (1u << i) : 0u;
    if (__builtin_amdgcn_ballot_w64(pending != 0) == 0) break;
    if (!poll_step(spins, L, ctl)) break;
    // (no unroll pragma: the compiler unrolls this loop by itself -- w[]
    // lives in registers, the resource test would see scratch otherwise --
    // and an explicit request only draws a warning for a peeled copy)
    for (int i = 0; i < 16; ++i)
      if (pending & (1u << i)) w[i] = ll_load(in + src(i));
  }
  float v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = __uint_as_float((uint32_t)w[i]);
  if (normw) {
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = (v[i] * scale) * pre[i];
    if (signs)
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] = v[i] * signs[c + 64 * i + lane];
  } else if (signs) {
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = v[i] * pre[i];
  }
  if (pd.block > 0) {
    slice_fwht_strided(v, lane, pd.block);
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = v[i] * pd.hs;
  }
  int lq = lane;
  asm volatile("" : "+v"(lq));  // lane tests formed here, not held from the kernel's start
  const int j = lq & 7, g = lq >> 3;
  // The four transpositions back to back (a wave's LDS operations complete
  // in order: each round's reads see every lane's writes, and the next
  // round's writes follow those reads; the empty asms keep the compiler's
  // order), then the four rounds' Q8 with no LDS wait between them.
  float* stg = L.stg[wave];
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  f32x4 x4[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
#pragma unroll
    for (int k = 0; k < 4; ++k) stg[64 * k + lq] = v[4 * r + k];
    asm volatile("" ::: "memory");
    x4[r] = *reinterpret_cast<const f32x4*>(stg + 4 * lq);
    asm volatile("" ::: "memory");
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float x[4] = {x4[r][0], x4[r][1], x4[r][2], x4[r][3]};
    float d;
    int s;
    const uint32_t wq = q8_oct(x, d, s);
    uint32_t* dst = &L.act[ob][(sl * 32 + 8 * r + g) * kWordsPerBlock];
    dst[j] = wq;
    if (j == 0) {
      dst[8] = __float_as_uint(d);
      dst[9] = (uint32_t)s;
    }
  }
}

// ---------------------------------------------------------------- compute waves
typedef const __attribute__((address_space(1))) u32x4 gvec4;
typedef const __attribute__((address_space(1))) _Float16 gf16;

// Work of an op inside a workgroup: items (unit u, K-slice s, row quad q),
// u < the workgroup's units of the op, s < S (1024-column slices), q < Qu
// (quads of 4 rows: 8 per unit, or for swiglu 8 of the gate and 8 of the up
// matrix), in the order t = (u*S + s)*Qu + q: a unit's items are consecutive,
// so the I/O waves can publish each unit as soon as it is done, and the items
// of a compute wave touch few slices of the input. One item is one 16-byte
// code chunk (64 columns) per lane: lane l reads chunk s*16 + (l & 15) of row
// (l >> 4) of the quad. Its partial sums land in part[s][local row] at
// virtual row 4q + (l >> 4) of the unit (swiglu: gate row j at
// 32*(j >> 4) + (j & 15), up row j 16 further).
struct Slot {
  u32x4 c;
  uint32_t s;  // the fp16 scale of the chunk's 128-column block, loaded as 16 bits and
               // zero-extended into a full register (two slots' scales packed into one
               // register would make the compiler wait for a refill right after issuing it)
};

// The items of an op are cut into batches of kRing, and each compute wave
// takes a contiguous run of whole batches (units hold a multiple of kRing
// items, so every batch lies in one (unit, slice) and is all real or all
// dummy); a wave with no batch runs one batch of dummies, which keeps every
// wave's ring in step across ops. All fields are uniform (SGPRs).
struct OpWork {
  int i;     // op index (>= nops: past the program's end; a dummy batch)
  int next;  // the GEMV op after it
  int S, qlog, first;  // slices, log2 quads per unit, first unit
  int t0, n, P;        // the wave's first item, real items, entries (a multiple of kRing)
  int u0, s0, q0;      // (u, s, q) of item t0
  int R;               // rows of part[slice][.] (the workgroup's units x 4 * Qu)
  int il;              // 1: unit-interleaved (the wave's batches are batch `wave` of each unit)
};
// Every field is assigned on every path (a partly assigned struct would be
// kept in scratch memory, whose accesses count in vmcnt).
template <class LT>
__device__ __forceinline__ OpWork op_work_calc(const LT& L, int nops, int wave, int wg, int G, int i) {
  OpWork w;
  const bool past = i >= nops;
  const OpDev& o = L.opd[past ? 0 : i];
  w.i = i;
  w.next = past ? nops : sgpr(o.next);
  w.first = past ? 0 : first_unit(sgpr(o.rot), wg, G);
  const int nunits = past ? 0 : units_of(sgpr(o.units), w.first, G);
  w.S = past ? 1 : (sgpr(o.cpr) + 15) >> 4;
  w.qlog = past ? 3 : sgpr(o.qpu_log2);
  const int Qu = 1 << w.qlog;
  w.R = (nunits << w.qlog) * 4;
  const int U = w.S << w.qlog;  // items per unit
  const int T = nunits * U;
  // Plain programs, one batch per wave per unit (gate+up at 5120 columns:
  // 5 slices x 16 quads): wave w takes batch w of every unit, in unit order,
  // so that the workgroup's units complete one after the other (the I/O waves
  // publish the first while the others are computed) instead of all at the
  // op's end. A consumer then finds the units of the workgroups with one unit
  // more than the rest late in one input slice, not in every slice that
  // holds one of them. The wave's batches all read the same slice. (With
  // prepped inputs the contiguous runs are kept: a wave with one slice holds
  // all its batches behind that slice's prep, and the waves of the slice
  // prepped last then finish last; measured 0.6 % slower per token.)
  // With 10 compute waves (il = 2) SIMDs 0 and 1 hold three of them and
  // SIMDs 2 and 3 two (beside the I/O waves), so in every odd unit the
  // batches of positions 8 and 9 go to waves 2 and 3 instead of waves 8 and
  // 9: each SIMD then runs 5 batches per two units, not 6 / 6 / 4 / 4
  // (sweep 1.789 -> 1.783 ms over 6 alternating A/B pairs, bit-exact).
  w.il = !LT::kPrepped && U == LT::kCW * kRing ? (LT::kCW == 10 ? 2 : 1) : 0;
  if (w.il) {
    const int cnt = w.il == 2 && (wave == 2 || wave == 3) ? nunits + nunits / 2
                    : w.il == 2 && (wave == 8 || wave == 9) ? (nunits + 1) / 2 : nunits;
    w.t0 = wave * kRing;
    w.n = cnt * kRing;
    w.P = (cnt > 0 ? cnt : 1) * kRing;
    w.u0 = 0;
    w.s0 = w.t0 >> w.qlog;
    w.q0 = w.t0 & (Qu - 1);
    return w;
  }
  // Batches are spread evenly over the waves, floor(B / kCW) each, the
  // remaining B % kCW one more each: a wave's batches are rounds of its ring
  // (each waits for the loads issued during the previous one), so the op
  // takes as many rounds as its busiest wave has batches. Runs follow in
  // wave order. Which waves take the extra batches: wave v runs on SIMD
  // v % 4, and the I/O waves, the last two, sit on SIMDs 2 and 3. In plain
  // programs the waves without items only pace their refills, and the extras
  // go to waves 0, 1, 2, ... (SIMDs 0 and 1 first: the I/O waves' SIMDs keep
  // fewer real batches; sweep 1.783 -> 1.768 ms against the order below).
  // With preps the waves without items run a dummy batch, and the extras go
  // first to the compute waves of SIMDs 2 and 3, which hold one compute wave
  // fewer: 2, 3, 6, 7, then 0, 1, 4, 5, 8, 9 (whole token 2.784 against
  // 2.821 ms for the plain programs' order).
  constexpr int kCW = LT::kCW;
  static_assert((kCW + kIW) % 4 == 0 && kIW == 2, "the extra-batch order assumes the I/O waves on SIMDs 2 and 3");
  constexpr int n23 = 2 * ((kCW + kIW) / 4 - 1);  // compute waves on SIMDs 2 and 3
  const int B = (T + kRing - 1) / kRing;
  const int base = B / kCW, extra = B % kCW;
  auto xrank = [](int v) {  // rank of wave v in the order of the extra batches
    if (!LT::kPrepped) return v;
    const int sm = v & 3, sl = v >> 2;
    return sm >= 2 ? (sm - 2) + 2 * sl : n23 + sm + 2 * sl;
  };
  int b0 = base * wave;
  for (int v = 0; v < wave; ++v) b0 += xrank(v) < extra ? 1 : 0;
  const int b1 = b0 + base + (xrank(wave) < extra ? 1 : 0);
  w.t0 = b0 * kRing;
  const int t1 = b1 * kRing < T ? b1 * kRing : T;
  w.n = t1 > w.t0 ? t1 - w.t0 : 0;
  w.P = (b1 > b0 ? b1 - b0 : 1) * kRing;
  const int ua = U ? w.t0 / U : 0, ra = w.t0 - ua * U;
  w.u0 = ua;  // (w.il: 0 on this path)
  w.s0 = ra >> w.qlog;
  w.q0 = ra & (Qu - 1);
  return w;
}

// Stage the records of op i (lanes 0 .. kCW-1 of the first I/O wave, one
// per compute wave); read by the compute waves after the next barrier B.
template <class LT>
__device__ __forceinline__ void stage_work(LT& L, int nops, int wg, int G, int i, int iol) {
  asm volatile("" : "+v"(iol));  // lane tests formed here, not held from the kernel's start
  if (iol < LT::kCW) {
    const OpWork w = op_work_calc(L, nops, iol, wg, G, i);
    const int slot = i % kRecSlots;
    L.wrec[slot][iol] = WorkRec{w.t0, w.n, w.P, w.u0 | (w.s0 << 8) | (w.q0 << 16)};
    if (iol == 0) L.orec[slot] = OpRec{w.first, w.R, w.next, w.S | (w.qlog << 8) | (w.il << 16)};
  }
}
template <class LT>
__device__ __forceinline__ OpWork op_work(const LT& L, int wave, int i) {
  const int slot = i % kRecSlots;
  const WorkRec& r = L.wrec[slot][wave];
  const OpRec& o = L.orec[slot];
  OpWork w;
  w.i = i;
  w.t0 = sgpr(r.t0);
  w.n = sgpr(r.n);
  w.P = sgpr(r.P);
  const int uq = sgpr(r.uq);
  w.u0 = uq & 255;
  w.s0 = (uq >> 8) & 255;
  w.q0 = uq >> 16;
  w.first = sgpr(o.first);
  w.R = sgpr(o.R);
  w.next = sgpr(o.next);
  const int sq = sgpr(o.sq);
  w.S = sq & 255;
  w.qlog = (sq >> 8) & 255;
  w.il = LT::kPrepped ? 0 : sq >> 16;  // (a constant in the prepped instance: no interleaved paths there)
  return w;
}

// The input slices the wave's real items read, as input LL word ranges
// [a0, a1) and [b0, b1) (one of them, or both, may be empty): the items run
// from (u0, s0) to the last one's (ub, sb).
__device__ __forceinline__ void input_words(const OpWork& w, int wave, int& a0, int& a1, int& b0, int& b1) {
  constexpr int kWS = 32 * kWordsPerBlock;  // input words per slice
  const int U = w.S << w.qlog;
  const int tl = w.t0 + w.n - 1;
  const int ub = tl / U, sb = (tl - ub * U) >> w.qlog;
  a0 = a1 = b0 = b1 = 0;
  if (w.il) {  // unit-interleaved: every batch in slice s0
    a0 = w.s0 * kWS, a1 = (w.s0 + 1) * kWS;
    if (w.il == 2 && (wave == 2 || wave == 3)) {  // and the slice of its extra position (odd units)
      const int s2 = ((wave + 6) * kRing) >> w.qlog;
      b0 = s2 * kWS, b1 = (s2 + 1) * kWS;
    }
  } else if (ub == w.u0) {
    a0 = w.s0 * kWS, a1 = (sb + 1) * kWS;
  } else if (ub == w.u0 + 1 && sb + 1 < w.s0) {
    a0 = w.s0 * kWS, a1 = w.S * kWS, b1 = (sb + 1) * kWS;
  } else {
    a1 = w.S * kWS;
  }
}

// Uniform load parameters of an op. A batch covers 8 row quads of one 32-row
// unit: for a plain op entries 0..7 read row quads 0..7 of the unit; for
// swiglu (Qu = 16: two batches per unit and slice, 16 rows each) entries 0-3
// read the batch's 4 row quads of the gate matrix and entries 4-7 the same
// rows of the up matrix. So each entry reads ONE matrix, through a buffer
// resource of that matrix (SGPRs) with the entry's uniform offset in soffset
// and the lane's part of the offset (row in the quad, chunk in the slice) in
// a VGPR fixed for the op: no address arithmetic on the vector ALU. A step
// program has K % 1024 == 0, so every chunk of every slice is inside the row,
// and every offset is below 4 GB (checked on the host); the resources span
// 4 GB, so no access is range-clamped.
struct OpLd {
  __amdgpu_buffer_rsrc_t clo, chi;  // codes read by entries 0-3 / 4-7
  __amdgpu_buffer_rsrc_t slo, shi;  // scales
  uint32_t rowc, rows;              // bytes per row: K/4 (codes), K/64 (scales)
  uint32_t lastc, lasts;            // offsets of the last row quad (N - 4)
  int sw;                           // swiglu
};
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p) {
  // stride 0, 4 GB of records, 32-bit data format (raw buffer loads)
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, -1, 0x00020000);
}
__device__ __forceinline__ OpLd make_ld(int mode, const uint8_t* c, const uint16_t* sc, const uint8_t* uc,
                                       const uint16_t* us, uint32_t K, uint32_t N) {
  OpLd d;
  d.sw = mode == BTF_GEMV_SWIGLU;
  d.clo = rsrc(c);
  d.slo = rsrc(sc);
  d.chi = rsrc(d.sw ? uc : c);
  d.shi = rsrc(d.sw ? us : sc);
  d.rowc = K >> 2;
  d.rows = K >> 6;
  d.lastc = (N - 4) * d.rowc;
  d.lasts = (N - 4) * d.rows;
  return d;
}
template <class LT>
__device__ __forceinline__ OpLd op_ld(const LT& L, int i) {
  const OpDev& o = L.opd[i];
  // Every field is read before any is tested, so the reads are in flight
  // together (one LDS round trip; reading the up matrix only for a swiglu
  // would make it a second, and this sits on the critical path of an op).
  return make_ld(sgpr(o.mode), sgpr_ptr(o.codes), sgpr_ptr(o.scales), sgpr_ptr(o.up_codes), sgpr_ptr(o.up_scales),
                 (uint32_t)sgpr(o.K), (uint32_t)sgpr(o.N));
}
// What the loads of op i's first batch need -- its descriptor's matrix
// fields, and the op's first unit and this wave's item count and position --
// read from LDS into vector registers (uniform values, pinned there by empty
// asms): a wave holds them through the op before, whose last batch issues
// those loads, and forms the load parameters there with scalar reads of its
// own registers instead of an LDS round trip. (In scalar registers they
// would be spilled: the op's own parameters fill them.)
struct NextRec {
  int mode, K, N, first, n, uq;
  uint32_t p[8];  // codes, scales, up_codes, up_scales (low, high words)
};
template <class LT>
__device__ __forceinline__ NextRec next_rec(const LT& L, int wave, int di, int wi) {
  const OpDev& o = L.opd[di];
  NextRec r;
  r.mode = o.mode;
  r.K = o.K;
  r.N = o.N;
  const uint32_t* pc = reinterpret_cast<const uint32_t*>(&o.codes);
  const uint32_t* ps = reinterpret_cast<const uint32_t*>(&o.scales);
  const uint32_t* puc = reinterpret_cast<const uint32_t*>(&o.up_codes);
  const uint32_t* pus = reinterpret_cast<const uint32_t*>(&o.up_scales);
  for (int k = 0; k < 2; ++k) {
    r.p[k] = pc[k];
    r.p[2 + k] = ps[k];
    r.p[4 + k] = puc[k];
    r.p[6 + k] = pus[k];
  }
  const int slot = wi % kRecSlots;
  r.first = L.orec[slot].first;
  r.n = L.wrec[slot][wave].n;
  r.uq = L.wrec[slot][wave].uq;
  asm volatile("" : "+v"(r.mode), "+v"(r.K), "+v"(r.N), "+v"(r.first), "+v"(r.n), "+v"(r.uq));
  asm volatile("" : "+v"(r.p[0]), "+v"(r.p[1]), "+v"(r.p[2]), "+v"(r.p[3]), "+v"(r.p[4]), "+v"(r.p[5]),
               "+v"(r.p[6]), "+v"(r.p[7]));
  return r;
}
template <class T>
__device__ __forceinline__ T* sgpr_ptr2(uint32_t lo, uint32_t hi) {  // (each half unsigned: no sign extension)
  const uint32_t l = (uint32_t)__builtin_amdgcn_readfirstlane(lo), h = (uint32_t)__builtin_amdgcn_readfirstlane(hi);
  return reinterpret_cast<T*>(((uint64_t)h << 32) | l);
}
__device__ __forceinline__ OpLd next_ld(const NextRec& r) {
  return make_ld(sgpr(r.mode), sgpr_ptr2<const uint8_t>(r.p[0], r.p[1]), sgpr_ptr2<const uint16_t>(r.p[2], r.p[3]),
                 sgpr_ptr2<const uint8_t>(r.p[4], r.p[5]), sgpr_ptr2<const uint16_t>(r.p[6], r.p[7]),
                 (uint32_t)sgpr(r.K), (uint32_t)sgpr(r.N));
}
// This lane's part of an entry's offsets: row grp of the quad, chunk l16 of
// the slice (16 code bytes; the fp16 scale of its 128-column block).
struct LaneOff {
  uint32_t c, s;
};
__device__ __forceinline__ LaneOff lane_off(const OpLd& d, int l16, int grp) {
  // (the lane's scale: the fp16 of 128-column block l16 / 2, 16 bits loaded directly: no shift to
  // its half of a word when it is consumed; sweep -0.55 %, whole token -0.7 %)
  return LaneOff{(uint32_t)grp * d.rowc + (uint32_t)l16 * 16u, (uint32_t)grp * d.rows + (uint32_t)(l16 >> 1) * 2u};
}

// Position of a batch in the op's items: local unit, slice, first quad.
struct BPos {
  int u, s, qb;
};
__device__ __forceinline__ void bpos_next(int qlog, int S, int il, int wave, BPos& p) {
  if (il == 2) {  // balanced unit-interleaved (10 compute waves)
    const int tb = wave * kRing, te = tb + 6 * kRing;  // the wave's position and, in odd units, its extra one
    if ((wave == 2 || wave == 3) && (p.u & 1) && p.s == (tb >> qlog)) {
      p.s = te >> qlog;
      p.qb = te & ((1 << qlog) - 1);
    } else {
      p.u += (wave == 8 || wave == 9) ? 2 : 1;
      p.s = tb >> qlog;
      p.qb = tb & ((1 << qlog) - 1);
    }
    return;
  }
  if (il) {  // unit-interleaved: the same position of the next unit
    ++p.u;
    return;
  }
  p.qb += kRing;
  if (p.qb == (1 << qlog)) {
    p.qb = 0;
    if (++p.s == S) {
      p.s = 0;
      ++p.u;
    }
  }
}
// Uniform offsets of a batch's entry 0 and the largest valid ones (the last
// row quad's chunk of the same slice).
struct BAddr {
  uint32_t oc, os, mc, ms;
};
__device__ __forceinline__ BAddr batch_addr(const OpLd& d, int first, int G, const BPos& p) {
  const uint32_t row = (uint32_t)(first + p.u * G) * 32u + ((uint32_t)p.qb << (d.sw ? 1 : 2));
  BAddr a;
  a.oc = row * d.rowc + (uint32_t)p.s * 256u;
  a.os = row * d.rows + (uint32_t)p.s * 16u;
  a.mc = d.lastc + (uint32_t)p.s * 256u;
  a.ms = d.lasts + (uint32_t)p.s * 16u;
  return a;
}
// Load entry r of a batch into its ring slot: an unconditional load pair into
// the slot's own registers (non-temporal: the weights are read once). Rows
// past N (only in an op's last unit; N % 4 == 0: a quad is all in or all out)
// read the last row quad instead (never stored). A dummy batch (`real`
// false: past the wave's items, whose dot products are computed and
// dropped) loads through a zero-length buffer resource: the loads return
// zeros without touching memory, so they do not queue in front of the real
// loads (a third of the step's loads were such dummies: 1.93 -> 1.87 ms).
constexpr int kNT = 2;  // cache policy: non-temporal
__device__ __forceinline__ void issue_entry(const OpLd& d, const LaneOff& lo, const BAddr& a, int r, Slot& sl,
                                            bool real) {
  const bool hi = r >= 4;
  const uint32_t dr = 4u * (uint32_t)(r & 3) + (hi && !d.sw ? 16u : 0u);  // rows past the batch's first
  const uint32_t oc = min(a.oc + dr * d.rowc, a.mc);
  const uint32_t os = min(a.os + dr * d.rows, a.ms);
  const __amdgpu_buffer_rsrc_t z = __builtin_amdgcn_make_buffer_rsrc((void*)0, (short)0, 0, 0x00020000);
  sl.c = __builtin_amdgcn_raw_buffer_load_b128(real ? (hi ? d.chi : d.clo) : z, (int)lo.c, (int)oc, kNT);
  sl.s = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(real ? (hi ? d.shi : d.slo) : z, (int)lo.s, (int)os, kNT);
}

// The activation of this lane's chunk of slice s (64 columns = two Q8
// blocks): 64 q bytes, and per sub-block d/16 and -16 s (the dot returns
// 16 * I; both conversions are exact). The 4 row groups of a wave read the
// same addresses (LDS broadcasts).
template <class LT>
__device__ __forceinline__ void load_act(const LT& L, int ob, int s, int l16, uint32_t (&aq)[16], float (&ad)[2],
                                         int (&an)[2]) {
  const int blk = 2 * (s * 16 + l16);
  const uint2* p = reinterpret_cast<const uint2*>(&L.act[ob][blk * kWordsPerBlock]);  // 8-byte aligned
#pragma unroll
  for (int h = 0; h < 2; ++h) {  // block blk + h: words 10 h .. 10 h + 9
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint2 v = p[5 * h + i];
      aq[8 * h + 2 * i] = v.x;
      aq[8 * h + 2 * i + 1] = v.y;
    }
    const uint2 ds = p[5 * h + 4];
    ad[h] = __uint_as_float(ds.x) * 0.0625f;
    an[h] = -16 * (int)ds.y;
  }
}

// 16 * (code . q - s) over the two 32-column sub-blocks of a 16-byte chunk,
// as subblock_dot16 (common.h): the same masks, and the partial sums
// recombined as 16*c0 + 4*c1 + c23, but each chain starts from the previous
// one shifted (c1 from c0 << 2, c23 from (c1 << 2) - 16 s), so every dot but
// the first accumulates into a dead register (the two-operand form, no
// copies). The first has a zero accumulator and the clamp bit, which keeps
// it in the three-operand form (no register clear; the sums are far from
// saturating: |result| < 2^18). The two sub-blocks' chains are interleaved so
// that no instruction waits on the one just before it. ns16 = -16 s.
__device__ __forceinline__ void chunk_dot16(const u32x4& w, const uint32_t (&a)[16], const int (&ns16)[2], int& y0,
                                            int& y1) {
  int c = __builtin_amdgcn_sdot4((int)(w.x & 0x03030303u), (int)a[0], 0, true);
  int e = __builtin_amdgcn_sdot4((int)(w.z & 0x03030303u), (int)a[8], 0, true);
  c = sdot4(w.y & 0x03030303u, a[4], c);
  e = sdot4(w.w & 0x03030303u, a[12], e);
  c = sdot4(w.x & 0x0C0C0C0Cu, a[1], c << 2);
  e = sdot4(w.z & 0x0C0C0C0Cu, a[9], e << 2);
  c = sdot4(w.y & 0x0C0C0C0Cu, a[5], c);
  e = sdot4(w.w & 0x0C0C0C0Cu, a[13], e);
  c = sdot4(w.x & 0x30303030u, a[2], (c << 2) + ns16[0]);
  e = sdot4(w.z & 0x30303030u, a[10], (e << 2) + ns16[1]);
  c = sdot4((w.x >> 2) & 0x30303030u, a[3], c);
  e = sdot4((w.z >> 2) & 0x30303030u, a[11], e);
  c = sdot4(w.y & 0x30303030u, a[6], c);
  e = sdot4(w.w & 0x30303030u, a[14], e);
  c = sdot4((w.y >> 2) & 0x30303030u, a[7], c);
  e = sdot4((w.w >> 2) & 0x30303030u, a[15], e);
  y0 = c;
  y1 = e;
}

// One consumed entry: the dot products and the scale of ring slot `sl`,
// taken before the slot is refilled (the empty asm pins them there, so they
// are neither sunk past the refill nor folded into a later v_fma_mix).
struct Consumed {
  int y0, y1;
  float f;
};
__device__ __forceinline__ Consumed consume(const Slot& sl, const uint32_t (&aq)[16], const int (&an)[2]) {
  Consumed r;
  const u32x4 wv = sl.c;
  r.f = h2f((uint16_t)sl.s);
  chunk_dot16(wv, aq, an, r.y0, r.y1);
  asm volatile("" : "+v"(r.f), "+v"(r.y0), "+v"(r.y1));
  return r;
}

// The 16-lane row sums of a batch's 8 entry values, each in the addition
// tree of row16_sum (partners across lane bit 0, then 1, 2, 3; the same
// floating-point result), for all 8 at once: the first two levels also sort
// the entries over the lanes (lane l keeps entry l & 3 in z0, entry
// 4 + (l & 3) in z1); the last two are row rotations by 4 and 8. A rotation
// by 8 pairs every lane with its exact bit-3 partner l ^ 8; a rotation by 4
// brings lane l ^ 4 to half of the lanes (those with bit 2 clear or those
// with it set, by the rotation's direction), and there the sums are exact:
// sum_lanes() names them.
__device__ __forceinline__ void reduce8(const float (&v)[kRing], bool b0, bool b1, float& z0, float& z1) {
  float w[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float keep = b0 ? v[2 * k + 1] : v[2 * k];
    const float send = b0 ? v[2 * k] : v[2 * k + 1];
    w[k] = keep + dpp_f<0xB1>(send);  // quad_perm(1,0,3,2): lane l ^ 1
  }
  float x[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const float keep = b1 ? w[2 * k + 1] : w[2 * k];
    const float send = b1 ? w[2 * k] : w[2 * k + 1];
    x[k] = keep + dpp_f<0x4E>(send);  // quad_perm(2,3,0,1): lane l ^ 2
  }
  z0 = x[0] + dpp_f<0x124>(x[0]);  // row_ror:4
  z1 = x[1] + dpp_f<0x124>(x[1]);
  z0 = z0 + dpp_f<0x128>(z0);      // row_ror:8
  z1 = z1 + dpp_f<0x128>(z1);
}
// Lanes 0-7 of a row whose row_ror:4 source is their bit-2 partner: 4 lanes
// per row, holding reduce8's sums of entries (l & 3) and 4 + (l & 3).
__device__ __forceinline__ bool sum_lanes(int l16) {
  return l16 < 8 && dpp_i<0x124>(l16) == (l16 ^ 4);
}

// The compute waves' whole program. Per op: wait for the input slices the
// wave's items read (fetch them, or for an early op wait until the I/O waves
// have), the op's batches of kRing entries, barrier B (every wave done with
// the op). Entry r of a batch lives in ring slot r; consuming it refills the
// slot with entry r of the next batch, which for the op's last batch is the
// NEXT op's first batch: the ring stays full across op boundaries (the next
// op's first loads are in flight while this op finishes and while the wave
// waits for its input), with no dummy loads to drain. The loop body is
// straight-line code with one unconditional load pair per entry, so the
// compiler keeps each slot in fixed registers with exact wait counts; the
// per-batch bookkeeping (addresses, partial-sum slots, the unit's count, the
// activation reload at a new slice) is uniform and done once per batch.
template <bool kFull>
__device__ __forceinline__ void compute_waves(Lds<kFull>& L, int nops, int first, int wave, int lane, int wg, int G, Ctl* ctl,
                                              uint32_t base_tag) {
  const int l16 = lane & 15, grp = lane >> 4;
  const bool b0 = (lane & 1) != 0, b1 = (lane & 2) != 0;
  const bool sum_lane = sum_lanes(l16);
  Slot ring[kRing];
  {
    const OpWork w0 = op_work(L, wave, first);
    const OpLd d0 = op_ld(L, first);
    const LaneOff l0 = lane_off(d0, l16, grp);
    const BAddr a = batch_addr(d0, w0.first, G, BPos{w0.u0, w0.s0, w0.q0});
#pragma unroll
    for (int r = 0; r < kRing; ++r) issue_entry(d0, l0, a, r, ring[r], w0.n > 0);
  }
  // Per op, the op's work record and load parameters are read from LDS
  // before the input wait: after it they would be LDS round trips on the op's
  // critical path (measured: sweep 1.850 -> 1.810 ms, whole token 2.841 ->
  // 2.788 ms). Plain programs also read the next op's there (into vector
  // registers, NextRec), for the last batch's refill (sweep 1.810 -> 1.794
  // ms); programs with preps read those in the last batch, as the registers
  // that would hold them across the op are what the prep needs. Op i + 1's
  // records are staged by the I/O waves during op i - 1 and visible after
  // that op's barrier B.
  for (int opi = first;;) {
    const int ob = opi & 1;  // LDS buffers of this op
    const OpLd ld_pre = op_ld(L, opi);
    const OpWork w_pre = op_work(L, wave, opi);
    NextRec nx;  // plain programs: the next op's, which the last batch loads from
    if constexpr (!kFull) nx = next_rec(L, wave, w_pre.next < nops ? w_pre.next : opi, w_pre.next);
    {
    // An input with a prep: the op's slices are shared out over the compute
    // waves (wave w takes slices w, w + kCW, ...), each slice prepped once
    // per workgroup into the LDS image and flagged -- by every wave with a
    // share, whether or not it has items of the op; below, every wave with
    // items waits for the flags of the slices its items read.
    const int pi = kFull ? sgpr(L.opd[opi].prep) : -1;
    if (pi >= 0 && wave < sgpr(L.opd[opi].K) / kSliceVals) {
      float scale = 1.0f;
      const int pf = sgpr(L.opd[opi].prep_flags);
      const bool norm = (pf & 1) != 0, perm = (pf & 2) != 0;
      auto mine = [&](auto pm) {
        for (int sl = wave; sl < sgpr(L.opd[opi].K) / kSliceVals; sl += Lds<kFull>::kCW) {
          fetch_prep_slice<decltype(pm)::value>(L.opd[opi], sgpr_ptr(L.preps), sgpr(L.opd[opi].prep), scale,
                                                norm && sl == wave, L, wave, lane, ctl, base_tag, ob, sl);
          asm volatile("" ::: "memory");  // the image words before the flag (LDS ops of a wave complete in order)
          __hip_atomic_store(&L.sready[ob][sl], (uint32_t)opi + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
      };
      // raised priority: every wave with items of the op waits for these
      // slices, so their instructions go before those of the I/O waves and
      // of the waves that poll
      __builtin_amdgcn_s_setprio(2);
      if (perm)
        mine(std::true_type{});
      else
        mine(std::false_type{});
      __builtin_amdgcn_s_setprio(0);
    }
    const OpWork cur = w_pre;
    if (cur.n > 0) {
      if (sgpr(L.opd[cur.i].early)) {
        // fetched by the I/O waves (early_seq only grows within a launch:
        // they may have gone on to fetch the next early op's input, into
        // the other buffer)
        uint32_t spins = 0;
        for (;;) {
          bool ready = true;
#pragma unroll
          for (int k = 0; k < kIW; ++k)
            ready &= __hip_atomic_load(&L.early_seq[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >=
                     (uint32_t)cur.i + 1;
          if (ready || !poll_step(spins, L, ctl)) break;
          __builtin_amdgcn_s_sleep(2);  // (an LDS poll: paced)
        }
        asm volatile("" ::: "memory");
      } else {
        int a0, a1, b0w, b1w;
        input_words(cur, wave, a0, a1, b0w, b1w);
        if (pi >= 0) {  // wait for the prepped slices this wave's items read
          constexpr int kWS = 32 * kWordsPerBlock;  // input words per slice
          const int s1 = a0 / kWS, n1 = a1 / kWS - s1, s2 = b0w / kWS, n = n1 + b1w / kWS - s2;
          for (int k = 0; k < n; ++k) {
            const int sl = k < n1 ? s1 + k : s2 + (k - n1);
            uint32_t spins = 0;
            while (__hip_atomic_load(&L.sready[ob][sl], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) !=
                   (uint32_t)cur.i + 1) {
              if (!poll_step(spins, L, ctl)) break;
              // an LDS poll returns at once: paced, so that the waves preparing
              // the slices on the same SIMD keep its issue slots
              __builtin_amdgcn_s_sleep(2);
            }
          }
          asm volatile("" ::: "memory");
        } else {
          fetch_words(L.opd[cur.i], L, lane, ctl, base_tag, ob, a0, a1, b0w, b1w);
          // the words other lanes of this wave wrote are read below
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
      }
    }
    }
    OpLd ld_cur = ld_pre;
    const OpWork cur = w_pre;
    LaneOff lo_cur = lane_off(ld_cur, l16, grp);
    const int U = cur.S << cur.qlog;  // items per unit
    BPos cp{cur.u0, cur.s0, cur.q0};  // the batch being consumed
    uint32_t aq[16];
    float ad[2];
    int an[2];
    load_act(L, ob, cp.s, l16, aq, ad, an);
    const int nb = cur.P / kRing;
    // One batch: consume ring slot r, refill it with entry r of the batch at
    // `a` (loads through `ld` / `lo`), then the batch's row sums and count.
    auto run_batch = [&](int b, const OpLd& ld, const LaneOff& lo, const BAddr& a, const BPos& np, bool last,
                         bool real) {
      // With preps in the program, a wave still holding real items of the op
      // issues ahead of the waves that only refill (their batches past the
      // op's items) or prepare slices; the plain kernel measured slower with it.
      if constexpr (kFull) {
        if (b * kRing < cur.n) __builtin_amdgcn_s_setprio(1);
        else __builtin_amdgcn_s_setprio(0);
      }
      if (!kFull && cur.n == 0) {
        // Plain programs, a wave without items of the op: its refills (the
        // next op's first batch) paced ~770 cycles apart instead of behind a
        // dummy batch's dot products, which took issue slots from the real
        // batches on the same SIMD (sweep -0.4 to -0.8 %). Issued back to
        // back they queue in front of the op's real loads (1.828 ms); paced
        // past the op's length, they hold barrier B (~1540 cycles apart:
        // 1.914 ms). With preps the dummy batch stays: an idle wave there may
        // have prepped slices first, and paced refills then outlast the op
        // (2.806 against 2.779 ms per token).
#pragma unroll
        for (int r = 0; r < kRing; ++r) {
          issue_entry(ld, lo, a, r, ring[r], real);
          __builtin_amdgcn_s_sleep(12);
        }
        cp = np;
        return;
      }
      float v[kRing];
#pragma unroll
      for (int r = 0; r < kRing; ++r) {
        const Consumed c = consume(ring[r], aq, an);
        __builtin_amdgcn_sched_barrier(0);
        issue_entry(ld, lo, a, r, ring[r], real);
        __builtin_amdgcn_sched_barrier(0);
        float p = ad[0] * (float)c.y0;
        p = fmaf(ad[1], (float)c.y1, p);
        v[r] = c.f * p;
      }
      float z0, z1;
      reduce8(v, b0, b1, z0, z1);
      if (b * kRing < cur.n) {  // a real batch: its partial sums into part[slice][local row]
        const int pb = cp.s * cur.R + (((cp.u << cur.qlog) + cp.qb) << 2) + grp;
        if (sum_lane) {
          L.part[pb + 4 * (l16 & 3)] = z0;
          L.part[pb + 4 * (l16 & 3) + 16] = z1;
        }
        // then the wave's count of done items of the unit (a plain store of a
        // uniform value: LDS operations of a wave complete in order, so the
        // I/O waves see the partial sums once they see the count)
        asm volatile("" ::: "memory");
        // (il = 2: a wave's extra batch of an odd unit counts both of its batches)
        L.ucnt[wave][cp.u] = cur.il ? (uint32_t)(cur.il == 2 && cp.s != cur.s0 ? 2 * kRing : kRing)
                                    : (uint32_t)(cur.t0 + (b + 1) * kRing - max(cur.t0, cp.u * U));
      }
      if (!last && np.s != cp.s) load_act(L, ob, np.s, l16, aq, ad, an);
      cp = np;
    };
    for (int b = 0; b < nb - 1; ++b) {  // refills: the next batch of this op
      BPos np = cp;
      bpos_next(cur.qlog, cur.S, cur.il, wave, np);
      run_batch(b, ld_cur, lo_cur, batch_addr(ld_cur, cur.first, G, np), np, false, (b + 1) * kRing < cur.n);
    }
    {
      // the last batch refills with the next op's first batch (past the
      // program's end: this op's matrices again). Its addresses are formed
      // only here, so they hold no vector registers through the op's other
      // batches. (read unconditionally -- past the program's end this op's
      // own descriptor again -- so that no branch splits the reads)
      int nfirst, nn, nuq;
      if constexpr (kFull) {
        ld_cur = op_ld(L, cur.next < nops ? cur.next : opi);
        const OpWork nw = op_work(L, wave, cur.next);
        nfirst = nw.first;
        nn = nw.n;
        nuq = nw.u0 | nw.s0 << 8 | nw.q0 << 16;
      } else {
        ld_cur = next_ld(nx);
        nfirst = sgpr(nx.first);
        nn = sgpr(nx.n);
        nuq = sgpr(nx.uq);
      }
      lo_cur = lane_off(ld_cur, l16, grp);
      run_batch(nb - 1, ld_cur, lo_cur, batch_addr(ld_cur, nfirst, G, BPos{nuq & 255, (nuq >> 8) & 255, nuq >> 16}), cp,
                true, nn > 0);
    }
    if constexpr (kFull) __builtin_amdgcn_s_setprio(0);
    lds_barrier();  // B: every wave is done with the op
    if (cur.next >= nops) break;
    opi = cur.next;
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the trailing dummy loads
}

// ---------------------------------------------------------------- I/O waves
// Publish one 32-value unit held by a half-wave: fp32 LL words, plain output
// and the Q8 LL words.
__device__ __forceinline__ void publish_unit(const OpDev& op, int unit, int j, float v, bool valid, uint32_t tag) {
  const int row = unit_row(unit, j);
  float* out_plain = sgpr_ptr(op.out_plain);
  uint64_t* out_f32 = sgpr_ptr(op.out_f32);
  uint64_t* out_q8 = sgpr_ptr(op.out_q8);
  if (valid && out_plain) *(__attribute__((address_space(1))) float*)(out_plain + row) = v;
  if (valid && out_f32) ll_store(out_f32 + row, ((uint64_t)tag << 32) | __float_as_uint(v));
  if (out_q8) {
    float d;
    int s;
    const int q = q8_half(v, d, s);
    // pack 4 consecutive q bytes into one word (lanes 4w..4w+3)
    const uint32_t b = (uint32_t)(q & 0xff) << (8 * (j & 3));
    uint32_t w = b | (uint32_t)dpp_i<0xB1>((int)b);  // quad_perm(1,0,3,2)
    w |= (uint32_t)dpp_i<0x4E>((int)w);              // quad_perm(2,3,0,1)
    uint64_t* dst = out_q8 + q8_block_word(unit);
    if ((j & 3) == 0) ll_store(dst + (j >> 2), ((uint64_t)tag << 32) | w);
    if (j == 0) ll_store(dst + 8, ((uint64_t)tag << 32) | __float_as_uint(d));
    if (j == 1) ll_store(dst + 9, ((uint64_t)tag << 32) | (uint32_t)s);
  }
  if (sgpr(op.out_sq)) {
    // the unit's sum of squares in the canonical tree over the value index
    // bits 0..4 (= lane bits of the half-wave), as pair_sumsq
    const double x = valid ? (double)v : 0.0;
    double t = x * x;
    t += lane_xor_d<1>(t);
    t += lane_xor_d<2>(t);
    t += lane_xor_d<4>(t);
    t += lane_xor_d<8>(t);
    float llo, lhi, hlo, hhi;  // rows 0 / 1 (2 / 3) of the half-wave
    const uint64_t u = __double_as_longlong(t);
    pair16(__uint_as_float((uint32_t)u), llo, lhi);
    pair16(__uint_as_float((uint32_t)(u >> 32)), hlo, hhi);
    t = __longlong_as_double((long long)(((uint64_t)__float_as_uint(hlo) << 32) | __float_as_uint(llo))) +
        __longlong_as_double((long long)(((uint64_t)__float_as_uint(hhi) << 32) | __float_as_uint(lhi)));
    if (j == 0) {
      const uint64_t b = __double_as_longlong(t);
      uint64_t* dst = out_f32 + sq_word(sgpr(op.N), unit);
      ll_store(dst, ((uint64_t)tag << 32) | (uint32_t)b);
      ll_store(dst + 1, ((uint64_t)tag << 32) | (uint32_t)(b >> 32));
    }
  }
}

// Publish a 1024-value slice held by one wave, 16 values per lane (an
// embedding lookup's output): plain output, fp32 LL words, the block sums of
// squares and the Q8 LL words (each lane pair one 32-value block).
__device__ __forceinline__ void publish_slice(const OpDev& op, int c0, int lane, const float (&v)[16], uint32_t tag) {
  float* out_plain = sgpr_ptr(op.out_plain);
  uint64_t* out_f32 = sgpr_ptr(op.out_f32);
  uint64_t* out_q8 = sgpr_ptr(op.out_q8);
  if (out_plain) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(1))) f32x4 gf32x4;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      ((gf32x4*)(out_plain + c0))[k] = f32x4{v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
  }
  if (out_f32) {
#pragma unroll
    for (int i = 0; i < 16; ++i) ll_store(out_f32 + c0 + i, ((uint64_t)tag << 32) | __float_as_uint(v[i]));
  }
  const int blk = c0 >> 5, h = lane & 1;
  if (sgpr(op.out_sq)) {
    const uint64_t b = __double_as_longlong(pair_sumsq(v));
    if (!h) {
      uint64_t* dst = out_f32 + sq_word(sgpr(op.N), blk);
      ll_store(dst, ((uint64_t)tag << 32) | (uint32_t)b);
      ll_store(dst + 1, ((uint64_t)tag << 32) | (uint32_t)(b >> 32));
    }
  }
  if (out_q8) {
    uint32_t qw[4];
    float d;
    int s;
    q8_pair(v, qw, d, s);
    uint64_t* dst = out_q8 + q8_block_word(blk);
#pragma unroll
    for (int k = 0; k < 4; ++k) ll_store(dst + 4 * h + k, ((uint64_t)tag << 32) | qw[k]);
    if (!h) {
      ll_store(dst + 8, ((uint64_t)tag << 32) | __float_as_uint(d));
      ll_store(dst + 9, ((uint64_t)tag << 32) | (uint32_t)s);
    }
  }
}

// The embedding lookup (an op of the prologue, by the I/O waves of the
// workgroups that own its 1024-value units): as embed_slices_kernel, then
// published like a GEMV output.
__device__ __forceinline__ void io_embed(const OpDev& op, const PrepRegs& pd, int wg, int G, int iol, uint32_t tag) {
  const int iw = iol >> 6, lane = iol & 63;
  const int E = sgpr(op.N), units = sgpr(op.units);
  const int tok = sgpr(*(const __attribute__((address_space(1))) int*)sgpr_ptr(static_cast<const int*>(op.src)));
  const gptr<uint32_t> rowc = as_global(reinterpret_cast<const uint32_t*>(sgpr_ptr(op.codes) + (size_t)tok * (size_t)(E / 4)));
  const gptr<uint16_t> rows = as_global(sgpr_ptr(op.scales) + (size_t)tok * (size_t)(E / 128));
  for (int u = first_unit(sgpr(op.rot), wg, G) + iw * G; u < units; u += kIW * G) {
    const int c0 = slice_col(u, lane);
    const uint32_t w = rowc[c0 >> 4];
    const float sc = h2f(rows[c0 >> 7]);
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = (float)((int)((w >> (8 * (j & 3) + 2 * (j >> 2))) & 3u) - 1) * sc;
    if (pd.block > 0) {
      slice_fwht(v, lane, pd.block);
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = v[j] * pd.hs;
      if (const gptr<float> signs = as_global(pd.signs))
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = v[j] * signs[c0 + j];
    }
    publish_slice(op, c0, lane, v, tag);
  }
}

__device__ __forceinline__ void io_quantize(const OpDev& op, int wg, int G, int iol, uint32_t tag) {
  // half-wave h of the I/O waves handles units first + (h + t*nhalves)*G
  const int half = iol >> 5, j = iol & 31, nhalves = kIW * 2;
  const int N = sgpr(op.N), units = sgpr(op.units);
  const float* src = sgpr_ptr(static_cast<const float*>(op.src));
  for (int u = first_unit(sgpr(op.rot), wg, G) + half * G; u < units; u += nhalves * G) {
    const int row = unit_row(u, j);
    const bool valid = row < N;
    const float v = valid ? *(const __attribute__((address_space(1))) float*)(src + row) : 0.f;
    publish_unit(op, u, j, v, valid, tag);
  }
}

// Write-after-read guard: the version of the output vector this op replaces
// may still be needed by a workgroup that has not fetched the input of op
// `war_op` yet; wait until all G have. Each workgroup records its progress in
// a word of its own (prog[wg] = the tag of the last op with count_reads whose
// barrier B it has passed; tags only grow, launch after launch), so the wait
// reads G words (4 per lane) instead of a counter that
// G workgroups increment: same-address atomics from every workgroup
// serialize in the memory system, and the count then completes microseconds
// after the last workgroup passed.
template <class LT>
__device__ __forceinline__ void wait_readers(int war_op, const uint32_t* prog, int G, LT& L, Ctl* ctl,
                                             uint32_t base_tag, int lane) {
  if (war_op < 0) return;
  // (the target and this lane's words in vector registers: scalar registers
  // are short in the I/O waves)
  uint32_t want = base_tag + (uint32_t)war_op + 1;
  const uint32_t* mine = prog + lane;
  asm volatile("" : "+v"(want), "+v"(mine));
  uint32_t spins = 0;
  for (;;) {
    // lane l: workgroups l, l + 64, ... (the buffer has 256 words; G <= 256);
    // sign bits instead of compares: no lane masks held in scalar registers
    uint32_t behind = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t v = __hip_atomic_load((const __attribute__((address_space(1))) uint32_t*)(mine + 64 * k),
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      behind |= (v - want) & (uint32_t)(lane + 64 * k - G);  // sign: behind, and a workgroup of the grid
    }
    if (__builtin_amdgcn_ballot_w64((int32_t)behind < 0) == 0 || aborted(L)) break;
    if (++spins > L.spin_max || ((spins & 255) == 0 && grid_failed(ctl, L))) {
      set_abort(L, ctl);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Row lr's partial sums over the op's S slices, added in slice order. The
// loads go out in groups of kSumGroup before their adds (addresses clamped to
// slice S - 1; a slice past S adds -0.0f, which leaves every sum as it is,
// -0.0f included): at K = 5120 one LDS round trip with no padded load, at
// K = 17408 four instead of 17. (Groups of 10, five padded loads in every
// 5-slice sum: sweep 1.752 and whole token 2.722 ms against 1.740 and 2.690;
// groups of 6 and 8 in between, 17 slower still; groups of 3 and 4: 1.756
// and 1.762.)
constexpr int kSumGroup = 5;
template <class LT>
__device__ __forceinline__ float slice_sum(const LT& L, int S, int R, int lr) {
  float sum = 0.f;
  for (int s0 = 0; s0 < S; s0 += kSumGroup) {
    float p[kSumGroup];
#pragma unroll
    for (int k = 0; k < kSumGroup; ++k) p[k] = L.part[min(s0 + k, S - 1) * R + lr];
#pragma unroll
    for (int k = 0; k < kSumGroup; ++k) sum += s0 + k < S ? p[k] : -0.0f;
  }
  return sum;
}

// Publish the op's units as the compute waves complete them: half-wave h
// takes local units h, h + 4, ...; for each, it waits until the unit's
// items are all counted (the compute waves' counts add up), reduces
// part[slice][row] over the slices in order,
// applies the mode (old value: the LDS carry, or the LL word of the previous
// version, loaded one unit ahead) and publishes. Returns each counter to 0
// for the next op.
template <bool kFull, class LT>
__device__ __forceinline__ void io_publish(const OpDev& op, LT& L, int wg, int G, int iol, uint32_t base_tag,
                                           Ctl* ctl) {
  asm volatile("" : "+v"(iol));  // lane values formed here, not held from the kernel's start
  const int half = iol >> 5, j = iol & 31, nhalves = kIW * 2;
  const int first = first_unit(sgpr(op.rot), wg, G);
  const int nunits = units_of(sgpr(op.units), first, G);
  const int mode = sgpr(op.mode), N = sgpr(op.N);
  const int S = (sgpr(op.cpr) + 15) >> 4;                      // 1024-column slices: partial sums per row
  const uint32_t items = (uint32_t)S << sgpr(op.qpu_log2);     // items per unit
  const int R = nunits * (mode == BTF_GEMV_SWIGLU ? 64 : 32);  // rows of part[slice][row]
  const uint32_t tag = base_tag + sgpr(op.my_tag);
  const bool carry_in = sgpr(op.carry_in), carry_out = sgpr(op.carry_out);
  const bool old_ll = mode == BTF_GEMV_ADD && !carry_in;
  const uint64_t* old = sgpr_ptr(op.old_f32);
  const uint32_t told = base_tag + sgpr(op.old_tag);
  auto old_word = [&](int ui) {
    const int row = (first + ui * G) * 32 + j;
    return (old_ll && ui < nunits && row < N) ? ll_load(old + row) : ((uint64_t)told << 32);
  };
  uint64_t ov = old_word(half);
  const bool pick = kFull && sgpr(op.argmax);
  uint64_t best = 0;  // the largest pick key of the rows this lane published
  for (int ui = half; ui < nunits; ui += nhalves) {
    {
      // polled sparsely: the compute waves on the same SIMDs are producing
      // these items
      uint32_t spins = 0;
      for (;;) {
        uint32_t done = 0;
#pragma unroll
        for (int w = 0; w < LT::kCW; ++w)
          done += __hip_atomic_load(&L.ucnt[w][ui], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (done == items || !poll_step(spins, L, ctl)) break;
        __builtin_amdgcn_s_sleep(1);
      }
    }
    asm volatile("" ::: "memory");
    if (j < LT::kCW) __hip_atomic_store(&L.ucnt[j][ui], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    const int unit = first + ui * G;
    const int row = unit_row(unit, j);
    const bool valid = row < N;
    float v;
    if (mode == BTF_GEMV_SWIGLU) {
      const int lr = ui * 64 + 32 * (j >> 4) + (j & 15);  // virtual rows: gate row j; up row j at lr + 16
      const float g = slice_sum(L, S, R, lr), u = slice_sum(L, S, R, lr + 16);
      v = g / (1.0f + expf(-g)) * u;
    } else {
      const int lr = ui * 32 + j;
      const float sum = slice_sum(L, S, R, lr);
      if (mode == BTF_GEMV_ADD) {
        float o;
        if (carry_in) {
          o = L.carry[lr];
        } else {
          uint32_t spins = 0;
          while ((uint32_t)(ov >> 32) != told && poll_step(spins, L, ctl)) ov = ll_load(old + row);
          o = __uint_as_float((uint32_t)ov);
          ov = old_word(ui + nhalves);  // the next unit's, in flight while it computes
        }
        v = o + sum;
      } else {
        v = sum;
      }
      if (carry_out) L.carry[lr] = v;
    }
    publish_unit(op, unit, j, valid ? v : 0.f, valid, tag);
    if (pick && valid) best = key_max(best, argmax_key(v, row));
  }
  if (pick) {
    best = wave_max_key(best);
    L.argk[iol >> 6] = best;  // every lane stores the wave's key; combined after barrier B
  }
}

// The I/O waves' program. Per op: issue the early loads of the next op's
// input (if it is early), wait for the write-after-read guard, publish the
// units as they complete, barrier B, count this workgroup's reads of the
// op's input, finish the early fetch.
// The program's greedy pick (workgroup 0's first I/O wave, after its last
// op): the largest of the G workgroups' keys, polled from their LL words.
template <class LT>
__device__ __forceinline__ void io_pick(const HeadDev* head, LT& L, int G, int lane, Ctl* ctl, uint32_t base_tag) {
  const cptr<HeadDev> h = as_const(head);
  const uint64_t* parts = sgpr_ptr(h->parts);
  const uint32_t tag = base_tag + sgpr((int)h->tag);
  constexpr int kPer = 4;  // parts per lane (G <= 256)
  uint64_t lo[kPer], hi[kPer];
#pragma unroll
  for (int b = 0; b < kPer; ++b) {
    const int w = lane + 64 * b;
    lo[b] = w < G ? ll_load(parts + 2 * w) : ((uint64_t)tag << 32);
    hi[b] = w < G ? ll_load(parts + 2 * w + 1) : ((uint64_t)tag << 32);
  }
  uint32_t spins = 0;
  for (;;) {
    uint32_t pending = 0;
#pragma unroll
    for (int b = 0; b < kPer; ++b)
      pending |= ((uint32_t)(lo[b] >> 32) != tag || (uint32_t)(hi[b] >> 32) != tag) ? (1u << b) : 0u;
    if (__builtin_amdgcn_ballot_w64(pending != 0) == 0) break;
    if (!poll_step(spins, L, ctl)) break;
#pragma unroll
    for (int b = 0; b < kPer; ++b)
      if (pending & (1u << b)) {
        const int w = lane + 64 * b;
        lo[b] = ll_load(parts + 2 * w);
        hi[b] = ll_load(parts + 2 * w + 1);
      }
  }
  uint64_t best = 0;
#pragma unroll
  for (int b = 0; b < kPer; ++b)
    if (lane + 64 * b < G) best = key_max(best, ((uint64_t)(uint32_t)hi[b] << 32) | (uint32_t)lo[b]);
  best = wave_max_key(best);
  if (first_lane(lane)) {
    *(__attribute__((address_space(1))) int*)sgpr_ptr(h->tok_out) = argmax_key_index(best);
    if (int* pos = sgpr_ptr(h->pos))
      (void)__hip_atomic_fetch_add((__attribute__((address_space(1))) int*)pos, 1, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
  }
}

// The I/O waves' program. Per op: issue the early loads of the next op's
// input (if it is early), wait for the write-after-read guard, publish the
// units as they complete, barrier B, count this workgroup's reads of the
// op's input (and publish its pick key), finish the early fetch. Prologue ops
// (quantize, embedding) run before the first GEMV.
template <bool kFull>
__device__ __forceinline__ void io_waves(Lds<kFull>& L, int nops, Ctl* ctl, uint32_t* prog, int iol, int wg, int G,
                                         uint32_t base_tag) {
  for (int i = 0; i < nops; ++i) {
    const OpDev& op = L.opd[i];
    const int kind = sgpr(op.kind);
    if (kind == 0) {
      io_quantize(op, wg, G, iol, base_tag + sgpr(op.my_tag));
      continue;
    }
    if (kFull && kind == 2) {
      io_embed(op, prep_regs(op), wg, G, iol, base_tag + sgpr(op.my_tag));
      continue;
    }
    const int nx = sgpr(op.next);
    // the compute waves read op nx + 1's records at their next loop top (after B of this op)
    stage_work(L, nops, wg, G, nx < nops ? sgpr(L.opd[nx].next) : nx + 1, iol);
    const bool early = nx < nops && sgpr(L.opd[nx].early);
    EarlyFetch ef;
    bool early_done = !early;
    if (early) early_issue(L.opd[nx], iol, base_tag, ef);
    wait_readers(sgpr(op.war_op), prog, G, L, ctl, base_tag, iol & 63);
    // Finish the early fetch now if its input is all published (usual: its
    // producers are two or more ops back), while this op's first units are
    // still being computed. Waiting for these loads later would also wait
    // for the op's own output stores to complete (vmcnt counts both).
    if (early) early_done = early_finish(L.opd[nx], iol, base_tag, ef, L, nx & 1, ctl, false, (uint32_t)nx + 1);
    io_publish<kFull>(op, L, wg, G, iol, base_tag, ctl);
    lds_barrier();  // B: every compute wave is done with the op's input
    const bool io0 = sgpr(iol >> 6) == 0;  // the first I/O wave
    if (sgpr(op.count_reads) && io0 && first_lane(iol))  // this workgroup has fetched op i's input
      __hip_atomic_store((__attribute__((address_space(1))) uint32_t*)(prog + wg), base_tag + (uint32_t)i + 1,
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (kFull && sgpr(op.argmax) && io0 && first_lane(iol)) {  // this workgroup's pick key: the larger of the two I/O waves'
      const uint64_t k = key_max(L.argk[0], L.argk[1]);
      uint64_t* dst = sgpr_ptr(as_const(sgpr_ptr(L.head))->parts) + pick_word(wg);
      const uint32_t tag = base_tag + sgpr(op.my_tag);
      ll_store(dst, ((uint64_t)tag << 32) | (uint32_t)k);
      ll_store(dst + 1, ((uint64_t)tag << 32) | (uint32_t)(k >> 32));
    }
    if (!early_done) early_finish(L.opd[nx], iol, base_tag, ef, L, nx & 1, ctl, true, (uint32_t)nx + 1);
  }
  if (kFull && wg == 0 && sgpr(iol >> 6) == 0 && sgpr(as_const(sgpr_ptr(L.head))->present))
    io_pick(sgpr_ptr(L.head), L, G, iol, ctl, base_tag);
}

// ---------------------------------------------------------------- the kernel
// Two instances: kFull for programs with an activation prep, an embedding
// lookup or a greedy pick; the plain one (a chain of GEMVs on Q8 inputs)
// without that code.
template <bool kFull>
__global__ void __launch_bounds__(threads_of<kFull>()) step_kernel(const OpDev* __restrict__ ops, int nops, int first_gemv,
                                                        Ctl* ctl, uint32_t* prog, const PrepDev* __restrict__ preps,
                                                        const HeadDev* __restrict__ head) {
  constexpr int kCW = cw_of<kFull>(), kThreads = threads_of<kFull>();
  __shared__ Lds<kFull> L;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wg = blockIdx.x, G = gridDim.x;
  // stage the program in LDS
  {
    const u32x4* src = reinterpret_cast<const u32x4*>(ops);
    u32x4* dst = reinterpret_cast<u32x4*>(L.opd);
    const int nvec = nops * (int)(sizeof(OpDev) / 16);
    for (int k = threadIdx.x; k < nvec; k += kThreads) dst[k] = src[k];
  }
  for (int k = threadIdx.x; k < kCW * kMaxUnits; k += kThreads) (&L.ucnt[0][0])[k] = 0;
  for (int k = threadIdx.x; k < 2 * (kMaxK / kSliceVals); k += kThreads) (&L.sready[0][0])[k] = 0;
  if (threadIdx.x < kIW) L.early_seq[threadIdx.x] = 0;
  if (threadIdx.x == 0) {
    L.preps = preps;
    L.head = head;
    L.epoch = ctl_load(&ctl->epoch);
    const uint32_t sm = ctl_load(&ctl->spin_max);
    L.spin_max = sm ? sm : kSpinMax;
    __hip_atomic_store(&L.abort_, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the staged words have landed
  lds_barrier();
  if (wave == kCW) {  // the compute waves' records of the first two GEMV ops
    const int f2 = first_gemv < nops ? sgpr(L.opd[first_gemv].next) : first_gemv + 1;
    stage_work(L, nops, wg, G, first_gemv, lane);
    stage_work(L, nops, wg, G, f2, lane);
  }
  lds_barrier();
  const uint32_t base_tag = L.epoch * (uint32_t)(nops + 1);

  if (wave < kCW)
    compute_waves<kFull>(L, nops, first_gemv, wave, lane, wg, G, ctl, base_tag);
  else {
    // (at the compute waves' priority: raised above them, the I/O waves'
    // polls took issue slots from the preps of whole-token programs, 3.41
    // against 3.23 ms per token, and gained nothing for a plain chain)
    io_waves<kFull>(L, nops, ctl, prog, threadIdx.x - 64 * kCW, wg, G, base_tag);
  }

  // ---------------- end of step: count the workgroup out; the last one to
  // arrive advances the epoch for the next launch (it is read before any
  // workgroup of this launch can have finished its first op).
  lds_barrier();
  // (the thread index is re-read here: a lane mask computed at the start
  // would hold two SGPRs through the whole kernel)
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&ctl->done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == (uint32_t)G - 1) {
      __hip_atomic_store(&ctl->done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&ctl->epoch, L.epoch + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace

// ================================================================ host side
struct StepProgram {
  int device = 0;
  int G = 0;
  int nops = 0;
  int first = 0;  // index of the first GEMV op
  OpDev* d_ops = nullptr;
  Ctl* d_ctl = nullptr;
  uint32_t* d_cnt = nullptr;    // per-workgroup progress words (write-after-read guards)
  PrepDev* d_preps = nullptr;   // the ops' prep descriptors
  HeadDev* d_head = nullptr;    // the greedy pick
  bool full = false;            // any prep, embedding or pick: the kFull kernel
  int guards = 0;               // ops that keep a write-after-read wait (not implied by the data flow)
  std::vector<void*> bufs;      // every device buffer the program owns
  // A plan built without a device (btf_hip_step_audit): the buffers are host
  // memory, and the device program is kept here instead of uploaded.
  bool host = false;
  std::vector<size_t> buf_bytes;
  std::vector<OpDev> plan_ops;
  std::vector<PrepDev> plan_preps;
  HeadDev plan_head{};
};

void step_destroy(StepProgram* P) {
  if (!P) return;
  for (void* p : P->bufs) {
    if (P->host) std::free(p);
    else (void)hipFree(p);
  }
  delete P;
}

namespace {
bool pow2_upto(int b, int hi) { return b > 0 && b <= hi && (b & (b - 1)) == 0; }
bool has_prep(const btf_step_op& o) { return o.normw != nullptr || o.hx.block > 0; }
bool misaligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) != 0; }

int check_gemv_op(const btf_step_vec* vecs, int nvec, const btf_step_op& o) {
  const btf_step_gemv& g = o.gemv;
  if (g.in_vec < 0 || g.in_vec >= nvec || g.out_vec < 0 || g.out_vec >= nvec)
    return fail(BTF_ERR_ARGS, "step: vector index out of range");
  if (g.mode != BTF_GEMV_STORE && g.mode != BTF_GEMV_ADD && g.mode != BTF_GEMV_SWIGLU)
    return fail(BTF_ERR_ARGS, "step: unknown mode");
  if (g.K <= 0 || g.K % 1024 || g.K > kMaxK) return fail(BTF_ERR_ARGS, "step: K must be a multiple of 1024, <= 20480");
  if (g.N % 4) return fail(BTF_ERR_ARGS, "step: N must be a multiple of 4");
  if ((uint64_t)g.N * (uint64_t)(g.K / 4) >= (1ull << 32)) return fail(BTF_ERR_ARGS, "step: a matrix must be below 4 GB");
  if (g.K > vecs[g.in_vec].n) return fail(BTF_ERR_ARGS, "step: K exceeds the input vector");
  if (g.N != vecs[g.out_vec].n) return fail(BTF_ERR_ARGS, "step: N must equal the output vector length");
  if (g.in_vec == g.out_vec) return fail(BTF_ERR_ARGS, "step: a GEMV cannot read its own output vector");
  if (!g.codes || !g.scales || (g.mode == BTF_GEMV_SWIGLU && (!g.up_codes || !g.up_scales)))
    return fail(BTF_ERR_ARGS, "step: null weights");
  if (misaligned(g.codes, 16) || (g.up_codes && misaligned(g.up_codes, 16)) || misaligned(g.scales, 2) ||
      (g.up_scales && misaligned(g.up_scales, 2)))
    return fail(BTF_ERR_ARGS, "step: codes must be 16-byte and scales 2-byte aligned");
  if (has_prep(o)) {
    if (vecs[g.in_vec].n != g.K) return fail(BTF_ERR_ARGS, "step: a GEMV with a norm or transform needs an input of length K");
    if (o.hx.block < 0 || (o.hx.block > 0 && !pow2_upto(o.hx.block, 1024)))
      return fail(BTF_ERR_ARGS, "step: hadamard block must be 0 or a power of two <= 1024");
    if (o.hx.block > 0 && o.hx.perm_rep > 1 &&
        (o.hx.perm_hd <= 0 || o.hx.perm_nk <= 0 || (int64_t)o.hx.perm_hd * o.hx.perm_nk * o.hx.perm_rep != g.K))
      return fail(BTF_ERR_ARGS, "step: hadamard perm geometry");
    if (o.hx.block > 0 && o.hx.perm_rep > 1 && o.hx.perm_hd % 64)
      return fail(BTF_ERR_ARGS, "step: the perm's tile (perm_hd) must be a multiple of 64");
  } else if (o.hx.block < 0) {
    return fail(BTF_ERR_ARGS, "step: hadamard block must be 0 or a power of two <= 1024");
  }
  if (vecs[g.in_vec].n % 32) return fail(BTF_ERR_ARGS, "step: quantized vectors need n % 32 == 0");
  return BTF_OK;
}
}  // namespace

int step_validate_ops(const btf_step_vec* vecs, int nvec, const btf_step_op* ops, int nops) {
  for (int v = 0; v < nvec; ++v)
    if (vecs[v].n <= 0) return fail(BTF_ERR_ARGS, "step: vector length must be positive");
  std::vector<int> writes(nvec, 0);
  bool seen_gemv = false;
  int picks = 0;
  for (int i = 0; i < nops; ++i) {
    const btf_step_op& o = ops[i];
    if (o.kind == BTF_STEP_EMBED) {
      if (seen_gemv) return fail(BTF_ERR_ARGS, "step: embedding ops come before every GEMV");
      if (o.vec < 0 || o.vec >= nvec) return fail(BTF_ERR_ARGS, "step: vector index out of range");
      if (vecs[o.vec].n % 1024) return fail(BTF_ERR_ARGS, "step: an embedded vector's length must be a multiple of 1024");
      if (!o.table_codes || !o.table_scales || !o.d_tok) return fail(BTF_ERR_ARGS, "step: embedding needs its table and token");
      if (misaligned(o.table_codes, 4) || misaligned(o.table_scales, 2))
        return fail(BTF_ERR_ARGS, "step: embedding table codes must be 4-byte and scales 2-byte aligned");
      if (o.hx.block < 0 || (o.hx.block > 0 && !pow2_upto(o.hx.block, 1024)))
        return fail(BTF_ERR_ARGS, "step: hadamard block must be 0 or a power of two <= 1024");
      if (writes[o.vec]) return fail(BTF_ERR_ARGS, "step: a vector is embedded at most once");
      writes[o.vec]++;
    } else if (o.kind == BTF_STEP_GEMV) {
      seen_gemv = true;
      if (const int rc = check_gemv_op(vecs, nvec, o)) return rc;
      const btf_step_gemv& g = o.gemv;
      if (writes[g.in_vec] == 0 && !vecs[g.in_vec].data)
        return fail(BTF_ERR_ARGS, "step: a vector read before any write needs data");
      if (g.mode == BTF_GEMV_ADD && writes[g.out_vec] == 0 && !vecs[g.out_vec].data)
        return fail(BTF_ERR_ARGS, "step: a vector read before any write needs data");
      writes[g.out_vec]++;
    } else if (o.kind == BTF_STEP_ARGMAX) {
      if (++picks > 1) return fail(BTF_ERR_ARGS, "step: at most one greedy pick per program");
      if (o.vec < 0 || o.vec >= nvec) return fail(BTF_ERR_ARGS, "step: vector index out of range");
      if (!o.d_tok_out) return fail(BTF_ERR_ARGS, "step: null token output");
      if (i == 0 || ops[i - 1].kind != BTF_STEP_GEMV || ops[i - 1].gemv.out_vec != o.vec)
        return fail(BTF_ERR_ARGS, "step: a greedy pick must directly follow the GEMV that writes its vector");
    } else {
      return fail(BTF_ERR_ARGS, "step: unknown op kind");
    }
  }
  if (!seen_gemv) return fail(BTF_ERR_ARGS, "step: a program needs at least one GEMV");
  return BTF_OK;
}

std::vector<btf_step_op> step_ops_of(const btf_step_gemv* gemvs, int ngemv) {
  std::vector<btf_step_op> ops((size_t)ngemv);
  for (int i = 0; i < ngemv; ++i) {
    ops[i] = btf_step_op{};
    ops[i].kind = BTF_STEP_GEMV;
    ops[i].gemv = gemvs[i];
  }
  return ops;
}

int step_validate(const btf_step_vec* vecs, int nvec, const btf_step_gemv* gemvs, int ngemv) {
  const std::vector<btf_step_op> ops = step_ops_of(gemvs, ngemv);
  return step_validate_ops(vecs, nvec, ops.data(), ngemv);
}

namespace {
// Builds a program for a grid of G workgroups. host_G > 0: without a device
// (the buffers in host memory, the program kept in P instead of uploaded).
int step_build(const btf_step_vec* vecs, int nvec, const btf_step_op* uops, int nuops, StepProgram** out,
               const DevState* ds, int host_G) {
  const bool host = host_G > 0;
  if (const int rc = step_validate_ops(vecs, nvec, uops, nuops)) return rc;
  if (!host)
    if (const int rc = step_check_residency(*ds)) return rc;
  const int G = host ? host_G : ds->cu_count;
  if (G > 256) return fail(BTF_ERR_DEVICE, "step: more than 256 CUs");
  // ---- versions of every vector over the program. Version 0 of a vector
  // read before any write is its user data, published by a prologue op;
  // every GEMV and embedding writes a new version of its output vector. A
  // version has Q8 LL words if a GEMV without a prep reads it, fp32 LL words
  // (with room for the block sums of squares) if an op wrote it (read later
  // or not) or an add-mode GEMV or a GEMV with a prep reads it, and the sums
  // of squares if a GEMV with a norm reads it.
  struct Version {
    int writer;                  // user op index, -1 = prologue
    int last_q8_reader = -1;     // user op index
    int last_f32_reader = -1;    // GEMV with a prep reading the fp32 words
    std::vector<int> old_readers;  // add-mode GEMVs reading it as their old value
    bool needs_sq = false;
    int q8_slot = -1, f32_slot = -1;
  };
  std::vector<std::vector<Version>> versions(nvec);
  std::vector<int> in_ver(nuops, -1), old_ver(nuops, -1), out_ver(nuops, -1);
  int pick_gemv = -1;  // user index of the GEMV whose output the greedy pick reads
  const btf_step_op* pick = nullptr;
  for (int i = 0; i < nuops; ++i) {
    const btf_step_op& o = uops[i];
    if (o.kind == BTF_STEP_ARGMAX) {
      pick = &o;
      pick_gemv = i - 1;
      continue;
    }
    if (o.kind == BTF_STEP_EMBED) {
      out_ver[i] = (int)versions[o.vec].size();
      versions[o.vec].push_back(Version{i});
      continue;
    }
    const btf_step_gemv& g = o.gemv;
    if (versions[g.in_vec].empty()) versions[g.in_vec].push_back(Version{-1});
    in_ver[i] = (int)versions[g.in_vec].size() - 1;
    Version& iv = versions[g.in_vec].back();
    if (has_prep(o)) {
      iv.last_f32_reader = i;
      iv.needs_sq |= o.normw != nullptr;
    } else {
      iv.last_q8_reader = i;
    }
    if (g.mode == BTF_GEMV_ADD) {
      if (versions[g.out_vec].empty()) versions[g.out_vec].push_back(Version{-1});
      old_ver[i] = (int)versions[g.out_vec].size() - 1;
      versions[g.out_vec].back().old_readers.push_back(i);
    }
    out_ver[i] = (int)versions[g.out_vec].size();
    versions[g.out_vec].push_back(Version{i});
  }
  std::vector<int> final_writer(nvec, -1);
  for (int v = 0; v < nvec; ++v)
    if (!versions[v].empty()) final_writer[v] = versions[v].back().writer;
  StepProgram* P = new StepProgram();
  P->G = G;
  P->host = host;
  auto alloc = [&](size_t bytes) -> void* {
    void* p = nullptr;
    if (host) {
      if (!(p = std::calloc(bytes, 1))) return nullptr;
    } else if (hipMalloc(&p, bytes) != hipSuccess) {
      return nullptr;
    }
    P->bufs.push_back(p);
    P->buf_bytes.push_back(bytes);
    if (!host && hipMemset(p, 0, bytes) != hipSuccess) return nullptr;
    return p;
  };
  auto bail = [&](int code, const char* msg) {
    step_destroy(P);
    return fail(code, msg);
  };
  // kSlots buffers of each kind per vector, taken in turn by the versions
  // that need one, so a version overwrites the one kSlots such versions
  // earlier (whose readers have long finished, normally).
  std::vector<uint64_t*> f32buf[kSlots], q8buf[kSlots];
  for (int b = 0; b < kSlots; ++b) {
    f32buf[b].assign(nvec, nullptr);
    q8buf[b].assign(nvec, nullptr);
  }
  for (int v = 0; v < nvec; ++v) {
    int nq = 0, nf = 0;
    for (Version& ve : versions[v]) {
      if (ve.last_q8_reader >= 0) ve.q8_slot = nq++ % kSlots;
      if (ve.writer >= 0 || !ve.old_readers.empty() || ve.last_f32_reader >= 0) ve.f32_slot = nf++ % kSlots;
    }
    const size_t n = (size_t)vecs[v].n, nb = (n + 31) / 32;
    for (int b = 0; b < kSlots && b < nq; ++b)
      if (!(q8buf[b][v] = static_cast<uint64_t*>(alloc(nb * kWordsPerBlock * 8))))
        return bail(BTF_ERR_LAUNCH, "step: device allocation failed");
    for (int b = 0; b < kSlots && b < nf; ++b)
      if (!(f32buf[b][v] = static_cast<uint64_t*>(alloc((n + 2 * nb) * 8))))
        return bail(BTF_ERR_LAUNCH, "step: device allocation failed");
  }
  auto q8_of = [&](int v, int k) { return versions[v][k].q8_slot >= 0 ? q8buf[versions[v][k].q8_slot][v] : nullptr; };
  auto f32_of = [&](int v, int k) { return versions[v][k].f32_slot >= 0 ? f32buf[versions[v][k].f32_slot][v] : nullptr; };
  std::vector<PrepDev> preps;
  std::vector<std::vector<int>> run_tables;  // uploaded after the program is built
  std::vector<int> run_of;                   // the prep each table belongs to
  auto add_prep = [&](const float* normw, float eps, const btf_hx& hx, int n) {
    PrepDev p{};
    p.normw = normw;
    p.eps = eps;
    p.block = hx.block > 0 ? hx.block : 0;
    p.hs = hx.block > 0 ? 1.0f / std::sqrt((float)hx.block) : 1.0f;
    p.signs = hx.block > 0 ? hx.signs : nullptr;
    if (hx.block > 0 && hx.perm_rep > 1) {  // the gather's runs (perm_hd % 64 == 0: runs of 64 are contiguous)
      std::vector<int> runs((size_t)n / 64);
      for (size_t j = 0; j < runs.size(); ++j) {
        const int og = (int)j * 64, dd = og % hx.perm_hd, t = og / hx.perm_hd;
        runs[j] = dd + hx.perm_hd * (t / hx.perm_rep + hx.perm_nk * (t % hx.perm_rep));
      }
      run_tables.push_back(std::move(runs));
      run_of.push_back((int)preps.size());
    }
    preps.push_back(p);
    return (int)preps.size() - 1;
  };
  auto prep_flags_of = [](const float* normw, const btf_hx& hx) {
    return (uint8_t)((normw ? 1 : 0) | (hx.block > 0 && hx.perm_rep > 1 ? 2 : 0));
  };
  auto set_prep = [&](OpDev& o, int pi, const btf_hx& hx) {  // the op's copy of the prep's fields
    o.prep = pi;
    if (pi < 0) return;
    const PrepDev& p = preps[(size_t)pi];
    o.normw = p.normw;
    o.signs = p.signs;
    o.eps = p.eps;
    o.hs = p.hs;
    o.block = p.block;
    o.prep_flags = prep_flags_of(p.normw, hx);
  };
  // ---- the device program: prologue quantize ops, embeddings, then the GEMVs in order
  std::vector<OpDev> ops;
  // known[v * G + w]: the last GEMV whose barrier B workgroup w has surely
  // passed, as far as workgroup v can tell when it reaches a later op. A
  // workgroup that owns units of an op reads all of its input (every unit
  // spans all slices), published unit by unit by the writers of the input's
  // producer X, each of which had passed B of the GEMV before X. Workgroup v
  // has passed B of every earlier op before starting an op.
  std::vector<int> known((size_t)G * G, -1);
  // allk[v]: the last GEMV whose barrier B every workgroup has surely
  // passed, as far as workgroup v can tell; ax[op]: what every writer of op
  // knew of all workgroups when it published (the minimum over them), which
  // a reader of op's output learns too (its writers published after
  // knowing it). If every workgroup writes units of an op, its readers know
  // that all had passed B of the GEMV before it.
  std::vector<int> allk(G, -1);
  std::vector<int> ax;  // per device op
  int last_gemv = -1;                   // device index of the previous GEMV
  std::vector<int> prev_gemv;           // per device op: the GEMV before it (-1: none)
  auto owns = [&](const OpDev& x, int w) { return (w - x.rot + G) % G < x.units; };
  std::vector<int> dev_of(nuops, -1);        // device op index of each user op
  std::vector<int> prologue_of(nvec, -1);    // device op index of each prologue op
  // Unit placement: unit u of an op goes to workgroup (u + rot) % G. An
  // add-mode op takes the rotation of the op that wrote its old value when
  // they have the same units, so each row's old value was published by the
  // same workgroup (no cross-workgroup wait on an add chain). Any other op
  // takes the rotation that keeps the most-loaded workgroup's weight bytes
  // lowest.
  std::vector<double> load(G, 0.0);
  auto place = [&](OpDev& o, double cost_per_unit, int align_to) {
    const int extra = o.units % G;
    int best = 0;
    if (align_to >= 0 && ops[align_to].units == o.units) {
      best = ops[align_to].rot;
    } else if (extra) {
      // the `extra` workgroups with one more unit form a window of length
      // extra starting at rot: pick the window with the least load
      double best_max = 1e300;
      for (int r = 0; r < G; ++r) {
        double mx = 0.0;
        for (int k = 0; k < extra; ++k) mx = std::max(mx, load[(r + k) % G]);
        if (mx < best_max) {
          best_max = mx;
          best = r;
        }
      }
    }
    o.rot = best;
    for (int w = 0; w < G; ++w) {
      const int first = (w - best + G) % G;
      const int n = first < o.units ? (o.units - 1 - first) / G + 1 : 0;
      load[w] += n * cost_per_unit;
    }
  };
  for (int v = 0; v < nvec; ++v) {
    if (versions[v].empty() || versions[v][0].writer >= 0) continue;
    OpDev o{};
    o.kind = 0;
    o.N = vecs[v].n;
    o.units = (o.N + 31) / 32;
    o.src = vecs[v].data;
    o.out_q8 = q8_of(v, 0);
    o.out_f32 = f32_of(v, 0);
    o.out_sq = versions[v][0].needs_sq;
    o.my_tag = (uint32_t)ops.size() + 1;
    o.war_op = -1;
    o.prep = -1;
    place(o, 1.0, -1);
    prologue_of[v] = (int)ops.size();
    ops.push_back(o);
    ax.push_back(-1);
    prev_gemv.push_back(-1);
  }
  for (int i = 0; i < nuops; ++i) {
    const btf_step_op& u = uops[i];
    if (u.kind != BTF_STEP_EMBED) continue;
    const int v = u.vec;
    const Version& ve = versions[v][out_ver[i]];
    OpDev o{};
    o.kind = 2;
    o.N = vecs[v].n;
    o.units = o.N / kSliceVals;
    o.codes = u.table_codes;
    o.scales = u.table_scales;
    o.src = u.d_tok;
    set_prep(o, add_prep(nullptr, 0.0f, u.hx, o.N), u.hx);
    o.out_plain = final_writer[v] == i ? vecs[v].data : nullptr;
    o.out_q8 = q8_of(v, out_ver[i]);
    o.out_f32 = f32_of(v, out_ver[i]);
    o.out_sq = ve.needs_sq;
    o.my_tag = (uint32_t)ops.size() + 1;
    o.war_op = -1;
    place(o, 1.0, -1);
    dev_of[i] = (int)ops.size();
    ops.push_back(o);
    ax.push_back(-1);
    prev_gemv.push_back(-1);
  }
  auto dev_writer = [&](int v, int k) {
    const int w = versions[v][k].writer;
    return w < 0 ? prologue_of[v] : dev_of[w];
  };
  for (int i = 0; i < nuops; ++i) {
    const btf_step_op& u = uops[i];
    if (u.kind != BTF_STEP_GEMV) continue;
    const btf_step_gemv& g = u.gemv;
    const int me = (int)ops.size();
    dev_of[i] = me;
    OpDev o{};
    o.kind = 1;
    o.mode = g.mode;
    o.K = g.K;
    o.N = g.N;
    o.units = (g.N + 31) / 32;
    o.cpr = g.K / 64;
    o.qpu_log2 = g.mode == BTF_GEMV_SWIGLU ? 4 : 3;
    o.codes = g.codes;
    o.scales = g.scales;
    o.up_codes = g.up_codes;
    o.up_scales = g.up_scales;
    const bool pre = has_prep(u);
    set_prep(o, pre ? add_prep(u.normw, u.eps, u.hx, g.K) : -1, u.hx);
    o.in_ll = pre ? f32_of(g.in_vec, in_ver[i]) : q8_of(g.in_vec, in_ver[i]);
    o.in_tag = (uint32_t)dev_writer(g.in_vec, in_ver[i]) + 1;
    o.argmax = i == pick_gemv;
    int align_to = -1;
    if (g.mode == BTF_GEMV_ADD) {
      o.old_f32 = f32_of(g.out_vec, old_ver[i]);
      o.old_tag = (uint32_t)dev_writer(g.out_vec, old_ver[i]) + 1;
      align_to = dev_writer(g.out_vec, old_ver[i]);
    }
    const int kv = out_ver[i];
    const Version& nv = versions[g.out_vec][kv];
    // Plain output: only the final version goes to the user's buffer (plain
    // stores of two ops to one address from different XCDs reach HBM in the
    // order their L2s write back, not in program order).
    o.out_plain = final_writer[g.out_vec] == i ? vecs[g.out_vec].data : nullptr;
    o.out_q8 = q8_of(g.out_vec, kv);
    o.out_f32 = f32_of(g.out_vec, kv);
    o.out_sq = nv.needs_sq;
    o.my_tag = (uint32_t)me + 1;
    place(o, (double)g.K * (g.mode == BTF_GEMV_SWIGLU ? 2 : 1), align_to);
    // Write-after-read: the buffers this version takes held the version
    // kSlots such versions earlier; wait until every workgroup has fetched the
    // input of its last reader. Old-value reads by an op with the same unit
    // placement are reads of the workgroup's own rows, already ordered by
    // program order. The final writer also stores into the user's buffer,
    // which the prologue read (version 0): after every reader of version 0.
    int war = -1;
    auto dev_reader = [&](int r) { return r >= 0 ? dev_of[r] : -1; };
    for (int k = kv - 1; k >= 0; --k) {
      const Version& pv = versions[g.out_vec][k];
      if (nv.q8_slot >= 0 && pv.q8_slot == nv.q8_slot) {
        war = std::max(war, dev_reader(pv.last_q8_reader));
        break;
      }
    }
    for (int k = kv - 1; k >= 0; --k) {
      const Version& pv = versions[g.out_vec][k];
      if (nv.f32_slot >= 0 && pv.f32_slot == nv.f32_slot) {
        war = std::max(war, dev_reader(pv.last_f32_reader));
        for (int r : pv.old_readers) {
          const OpDev& ro = ops[dev_of[r]];
          if (!(ro.units == o.units && ro.rot == o.rot)) war = std::max(war, dev_of[r]);
        }
        break;
      }
    }
    if (o.out_plain && versions[g.out_vec][0].writer < 0) {
      const Version& v0 = versions[g.out_vec][0];
      int last = std::max(v0.last_q8_reader, v0.last_f32_reader);
      for (int r : v0.old_readers) last = std::max(last, r);
      if (last >= 0 && last != i) war = std::max(war, dev_of[last]);
    }
    // What this op's writers learn from its input: they read all of the
    // first K values before publishing any unit (a unit spans every slice),
    // so it counts for this op's own guard -- but only the writers of the
    // input units below K are observed (an op without a prep may read a
    // prefix of a longer vector).
    {
      const int x = (int)o.in_tag - 1;  // input producer
      const int px = x < (int)prev_gemv.size() ? prev_gemv[x] : -1;
      if (ops[x].kind == 1) {
        const int nread = std::min(ops[x].units, (o.K + 31) / 32);
        auto observed = [&](int w) { return (w - ops[x].rot + G) % G < nread; };
        int a_in = ax[x];
        bool all_write = px >= 0;
        for (int w = 0; w < G && all_write; ++w) all_write = observed(w);
        if (all_write) a_in = std::max(a_in, px);
        for (int v = 0; v < G; ++v) {
          if (!owns(o, v)) continue;
          allk[v] = std::max(allk[v], a_in);
          if (px >= 0)
            for (int w = 0; w < G; ++w)
              if (observed(w)) known[(size_t)v * G + w] = std::max(known[(size_t)v * G + w], px);
        }
      }
    }
    if (war >= 0) {  // implied for every workgroup that writes this op's output?
      bool implied = true;
      for (int v = 0; v < G && implied; ++v) {
        if (!owns(o, v) || allk[v] >= war) continue;
        for (int w = 0; w < G; ++w)
          if (w != v && known[(size_t)v * G + w] < war) {
            implied = false;
            break;
          }
      }
      if (implied) war = -1;
    }
    {
      int axo = INT_MAX;
      for (int v = 0; v < G; ++v)
        if (owns(o, v)) axo = std::min(axo, allk[v]);
      ax.push_back(axo == INT_MAX ? -1 : axo);
    }
    o.war_op = war;
    if (war >= 0) ops[war].count_reads = 1;
    // per-workgroup LDS bounds: partial sums, old values of add-mode rows
    const int max_units = (o.units + G - 1) / G;
    const int rows = max_units * (g.mode == BTF_GEMV_SWIGLU ? 64 : 32);
    if (rows * ((o.cpr + 15) / 16) > kMaxPart) return bail(BTF_ERR_ARGS, "step: output too tall for the partial-sum buffer");
    if (g.mode == BTF_GEMV_ADD && max_units * 32 > kMaxOld)
      return bail(BTF_ERR_ARGS, "step: add-mode output too tall for the old-value buffer");
    ops.push_back(o);
    prev_gemv.push_back(last_gemv);
    last_gemv = me;
  }
  if ((int)ops.size() > kMaxOps) return bail(BTF_ERR_ARGS, "step: more than 300 ops (prologue + GEMVs)");
  // Early fetch and carry. An op's input is fetched by the I/O waves while
  // the previous GEMV computes when every producer it reads from comes
  // before that previous GEMV (a workgroup then never waits for its own
  // unpublished output) and it is a plain Q8 input (a prep runs in the
  // compute waves). An add-mode op whose old value was produced by the
  // previous GEMV with the same unit placement takes it from the LDS carry
  // (the same workgroup computed it) -- unless that GEMV is a swiglu, whose
  // epilogue keeps its rows in another layout and writes no carry.
  {
    int pd = -1;  // previous GEMV in program order
    for (int d = 0; d < (int)ops.size(); ++d) {
      OpDev& o = ops[d];
      if (o.kind != 1) continue;
      if (o.mode == BTF_GEMV_ADD && pd >= 0 && (int)o.old_tag - 1 == pd && ops[pd].mode != BTF_GEMV_SWIGLU &&
          ops[pd].units == o.units && ops[pd].rot == o.rot) {
        o.carry_in = 1;
        ops[pd].carry_out = 1;
      }
      const bool in_ok = (int)o.in_tag - 1 < pd;
      const bool no_old = o.mode != BTF_GEMV_ADD || o.carry_in;
      const bool fits = (o.K / 32) * kWordsPerBlock <= kIL * kEIn;  // one round of the I/O waves
      o.early = pd >= 0 && in_ok && no_old && fits && o.prep < 0;
      pd = d;
    }
  }
  // next GEMV after each op
  {
    int nxt = (int)ops.size();
    for (int i = (int)ops.size() - 1; i >= 0; --i) {
      ops[i].next = nxt;
      if (ops[i].kind == 1) nxt = i;
    }
    P->first = nxt;
  }
  HeadDev head{};
  if (pick) {
    head.present = 1;
    head.tag = (uint32_t)dev_of[pick_gemv] + 1;
    head.tok_out = pick->d_tok_out;
    head.pos = pick->d_pos;
    if (!(head.parts = static_cast<uint64_t*>(alloc((size_t)G * 2 * 8))))
      return bail(BTF_ERR_LAUNCH, "step: device allocation failed");
  }
  for (size_t t = 0; t < run_tables.size(); ++t) {
    int* d = static_cast<int*>(alloc(run_tables[t].size() * sizeof(int)));
    if (d && host) std::memcpy(d, run_tables[t].data(), run_tables[t].size() * sizeof(int));
    if (!d || (!host && hipMemcpy(d, run_tables[t].data(), run_tables[t].size() * sizeof(int),
                                  hipMemcpyHostToDevice) != hipSuccess))
      return bail(BTF_ERR_LAUNCH, "step: gather table upload failed");
    preps[run_of[t]].runs = d;
  }
  P->full = pick != nullptr || std::any_of(ops.begin(), ops.end(), [](const OpDev& o) { return o.prep >= 0 || o.kind == 2; });
  if (preps.empty()) preps.push_back(PrepDev{});
  P->nops = (int)ops.size();
  P->guards = (int)std::count_if(ops.begin(), ops.end(), [](const OpDev& o) { return o.war_op >= 0; });
  if (!(P->d_ops = static_cast<OpDev*>(alloc(ops.size() * sizeof(OpDev)))) ||
      !(P->d_ctl = static_cast<Ctl*>(alloc(sizeof(Ctl)))) ||
      !(P->d_cnt = static_cast<uint32_t*>(alloc(256 * sizeof(uint32_t)))) ||
      !(P->d_preps = static_cast<PrepDev*>(alloc(preps.size() * sizeof(PrepDev)))) ||
      !(P->d_head = static_cast<HeadDev*>(alloc(sizeof(HeadDev)))))
    return bail(BTF_ERR_LAUNCH, "step: device allocation failed");
  const Ctl c0{1u, 0u, 0u, 0u};
  if (host) {
    P->plan_ops = ops;
    P->plan_preps = preps;
    P->plan_head = head;
    *P->d_ctl = c0;
    *out = P;
    return BTF_OK;
  }
  if (hipMemcpy(P->d_ops, ops.data(), ops.size() * sizeof(OpDev), hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(P->d_ctl, &c0, sizeof c0, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(P->d_preps, preps.data(), preps.size() * sizeof(PrepDev), hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(P->d_head, &head, sizeof head, hipMemcpyHostToDevice) != hipSuccess)
    return bail(BTF_ERR_LAUNCH, "step: program upload failed");
  (void)hipGetDevice(&P->device);
  *out = P;
  return BTF_OK;
}
}  // namespace

int step_create_ops(const btf_step_vec* vecs, int nvec, const btf_step_op* uops, int nuops, StepProgram** out,
                    const DevState& ds) {
  return step_build(vecs, nvec, uops, nuops, out, &ds, 0);
}

// The global stores of a program's launch, replayed on the host over every
// workgroup with the kernel's own placement and address functions
// (first_unit, units_of, unit_row, q8_block_word, sq_word, slice_col,
// pick_word) and the store pattern of publish_unit, publish_slice,
// io_quantize, io_embed, io_publish, io_waves, io_pick and the kernel's
// epilogue; each store must lie inside a buffer the program owns or one it
// was given (a vector's data, the pick's token and position).
int step_audit(const btf_step_vec* vecs, int nvec, const btf_step_op* uops, int nuops, int G, btf_step_audit* res) {
  if (G <= 0 || G > 256) return fail(BTF_ERR_ARGS, "step audit: G must be in 1..256");
  StepProgram* P = nullptr;
  if (const int rc = step_build(vecs, nvec, uops, nuops, &P, nullptr, G)) return rc;
  struct Range {
    uintptr_t a, b;
    const char* what;
  };
  std::vector<Range> rs;
  for (size_t i = 0; i < P->bufs.size(); ++i)
    rs.push_back({reinterpret_cast<uintptr_t>(P->bufs[i]), reinterpret_cast<uintptr_t>(P->bufs[i]) + P->buf_bytes[i],
                  "program buffer"});
  for (int v = 0; v < nvec; ++v)
    if (vecs[v].data)
      rs.push_back({reinterpret_cast<uintptr_t>(vecs[v].data),
                    reinterpret_cast<uintptr_t>(vecs[v].data) + 4 * (size_t)vecs[v].n, "vector data"});
  const HeadDev& head = P->plan_head;
  if (head.present) {
    rs.push_back({reinterpret_cast<uintptr_t>(head.tok_out), reinterpret_cast<uintptr_t>(head.tok_out) + 4, "token"});
    if (head.pos)
      rs.push_back({reinterpret_cast<uintptr_t>(head.pos), reinterpret_cast<uintptr_t>(head.pos) + 4, "position"});
  }
  std::sort(rs.begin(), rs.end(), [](const Range& x, const Range& y) { return x.a < y.a; });
  *res = btf_step_audit{};
  res->ops = P->nops;
  res->guards = P->guards;
  res->full = P->full ? 1 : 0;
  auto store = [&](const void* p, size_t bytes, int op, int wg, const char* site) {
    ++res->stores;
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    auto it = std::upper_bound(rs.begin(), rs.end(), a, [](uintptr_t x, const Range& r) { return x < r.a; });
    if (it != rs.begin() && a >= std::prev(it)->a && a + bytes <= std::prev(it)->b) return;
    if (res->outside++ == 0)
      std::snprintf(res->first_outside, sizeof res->first_outside, "op %d workgroup %d: %s, %zu bytes at %p", op, wg,
                    site, bytes, p);
  };
  auto unit_stores = [&](const OpDev& o, int d, int wg, int unit) {  // publish_unit, j = 0..31
    for (int j = 0; j < 32; ++j) {
      const int row = unit_row(unit, j);
      const bool valid = row < o.N;
      if (valid && o.out_plain) store(o.out_plain + row, 4, d, wg, "plain output");
      if (valid && o.out_f32) store(o.out_f32 + row, 8, d, wg, "fp32 LL word");
      if (o.out_q8) {
        uint64_t* dst = o.out_q8 + q8_block_word(unit);
        if ((j & 3) == 0) store(dst + (j >> 2), 8, d, wg, "Q8 q word");
        if (j == 0) store(dst + 8, 8, d, wg, "Q8 d word");
        if (j == 1) store(dst + 9, 8, d, wg, "Q8 s word");
      }
      if (o.out_sq && j == 0) {
        store(o.out_f32 + sq_word(o.N, unit), 8, d, wg, "sum of squares (low)");
        store(o.out_f32 + sq_word(o.N, unit) + 1, 8, d, wg, "sum of squares (high)");
      }
    }
  };
  for (int wg = 0; wg < G; ++wg) {
    for (int d = 0; d < P->nops; ++d) {
      const OpDev& o = P->plan_ops[(size_t)d];
      const int first = first_unit(o.rot, wg, G);
      if (o.kind == 0) {  // io_quantize: half-waves 0..3, units first + h G + 4 G t
        for (int h = 0; h < 2 * kIW; ++h)
          for (int u = first + h * G; u < o.units; u += 2 * kIW * G) unit_stores(o, d, wg, u);
      } else if (o.kind == 2) {  // io_embed: I/O waves 0..1, units first + w G + 2 G t; publish_slice per lane
        for (int iw = 0; iw < kIW; ++iw)
          for (int u = first + iw * G; u < o.units; u += kIW * G)
            for (int lane = 0; lane < 64; ++lane) {
              const int c0 = slice_col(u, lane), blk = c0 >> 5, h = lane & 1;
              if (o.out_plain) store(o.out_plain + c0, 64, d, wg, "plain output (slice)");
              if (o.out_f32)
                for (int i = 0; i < 16; ++i) store(o.out_f32 + c0 + i, 8, d, wg, "fp32 LL word (slice)");
              if (o.out_sq && !h) {
                store(o.out_f32 + sq_word(o.N, blk), 8, d, wg, "sum of squares (slice)");
                store(o.out_f32 + sq_word(o.N, blk) + 1, 8, d, wg, "sum of squares (slice)");
              }
              if (o.out_q8) {
                uint64_t* dst = o.out_q8 + q8_block_word(blk);
                for (int k = 0; k < 4; ++k) store(dst + 4 * h + k, 8, d, wg, "Q8 q word (slice)");
                if (!h) {
                  store(dst + 8, 8, d, wg, "Q8 d word (slice)");
                  store(dst + 9, 8, d, wg, "Q8 s word (slice)");
                }
              }
            }
      } else {  // io_publish: local units ui = half + 4 t of the workgroup's nunits
        const int nunits = units_of(o.units, first, G);
        for (int half = 0; half < 2 * kIW; ++half)
          for (int ui = half; ui < nunits; ui += 2 * kIW) unit_stores(o, d, wg, first + ui * G);
        if (o.count_reads) store(P->d_cnt + wg, 4, d, wg, "progress word");
        if (o.argmax) {
          store(head.parts + pick_word(wg), 8, d, wg, "pick key (low)");
          store(head.parts + pick_word(wg) + 1, 8, d, wg, "pick key (high)");
        }
      }
    }
    if (wg == 0 && head.present) {  // io_pick
      store(head.tok_out, 4, P->nops, wg, "token");
      if (head.pos) store(head.pos, 4, P->nops, wg, "position");
    }
    // set_abort, the end-of-step count and the epoch advance
    store(&P->d_ctl->error, 4, P->nops, wg, "control: error");
    store(&P->d_ctl->done, 4, P->nops, wg, "control: done");
    store(&P->d_ctl->epoch, 4, P->nops, wg, "control: epoch");
  }
  step_destroy(P);
  return BTF_OK;
}

int step_create(const btf_step_vec* vecs, int nvec, const btf_step_gemv* gemvs, int ngemv, StepProgram** out,
                const DevState& ds) {
  const std::vector<btf_step_op> ops = step_ops_of(gemvs, ngemv);
  return step_create_ops(vecs, nvec, ops.data(), ngemv, out, ds);
}

int step_set_spin_limit(StepProgram* P, uint32_t polls) {
  if (hipMemcpy(&P->d_ctl->spin_max, &polls, sizeof polls, hipMemcpyHostToDevice) != hipSuccess)
    return fail(BTF_ERR_LAUNCH, "step: control block write failed");
  return BTF_OK;
}

int step_check_residency(const DevState& ds) {
  int dev = 0, coop = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess)
    return fail(BTF_ERR_DEVICE, "step: device query failed");
  if (!coop) return fail(BTF_ERR_DEVICE, "step: the device does not support cooperative launches");
  int per_cu = 0;
  for (const void* k : {reinterpret_cast<const void*>(step_kernel<false>), reinterpret_cast<const void*>(step_kernel<true>)}) {
    const int threads = k == reinterpret_cast<const void*>(step_kernel<true>) ? threads_of<true>() : threads_of<false>();
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, threads, 0) != hipSuccess)
      return fail(BTF_ERR_LAUNCH, "step: occupancy query failed");
    if (per_cu < 1) return fail(BTF_ERR_LAUNCH, "step: the step kernel does not fit on a CU");
  }
  (void)ds;
  return BTF_OK;
}

int step_launch(StepProgram* P, hipStream_t st) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != P->device)
    return fail(BTF_ERR_ARGS, "step: launch on a device other than the program's");
  void* args[] = {&P->d_ops, &P->nops, &P->first, &P->d_ctl, &P->d_cnt, &P->d_preps, &P->d_head};
  const hipError_t e =
      hipLaunchCooperativeKernel(P->full ? reinterpret_cast<const void*>(step_kernel<true>)
                                         : reinterpret_cast<const void*>(step_kernel<false>),
                                 dim3(P->G), dim3(P->full ? threads_of<true>() : threads_of<false>()), args, 0, st);
  if (e != hipSuccess) return fail(BTF_ERR_LAUNCH, std::string("step kernel: ") + hipGetErrorString(e));
  return launch_status("step_kernel");
}

int step_guards(StepProgram* P, int* guards) {
  *guards = P->guards;
  return BTF_OK;
}

int step_error(StepProgram* P, int* err) {
  Ctl c{};
  if (hipMemcpy(&c, P->d_ctl, sizeof c, hipMemcpyDeviceToHost) != hipSuccess)
    return fail(BTF_ERR_LAUNCH, "step: control block read failed");
  *err = c.error != 0;
  if (c.error) {
    const uint32_t zero = 0;
    if (hipMemcpy(&P->d_ctl->error, &zero, sizeof zero, hipMemcpyHostToDevice) != hipSuccess)
      return fail(BTF_ERR_LAUNCH, "step: control block write failed");
  }
  return BTF_OK;
}

}  // namespace btfhip

