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
#include <cstring>
#include <vector>

#include "../../include/btf/hip_abi.h"
#include "common.h"

namespace btfhip {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kCW = 10;                     // compute waves
constexpr int kIW = 2;                      // I/O waves
constexpr int kThreads = 64 * (kCW + kIW);  // 768
constexpr int kRing = 8;                    // weight items (16 B per lane) in flight per compute wave
constexpr int kMaxK = 20480;                // widest GEMV input
constexpr int kMaxPart = 8192;              // partial sums per op per workgroup
constexpr int kMaxOps = 384;                // ops per program (descriptors live in LDS)
constexpr int kMaxOld = 1024;               // rows per workgroup of an add-mode op (the LDS carry)
constexpr int kMaxUnits = 256;              // units of one op per workgroup (kMaxPart / 32)
constexpr int kWordsPerBlock = 10;          // LL words per 32-value Q8 block
constexpr int kSlots = 3;                   // LL buffers of each kind per vector (versions in turn)
constexpr uint32_t kSpinMax = 1u << 20;     // poll bound (each poll is a memory round trip: ~1 s)

// 144 bytes (a multiple of 16: copied into LDS in 16-byte words).
struct OpDev {
  int kind;  // 0 = quantize a user vector (prologue), 1 = GEMV
  int mode;
  int K, N;
  int cpr;
  int units, rot, qpu_log2;  // 32-row units, unit rotation, log2 row quads per unit (3; swiglu 4)
  int next;                  // index of the next GEMV op (nops: none)
  int count_reads;           // 1: count the workgroups that have fetched this op's input
  int war_op;                // >= 0: wait until every workgroup has fetched that op's input
                             // (the last reader of the version this op overwrites)
  uint32_t in_tag;           // relative tag of the input's producer
  uint32_t old_tag;          // add mode: relative tag of the output's previous version
  uint32_t my_tag;
  uint8_t early;      // 1: the I/O waves fetch this op's input during the previous op
  uint8_t carry_in;   // 1: add-mode old values come from the previous op's epilogue (LDS carry)
  uint8_t carry_out;  // 1: the epilogue keeps its outputs in the LDS carry for the next op
  uint8_t pad0;
  int pad1;
  const uint8_t* codes;
  const uint16_t* scales;
  const uint8_t* up_codes;
  const uint16_t* up_scales;
  const uint64_t* in_q8;    // LL Q8 words of the input vector
  float* out_plain;         // user output (nullable)
  uint64_t* out_f32;        // LL fp32 of the output vector (nullable)
  uint64_t* out_q8;         // LL Q8 of the output vector (nullable)
  const uint64_t* old_f32;  // add mode: previous value of the output vector
  const float* src;         // quantize op: user vector
};
static_assert(sizeof(OpDev) == 144, "descriptor layout");

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

struct Lds {
  OpDev opd[kMaxOps];        // the program
  uint32_t act_q[2][kMaxK / 4];  // q bytes of an op's input (by op parity)
  float act_d[2][kMaxK / 32];    // d
  int32_t act_s[2][kMaxK / 32];  // s
  float part[kMaxPart];       // [1024-column slice][local row]
  float carry[kMaxOld];       // outputs of the workgroup's rows kept for the next (add-mode) op
  uint32_t ucnt[kCW][kMaxUnits];  // per compute wave: items of each local unit of the current op it has done
  uint32_t early_seq[kIW];    // per I/O wave: op index + 1 of the last input it fetched early
  uint32_t epoch;
  uint32_t abort_;
  uint32_t spin_max;
};

__device__ __forceinline__ bool aborted(Lds& L) {
  return __hip_atomic_load(&L.abort_, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0;
}
// Has another workgroup of this launch failed?
__device__ __forceinline__ bool grid_failed(const Ctl* ctl, const Lds& L) {
  return __hip_atomic_load(&ctl->error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == L.epoch;
}
// The error word holds the epoch of the failing launch, so a failure that the
// host has not cleared yet does not abort later launches.
__device__ __forceinline__ void set_abort(Lds& L, Ctl* ctl) {
  __hip_atomic_store(&ctl->error, L.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(&L.abort_, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ int sgpr(int v) { return __builtin_amdgcn_readfirstlane(v); }
template <class T>
__device__ __forceinline__ T* sgpr_ptr(T* p) {
  const uint64_t u = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

// First workgroup-local unit of an op: units u with u % G == (wg - rot) mod G.
__device__ __forceinline__ int first_unit(int rot, int wg, int G) {
  const int f = wg - rot;
  return f < 0 ? f + G : f;
}
__device__ __forceinline__ int units_of(int units, int first, int G) {
  return first < units ? (units - 1 - first) / G + 1 : 0;
}

// ---------------------------------------------------------------- input fetch
__device__ __forceinline__ bool poll_step(uint32_t& spins, Lds& L, Ctl* ctl) {
  if (aborted(L)) return false;
  if (++spins > L.spin_max || ((spins & 255) == 0 && grid_failed(ctl, L))) {
    set_abort(L, ctl);
    return false;
  }
  __builtin_amdgcn_s_sleep(1);
  return true;
}

// Fetch LL words [a0, a1) and [b0, b1) of an op's input (its Q8 words, tag = the input
// producer's) into LDS buffer `ob`, by the 64 lanes of one compute wave in
// rounds of kFB words per lane, polling until every tag matches. A slice
// whose items two waves share is fetched by both: the same values land twice.
constexpr int kFB = 10;
__device__ __forceinline__ void fetch_words(const OpDev& op, Lds& L, int lane, Ctl* ctl, uint32_t base_tag, int ob,
                                            int a0, int a1, int b0, int b1) {
  const uint64_t* in = sgpr_ptr(op.in_q8);
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
    for (int b = 0; b < kFB; ++b) {
      const int idx = at[b];
      if (idx >= 0) {
        const uint32_t data = (uint32_t)v[b];
        const int blk = idx / kWordsPerBlock, w = idx - blk * kWordsPerBlock;
        if (w < 8)
          L.act_q[ob][blk * 8 + w] = data;
        else if (w == 8)
          L.act_d[ob][blk] = __uint_as_float(data);
        else
          L.act_s[ob][blk] = (int32_t)data;
      }
    }
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
  const uint64_t* in = sgpr_ptr(op.in_q8);
  const uint32_t tin = base_tag + sgpr(op.in_tag);
  const int nin = (sgpr(op.K) / 32) * kWordsPerBlock;
#pragma unroll
  for (int b = 0; b < kEIn; ++b) {
    const int idx = lid + b * kIL;
    f.v[b] = idx < nin ? ll_load(in + idx) : ((uint64_t)tin << 32);
  }
}
__device__ __forceinline__ void early_finish(const OpDev& op, int lid, uint32_t base_tag, EarlyFetch& f, Lds& L, int ob,
                                             Ctl* ctl) {
  const uint64_t* in = sgpr_ptr(op.in_q8);
  const uint32_t tin = base_tag + sgpr(op.in_tag);
  const int nin = (sgpr(op.K) / 32) * kWordsPerBlock;
  uint32_t spins = 0;
  for (;;) {
    uint32_t pending = 0;
#pragma unroll
    for (int b = 0; b < kEIn; ++b) pending |= ((uint32_t)(f.v[b] >> 32) != tin) ? (1u << b) : 0u;
    if (pending == 0) break;
    if (!poll_step(spins, L, ctl)) break;
    for (int b = 0; b < kEIn; ++b) {
      const int idx = lid + b * kIL;
      if ((pending & (1u << b)) && idx < nin) f.v[b] = ll_load(in + idx);
    }
  }
#pragma unroll
  for (int b = 0; b < kEIn; ++b) {
    const int idx = lid + b * kIL;
    if (idx < nin) {
      const uint32_t data = (uint32_t)f.v[b];
      const int blk = idx / kWordsPerBlock, w = idx - blk * kWordsPerBlock;
      if (w < 8)
        L.act_q[ob][blk * 8 + w] = data;
      else if (w == 8)
        L.act_d[ob][blk] = __uint_as_float(data);
      else
        L.act_s[ob][blk] = (int32_t)data;
    }
  }
}

// ---------------------------------------------------------------- compute waves
typedef const __attribute__((address_space(1))) u32x4 gvec4;
typedef const __attribute__((address_space(1))) _Float16 gf16;

// The fields of an op the compute waves need, in SGPRs (read from LDS and
// made uniform, so lane-dependent selects never become vector loads).
struct OpR {
  int mode, K, N, cpr, units, rot, qpu_log2, next;
  const uint8_t* codes;
  const uint16_t* scales;
  const uint8_t* up_codes;
  const uint16_t* up_scales;
};
__device__ __forceinline__ OpR op_r(const Lds& L, int i) {
  const OpDev& o = L.opd[i];
  OpR r;
  r.mode = sgpr(o.mode);
  r.K = sgpr(o.K);
  r.N = sgpr(o.N);
  r.cpr = sgpr(o.cpr);
  r.units = sgpr(o.units);
  r.rot = sgpr(o.rot);
  r.qpu_log2 = sgpr(o.qpu_log2);
  r.next = sgpr(o.next);
  r.codes = sgpr_ptr(o.codes);
  r.scales = sgpr_ptr(o.scales);
  r.up_codes = sgpr_ptr(o.up_codes);
  r.up_scales = sgpr_ptr(o.up_scales);
  return r;
}

// Work of an op inside a workgroup: items (unit u, K-slice s, row quad q),
// u < the workgroup's units of the op, s < S (1024-column slices), q < Qu
// (quads of a unit: 4 rows each, or for swiglu 2 gate + 2 up rows), in the
// order t = (u*S + s)*Qu + q: a unit's items are consecutive, so the I/O
// waves can publish each unit as soon as it is done, and the items of a
// compute wave touch few slices of the input. One item is one 16-byte code
// chunk (64 columns) per lane: lane l reads chunk s*16 + (l & 15) of row
// quad row + (l >> 4).
struct Slot {
  u32x4 c;
  _Float16 s;  // fp16 scale of the chunk's 128-column block
};

// The items of an op are cut into batches of kRing, and each compute wave
// takes a contiguous run of whole batches (so only the op's last batch in
// the workgroup is partial); a wave with no batch runs one batch of dummies,
// which keeps every wave's ring in step across ops. Entries past n are
// dummies (dummy load, no store).
struct OpWork {
  int i;  // op index (>= nops: past the program's end; every entry is a dummy)
  OpR op;
  int S, Qu, Q, first;  // slices, quads per unit, quads of the workgroup, first unit
  int t0, n, P;         // the wave's first item, real items, entries (a multiple of kRing)
  int u0, s0, q0;       // (u, s, q) of item t0
};
// Every field is assigned on every path (a partly assigned struct would be
// kept in scratch memory, whose accesses count in vmcnt).
__device__ __forceinline__ OpWork op_work(const Lds& L, int nops, int wave, int wg, int G, int i, const OpR& prev) {
  OpWork w;
  const bool past = i >= nops;  // past the end: the previous op's pointers stay valid dummy addresses
  w.i = i;
  w.op = past ? prev : op_r(L, i);
  w.first = first_unit(w.op.rot, wg, G);
  const int nunits = past ? 0 : units_of(w.op.units, w.first, G);
  w.S = (w.op.cpr + 15) >> 4;
  w.Qu = 1 << w.op.qpu_log2;
  w.Q = nunits << w.op.qpu_log2;
  const int U = w.S << w.op.qpu_log2;  // items per unit
  const int T = nunits * U;
  // Batches are balanced over the four SIMDs, not over the waves: wave w
  // sits on SIMD w % 4, SIMDs 0 and 1 hold three compute waves and SIMDs 2
  // and 3 two (beside the I/O waves), and a SIMD's waves mostly run one after
  // another (the oldest issues first), so an op ends when its busiest SIMD
  // does. SIMD k takes B/4 batches (the first B % 4 SIMDs one more), split
  // over its waves the same way; runs follow in SIMD-major wave order.
  const int B = (T + kRing - 1) / kRing;
  const int simd = wave & 3, slot = wave >> 2;         // slot: the wave's rank on its SIMD
  const int nws = simd < kCW - 8 ? 3 : 2;              // compute waves on this SIMD
  const int bs = B / 4 + (simd < B % 4 ? 1 : 0);       // batches of this SIMD
  const int sb0 = simd * (B / 4) + (simd < B % 4 ? simd : B % 4);  // its first batch
  const int b0 = sb0 + slot * (bs / nws) + (slot < bs % nws ? slot : bs % nws);
  const int b1 = b0 + bs / nws + (slot < bs % nws ? 1 : 0);
  w.t0 = b0 * kRing;
  const int t1 = b1 * kRing < T ? b1 * kRing : T;
  w.n = t1 > w.t0 ? t1 - w.t0 : 0;
  w.P = (b1 > b0 ? b1 - b0 : 1) * kRing;
  const int ua = U ? w.t0 / U : 0, ra = w.t0 - ua * U;
  w.u0 = ua;
  w.s0 = ra >> w.op.qpu_log2;
  w.q0 = ra & (w.Qu - 1);
  return w;
}

// The input slices the wave's real items read, as input LL word ranges
// [a0, a1) and [b0, b1) (one of them, or both, may be empty): the items run
// from (u0, s0) to the last one's (ub, sb).
__device__ __forceinline__ void input_words(const OpWork& w, int& a0, int& a1, int& b0, int& b1) {
  constexpr int kWS = 32 * kWordsPerBlock;  // input words per slice
  const int U = w.S << w.op.qpu_log2;
  const int tl = w.t0 + w.n - 1;
  const int ub = tl / U, sb = (tl - ub * U) >> w.op.qpu_log2;
  a0 = a1 = b0 = b1 = 0;
  if (ub == w.u0) {
    a0 = w.s0 * kWS, a1 = (sb + 1) * kWS;
  } else if (ub == w.u0 + 1 && sb + 1 < w.s0) {
    a0 = w.s0 * kWS, a1 = w.S * kWS, b1 = (sb + 1) * kWS;
  } else {
    a1 = w.S * kWS;
  }
}

// Per-op, per-lane part of the load addresses: the lane's matrix (swiglu: odd
// row groups read the up matrix), its row within the quad and its chunk
// within the slice. A step program has K % 1024 == 0, so every chunk of
// every slice is inside the row.
struct LaneAddr {
  uintptr_t cbase, sbase;  // codes / scales of (quad row 0, slice 0) for this lane
};
__device__ __forceinline__ LaneAddr lane_addr(const OpR& op, int l16, int grp) {
  LaneAddr a;
  const bool swiglu = op.mode == BTF_GEMV_SWIGLU;
  const bool up = swiglu && (grp & 1);
  const int rq = swiglu ? (grp >> 1) : grp;  // row within the quad
  const uintptr_t cm = up ? reinterpret_cast<uintptr_t>(op.up_codes) : reinterpret_cast<uintptr_t>(op.codes);
  const uintptr_t sm = up ? reinterpret_cast<uintptr_t>(op.up_scales) : reinterpret_cast<uintptr_t>(op.scales);
  a.cbase = cm + (size_t)rq * (op.K >> 2) + (size_t)l16 * 16;
  a.sbase = sm + (size_t)rq * (op.K >> 6) + (size_t)(l16 >> 1) * 2;
  return a;
}

// (u, s, q) cursor advanced without divisions.
struct Cur {
  int u, s, q;
};
__device__ __forceinline__ void cur_next(int Qu, int S, Cur& c) {
  if (++c.q == Qu) {
    c.q = 0;
    if (++c.s == S) {
      c.s = 0;
      ++c.u;
    }
  }
}

// Load item (u, s, q) into a ring slot, or (real == false) the lane's chunk of
// the op's first quad and slice, so every refill is an unconditional load
// into the slot's own registers. The item's offset is uniform (SGPRs); quads
// past N (N % 4 == 0, swiglu N % 2 == 0: a quad is all in or all out) read
// quad 0.
__device__ __forceinline__ void issue_item(const OpR& op, const LaneAddr& la, int first, const Cur& c, bool real,
                                           int G, Slot& sl) {
  int row0 = (first + c.u * G) * 32 + (op.mode == BTF_GEMV_SWIGLU ? 2 * c.q : 4 * c.q);
  row0 = real && row0 < op.N ? row0 : 0;
  const int s = real ? c.s : 0;
  // 32-bit uniform offsets (a matrix is below 4 GB, checked on the host)
  const uint32_t co = (uint32_t)row0 * (uint32_t)(op.K >> 2) + (uint32_t)s * 256u;
  const uint32_t so = (uint32_t)row0 * (uint32_t)(op.K >> 6) + (uint32_t)s * 16u;
  sl.c = __builtin_nontemporal_load(reinterpret_cast<gvec4*>(la.cbase + co));
  sl.s = __builtin_nontemporal_load(reinterpret_cast<gf16*>(la.sbase + so));
}

// The activation of this lane's chunk of slice s (64 q bytes, d/16, -s of
// its two sub-blocks). The 4 row groups of a wave read the same addresses
// (LDS broadcasts).
__device__ __forceinline__ void load_act(const Lds& L, int ob, int s, int l16, uint32_t (&aq)[16], float (&ad)[2],
                                         int (&an)[2]) {
  const int chunk = s * 16 + l16;
  const u32x4* qp = reinterpret_cast<const u32x4*>(&L.act_q[ob][chunk * 16]);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32x4 v = qp[i];
    aq[4 * i] = v.x;
    aq[4 * i + 1] = v.y;
    aq[4 * i + 2] = v.z;
    aq[4 * i + 3] = v.w;
  }
  const float2 d = *reinterpret_cast<const float2*>(&L.act_d[ob][2 * chunk]);
  const int2 sv = *reinterpret_cast<const int2*>(&L.act_s[ob][2 * chunk]);
  ad[0] = d.x * 0.0625f;  // exact: the dot returns 16 * I
  ad[1] = d.y * 0.0625f;
  an[0] = -sv.x;
  an[1] = -sv.y;
}

// dot4 with a zero accumulator in one VOP3P instruction (the builtin with a
// constant 0 becomes a register clear plus the two-operand form).
__device__ __forceinline__ int sdot4_0(uint32_t a, uint32_t b) {
  int r;
  asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
// subblock_dot16 (common.h) with the zero-started chains in VOP3P form; the
// same integer result.
__device__ __forceinline__ int subblock_dot16_z(uint32_t w0, uint32_t w1, const uint32_t* a, int ns) {
  int c0 = sdot4(w0 & 0x03030303u, a[0], ns);
  c0 = sdot4(w1 & 0x03030303u, a[4], c0);
  int c1 = sdot4_0(w0 & 0x0C0C0C0Cu, a[1]);
  c1 = sdot4(w1 & 0x0C0C0C0Cu, a[5], c1);
  int c2 = sdot4_0(w0 & 0x30303030u, a[2]);
  c2 = sdot4((w0 >> 2) & 0x30303030u, a[3], c2);
  c2 = sdot4(w1 & 0x30303030u, a[6], c2);
  c2 = sdot4((w1 >> 2) & 0x30303030u, a[7], c2);
  return (((c0 << 2) + c1) << 2) + c2;
}

// One consumed entry: the dot products of ring slot `sl` (read before the
// slot is refilled), then the refill.
struct Consumed {
  int y0, y1;
  float f;
};
__device__ __forceinline__ Consumed consume(const Slot& sl, const uint32_t (&aq)[16], const int (&an)[2]) {
  // The empty asm keeps the fp16 -> f32 conversion from being folded into a
  // later v_fma_mix that would read the slot after the refill.
  Consumed r;
  const u32x4 wv = sl.c;
  r.f = (float)sl.s;
  asm volatile("" : "+v"(r.f));
  r.y0 = subblock_dot16_z(wv.x, wv.y, &aq[0], an[0]);
  r.y1 = subblock_dot16_z(wv.z, wv.w, &aq[8], an[1]);
  return r;
}
// Finish an entry: scale, 16-lane DPP reduction, store of the slice's
// partial sum of the row into LDS part[s][local row], then the wave's count
// of done items of the unit (a plain store of a uniform value: LDS
// operations of a wave complete in order, so the I/O waves see the partial
// sums once they see the count).
__device__ __forceinline__ void finish(const Consumed& c, const float (&ad)[2], bool store, int part_idx,
                                       uint32_t* count, uint32_t done, int lane, Lds& L) {
  float p = ad[0] * (float)c.y0;
  p = fmaf(ad[1], (float)c.y1, p);
  float acc = c.f * p;
  acc = row16_sum(acc);
  if (store) {
    if ((lane & 15) == 0) L.part[part_idx] = acc;
    asm volatile("" ::: "memory");
    *count = done;
  }
}

// The compute waves' whole program. Per op: wait for the input slices the
// wave's items read (fetch them, or for an early op wait until the I/O waves
// have), the op's batches of kRing entries, barrier B (every wave done with
// the op). Entry e of the op lives in ring slot e % kRing; consuming it
// refills the slot with entry e + kRing of the op, and in the op's last
// batch (a separate copy of the loop body) with entry e + kRing - P of the
// NEXT op: the ring stays full across op boundaries (the next op's first
// loads are in flight while this op finishes and while the wave waits for
// its input), with no dummy loads to drain. Each copy of the body is
// straight-line code with one unconditional load pair per entry, so the
// compiler keeps each slot in fixed registers with exact wait counts. The
// activation stays in registers and is reloaded from LDS when the slice
// changes.
__device__ __forceinline__ void compute_waves(Lds& L, int nops, int first, int wave, int lane, int wg, int G, Ctl* ctl,
                                              uint32_t base_tag) {
  const int l16 = lane & 15, grp = lane >> 4;
  Slot ring[kRing];
  OpWork cur = op_work(L, nops, wave, wg, G, first, op_r(L, first));
  OpWork nxt = op_work(L, nops, wave, wg, G, cur.op.next, cur.op);
  LaneAddr la_cur = lane_addr(cur.op, l16, grp);
  LaneAddr la_nxt = lane_addr(nxt.op, l16, grp);
  {
    Cur c{cur.u0, cur.s0, cur.q0};
#pragma unroll
    for (int r = 0; r < kRing; ++r) {
      issue_item(cur.op, la_cur, cur.first, c, r < cur.n, G, ring[r]);
      cur_next(cur.Qu, cur.S, c);
    }
  }
  for (;;) {
    const int ob = cur.i & 1;  // LDS buffers of this op
    if (cur.n > 0) {
      if (sgpr(L.opd[cur.i].early)) {
        // fetched by the I/O waves after the previous op's barrier B
        uint32_t spins = 0;
        for (;;) {
          bool ready = true;
#pragma unroll
          for (int k = 0; k < kIW; ++k)
            ready &= __hip_atomic_load(&L.early_seq[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) ==
                     (uint32_t)cur.i + 1;
          if (ready || !poll_step(spins, L, ctl)) break;
        }
        asm volatile("" ::: "memory");
      } else {
        int a0, a1, b0, b1;
        input_words(cur, a0, a1, b0, b1);
        fetch_words(L.opd[cur.i], L, lane, ctl, base_tag, ob, a0, a1, b0, b1);
        // the words other lanes of this wave wrote are read below
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      }
    }
    const int R = cur.Q * 4;  // rows (virtual: swiglu gate/up interleaved) of this workgroup
    const int U = cur.S << cur.op.qpu_log2;  // items per unit
    Cur cc{cur.u0, cur.s0, cur.q0};  // entry being consumed
    Cur lc = cc;                     // entry being loaded (kRing ahead)
#pragma unroll
    for (int r = 0; r < kRing; ++r) cur_next(cur.Qu, cur.S, lc);
    uint32_t aq[16];
    float ad[2];
    int an[2];
    load_act(L, ob, cc.s, l16, aq, ad, an);
    const int nb = cur.P / kRing;
    for (int b = 0; b < nb - 1; ++b) {
#pragma unroll
      for (int r = 0; r < kRing; ++r) {
        const int e = b * kRing + r;
        const Consumed c = consume(ring[r], aq, an);
        __builtin_amdgcn_sched_barrier(0);
        issue_item(cur.op, la_cur, cur.first, lc, e + kRing < cur.n, G, ring[r]);
        __builtin_amdgcn_sched_barrier(0);
        cur_next(cur.Qu, cur.S, lc);
        finish(c, ad, e < cur.n, cc.s * R + ((cc.u << cur.op.qpu_log2) + cc.q) * 4 + grp, &L.ucnt[wave][cc.u],
               (uint32_t)(cur.t0 + e + 1 - max(cur.t0, cc.u * U)), lane, L);
        const int s_prev = cc.s;
        cur_next(cur.Qu, cur.S, cc);
        if (cc.s != s_prev) load_act(L, ob, cc.s, l16, aq, ad, an);
      }
    }
    if (cur.n == 0) {  // no real entry: only the refills with the next op's first entries
      Cur ln{nxt.u0, nxt.s0, nxt.q0};
#pragma unroll
      for (int r = 0; r < kRing; ++r) {
        issue_item(nxt.op, la_nxt, nxt.first, ln, r < nxt.n, G, ring[r]);
        cur_next(nxt.Qu, nxt.S, ln);
      }
    } else {  // last batch: the refills load the next op's first entries
      Cur ln{nxt.u0, nxt.s0, nxt.q0};
#pragma unroll
      for (int r = 0; r < kRing; ++r) {
        const int e = cur.P - kRing + r;
        const Consumed c = consume(ring[r], aq, an);
        __builtin_amdgcn_sched_barrier(0);
        issue_item(nxt.op, la_nxt, nxt.first, ln, r < nxt.n, G, ring[r]);
        __builtin_amdgcn_sched_barrier(0);
        cur_next(nxt.Qu, nxt.S, ln);
        finish(c, ad, e < cur.n, cc.s * R + ((cc.u << cur.op.qpu_log2) + cc.q) * 4 + grp, &L.ucnt[wave][cc.u],
               (uint32_t)(cur.t0 + e + 1 - max(cur.t0, cc.u * U)), lane, L);
        const int s_prev = cc.s;
        cur_next(cur.Qu, cur.S, cc);
        if (r + 1 < kRing && cc.s != s_prev) load_act(L, ob, cc.s, l16, aq, ad, an);
      }
    }
    lds_barrier();  // B: every wave is done with the op
    if (nxt.i >= nops) break;
    cur = nxt;
    la_cur = la_nxt;
    nxt = op_work(L, nops, wave, wg, G, cur.op.next, cur.op);
    la_nxt = lane_addr(nxt.op, l16, grp);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the trailing dummy loads
}

// ---------------------------------------------------------------- I/O waves
// Publish one 32-value unit held by a half-wave: fp32 LL words, plain output
// and the Q8 LL words.
__device__ __forceinline__ void publish_unit(const OpDev& op, int unit, int j, float v, bool valid, uint32_t tag) {
  const int row = unit * 32 + j;
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
    uint64_t* dst = out_q8 + (size_t)unit * kWordsPerBlock;
    if ((j & 3) == 0) ll_store(dst + (j >> 2), ((uint64_t)tag << 32) | w);
    if (j == 0) ll_store(dst + 8, ((uint64_t)tag << 32) | __float_as_uint(d));
    if (j == 1) ll_store(dst + 9, ((uint64_t)tag << 32) | (uint32_t)s);
  }
}

__device__ __forceinline__ void io_quantize(const OpDev& op, int wg, int G, int iol, uint32_t tag) {
  // half-wave h of the I/O waves handles units first + (h + t*nhalves)*G
  const int half = iol >> 5, j = iol & 31, nhalves = kIW * 2;
  const int N = sgpr(op.N), units = sgpr(op.units);
  const float* src = sgpr_ptr(op.src);
  for (int u = first_unit(sgpr(op.rot), wg, G) + half * G; u < units; u += nhalves * G) {
    const int row = u * 32 + j;
    const bool valid = row < N;
    const float v = valid ? *(const __attribute__((address_space(1))) float*)(src + row) : 0.f;
    publish_unit(op, u, j, v, valid, tag);
  }
}

// Write-after-read guard: the version of the output vector this op replaces
// may still be needed by a workgroup that has not fetched the input of op
// `war_op` yet; wait until all G have (rd_cnt counts them, G per launch).
__device__ __forceinline__ void wait_readers(int war_op, const uint32_t* rd_cnt, int G, Lds& L, Ctl* ctl) {
  if (war_op < 0) return;
  const uint32_t want = L.epoch * (uint32_t)G;
  uint32_t spins = 0;
  while ((int32_t)(ctl_load(rd_cnt + war_op) - want) < 0 && !aborted(L)) {
    if (++spins > L.spin_max || ((spins & 255) == 0 && grid_failed(ctl, L))) {
      set_abort(L, ctl);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Publish the op's units as the compute waves complete them: half-wave h
// takes local units h, h + 4, ...; for each, it waits until the unit's
// items are all counted (the compute waves' counts add up), reduces
// part[slice][row] over the slices in order,
// applies the mode (old value: the LDS carry, or the LL word of the previous
// version, loaded one unit ahead) and publishes. Returns each counter to 0
// for the next op.
__device__ __forceinline__ void io_publish(const OpDev& op, Lds& L, int wg, int G, int iol, uint32_t base_tag,
                                           Ctl* ctl) {
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
  for (int ui = half; ui < nunits; ui += nhalves) {
    {
      // polled at normal priority and sparsely: the compute waves on the
      // same SIMDs are producing these items
      __builtin_amdgcn_s_setprio(0);
      uint32_t spins = 0;
      for (;;) {
        uint32_t done = 0;
#pragma unroll
        for (int w = 0; w < kCW; ++w) done += __hip_atomic_load(&L.ucnt[w][ui], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (done == items || !poll_step(spins, L, ctl)) break;
        __builtin_amdgcn_s_sleep(3);
      }
      __builtin_amdgcn_s_setprio(3);
    }
    asm volatile("" ::: "memory");
    if (j < kCW) __hip_atomic_store(&L.ucnt[j][ui], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    const int unit = first + ui * G;
    const int row = unit * 32 + j;
    const bool valid = row < N;
    float v;
    if (mode == BTF_GEMV_SWIGLU) {
      const int lr = ui * 64 + 2 * j;  // virtual rows: gate 2j, up 2j+1 of this unit
      float g = 0.f, u = 0.f;
      for (int s = 0; s < S; ++s) {
        g += L.part[s * R + lr];
        u += L.part[s * R + lr + 1];
      }
      v = g / (1.0f + expf(-g)) * u;
    } else {
      const int lr = ui * 32 + j;
      float sum = 0.f;
      for (int s = 0; s < S; ++s) sum += L.part[s * R + lr];
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
  }
}

// The I/O waves' program. Per op: issue the early loads of the next op's
// input (if it is early), wait for the write-after-read guard, publish the
// units as they complete, barrier B, count this workgroup's reads of the
// op's input, finish the early fetch.
__device__ __forceinline__ void io_waves(Lds& L, int nops, Ctl* ctl, uint32_t* rd_cnt, int iol, int wg, int G,
                                         uint32_t base_tag) {
  for (int i = 0; i < nops; ++i) {
    const OpDev& op = L.opd[i];
    if (sgpr(op.kind) == 0) {
      io_quantize(op, wg, G, iol, base_tag + sgpr(op.my_tag));
      continue;
    }
    const int nx = sgpr(op.next);
    const bool early = nx < nops && sgpr(L.opd[nx].early);
    EarlyFetch ef;
    if (early) early_issue(L.opd[nx], iol, base_tag, ef);
    wait_readers(sgpr(op.war_op), rd_cnt, G, L, ctl);
    io_publish(op, L, wg, G, iol, base_tag, ctl);
    lds_barrier();  // B: every compute wave is done with the op's input
    if (sgpr(op.count_reads) && iol == 0)
      (void)__hip_atomic_fetch_add(rd_cnt + i, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (early) {
      early_finish(L.opd[nx], iol, base_tag, ef, L, nx & 1, ctl);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the input words are in LDS
      if ((iol & 63) == 0)
        __hip_atomic_store(&L.early_seq[iol >> 6], (uint32_t)nx + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }
}

// ---------------------------------------------------------------- the kernel
__global__ void __launch_bounds__(kThreads) step_kernel(const OpDev* __restrict__ ops, int nops, int first_gemv,
                                                        Ctl* ctl, uint32_t* rd_cnt) {
  __shared__ Lds L;
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
  if (threadIdx.x < kIW) L.early_seq[threadIdx.x] = 0;
  if (threadIdx.x == 0) {
    L.epoch = ctl_load(&ctl->epoch);
    const uint32_t sm = ctl_load(&ctl->spin_max);
    L.spin_max = sm ? sm : kSpinMax;
    __hip_atomic_store(&L.abort_, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the staged words have landed
  lds_barrier();
  const uint32_t base_tag = L.epoch * (uint32_t)(nops + 1);

  if (wave < kCW)
    compute_waves(L, nops, first_gemv, wave, lane, wg, G, ctl, base_tag);
  else {
    // The I/O waves' epilogue of an op is on the chain's critical path while
    // the compute waves already run the next op's dot products on the same
    // SIMDs: their instructions issue first (the waits in between sleep).
    __builtin_amdgcn_s_setprio(3);
    io_waves(L, nops, ctl, rd_cnt, threadIdx.x - 64 * kCW, wg, G, base_tag);
    __builtin_amdgcn_s_setprio(0);
  }

  // ---------------- end of step: count the workgroup out; the last one to
  // arrive advances the epoch for the next launch (it is read before any
  // workgroup of this launch can have finished its first op).
  lds_barrier();
  if (threadIdx.x == 0) {
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
  uint32_t* d_cnt = nullptr;  // per-op reader counters
  std::vector<void*> bufs;    // every device buffer the program owns
};

void step_destroy(StepProgram* P) {
  if (!P) return;
  for (void* p : P->bufs) (void)hipFree(p);
  delete P;
}

int step_validate(const btf_step_vec* vecs, int nvec, const btf_step_gemv* gemvs, int ngemv) {
  for (int v = 0; v < nvec; ++v)
    if (vecs[v].n <= 0) return fail(BTF_ERR_ARGS, "step: vector length must be positive");
  for (int i = 0; i < ngemv; ++i) {
    const btf_step_gemv& g = gemvs[i];
    if (g.in_vec < 0 || g.in_vec >= nvec || g.out_vec < 0 || g.out_vec >= nvec)
      return fail(BTF_ERR_ARGS, "step: vector index out of range");
    if (g.mode != BTF_GEMV_STORE && g.mode != BTF_GEMV_ADD && g.mode != BTF_GEMV_SWIGLU)
      return fail(BTF_ERR_ARGS, "step: unknown mode");
    if (g.K <= 0 || g.K % 1024 || g.K > kMaxK)
      return fail(BTF_ERR_ARGS, "step: K must be a multiple of 1024, <= 20480");
    if (g.N % 4) return fail(BTF_ERR_ARGS, "step: N must be a multiple of 4");
    if ((uint64_t)g.N * (uint64_t)(g.K / 4) >= (1ull << 32)) return fail(BTF_ERR_ARGS, "step: a matrix must be below 4 GB");
    if (g.K > vecs[g.in_vec].n) return fail(BTF_ERR_ARGS, "step: K exceeds the input vector");
    if (g.N != vecs[g.out_vec].n) return fail(BTF_ERR_ARGS, "step: N must equal the output vector length");
    if (g.in_vec == g.out_vec) return fail(BTF_ERR_ARGS, "step: a GEMV cannot read its own output vector");
    if (!g.codes || !g.scales || (g.mode == BTF_GEMV_SWIGLU && (!g.up_codes || !g.up_scales)))
      return fail(BTF_ERR_ARGS, "step: null weights");
    if ((reinterpret_cast<uintptr_t>(g.codes) & 15) || (g.up_codes && (reinterpret_cast<uintptr_t>(g.up_codes) & 15)) ||
        (reinterpret_cast<uintptr_t>(g.scales) & 1) || (g.up_scales && (reinterpret_cast<uintptr_t>(g.up_scales) & 1)))
      return fail(BTF_ERR_ARGS, "step: codes must be 16-byte and scales 2-byte aligned");
  }
  {
    std::vector<int> writes(nvec, 0);
    for (int i = 0; i < ngemv; ++i) {
      const btf_step_gemv& g = gemvs[i];
      if (writes[g.in_vec] == 0 && !vecs[g.in_vec].data)
        return fail(BTF_ERR_ARGS, "step: a vector read before any write needs data");
      if (g.mode == BTF_GEMV_ADD && writes[g.out_vec] == 0 && !vecs[g.out_vec].data)
        return fail(BTF_ERR_ARGS, "step: a vector read before any write needs data");
      if (vecs[g.in_vec].n % 32) return fail(BTF_ERR_ARGS, "step: quantized vectors need n % 32 == 0");
      writes[g.out_vec]++;
    }
  }
  return BTF_OK;
}

int step_create(const btf_step_vec* vecs, int nvec, const btf_step_gemv* gemvs, int ngemv, StepProgram** out,
                const DevState& ds) {
  if (const int rc = step_validate(vecs, nvec, gemvs, ngemv)) return rc;
  if (const int rc = step_check_residency(ds)) return rc;
  const int G = ds.cu_count;
  // ---- which vectors need an initial quantize / an fp32 or Q8 copy
  std::vector<bool> needs_init(nvec, false), needs_f32(nvec, false), needs_q8(nvec, false);
  std::vector<int> final_writer(nvec, -1);  // GEMV index of each vector's last writer
  {
    std::vector<int> writes(nvec, 0);
    for (int i = 0; i < ngemv; ++i) {
      const btf_step_gemv& g = gemvs[i];
      if (writes[g.in_vec] == 0) needs_init[g.in_vec] = true;
      needs_q8[g.in_vec] = true;
      if (g.mode == BTF_GEMV_ADD) {
        if (writes[g.out_vec] == 0) needs_init[g.out_vec] = true;
        needs_f32[g.out_vec] = true;
      }
      writes[g.out_vec]++;
      final_writer[g.out_vec] = i;
    }
  }
  StepProgram* P = new StepProgram();
  P->G = G;
  auto alloc = [&](size_t bytes) -> void* {
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) return nullptr;
    P->bufs.push_back(p);
    if (hipMemset(p, 0, bytes) != hipSuccess) return nullptr;
    return p;
  };
  auto bail = [&](int code, const char* msg) {
    step_destroy(P);
    return fail(code, msg);
  };
  // ---- versions of every vector over the program (pre-pass). Version 0 of a
  // vector read before any write is its user data, quantized by a prologue
  // op; every GEMV writes a new version of its output vector. A version gets
  // Q8 LL words only if a later op reads it as input; every GEMV output gets
  // fp32 LL words (read by a later add-mode op as its old value, or not).
  struct Version {
    int writer;                 // GEMV index, -1 = prologue
    int last_q8_reader = -1;    // GEMV index
    std::vector<int> f32_readers;
    int q8_slot = -1, f32_slot = -1;
  };
  std::vector<std::vector<Version>> versions(nvec);
  std::vector<int> op_in_ver(ngemv), op_old_ver(ngemv, -1), op_out_ver(ngemv);
  for (int v = 0; v < nvec; ++v)
    if (needs_init[v]) versions[v].push_back(Version{-1});
  for (int i = 0; i < ngemv; ++i) {
    const btf_step_gemv& g = gemvs[i];
    op_in_ver[i] = (int)versions[g.in_vec].size() - 1;
    versions[g.in_vec].back().last_q8_reader = i;
    if (g.mode == BTF_GEMV_ADD) {
      op_old_ver[i] = (int)versions[g.out_vec].size() - 1;
      versions[g.out_vec].back().f32_readers.push_back(i);
    }
    op_out_ver[i] = (int)versions[g.out_vec].size();
    versions[g.out_vec].push_back(Version{i});
  }
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
      // every GEMV's result is written to device memory (fp32 words), read
      // later or not; the prologue's version 0 only if an add reads it
      if (ve.writer >= 0 || !ve.f32_readers.empty()) ve.f32_slot = nf++ % kSlots;
    }
    for (int b = 0; b < kSlots && b < nq; ++b)
      if (!(q8buf[b][v] = static_cast<uint64_t*>(alloc((size_t)(vecs[v].n / 32) * kWordsPerBlock * 8))))
        return bail(BTF_ERR_LAUNCH, "step: device allocation failed");
    for (int b = 0; b < kSlots && b < nf; ++b)
      if (!(f32buf[b][v] = static_cast<uint64_t*>(alloc((size_t)vecs[v].n * 8))))
        return bail(BTF_ERR_LAUNCH, "step: device allocation failed");
  }
  auto q8_of = [&](int v, int k) { return versions[v][k].q8_slot >= 0 ? q8buf[versions[v][k].q8_slot][v] : nullptr; };
  auto f32_of = [&](int v, int k) { return versions[v][k].f32_slot >= 0 ? f32buf[versions[v][k].f32_slot][v] : nullptr; };
  // ---- the device program: prologue quantize ops, then the GEMVs in order
  std::vector<OpDev> ops;
  // known[v * G + w]: the last GEMV whose barrier B workgroup w has surely
  // passed, as far as workgroup v can tell when it reaches a later op. A
  // workgroup that owns units of an op reads all of its input (every unit
  // spans all slices), published unit by unit by the writers of the input's
  // producer X, each of which had passed B of the GEMV before X. Workgroup v
  // has passed B of every earlier op before starting an op.
  std::vector<int> known((size_t)G * G, -1);
  int last_gemv = -1;                   // device index of the previous GEMV
  std::vector<int> prev_gemv;           // per device op: the GEMV before it (-1: none)
  auto owns = [&](const OpDev& x, int w) { return (w - x.rot + G) % G < x.units; };
  std::vector<int> dev_of(ngemv, -1);        // device op index of each GEMV
  std::vector<int> prologue_of(nvec, -1);    // device op index of each prologue op
  // Unit placement: unit u of an op goes to workgroup (u + rot) % G. An
  // add-mode op takes the rotation of the op that wrote its old value when
  // they have the same units, so each row's old value was published by the
  // same workgroup (no cross-workgroup wait on an add chain). Any other op
  // takes the rotation that keeps the most-loaded workgroup's weight bytes
  // lowest.
  std::vector<double> load(G, 0.0);
  auto place = [&](OpDev& o, double cost_per_unit, int align_to) {
    o.units = (o.N + 31) / 32;
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
    if (!needs_init[v]) continue;
    OpDev o{};
    o.kind = 0;
    o.N = vecs[v].n;
    o.src = vecs[v].data;
    o.out_q8 = q8_of(v, 0);
    o.out_f32 = f32_of(v, 0);
    o.my_tag = (uint32_t)ops.size() + 1;
    o.war_op = -1;
    place(o, 1.0, -1);
    prologue_of[v] = (int)ops.size();
    ops.push_back(o);
    prev_gemv.push_back(-1);
  }
  auto dev_writer = [&](int v, int k) {
    const int w = versions[v][k].writer;
    return w < 0 ? prologue_of[v] : dev_of[w];
  };
  for (int i = 0; i < ngemv; ++i) {
    const btf_step_gemv& g = gemvs[i];
    const int me = (int)ops.size();
    dev_of[i] = me;
    OpDev o{};
    o.kind = 1;
    o.mode = g.mode;
    o.K = g.K;
    o.N = g.N;
    o.cpr = g.K / 64;
    o.qpu_log2 = g.mode == BTF_GEMV_SWIGLU ? 4 : 3;
    o.codes = g.codes;
    o.scales = g.scales;
    o.up_codes = g.up_codes;
    o.up_scales = g.up_scales;
    o.in_q8 = q8_of(g.in_vec, op_in_ver[i]);
    o.in_tag = (uint32_t)dev_writer(g.in_vec, op_in_ver[i]) + 1;
    int align_to = -1;
    if (g.mode == BTF_GEMV_ADD) {
      o.old_f32 = f32_of(g.out_vec, op_old_ver[i]);
      o.old_tag = (uint32_t)dev_writer(g.out_vec, op_old_ver[i]) + 1;
      align_to = dev_writer(g.out_vec, op_old_ver[i]);
    }
    const int kv = op_out_ver[i];
    const Version& nv = versions[g.out_vec][kv];
    // Plain output: only the final version goes to the user's buffer (plain
    // stores of two ops to one address from different XCDs reach HBM in the
    // order their L2s write back, not in program order).
    o.out_plain = final_writer[g.out_vec] == i ? vecs[g.out_vec].data : nullptr;
    o.out_q8 = q8_of(g.out_vec, kv);
    o.out_f32 = f32_of(g.out_vec, kv);
    o.my_tag = (uint32_t)me + 1;
    place(o, (double)g.K * (g.mode == BTF_GEMV_SWIGLU ? 2 : 1), align_to);
    // Write-after-read: the buffers this version takes held the version
    // kSlots such versions earlier; wait until every workgroup has fetched the
    // input of its last reader. Old-value reads by an op with the same unit
    // placement are reads of the workgroup's own rows, already ordered by
    // program order. The final writer also stores into the user's buffer,
    // which the prologue read (version 0): after every reader of version 0.
    int war = -1;
    for (int k = kv - 1; k >= 0; --k) {
      const Version& pv = versions[g.out_vec][k];
      if (nv.q8_slot >= 0 && pv.q8_slot == nv.q8_slot) {
        war = std::max(war, pv.last_q8_reader >= 0 ? dev_of[pv.last_q8_reader] : -1);
        break;
      }
    }
    for (int k = kv - 1; k >= 0; --k) {
      const Version& pv = versions[g.out_vec][k];
      if (nv.f32_slot >= 0 && pv.f32_slot == nv.f32_slot) {
        for (int r : pv.f32_readers) {
          const OpDev& ro = ops[dev_of[r]];
          if (!(ro.units == o.units && ro.rot == o.rot)) war = std::max(war, dev_of[r]);
        }
        break;
      }
    }
    if (o.out_plain && needs_init[g.out_vec]) {
      const Version& v0 = versions[g.out_vec][0];
      int last = v0.last_q8_reader;
      for (int r : v0.f32_readers) last = std::max(last, r);
      if (last >= 0 && last != i) war = std::max(war, dev_of[last]);
    }
    if (war >= 0) {  // implied for every workgroup that writes this op's output?
      bool implied = true;
      for (int v = 0; v < G && implied; ++v) {
        if (!owns(o, v)) continue;
        for (int w = 0; w < G; ++w)
          if (w != v && known[(size_t)v * G + w] < war) {
            implied = false;
            break;
          }
      }
      if (implied) war = -1;
    }
    {
      const int x = (int)o.in_tag - 1;  // input producer
      const int px = x < (int)prev_gemv.size() ? prev_gemv[x] : -1;
      if (ops[x].kind == 1 && px >= 0)
        for (int v = 0; v < G; ++v) {
          if (!owns(o, v)) continue;
          for (int w = 0; w < G; ++w)
            if (owns(ops[x], w)) known[(size_t)v * G + w] = std::max(known[(size_t)v * G + w], px);
        }
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
  if ((int)ops.size() > kMaxOps) return bail(BTF_ERR_ARGS, "step: more than 384 ops (quantize prologue + GEMVs)");
  // Early fetch and carry. An op's input is fetched by the I/O waves while
  // the previous GEMV computes when every producer it reads from comes
  // before that previous GEMV (a workgroup then never waits for its own
  // unpublished output). An add-mode op whose old value was produced by the
  // previous GEMV with the same unit placement takes it from the LDS carry
  // (the same workgroup computed it).
  {
    int pd = -1;  // previous GEMV in program order
    for (int d = 0; d < (int)ops.size(); ++d) {
      OpDev& o = ops[d];
      if (o.kind != 1) continue;
      if (o.mode == BTF_GEMV_ADD && pd >= 0 && (int)o.old_tag - 1 == pd && ops[pd].units == o.units &&
          ops[pd].rot == o.rot) {
        o.carry_in = 1;
        ops[pd].carry_out = 1;
      }
      const bool in_ok = (int)o.in_tag - 1 < pd;
      const bool no_old = o.mode != BTF_GEMV_ADD || o.carry_in;
      const bool fits = (o.K / 32) * kWordsPerBlock <= kIL * kEIn;  // one round of the I/O waves
      o.early = pd >= 0 && in_ok && no_old && fits;
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
  P->nops = (int)ops.size();
  if (!(P->d_ops = static_cast<OpDev*>(alloc(ops.size() * sizeof(OpDev)))) ||
      !(P->d_ctl = static_cast<Ctl*>(alloc(sizeof(Ctl)))) ||
      !(P->d_cnt = static_cast<uint32_t*>(alloc(ops.size() * sizeof(uint32_t)))))
    return bail(BTF_ERR_LAUNCH, "step: device allocation failed");
  const Ctl c0{1u, 0u, 0u, 0u};
  if (hipMemcpy(P->d_ops, ops.data(), ops.size() * sizeof(OpDev), hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(P->d_ctl, &c0, sizeof c0, hipMemcpyHostToDevice) != hipSuccess)
    return bail(BTF_ERR_LAUNCH, "step: program upload failed");
  (void)hipGetDevice(&P->device);
  *out = P;
  return BTF_OK;
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
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, step_kernel, kThreads, 0) != hipSuccess)
    return fail(BTF_ERR_LAUNCH, "step: occupancy query failed");
  if (per_cu < 1) return fail(BTF_ERR_LAUNCH, "step: the step kernel does not fit on a CU");
  (void)ds;
  return BTF_OK;
}

int step_launch(StepProgram* P, hipStream_t st) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != P->device)
    return fail(BTF_ERR_ARGS, "step: launch on a device other than the program's");
  void* args[] = {&P->d_ops, &P->nops, &P->first, &P->d_ctl, &P->d_cnt};
  const hipError_t e =
      hipLaunchCooperativeKernel(reinterpret_cast<const void*>(step_kernel), dim3(P->G), dim3(kThreads), args, 0, st);
  if (e != hipSuccess) return fail(BTF_ERR_LAUNCH, std::string("step kernel: ") + hipGetErrorString(e));
  return launch_status("step_kernel");
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

