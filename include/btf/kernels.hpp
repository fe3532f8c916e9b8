// kernels.hpp -- C++ mirror of the reference's kernel-launch API for the
// fused ternary matmul path (src/cuda/kernels.cuh:13-56, namespace
// btf::cuda), implemented over the C ABI of libbtf_hip.so (hip_abi.h).
//
// Same names, struct fields, defaults and argument meaning as the reference;
// the namespace is btf::hip and the stream is a hipStream_t (any pointer-
// sized stream handle converts to btf_stream_t). Failures throw
// std::runtime_error with the library's message, as the reference launchers
// do. Header-only; link with -lbtf_hip.
#pragma once
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>

#include "hip_abi.h"

namespace btf {
namespace hip {

namespace detail {
inline void check(int rc, const char* what) {
  if (rc != BTF_OK) {
    const char* msg = btf_hip_last_error();
    throw std::runtime_error(std::string(what) + ": " + (msg && *msg ? msg : "error " + std::to_string(rc)));
  }
}
}  // namespace detail

// kernels.cuh:17 -- once per device before any launch or capture.
inline void kernels_init(int device) { detail::check(btf_hip_kernels_init(device), "kernels_init"); }

// kernels.cuh:20
inline int gemv_max_nb(int K) { return btf_hip_gemv_max_nb(K); }

// kernels.cuh:22-24
inline void launch_repack(const uint8_t* src, int64_t nblocks, uint8_t* codes, uint16_t* scales,
                          btf_stream_t st) {
  detail::check(btf_hip_launch_repack(src, nblocks, codes, scales, st), "launch_repack");
}

// kernels.cuh:26-31
struct Q8Act {
  int8_t* q = nullptr;  // [M][K]
  float* d = nullptr;   // [M][K/32]
  int* s = nullptr;     // [M][K/32] sum of q per block
};

// kernels.cuh:33-38
struct Hx {
  int block = 0;
  int perm_hd = 0, perm_nk = 0, perm_rep = 0;
  const float* signs = nullptr;
};

// kernels.cuh:40-43
inline void launch_prep(const float* x, int ldx, int M, int n, const float* normw, float eps, const Hx& hx,
                        float* xn_out, int ldxn, const Q8Act& a, btf_stream_t st) {
  const btf_hx h{hx.block, hx.perm_hd, hx.perm_nk, hx.perm_rep, hx.signs};
  const btf_q8act q{a.q, a.d, reinterpret_cast<int32_t*>(a.s)};
  detail::check(btf_hip_launch_prep(x, ldx, M, n, normw, eps, &h, xn_out, ldxn, &q, st), "launch_prep");
}

// kernels.cuh:45-52
struct GemvSeg {
  const uint8_t* codes = nullptr;
  const uint16_t* scales = nullptr;
  int N = 0;
  float* y = nullptr;
  int ldy = 0;
};
enum GemvMode { kStore = BTF_GEMV_STORE, kAdd = BTF_GEMV_ADD, kSwiglu = BTF_GEMV_SWIGLU };

// kernels.cuh:53-56
inline void launch_gemv(const GemvSeg* segs, int nseg, int K, int M, const Q8Act& a, GemvMode mode,
                        btf_stream_t st) {
  if (nseg < 1 || nseg > 3) throw std::runtime_error("launch_gemv: gemv: 1..3 segments");
  btf_gemv_seg s[3] = {};
  for (int i = 0; i < nseg; ++i) s[i] = btf_gemv_seg{segs[i].codes, segs[i].scales, segs[i].N, segs[i].y, segs[i].ldy};
  const btf_q8act q{a.q, a.d, reinterpret_cast<int32_t*>(a.s)};
  detail::check(btf_hip_launch_gemv(s, nseg, K, M, &q, mode, st), "launch_gemv");
}

// kernels.cuh:82-85
inline void launch_embed(const uint8_t* codes, const uint16_t* scales, const int* d_tok, int M, int E, const Hx& inv,
                         float* x, btf_stream_t st) {
  const btf_hx h{inv.block, inv.perm_hd, inv.perm_nk, inv.perm_rep, inv.signs};
  detail::check(btf_hip_launch_embed(codes, scales, d_tok, M, E, &h, x, st), "launch_embed");
}

// kernels.cuh:89-90
inline size_t argmax_part_bytes(int V) { return (size_t)btf_hip_argmax_part_bytes(V); }
inline void launch_argmax(const float* logits, int V, void* part, int* d_tok_out, btf_stream_t st) {
  detail::check(btf_hip_launch_argmax(logits, V, part, d_tok_out, st), "launch_argmax");
}
// no counterpart in kernels.cuh: launch_argmax without a workspace, for
// callers that cannot allocate (the library's static per-GPU scratch;
// overlapping calls on one GPU race)
inline void launch_argmax_noalloc(const float* logits, int V, int* d_tok_out, btf_stream_t st) {
  detail::check(btf_hip_launch_argmax_noalloc(logits, V, d_tok_out, st), "launch_argmax_noalloc");
}

// kernels.cuh:92
inline void launch_pos_add(int* d_pos, int M, btf_stream_t st) {
  detail::check(btf_hip_launch_pos_add(d_pos, M, st), "launch_pos_add");
}

// launch_gemv with the chain's quantizes fused in (no counterpart in
// kernels.cuh: the decoder's launch_prep + launch_gemv pairs without norm or
// transform, src/cuda/gpu_decoder.cu:411-418): input from Q8 rows `a` or fp32
// rows `x`; `out` (optional) receives the Q8 rows of the output.
inline void launch_gemv_ex(const GemvSeg* segs, int nseg, int K, int M, const Q8Act* a, const float* x, int ldx,
                           GemvMode mode, const Q8Act* out, btf_stream_t st) {
  if (nseg < 1 || nseg > 3) throw std::runtime_error("launch_gemv_ex: gemv: 1..3 segments");
  btf_gemv_seg s[3] = {};
  for (int i = 0; i < nseg; ++i) s[i] = btf_gemv_seg{segs[i].codes, segs[i].scales, segs[i].N, segs[i].y, segs[i].ldy};
  btf_q8act qa{}, qo{};
  if (a) qa = btf_q8act{a->q, a->d, reinterpret_cast<int32_t*>(a->s)};
  if (out) qo = btf_q8act{out->q, out->d, reinterpret_cast<int32_t*>(out->s)};
  detail::check(btf_hip_launch_gemv_ex(s, nseg, K, M, a ? &qa : nullptr, x, ldx, mode, out ? &qo : nullptr, st),
                "launch_gemv_ex");
}

// launch_gemv on PTQ1_0 matrices read directly (the native 1.75-bit GEMV the
// reference plans in docs/kernel-design.md:53): GemvSeg::codes holds N rows
// of K/128 28-byte PTQ1_0 blocks and GemvSeg::scales is nullptr.
inline void launch_gemv_ptq1_0(const GemvSeg* segs, int nseg, int K, int M, const Q8Act& a, GemvMode mode,
                               btf_stream_t st) {
  if (nseg < 1 || nseg > 3) throw std::runtime_error("launch_gemv_ptq1_0: gemv: 1..3 segments");
  btf_gemv_seg s[3] = {};
  for (int i = 0; i < nseg; ++i) s[i] = btf_gemv_seg{segs[i].codes, segs[i].scales, segs[i].N, segs[i].y, segs[i].ldy};
  const btf_q8act q{a.q, a.d, reinterpret_cast<int32_t*>(a.s)};
  detail::check(btf_hip_launch_gemv_ptq1_0(s, nseg, K, M, &q, mode, st), "launch_gemv_ptq1_0");
}

// ---- the decode-step program (no counterpart in kernels.cuh: it replaces
// the per-step graph of GEMV launches, src/cuda/gpu_decoder.cu:452-486)
class StepProgram {
 public:
  StepProgram(const btf_step_vec* vecs, int nvec, const btf_step_gemv* ops, int nops) {
    detail::check(btf_hip_step_create(vecs, nvec, ops, nops, &p_), "step_create");
  }
  // a whole token: embed ops, GEMVs with their full input prep, the greedy pick
  StepProgram(const btf_step_vec* vecs, int nvec, const btf_step_op* ops, int nops) {
    detail::check(btf_hip_step_create_ops(vecs, nvec, ops, nops, &p_), "step_create_ops");
  }
  StepProgram(const StepProgram&) = delete;
  StepProgram& operator=(const StepProgram&) = delete;
  ~StepProgram() { (void)btf_hip_step_destroy(p_); }
  void launch(btf_stream_t st) { detail::check(btf_hip_step_launch(p_, st), "step_launch"); }
  // true if a launch since the last call timed out (synchronise first); clears it
  bool failed() {
    int e = 0;
    detail::check(btf_hip_step_error(p_, &e), "step_error");
    return e != 0;
  }

 private:
  btf_step_t p_ = nullptr;
};

// ---- load path (no counterpart in kernels.cuh): the reader of the model file
// and the staged upload. Gguf offers what the reference's bd::Gguf offers for
// loading (ref/bonsai-decoder/include/bd/gguf.hpp:49-85: open, tensor lookup,
// need_tensor, get_i / get_f / get_s / get_b); Loader is GpuDecoder::upload_mat
// (src/cuda/gpu_decoder.cu:284-300) as an object. Both throw
// std::runtime_error on failure.
struct GgufTensor {
  std::string name;
  int n_dims = 0;
  int64_t ne[4] = {1, 1, 1, 1};
  uint32_t type = 0;
  uint64_t offset = 0, bytes = 0;
  const uint8_t* data = nullptr;
  int64_t n_elements() const { return ne[0] * ne[1] * ne[2] * ne[3]; }
  int64_t dim(int d) const { return d < n_dims ? ne[d] : 1; }
};

class Gguf {
 public:
  explicit Gguf(const std::string& path, bool header_only = false) {
    detail::check(btf_hip_gguf_open(path.c_str(), header_only ? 1 : 0, &g_), "gguf_open");
    detail::check(btf_hip_gguf_info(g_, &h_), "gguf_info");
  }
  Gguf(const Gguf&) = delete;
  Gguf& operator=(const Gguf&) = delete;
  ~Gguf() { (void)btf_hip_gguf_close(g_); }
  uint32_t version() const { return h_.version; }
  uint64_t alignment() const { return h_.alignment; }
  uint64_t data_offset() const { return h_.data_offset; }
  int64_t n_tensors() const { return h_.n_tensors; }
  GgufTensor tensor_at(int64_t i) const {
    btf_gguf_tensor t;
    detail::check(btf_hip_gguf_tensor(g_, i, &t), "gguf_tensor");
    GgufTensor r;
    r.name = t.name;
    r.n_dims = t.n_dims;
    for (int d = 0; d < 4; ++d) r.ne[d] = t.ne[d];
    r.type = t.type;
    r.offset = t.offset;
    r.bytes = t.bytes;
    r.data = t.data;
    return r;
  }
  bool has_tensor(const std::string& name) const { return btf_hip_gguf_find_tensor(g_, name.c_str()) >= 0; }
  GgufTensor need_tensor(const std::string& name) const {
    const int64_t i = btf_hip_gguf_find_tensor(g_, name.c_str());
    if (i < 0) throw std::runtime_error("missing tensor " + name);
    return tensor_at(i);
  }
  bool has(const std::string& key) const { return btf_hip_gguf_find_kv(g_, key.c_str()) >= 0; }
  int64_t get_i(const std::string& key) const { return num(key).first; }
  int64_t get_i(const std::string& key, int64_t def) const { return has(key) ? get_i(key) : def; }
  double get_f(const std::string& key) const { return num(key).second; }
  double get_f(const std::string& key, double def) const { return has(key) ? get_f(key) : def; }
  bool get_b(const std::string& key, bool def) const { return has(key) ? get_i(key) != 0 : def; }
  std::string get_s(const std::string& key, const std::string& def = "") const {
    const int64_t i = btf_hip_gguf_find_kv(g_, key.c_str());
    const char* s = nullptr;
    uint64_t n = 0;
    if (i < 0 || btf_hip_gguf_kv_str(g_, i, 0, &s, &n) != BTF_OK) return def;
    return std::string(s, (size_t)n);
  }
  btf_pack_plan plan(uint64_t staging_bytes) const {
    btf_pack_plan p;
    detail::check(btf_hip_gguf_plan(g_, staging_bytes, &p), "gguf_plan");
    return p;
  }
  btf_gguf_t handle() const { return g_; }

 private:
  std::pair<int64_t, double> num(const std::string& key) const {
    const int64_t i = btf_hip_gguf_find_kv(g_, key.c_str());
    if (i < 0) throw std::runtime_error("gguf: missing key " + key);
    int64_t v = 0;
    double f = 0.0;
    detail::check(btf_hip_gguf_kv_num(g_, i, 0, &v, &f), "gguf_kv_num");
    return {v, f};
  }
  btf_gguf_t g_ = nullptr;
  btf_gguf_header h_{};
};

class Loader {
 public:
  explicit Loader(uint64_t staging_bytes) { detail::check(btf_hip_loader_create(staging_bytes, &l_), "loader_create"); }
  Loader(const Loader&) = delete;
  Loader& operator=(const Loader&) = delete;
  ~Loader() { (void)btf_hip_loader_destroy(l_); }
  void upload_ptq1_0(const uint8_t* src, int64_t N, int64_t K, uint8_t* codes, uint16_t* scales, btf_stream_t st) {
    detail::check(btf_hip_loader_upload_ptq1_0(l_, src, N, K, codes, scales, st), "loader_upload");
  }
  uint64_t finish() {
    uint64_t n = 0;
    detail::check(btf_hip_loader_finish(l_, &n), "loader_finish");
    return n;
  }

 private:
  btf_loader_t l_ = nullptr;
};

}  // namespace hip
}  // namespace btf
