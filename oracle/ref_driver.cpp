// ref_driver.cpp -- TEST INFRASTRUCTURE. Compiled by oracle/Makefile together
// with the reference's own CPU sources, read where they lie in the reference
// checkout (nothing is copied), into oracle/_ref/libbtf_ref.so. It exposes the
// reference's functions through a C ABI so tests can pin the oracle
// (btf_oracle.c) against the real code. tests/golden/make_golden.py, the CPU
// tests and bench.py's CPU-baseline leg (which times the reference emulator's
// GEMV) load it; it never links into the product library.
//
// EmuDecoder (src/emu_decoder.cpp) keeps gemv() and prep() private inside an
// anonymous namespace, so this translation unit includes that source file and
// reaches them on an emulator built from the reference's tiny synthetic model
// (ref/bonsai-decoder/src/synth.cpp).
#include <algorithm>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <sstream>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "bd/cpu_ops.hpp"
#include "bd/gguf.hpp"
#include "bd/model.hpp"
#include "bd/sampler.hpp"
#include "bd/synth.hpp"
#include "bd/types.hpp"
#include "btf/fast.hpp"
#include "btf/packed.hpp"

#define private public
#include "emu_decoder.cpp"
#undef private

namespace {

struct RefEmu {
  std::unique_ptr<bd::Model> model;
  std::unique_ptr<btf::FastDecoder> dec;
};

int g_threads = 1;

// The emulator on the reference's smallest synthetic model; rebuilt when the
// requested thread count changes (its ThreadPool is sized at construction).
RefEmu& emu() {
  static RefEmu e;
  static int built_threads = -1;
  if (built_threads != g_threads) {
    e.dec.reset();
    if (!e.model) {
      bd::SynthOptions so;
      so.n_layer = 1;
      e.model = bd::Model::from_gguf(bd::Gguf::from_memory(bd::make_synth_qwen35(so)));
    }
    btf::FastOptions o;
    o.threads = g_threads;
    o.n_ctx = 16;
    e.dec = btf::make_emu_decoder(*e.model, o);
    built_threads = g_threads;
  }
  return e;
}

btf::EmuDecoder* emu_dec() { return static_cast<btf::EmuDecoder*>(emu().dec.get()); }

}  // namespace

extern "C" {

float ref_fp16_to_f32(uint16_t h) { return bd::fp16_to_f32(h); }
uint16_t ref_f32_to_fp16(float f) { return bd::f32_to_fp16(f); }
int ref_ptq1_0_trit(const uint8_t* blk, int e) { return bd::ptq1_0_trit(blk, e); }

void ref_quant_ptq1_0(const float* x, uint8_t* dst, int64_t n) { bd::quant_row(bd::T_PTQ1_0, x, dst, n); }
void ref_quant_q8_0(const float* x, uint8_t* dst, int64_t n) { bd::quant_row(bd::T_Q8_0, x, dst, n); }
void ref_dequant_ptq1_0(const uint8_t* src, float* dst, int64_t n) { bd::dequant_row(bd::T_PTQ1_0, src, dst, n); }

void ref_repack_rows(const uint8_t* src, int64_t rows, int64_t K, uint8_t* codes, uint16_t* scales) {
  btf::repack_rows(src, rows, K, codes, scales);
}
int ref_packed_code(const uint8_t* row_codes, int64_t e) { return btf::packed_code(row_codes, e); }
int ref_code_byte(int e) { return btf::code_byte(e); }
int ref_code_shift(int e) { return btf::code_shift(e); }

int ref_q8_block(const float* x, int8_t* q, float* d) { return btf::q8_block_host(x, q, d); }
void ref_round_q8_0(const float* x, int64_t n, float* out) { bd::round_q8_0(x, n, out); }
int ref_sub_dot(uint32_t w0, uint32_t w1, const uint32_t* aw) { return btf::sub_dot_host(w0, w1, aw); }
float ref_silu(float x) { return bd::silu(x); }

void ref_rmsnorm(const float* x, const float* w, int64_t n, float eps, float* y) { bd::rmsnorm(x, w, n, eps, y); }
void ref_fwht(float* x, int n) { bd::fwht(x, n); }

// bd::matvec_raw on a PTQ1_0 tensor [N][K] (ggml_act != 0: activations
// rounded through round_q8_0 first), ref/bonsai-decoder/src/cpu_ops.cpp:199-221.
void ref_matvec_ptq1_0(const uint8_t* src, int64_t N, int64_t K, const float* x, float* y, int ggml_act) {
  bd::GgufTensor t;
  t.name = "w";
  t.ne = {K, N};
  t.type = bd::T_PTQ1_0;
  t.data = src;
  bd::ThreadPool pool(1);
  bd::matvec_raw(pool, t, x, y, ggml_act != 0);
}

// The emulator's GEMV (src/emu_decoder.cpp:143-165) on caller data.
int ref_emu_gemv(const uint8_t* codes, const uint16_t* scales, int64_t N, int64_t K, const int8_t* q, const float* d,
                 const int32_t* s, int M, float* y, int64_t ldy, int add) {
  try {
    btf::PackedMatrix P;
    P.N = N;
    P.K = K;
    P.codes.assign(codes, codes + (size_t)N * (K / 4));
    P.scales.assign(scales, scales + (size_t)N * (K / 128));
    btf::Q8 a;
    a.resize(M, (int)K);
    std::memcpy(a.q.data(), q, (size_t)M * K);
    std::memcpy(a.d.data(), d, (size_t)M * (K / 32) * 4);
    std::memcpy(a.s.data(), s, (size_t)M * (K / 32) * 4);
    emu_dec()->gemv(P, a, M, y, (int)ldy, add != 0);
    return 0;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "ref_emu_gemv: %s\n", e.what());
    return -1;
  }
}

// Threads of the emulator's ThreadPool (0 = hardware concurrency, as bd::ThreadPool).
void ref_emu_set_threads(int n) { g_threads = n; }

// The emulator's GEMV timed around the call only (steady_clock, the clock
// EmuDecoder::step uses, src/emu_decoder.cpp:102-105); reps calls, returns the
// total seconds or -1 on error. The packed matrix and Q8 rows are built once.
double ref_emu_gemv_timed(const uint8_t* codes, const uint16_t* scales, int64_t N, int64_t K, const int8_t* q,
                          const float* d, const int32_t* s, int M, float* y, int64_t ldy, int add, int reps) {
  try {
    btf::PackedMatrix P;
    P.N = N;
    P.K = K;
    P.codes.assign(codes, codes + (size_t)N * (K / 4));
    P.scales.assign(scales, scales + (size_t)N * (K / 128));
    btf::Q8 a;
    a.resize(M, (int)K);
    std::memcpy(a.q.data(), q, (size_t)M * K);
    std::memcpy(a.d.data(), d, (size_t)M * (K / 32) * 4);
    std::memcpy(a.s.data(), s, (size_t)M * (K / 32) * 4);
    btf::EmuDecoder* E = emu_dec();
    const auto t0 = std::chrono::steady_clock::now();
    for (int r = 0; r < reps; ++r) E->gemv(P, a, M, y, (int)ldy, add != 0);
    return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
  } catch (const std::exception& e) {
    std::fprintf(stderr, "ref_emu_gemv_timed: %s\n", e.what());
    return -1.0;
  }
}

// The emulator's embedding lookup (src/emu_decoder.cpp:171-180): the same
// calls on rows of a packed table -- btf::packed_code, bd::fp16_to_f32 and
// bd::hadamard_inverse with the emulator's transform (active when block > 0).
int ref_emu_embed(const uint8_t* codes, const uint16_t* scales, const int32_t* toks, int M, int E, int V, int block,
                  const float* signs, float* x) {
  try {
    std::vector<float> sg;
    bd::HadamardXform hx;
    hx.active = block > 0;
    hx.block = block;
    if (signs) {
      sg.assign(signs, signs + E);
      hx.signs = &sg;
    }
    for (int m = 0; m < M; ++m) {
      const int tok = toks[m];
      if (tok < 0 || tok >= V) throw std::runtime_error("token id out of range");
      float* xr = x + (size_t)m * E;
      const uint8_t* cr = codes + (size_t)tok * (E / 4);
      const uint16_t* sr = scales + (size_t)tok * (E / 128);
      for (int i = 0; i < E; ++i) xr[i] = (float)(btf::packed_code(cr, i) - 1) * bd::fp16_to_f32(sr[i / 128]);
      bd::hadamard_inverse(hx, xr, E);
    }
    return 0;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "ref_emu_embed: %s\n", e.what());
    return -1;
  }
}

// The greedy sampler (ref/bonsai-decoder/src/sampler.cpp:20-25).
int ref_argmax(const float* logits, int n) { return bd::Sampler::argmax(logits, n); }

// The emulator's fused prep (src/emu_decoder.cpp:122-140) on dense rows
// x [M][n]; block == 0 means no input transform.
int ref_emu_prep(const float* x, int M, int n, const float* normw, float eps, int block, int perm_hd, int perm_nk,
                 int perm_rep, const float* signs, float* xn_out, int8_t* q, float* d, int32_t* s) {
  try {
    std::vector<float> sg;
    bd::HadamardXform hx;
    hx.active = block > 0;
    hx.block = block;
    hx.perm_hd = perm_hd;
    hx.perm_nk = perm_nk;
    hx.perm_rep = perm_rep;
    if (signs) {
      sg.assign(signs, signs + n);
      hx.signs = &sg;
    }
    btf::EmuDecoder* E = emu_dec();
    E->d_.eps = eps;
    btf::Q8 a;
    E->prep(x, M, n, normw, hx, a, xn_out);
    std::memcpy(q, a.q.data(), (size_t)M * n);
    std::memcpy(d, a.d.data(), (size_t)M * (n / 32) * 4);
    std::memcpy(s, a.s.data(), (size_t)M * (n / 32) * 4);
    return 0;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "ref_emu_prep: %s\n", e.what());
    return -1;
  }
}

// ---- GGUF (ref/bonsai-decoder/src/gguf.cpp) ----
// Canonical text of everything bd::Gguf parsed from `path` (one line per
// header field, metadata key and tensor; strings in hex), written into out.
// Returns 0, or -1 with the reader's error message in out.
int ref_gguf_dump(const char* path, int header_only, char* out, size_t cap) {
  std::string txt;
  try {
    std::unique_ptr<bd::Gguf> g = bd::Gguf::open(path, header_only != 0);
    std::ostringstream o;
    auto hex = [](const std::string& s) {
      static const char* d = "0123456789abcdef";
      std::string h;
      for (unsigned char c : s) h += d[c >> 4], h += d[c & 15];
      return std::to_string(s.size()) + ":" + h;
    };
    auto num = [](double f) {
      char b[64];
      std::snprintf(b, sizeof b, "%.17g", f);
      return std::string(b);
    };
    o << "version " << g->version << "\nalignment " << g->alignment << "\ndata_offset " << g->data_offset
      << "\nn_tensors " << g->tensors.size() << "\nn_kv " << g->kv_order.size() << "\n";
    for (const std::string& k : g->kv_order) {
      const bd::GgufValue& v = g->kv.at(k);
      o << "kv " << hex(k) << " " << v.type;
      if (v.type == bd::GV_ARRAY) {
        o << " " << v.arr_type << " " << v.arr_len();
        for (size_t j = 0; j < v.arr_len(); ++j) {
          if (v.arr_type == bd::GV_STRING) o << " " << hex(v.as[j]);
          else if (v.arr_type == bd::GV_F32 || v.arr_type == bd::GV_F64) o << " " << num(v.af[j]);
          else o << " " << v.ai[j];
        }
      } else if (v.type == bd::GV_STRING) {
        o << " " << hex(v.s);
      } else {
        o << " " << v.i << " " << num(v.f);
      }
      o << "\n";
    }
    for (const bd::GgufTensor& t : g->tensors) {
      o << "tensor " << hex(t.name) << " " << t.type << " " << t.ne.size();
      for (int64_t x : t.ne) o << " " << x;
      o << " " << t.offset << " " << t.bytes << " " << (t.data ? 1 : 0) << "\n";
    }
    txt = o.str();
  } catch (const std::exception& e) {
    std::snprintf(out, cap, "%s", e.what());
    return -1;
  }
  if (txt.size() + 1 > cap) return -2;
  std::memcpy(out, txt.c_str(), txt.size() + 1);
  return 0;
}

// A GGUF file written by the reference's own bd::GgufWriter: metadata of
// every scalar kind and arrays, and tensors of several ggml types (PTQ1_0
// data from a seeded byte stream), at the given alignment.
int ref_gguf_write_example(const char* path, uint32_t alignment, uint64_t seed) {
  try {
    bd::GgufWriter w;
    w.kv_str("general.architecture", "qwen35");
    w.kv_u32("qwen35.block_count", 2);
    w.kv_i32("test.negative", -7);
    w.kv_f32("test.eps", 1e-6f);
    w.kv_bool("test.flag", true);
    w.kv_arr_i32("test.ints", {1, -2, 3, 400000});
    w.kv_arr_f32("test.floats", {0.5f, -1.25f, 3.0e-8f});
    w.kv_arr_str("test.strings", {"a", "", "bonsai ternary", "line\nbreak"});
    uint64_t x = seed;
    auto next = [&]() {
      x += 0x9e3779b97f4a7c15ull;
      uint64_t z = x;
      z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
      z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
      return z ^ (z >> 31);
    };
    auto bytes = [&](size_t n) {
      std::vector<uint8_t> b(n);
      for (auto& c : b) c = (uint8_t)next();
      return b;
    };
    w.tensor("blk.0.ffn_gate.weight", {256, 96}, bd::T_PTQ1_0, bytes(96 * 2 * 28));
    w.tensor("blk.0.attn_norm.weight", {256}, bd::T_F32, bytes(256 * 4));
    w.tensor("blk.1.ffn_down.weight", {384, 40}, bd::T_PTQ1_0, bytes(40 * 3 * 28));
    w.tensor("blk.1.scale.weight", {64, 2}, bd::T_F16, bytes(64 * 2 * 2));
    w.tensor("output.weight", {1024, 33}, bd::T_PTQ1_0, bytes(33 * 8 * 28));
    const std::vector<uint8_t> img = w.finish(alignment);
    FILE* f = std::fopen(path, "wb");
    if (!f) return -1;
    const size_t n = std::fwrite(img.data(), 1, img.size(), f);
    std::fclose(f);
    return n == img.size() ? 0 : -1;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "ref_gguf_write_example: %s\n", e.what());
    return -1;
  }
}

}  // extern "C"
