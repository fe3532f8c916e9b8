"""CPU tests of the C ABI boundary (include/btf/hip_abi.h, libbtf_hip.so):
the library loads without a GPU, exports exactly what the header declares,
rejects invalid arguments on the host before any HIP call (as the reference
launchers validate before launching, src/cuda/kernels.cu:737-822), and the
C header / C++ mirror (include/btf/kernels.hpp) compile and link as a
reference-side caller would use them.
"""
import ctypes as C
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include")
PKG = os.path.join(ROOT, "bonsai-ternary-fast_amd")
LIB = os.path.join(PKG, "libbtf_hip.so")

pytestmark = pytest.mark.skipif(not os.path.exists(LIB), reason="libbtf_hip.so not built")


def header_symbols():
    text = open(os.path.join(INC, "btf", "hip_abi.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(btf_hip_\w+)\s*\(", text)))


def test_header_symbols_exported():
    lib = C.CDLL(LIB)
    syms = header_symbols()
    assert len(syms) >= 30
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing


def test_python_mirror_lists_every_symbol():
    import btf_hip
    assert sorted(btf_hip.ABI_SYMBOLS) == header_symbols()


def test_exported_names_are_only_the_abi():
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    out = subprocess.run([nm, "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    exported = sorted({l.split()[-1] for l in out.splitlines() if l.split() and l.split()[-1].startswith("btf_")})
    assert exported == header_symbols()


def test_pure_host_queries():
    import btf_hip
    assert btf_hip.gemv_max_nb(5120) > 0
    assert btf_hip.gemv_max_nb(100) == 0
    assert btf_hip.gemv_max_nb(0) == 0
    prev = btf_hip.gemv_set_policy(7)
    assert btf_hip.gemv_set_policy(prev) == 7


def test_invalid_arguments_rejected_on_host():
    """Every one of these fails in the host-side checks (no device exists in
    this process, so reaching a HIP call would give another code)."""
    import btf_hip as h
    ARGS = h.BTF_ERR_ARGS
    codes, scales, y = 0x100000, 0x200000, 0x300000
    act = h.Q8Act(0x400000, 0x500000, 0x600000)
    seg = h.GemvSeg(codes, scales, 64, y, 64)
    assert h.launch_gemv_raw([seg], 1, 100, 1, act, 0) == ARGS                       # K % 128
    assert h.launch_gemv_raw([seg], 0, 1024, 1, act, 0) == ARGS                      # no segment
    assert h.launch_gemv_raw([seg] * 3, 4, 1024, 1, act, 0) == ARGS                  # > 3 segments
    assert h.launch_gemv_raw([seg], 1, 1024, 1, act, 9) == ARGS                      # mode
    assert h.launch_gemv_raw([seg], 1, 1024, 1, act, 2) == ARGS                      # swiglu needs 2 segs
    assert h.launch_gemv_raw([h.GemvSeg(codes + 4, scales, 64, y, 64)], 1, 1024, 1, act, 0) == ARGS  # align
    assert h.launch_gemv_raw([h.GemvSeg(codes, scales, 64, None, 64)], 1, 1024, 1, act, 0) == ARGS  # null y
    assert h.launch_gemv_raw([h.GemvSeg(codes, scales, 64, y, 32)], 1, 1024, 2, act, 0) == ARGS   # ldy < N
    assert h.launch_gemv_raw([seg], 1, 1024, 1, h.Q8Act(0x400001, 0x500000, 0x600000), 0) == ARGS  # q align
    assert "gemv" in h.last_error()
    assert h.launch_repack_raw(codes, -1, codes, scales) == h.BTF_OK                 # empty: no-op
    assert h.launch_repack_raw(codes + 2, 10, codes, scales) == ARGS                 # src alignment
    assert h.launch_repack_raw(codes, 10, codes + 8, scales) == ARGS                 # codes alignment
    assert h.launch_prep_raw(y, 100, 1, 100, None, 0.0, None, None, 0, act) == ARGS   # n % 32
    assert h.launch_prep_raw(y, 64, 1, 128, None, 0.0, None, None, 0, act) == ARGS    # ldx < n
    # fused-quantize GEMV: one input, x alignment / stride, K, the output's shape, and the launch_gemv checks
    xa = 0x700000
    ex = h.launch_gemv_ex_raw
    assert ex([seg], 1, 1024, 1, None, xa + 4, 1024, 0) == ARGS                # x alignment
    assert ex([seg], 1, 1024, 1, None, xa, 1000, 0) == ARGS                    # ldx < K
    assert ex([seg], 1, 1024, 1, None, xa, 1026, 0) == ARGS                    # ldx % 4
    assert ex([seg], 1, 1000, 1, None, xa, 1024, 0) == ARGS                    # K % 128
    assert ex([seg], 1, 40960, 1, None, xa, 40960, 0) == ARGS                  # K too large
    assert ex([seg], 1, 1024, 1, None, None, 1024, 0) == ARGS                  # no input
    assert ex([seg], 1, 1024, 1, act, xa, 1024, 0) == ARGS                     # two inputs
    assert ex([seg], 1, 1024, 1, None, xa, 1024, 2) == ARGS                    # swiglu needs 2 segs
    assert ex([h.GemvSeg(codes, scales, 48, y, 48)], 1, 1024, 1, act, None, 0, 0, act) == ARGS  # out: N % 32
    assert ex([seg, seg], 2, 1024, 1, act, None, 0, 0, act) == ARGS            # out: one segment
    assert ex([seg], 1, 1024, 1, act, None, 0, 0, h.Q8Act(0x400001, 0x500000, 0x600000)) == ARGS  # out align
    assert ex([seg], 1, 1024, 0, None, xa, 1024, 0) == h.BTF_OK                # M = 0: no-op
    # PTQ1_0 GEMV: blocks carry their scales (scales must be NULL), 4-byte alignment, K <= 32768
    b3 = h.launch_gemv_ptq1_0_raw
    pseg = h.GemvSeg(codes + 4, None, 64, y, 64)
    assert b3([h.GemvSeg(codes, scales, 64, y, 64)], 1, 1024, 1, act, 0) == ARGS  # scales given
    assert "NULL" in h.last_error()
    assert b3([h.GemvSeg(codes + 2, None, 64, y, 64)], 1, 1024, 1, act, 0) == ARGS  # block alignment
    assert b3([pseg], 1, 1000, 1, act, 0) == ARGS                                 # K % 128
    assert b3([pseg], 1, 32768 + 128, 1, act, 0) == ARGS                          # K too large
    assert b3([pseg], 1, 1024, 1, act, 2) == ARGS                                 # swiglu needs 2 segs
    assert b3([h.GemvSeg(codes, None, 64, None, 64)], 1, 1024, 1, act, 0) == ARGS  # null y
    assert b3([h.GemvSeg(None, None, 64, y, 64)], 1, 1024, 1, act, 0) == ARGS     # null blocks
    assert b3([pseg], 1, 1024, 1, h.Q8Act(0x400001, 0x500000, 0x600000), 0) == ARGS  # q alignment
    assert b3([pseg], 1, 1024, 0, act, 0) == h.BTF_OK                             # M = 0: no-op
    assert b3([pseg], 1, 1024, 1, act, 0) == h.BTF_ERR_NOT_INIT                   # valid: needs a device
    # decode-step ends: embedding lookup, greedy pick, position counter
    tok = 0x800000
    assert h.launch_embed_raw(codes, scales, tok, 1, 1000, None, y) == ARGS                 # E % 128
    assert h.launch_embed_raw(codes, scales, None, 1, 1024, None, y) == ARGS                # null ids
    assert h.launch_embed_raw(codes + 2, scales, tok, 1, 1024, None, y) == ARGS             # codes alignment
    assert h.launch_embed_raw(codes, scales, tok, 1, 1024, h.Hx(block=96), y) == ARGS       # block not 2^k
    assert h.launch_embed_raw(codes, scales, tok, 0, 1024, None, y) == h.BTF_OK            # M = 0: no-op
    # one 8-byte key per part of up to 2048 logits, at most 256 parts
    assert h.argmax_part_bytes(248320) == 8 * ((248320 + 2047) // 2048)
    assert h.argmax_part_bytes(10 ** 7) == 8 * 256 and h.argmax_part_bytes(1) == 8
    assert h.launch_argmax_raw(y, 0, y, tok) == ARGS                                        # empty vocabulary
    assert h.launch_argmax_raw(y, 100, y + 4, tok) == ARGS                                  # part alignment
    assert h.launch_argmax_raw(None, 100, y, tok) == ARGS                                   # null logits
    # step programs: every structural error is caught before the device is touched
    G = h.GemvMode
    vecs = [h.StepVec(1024, y), h.StepVec(1024, None)]
    bad = [
        h.StepGemv(G.kStore, 1024, 1024, codes, scales, 0, 0),
        h.StepGemv(G.kStore, 1000, 1024, codes, scales, 0, 1),
        h.StepGemv(G.kStore, 1024, 512, codes, scales, 0, 1),
        h.StepGemv(G.kStore, 1024, 1024, codes, scales, 0, 5),
        h.StepGemv(G.kSwiglu, 1024, 1024, codes, scales, 0, 1),
        h.StepGemv(G.kStore, 1024, 1024, codes + 8, scales, 0, 1),
        h.StepGemv(G.kStore, 1024, 1024, codes, scales, 1, 0),
    ]
    for b in bad:
        assert h.step_create_raw(vecs, [b]) == ARGS, b
    assert h.step_create_raw([], []) == ARGS


def test_whole_token_programs_checked_on_host():
    """btf_hip_step_create_ops rejects malformed whole-token programs before
    any HIP call (BTF_ERR_ARGS); a valid one only fails for want of a device."""
    import btf_hip as h
    ARGS = h.BTF_ERR_ARGS
    G = h.GemvMode
    codes, scales, y, tok = 0x100000, 0x200000, 0x300000, 0x400000
    E, F, V = 2048, 3072, 4000
    vecs = [h.StepVec(E, y), h.StepVec(F, None), h.StepVec(V, y + 0x10000)]
    emb = h.StepEmbed(0, codes, scales, tok, h.Hx(block=1024))
    up = h.StepGemv(G.kStore, E, F, codes, scales, 0, 1, normw=y, eps=1e-6, hx=h.Hx(block=256))
    down = h.StepGemv(G.kAdd, F, E, codes, scales, 1, 0, hx=h.Hx(block=1024))
    head = h.StepGemv(G.kStore, E, V, codes, scales, 0, 2, normw=y, eps=1e-6)
    pick = h.StepArgmax(2, tok, tok + 4)
    good = [emb, up, down, head, pick]
    assert h.step_create_ops_raw(vecs, good) == h.BTF_ERR_NOT_INIT  # valid: needs a device
    bad = {
        "embed after a GEMV": [up, emb, down, head, pick],
        "embed width": ([h.StepVec(1536, y)] + vecs[1:], [h.StepEmbed(0, codes, scales, tok), up]),
        "embed table": [h.StepEmbed(0, None, scales, tok), up],
        "embed token": [h.StepEmbed(0, codes, scales, None), up],
        "embed table alignment": [h.StepEmbed(0, codes + 2, scales, tok), up],
        "embed block": [h.StepEmbed(0, codes, scales, tok, h.Hx(block=96)), up],
        "embedded twice": [emb, h.StepEmbed(0, codes, scales, tok), up],
        "pick not after its GEMV": [emb, up, down, pick, head],
        "pick of another vector": [emb, up, down, head, h.StepArgmax(1, tok)],
        "two picks": [emb, up, down, head, pick, pick],
        "pick output": [emb, up, down, head, h.StepArgmax(2, None)],
        "prep input length": [emb, h.StepGemv(G.kStore, 1024, F, codes, scales, 0, 1, normw=y)],
        "prep block": [emb, h.StepGemv(G.kStore, E, F, codes, scales, 0, 1, hx=h.Hx(block=2048))],
        "prep block power of two": [emb, h.StepGemv(G.kStore, E, F, codes, scales, 0, 1, hx=h.Hx(block=384))],
        "perm geometry": [emb, h.StepGemv(G.kStore, E, F, codes, scales, 0, 1, hx=h.Hx(1024, 32, 16, 2))],
        "perm tile": [emb, h.StepGemv(G.kStore, E, F, codes, scales, 0, 1, hx=h.Hx(1024, 8, 128, 2))],
        "unknown kind": [emb, up, 7],
        "no GEMV": [emb],
    }
    for what, prog in bad.items():
        v, ops = prog if isinstance(prog, tuple) else (vecs, prog)
        assert h.step_create_ops_raw(v, ops) == ARGS, what
        assert h.last_error(), what


def _compile_and_run(tmp_path, name, src, compiler, std):
    cc = shutil.which(compiler)
    if cc is None:
        pytest.skip(f"{compiler} not available")
    path = tmp_path / name
    path.write_text(src)
    exe = tmp_path / (name + ".bin")
    subprocess.run([cc, std, "-Wall", "-Werror", "-I", INC, str(path), "-o", str(exe), "-L", PKG, "-lbtf_hip",
                    f"-Wl,-rpath,{PKG}"], check=True, capture_output=True, text=True)
    return subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)


C_SRC = r"""
#include <stdio.h>
#include "btf/hip_abi.h"
int main(void) {
  btf_gemv_seg seg = {0, 0, 64, 0, 64};
  btf_q8act a = {0, 0, 0};
  int rc = btf_hip_launch_gemv(&seg, 1, 100, 1, &a, BTF_GEMV_STORE, NULL);
  printf("%d %d %s\n", btf_hip_gemv_max_nb(5120) > 0, rc, btf_hip_last_error());
  return rc == BTF_ERR_ARGS ? 0 : 1;
}
"""

CPP_SRC = r"""
#include <cstdio>
#include <stdexcept>
#include "btf/kernels.hpp"
int main() {
  btf::hip::GemvSeg seg;
  seg.N = 64;
  btf::hip::Q8Act a;
  try {
    btf::hip::launch_gemv(&seg, 1, 100, 1, a, btf::hip::kStore, nullptr);
  } catch (const std::runtime_error& e) {
    std::printf("threw: %s\n", e.what());
    return btf::hip::gemv_max_nb(5120) > 0 ? 0 : 2;
  }
  return 1;
}
"""


def test_c_header_compiles_links_and_validates(tmp_path):
    r = _compile_and_run(tmp_path, "abi_c.c", C_SRC, "gcc", "-std=c11")
    assert r.returncode == 0, r.stdout + r.stderr
    assert "multiple of 128" in r.stdout


def test_cpp_mirror_throws_like_the_reference(tmp_path):
    r = _compile_and_run(tmp_path, "abi_cpp.cpp", CPP_SRC, "g++", "-std=c++17")
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("threw: launch_gemv:")
