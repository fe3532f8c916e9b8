"""ctypes bindings of the oracle (libbtf_oracle.so) and of the reference build
(_ref/libbtf_ref.so). TEST INFRASTRUCTURE ONLY: imported by tests/, by
__graft_entry__.smoke() and by bench.py's cpu_baseline leg, never by the
product package.

All array arguments are numpy arrays (C-contiguous); functions return new
arrays. Each wrapper names the reference file:line its C function restates.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "libbtf_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libbtf_ref.so")

_p = C.c_void_p
_i64 = C.c_int64
_i32 = C.c_int


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "array must be C-contiguous"
    return a.ctypes.data_as(C.c_void_p)


def _decl(lib, name, res, args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = args
    return f


class Oracle:
    """The C restatement (oracle/btf_oracle.c)."""

    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = self.lib = C.CDLL(path)
        _decl(L, "btf_or_fp16_to_f32", C.c_float, [C.c_uint16])
        _decl(L, "btf_or_f32_to_fp16", C.c_uint16, [C.c_float])
        _decl(L, "btf_or_ptq1_0_trit", _i32, [_p, _i32])
        _decl(L, "btf_or_quant_ptq1_0", None, [_p, _p, _i64])
        _decl(L, "btf_or_encode_trits", None, [_p, C.c_uint16, _p])
        _decl(L, "btf_or_code_byte", _i32, [_i32])
        _decl(L, "btf_or_code_shift", _i32, [_i32])
        _decl(L, "btf_or_packed_code", _i32, [_p, _i64])
        _decl(L, "btf_or_repack_rows", None, [_p, _i64, _i64, _p, _p])
        _decl(L, "btf_or_repack_blocks", None, [_p, _i64, _p, _p])
        _decl(L, "btf_or_q8_block", _i32, [_p, _p, _p])
        _decl(L, "btf_or_round_q8_0", None, [_p, _i64, _p])
        _decl(L, "btf_or_quantize_rows", None, [_p, _i32, _i32, _i32, _p, _p, _p])
        _decl(L, "btf_or_rmsnorm", None, [_p, _p, _i64, C.c_float, _p])
        _decl(L, "btf_or_fwht", None, [_p, _i32])
        _decl(L, "btf_or_hadamard_input", None, [_i32, _i32, _i32, _i32, _p, _p, _i64, _p])
        _decl(L, "btf_or_prep", _i32,
              [_p, _i32, _i32, _i32, _p, C.c_float, _i32, _i32, _i32, _i32, _p, _p, _i32, _p, _p, _p])
        _decl(L, "btf_or_dp4a", _i32, [C.c_uint32, C.c_uint32, _i32])
        _decl(L, "btf_or_sub_dot", _i32, [C.c_uint32, C.c_uint32, _p])
        _decl(L, "btf_or_gemv_i32", None, [_p, _i64, _i64, _p, _p, _i32, _p])
        _decl(L, "btf_or_gemv", None, [_p, _p, _i64, _i64, _p, _p, _p, _i32, _p, _i64, _i32, _i32])
        _decl(L, "btf_or_swiglu", None, [_p, _p, _i64])
        _decl(L, "btf_or_embed", _i32, [_p, _p, _p, _i32, _i32, _i32, _i32, _p, _p])
        _decl(L, "btf_or_argmax", _i32, [_p, _i32])
        _decl(L, "btf_or_gen_ptq1_0", None, [C.c_uint64, C.c_uint64, _i64, _i64, _p])
        _decl(L, "btf_or_hw_threads", _i32, [])

    # ---- fp16 (ref/bonsai-decoder/include/bd/types.hpp:37-57, src/types.cpp:42-62)
    def fp16_to_f32(self, h: int) -> float:
        return self.lib.btf_or_fp16_to_f32(h)

    def f32_to_fp16(self, f: float) -> int:
        return self.lib.btf_or_f32_to_fp16(f)

    # ---- PTQ1_0 (ref/bonsai-decoder/src/types.cpp:289-320, types.hpp:70-78)
    def quant_ptq1_0(self, w: np.ndarray) -> np.ndarray:
        """w float32 [N][K] -> PTQ1_0 bytes [N][K/128*28]."""
        w = np.ascontiguousarray(w, np.float32)
        N, K = w.shape
        out = np.zeros((N, K // 128 * 28), np.uint8)
        self.lib.btf_or_quant_ptq1_0(_ptr(w), _ptr(out), N * K)
        return out

    def trit(self, blk: np.ndarray, e: int) -> int:
        blk = np.ascontiguousarray(blk, np.uint8)
        return self.lib.btf_or_ptq1_0_trit(_ptr(blk), e)

    def encode_trits(self, trits: np.ndarray, scale_bits: int) -> np.ndarray:
        t = np.ascontiguousarray(trits, np.int8)
        out = np.zeros(28, np.uint8)
        self.lib.btf_or_encode_trits(_ptr(t), scale_bits, _ptr(out))
        return out

    def gen_ptq1_0(self, seed: int, mat: int, nblocks: int, first_block: int = 0) -> np.ndarray:
        out = np.zeros((nblocks, 28), np.uint8)
        self.lib.btf_or_gen_ptq1_0(seed, mat, first_block, nblocks, _ptr(out))
        return out

    # ---- T2 (include/btf/packed.hpp, src/repack.cpp:16-27)
    def repack_rows(self, src: np.ndarray, rows: int, K: int):
        src = np.ascontiguousarray(src, np.uint8)
        codes = np.zeros((rows, K // 4), np.uint8)
        scales = np.zeros((rows, K // 128), np.uint16)
        self.lib.btf_or_repack_rows(_ptr(src), rows, K, _ptr(codes), _ptr(scales))
        return codes, scales

    def repack_blocks(self, src: np.ndarray, nblocks: int):
        src = np.ascontiguousarray(src, np.uint8)
        codes = np.zeros((nblocks, 32), np.uint8)
        scales = np.zeros(nblocks, np.uint16)
        self.lib.btf_or_repack_blocks(_ptr(src), nblocks, _ptr(codes), _ptr(scales))
        return codes, scales

    def packed_code(self, row: np.ndarray, e: int) -> int:
        row = np.ascontiguousarray(row, np.uint8)
        return self.lib.btf_or_packed_code(_ptr(row), e)

    # ---- Q8 (include/btf/packed.hpp:117-134, src/emu_decoder.cpp:122-140)
    def quantize_rows(self, x: np.ndarray):
        x = np.ascontiguousarray(x, np.float32)
        M, K = x.shape
        q = np.zeros((M, K), np.int8)
        d = np.zeros((M, K // 32), np.float32)
        s = np.zeros((M, K // 32), np.int32)
        self.lib.btf_or_quantize_rows(_ptr(x), K, M, K, _ptr(q), _ptr(d), _ptr(s))
        return q, d, s

    def round_q8_0(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros_like(x)
        self.lib.btf_or_round_q8_0(_ptr(x), x.size, _ptr(out))
        return out

    def prep(self, x, normw=None, eps=1e-6, block=0, perm_hd=0, perm_nk=0, perm_rep=0, signs=None):
        """Fused prep on dense rows x [M][n] -> (q, d, s, xn)."""
        x = np.ascontiguousarray(x, np.float32)
        M, n = x.shape
        q = np.zeros((M, n), np.int8)
        d = np.zeros((M, n // 32), np.float32)
        s = np.zeros((M, n // 32), np.int32)
        xn = np.zeros((M, n), np.float32)
        nw = None if normw is None else np.ascontiguousarray(normw, np.float32)
        sg = None if signs is None else np.ascontiguousarray(signs, np.float32)
        rc = self.lib.btf_or_prep(_ptr(x), n, M, n, _ptr(nw), eps, block, perm_hd, perm_nk, perm_rep, _ptr(sg),
                                  _ptr(xn), n, _ptr(q), _ptr(d), _ptr(s))
        if rc != 0:
            raise ValueError("prep: bad geometry")
        return q, d, s, xn

    def fwht(self, x: np.ndarray) -> np.ndarray:
        y = np.array(x, np.float32, copy=True)
        self.lib.btf_or_fwht(_ptr(y), y.size)
        return y

    # ---- GEMV (src/emu_decoder.cpp:143-165)
    def sub_dot(self, w0: int, w1: int, aw: np.ndarray) -> int:
        aw = np.ascontiguousarray(aw, np.uint32)
        return self.lib.btf_or_sub_dot(w0, w1, _ptr(aw))

    def gemv_i32(self, codes, K, q, s):
        codes = np.ascontiguousarray(codes, np.uint8)
        q = np.ascontiguousarray(q, np.int8)
        s = np.ascontiguousarray(s, np.int32)
        N = codes.size // (K // 4)
        M = q.size // K
        out = np.zeros((M, N, K // 32), np.int32)
        self.lib.btf_or_gemv_i32(_ptr(codes), N, K, _ptr(q), _ptr(s), M, _ptr(out))
        return out

    def gemv(self, codes, scales, K, q, d, s, y=None, add=False, nthreads=0):
        """y [M][N] (= or +=) W x on packed weights; returns y."""
        codes = np.ascontiguousarray(codes, np.uint8)
        scales = np.ascontiguousarray(scales, np.uint16)
        q = np.ascontiguousarray(q, np.int8)
        d = np.ascontiguousarray(d, np.float32)
        s = np.ascontiguousarray(s, np.int32)
        N = codes.size // (K // 4)
        M = q.size // K
        if y is None:
            y = np.zeros((M, N), np.float32)
        assert y.dtype == np.float32 and y.flags["C_CONTIGUOUS"]
        ldy = y.shape[-1]
        self.lib.btf_or_gemv(_ptr(codes), _ptr(scales), N, K, _ptr(q), _ptr(d), _ptr(s), M, _ptr(y), ldy,
                             1 if add else 0, nthreads)
        return y

    def swiglu(self, g: np.ndarray, u: np.ndarray) -> np.ndarray:
        g = np.array(g, np.float32, copy=True)
        u = np.ascontiguousarray(u, np.float32)
        self.lib.btf_or_swiglu(_ptr(g), _ptr(u), g.size)
        return g

    # ---- either side of the chain (src/emu_decoder.cpp:171-180, 205-207;
    # ref/bonsai-decoder/src/sampler.cpp:20-25)
    def embed(self, codes, scales, toks, E, V, block=0, signs=None):
        codes = np.ascontiguousarray(codes, np.uint8)
        scales = np.ascontiguousarray(scales).view(np.uint16)
        toks = np.ascontiguousarray(toks, np.int32)
        sg = None if signs is None else np.ascontiguousarray(signs, np.float32)
        x = np.zeros((toks.size, E), np.float32)
        if self.lib.btf_or_embed(_ptr(codes), _ptr(scales), _ptr(toks), toks.size, E, V, block, _ptr(sg), _ptr(x)):
            raise ValueError("embed: token id out of range")
        return x

    def argmax(self, logits) -> int:
        logits = np.ascontiguousarray(logits, np.float32)
        return self.lib.btf_or_argmax(_ptr(logits), logits.size)

    def hw_threads(self) -> int:
        return self.lib.btf_or_hw_threads()


class Ref:
    """The reference's own CPU code, built from its sources by `make -C oracle ref`."""

    def __init__(self, path: str = REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle ref` (needs the reference checkout)")
        L = self.lib = C.CDLL(path)
        _decl(L, "ref_fp16_to_f32", C.c_float, [C.c_uint16])
        _decl(L, "ref_f32_to_fp16", C.c_uint16, [C.c_float])
        _decl(L, "ref_ptq1_0_trit", _i32, [_p, _i32])
        _decl(L, "ref_quant_ptq1_0", None, [_p, _p, _i64])
        _decl(L, "ref_dequant_ptq1_0", None, [_p, _p, _i64])
        _decl(L, "ref_repack_rows", None, [_p, _i64, _i64, _p, _p])
        _decl(L, "ref_packed_code", _i32, [_p, _i64])
        _decl(L, "ref_code_byte", _i32, [_i32])
        _decl(L, "ref_code_shift", _i32, [_i32])
        _decl(L, "ref_q8_block", _i32, [_p, _p, _p])
        _decl(L, "ref_round_q8_0", None, [_p, _i64, _p])
        _decl(L, "ref_sub_dot", _i32, [C.c_uint32, C.c_uint32, _p])
        _decl(L, "ref_silu", C.c_float, [C.c_float])
        _decl(L, "ref_rmsnorm", None, [_p, _p, _i64, C.c_float, _p])
        _decl(L, "ref_fwht", None, [_p, _i32])
        _decl(L, "ref_matvec_ptq1_0", None, [_p, _i64, _i64, _p, _p, _i32])
        _decl(L, "ref_emu_gemv", _i32, [_p, _p, _i64, _i64, _p, _p, _p, _i32, _p, _i64, _i32])
        _decl(L, "ref_emu_set_threads", None, [_i32])
        _decl(L, "ref_emu_gemv_timed", C.c_double, [_p, _p, _i64, _i64, _p, _p, _p, _i32, _p, _i64, _i32, _i32])
        _decl(L, "ref_emu_prep", _i32,
              [_p, _i32, _i32, _p, C.c_float, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _p])
        _decl(L, "ref_emu_embed", _i32, [_p, _p, _p, _i32, _i32, _i32, _i32, _p, _p])
        _decl(L, "ref_argmax", _i32, [_p, _i32])
        _decl(L, "ref_gguf_dump", _i32, [C.c_char_p, _i32, C.c_char_p, C.c_size_t])
        _decl(L, "ref_gguf_write_example", _i32, [C.c_char_p, C.c_uint32, C.c_uint64])

    def gguf_dump(self, path, header_only=False):
        """(ok, text): the reference reader's canonical dump of a GGUF file,
        or its error message."""
        buf = C.create_string_buffer(1 << 22)
        rc = self.lib.ref_gguf_dump(os.fsencode(path), int(header_only), buf, len(buf))
        if rc == -2:
            raise RuntimeError("ref_gguf_dump: output buffer too small")
        return rc == 0, buf.value.decode()

    def gguf_write_example(self, path, alignment=32, seed=1):
        if self.lib.ref_gguf_write_example(os.fsencode(path), alignment, seed) != 0:
            raise RuntimeError("ref_gguf_write_example failed")

    def quant_ptq1_0(self, w):
        w = np.ascontiguousarray(w, np.float32)
        N, K = w.shape
        out = np.zeros((N, K // 128 * 28), np.uint8)
        self.lib.ref_quant_ptq1_0(_ptr(w), _ptr(out), N * K)
        return out

    def dequant_ptq1_0(self, src, n):
        src = np.ascontiguousarray(src, np.uint8)
        out = np.zeros(n, np.float32)
        self.lib.ref_dequant_ptq1_0(_ptr(src), _ptr(out), n)
        return out

    def repack_rows(self, src, rows, K):
        src = np.ascontiguousarray(src, np.uint8)
        codes = np.zeros((rows, K // 4), np.uint8)
        scales = np.zeros((rows, K // 128), np.uint16)
        self.lib.ref_repack_rows(_ptr(src), rows, K, _ptr(codes), _ptr(scales))
        return codes, scales

    def q8_block(self, x):
        x = np.ascontiguousarray(x, np.float32)
        q = np.zeros(32, np.int8)
        d = np.zeros(1, np.float32)
        s = self.lib.ref_q8_block(_ptr(x), _ptr(q), _ptr(d))
        return q, d[0], s

    def round_q8_0(self, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros_like(x)
        self.lib.ref_round_q8_0(_ptr(x), x.size, _ptr(out))
        return out

    def matvec_ptq1_0(self, src, N, K, x, ggml_act=True):
        src = np.ascontiguousarray(src, np.uint8)
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(N, np.float32)
        self.lib.ref_matvec_ptq1_0(_ptr(src), N, K, _ptr(x), _ptr(y), 1 if ggml_act else 0)
        return y

    def emu_gemv(self, codes, scales, K, q, d, s, y=None, add=False):
        codes = np.ascontiguousarray(codes, np.uint8)
        scales = np.ascontiguousarray(scales, np.uint16)
        q = np.ascontiguousarray(q, np.int8)
        d = np.ascontiguousarray(d, np.float32)
        s = np.ascontiguousarray(s, np.int32)
        N = codes.size // (K // 4)
        M = q.size // K
        if y is None:
            y = np.zeros((M, N), np.float32)
        rc = self.lib.ref_emu_gemv(_ptr(codes), _ptr(scales), N, K, _ptr(q), _ptr(d), _ptr(s), M, _ptr(y),
                                   y.shape[-1], 1 if add else 0)
        if rc != 0:
            raise RuntimeError("ref_emu_gemv failed")
        return y

    def emu_gemv_timed(self, codes, scales, K, q, d, s, reps=1, threads=0, add=False):
        """Seconds spent in `reps` calls of the emulator GEMV on `threads` threads."""
        codes = np.ascontiguousarray(codes, np.uint8)
        scales = np.ascontiguousarray(scales, np.uint16)
        q = np.ascontiguousarray(q, np.int8)
        d = np.ascontiguousarray(d, np.float32)
        s = np.ascontiguousarray(s, np.int32)
        N = codes.size // (K // 4)
        M = q.size // K
        y = np.zeros((M, N), np.float32)
        self.lib.ref_emu_set_threads(threads)
        t = self.lib.ref_emu_gemv_timed(_ptr(codes), _ptr(scales), N, K, _ptr(q), _ptr(d), _ptr(s), M, _ptr(y),
                                        N, 1 if add else 0, reps)
        if t < 0:
            raise RuntimeError("ref_emu_gemv_timed failed")
        return t, y

    def emu_prep(self, x, normw=None, eps=1e-6, block=0, perm_hd=0, perm_nk=0, perm_rep=0, signs=None):
        x = np.ascontiguousarray(x, np.float32)
        M, n = x.shape
        q = np.zeros((M, n), np.int8)
        d = np.zeros((M, n // 32), np.float32)
        s = np.zeros((M, n // 32), np.int32)
        xn = np.zeros((M, n), np.float32)
        nw = None if normw is None else np.ascontiguousarray(normw, np.float32)
        sg = None if signs is None else np.ascontiguousarray(signs, np.float32)
        rc = self.lib.ref_emu_prep(_ptr(x), M, n, _ptr(nw), eps, block, perm_hd, perm_nk, perm_rep, _ptr(sg),
                                   _ptr(xn), _ptr(q), _ptr(d), _ptr(s))
        if rc != 0:
            raise ValueError("ref_emu_prep failed")
        return q, d, s, xn

    def emu_embed(self, codes, scales, toks, E, V, block=0, signs=None):
        codes = np.ascontiguousarray(codes, np.uint8)
        scales = np.ascontiguousarray(scales).view(np.uint16)
        toks = np.ascontiguousarray(toks, np.int32)
        sg = None if signs is None else np.ascontiguousarray(signs, np.float32)
        x = np.zeros((toks.size, E), np.float32)
        if self.lib.ref_emu_embed(_ptr(codes), _ptr(scales), _ptr(toks), toks.size, E, V, block, _ptr(sg), _ptr(x)):
            raise ValueError("embed: token id out of range")
        return x

    def argmax(self, logits) -> int:
        logits = np.ascontiguousarray(logits, np.float32)
        return self.lib.ref_argmax(_ptr(logits), logits.size)


def have_ref() -> bool:
    return os.path.exists(REF_SO)
