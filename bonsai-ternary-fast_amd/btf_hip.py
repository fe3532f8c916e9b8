"""Python mirror of the reference's kernel-launch API (src/cuda/kernels.cuh,
namespace btf::cuda) over the C ABI of libbtf_hip.so (include/btf/hip_abi.h).

Names, argument order and meaning follow the reference: kernels_init,
gemv_max_nb, launch_repack, launch_prep, launch_gemv, and the Q8Act / Hx /
GemvSeg structs and GemvMode enum. Pointers are device addresses given as
ints or as torch tensors (their data_ptr()); `stream` is a hipStream_t handle
as an int (e.g. torch.cuda.current_stream().cuda_stream) or None for the null
stream. Failures raise RuntimeError with the library's message, as the
reference launchers throw std::runtime_error.

There is no fallback: importing this module fails loudly when the HIP
library has not been built.
"""
from __future__ import annotations

import ctypes as C
import enum
import os
import sys
from dataclasses import dataclass

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libbtf_hip.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(f"{LIB_PATH} is missing: build it with `make -C {HERE}` (hipcc, gfx950)")

_lib = C.CDLL(LIB_PATH)

BTF_OK, BTF_ERR_ARGS, BTF_ERR_DEVICE, BTF_ERR_LAUNCH, BTF_ERR_NOT_INIT = 0, 1, 2, 3, 4


class _Q8Act(C.Structure):
    _fields_ = [("q", C.c_void_p), ("d", C.c_void_p), ("s", C.c_void_p)]


class _Hx(C.Structure):
    _fields_ = [("block", C.c_int), ("perm_hd", C.c_int), ("perm_nk", C.c_int), ("perm_rep", C.c_int),
                ("signs", C.c_void_p)]


class _GemvSeg(C.Structure):
    _fields_ = [("codes", C.c_void_p), ("scales", C.c_void_p), ("N", C.c_int), ("y", C.c_void_p),
                ("ldy", C.c_int)]


class _StepVec(C.Structure):
    _fields_ = [("n", C.c_int), ("data", C.c_void_p)]


class _StepGemv(C.Structure):
    _fields_ = [("mode", C.c_int), ("K", C.c_int), ("N", C.c_int), ("codes", C.c_void_p), ("scales", C.c_void_p),
                ("up_codes", C.c_void_p), ("up_scales", C.c_void_p), ("in_vec", C.c_int), ("out_vec", C.c_int)]


class _StepOp(C.Structure):
    _fields_ = [("kind", C.c_int), ("gemv", _StepGemv), ("normw", C.c_void_p), ("eps", C.c_float), ("hx", _Hx),
                ("vec", C.c_int), ("table_codes", C.c_void_p), ("table_scales", C.c_void_p), ("d_tok", C.c_void_p),
                ("d_tok_out", C.c_void_p), ("d_pos", C.c_void_p)]


class _StepAudit(C.Structure):
    _fields_ = [("stores", C.c_int64), ("outside", C.c_int64), ("ops", C.c_int), ("guards", C.c_int),
                ("full", C.c_int), ("first_outside", C.c_char * 160)]


class _DeviceInfo(C.Structure):
    _fields_ = [("cu_count", C.c_int), ("lds_bytes_per_block", C.c_int), ("max_clock_khz", C.c_int),
                ("mem_clock_khz", C.c_int), ("mem_bus_width_bits", C.c_int), ("l2_bytes", C.c_int),
                ("wavefront_size", C.c_int), ("arch_major", C.c_int), ("arch_minor", C.c_int),
                ("total_mem_bytes", C.c_int64), ("name", C.c_char * 256), ("gcn_arch", C.c_char * 64)]


class _GgufHeader(C.Structure):
    _fields_ = [("version", C.c_uint32), ("alignment", C.c_uint64), ("data_offset", C.c_uint64),
                ("file_bytes", C.c_uint64), ("n_tensors", C.c_int64), ("n_kv", C.c_int64)]


class _GgufTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("n_dims", C.c_int), ("ne", C.c_int64 * 4), ("type", C.c_uint32),
                ("offset", C.c_uint64), ("bytes", C.c_uint64), ("data", C.c_void_p)]


class _GgufKv(C.Structure):
    _fields_ = [("key", C.c_void_p), ("key_len", C.c_uint64), ("type", C.c_uint32), ("arr_type", C.c_uint32),
                ("len", C.c_uint64)]


class _PackPlan(C.Structure):
    _fields_ = [("n_matrices", C.c_int64), ("codes_bytes", C.c_uint64), ("scales_bytes", C.c_uint64),
                ("arena_bytes", C.c_uint64), ("source_bytes", C.c_uint64), ("other_bytes", C.c_uint64),
                ("staging_host_bytes", C.c_uint64), ("staging_device_bytes", C.c_uint64)]


def _decl(name, args, res=C.c_int):
    f = getattr(_lib, name)
    f.argtypes = args
    f.restype = res
    return f


_vp, _i, _i64 = C.c_void_p, C.c_int, C.c_int64
_kernels_init = _decl("btf_hip_kernels_init", [_i])
_gemv_max_nb = _decl("btf_hip_gemv_max_nb", [_i])
_launch_repack = _decl("btf_hip_launch_repack", [_vp, _i64, _vp, _vp, _vp])
_launch_prep = _decl("btf_hip_launch_prep",
                     [_vp, _i, _i, _i, _vp, C.c_float, C.POINTER(_Hx), _vp, _i, C.POINTER(_Q8Act), _vp])
_launch_gemv = _decl("btf_hip_launch_gemv", [C.POINTER(_GemvSeg), _i, _i, _i, C.POINTER(_Q8Act), _i, _vp])
_launch_embed = _decl("btf_hip_launch_embed", [_vp, _vp, _vp, _i, _i, C.POINTER(_Hx), _vp, _vp])
_argmax_part_bytes = _decl("btf_hip_argmax_part_bytes", [_i], _i64)
_launch_argmax = _decl("btf_hip_launch_argmax", [_vp, _i, _vp, _vp, _vp])
_launch_argmax_noalloc = _decl("btf_hip_launch_argmax_noalloc", [_vp, _i, _vp, _vp])
_launch_pos_add = _decl("btf_hip_launch_pos_add", [_vp, _i, _vp])
_launch_gemv_ex = _decl("btf_hip_launch_gemv_ex", [C.POINTER(_GemvSeg), _i, _i, _i, C.POINTER(_Q8Act), _vp, _i, _i,
                                                    C.POINTER(_Q8Act), _vp])
_launch_gemv_ptq1_0 = _decl("btf_hip_launch_gemv_ptq1_0",
                            [C.POINTER(_GemvSeg), _i, _i, _i, C.POINTER(_Q8Act), _i, _vp])
_dump = _decl("btf_hip_gemv_i32_dump", [_vp, _i, _i, _i, C.POINTER(_Q8Act), _vp, _vp])
_set_policy = _decl("btf_hip_gemv_set_policy", [_i])
_gen = _decl("btf_hip_gen_ptq1_0", [C.c_uint64, C.c_uint64, _i64, _i64, _vp, _vp])
_stream_read = _decl("btf_hip_stream_read", [_vp, C.c_uint64, C.c_uint32, _vp, _vp])
_last_error = _decl("btf_hip_last_error", [], C.c_char_p)
_device_info = _decl("btf_hip_device_info", [_i, C.POINTER(_DeviceInfo)])
_graph_begin = _decl("btf_hip_graph_begin", [_vp])
_graph_end = _decl("btf_hip_graph_end", [_vp, C.POINTER(C.c_void_p)])
_graph_launch = _decl("btf_hip_graph_launch", [_vp, _vp])
_graph_destroy = _decl("btf_hip_graph_destroy", [_vp])
_event_create = _decl("btf_hip_event_create", [C.POINTER(C.c_void_p)])
_event_destroy = _decl("btf_hip_event_destroy", [_vp])
_event_record = _decl("btf_hip_event_record", [_vp, _vp])
_event_elapsed = _decl("btf_hip_event_elapsed_ms", [C.POINTER(C.c_float), _vp, _vp])
_host_alloc_mapped = _decl("btf_hip_host_alloc_mapped", [C.POINTER(C.c_void_p), C.POINTER(C.c_void_p), C.c_size_t])
_host_free = _decl("btf_hip_host_free", [_vp])
_step_create = _decl("btf_hip_step_create",
                     [C.POINTER(_StepVec), _i, C.POINTER(_StepGemv), _i, C.POINTER(C.c_void_p)])
_step_create_ops = _decl("btf_hip_step_create_ops",
                         [C.POINTER(_StepVec), _i, C.POINTER(_StepOp), _i, C.POINTER(C.c_void_p)])
_step_launch = _decl("btf_hip_step_launch", [_vp, _vp])
_step_error = _decl("btf_hip_step_error", [_vp, C.POINTER(C.c_int)])
_step_destroy = _decl("btf_hip_step_destroy", [_vp])
_step_spin = _decl("btf_hip_step_set_spin_limit", [_vp, C.c_uint32])
_step_guards = _decl("btf_hip_step_guards", [_vp, C.POINTER(C.c_int)])
_step_audit = _decl("btf_hip_step_audit",
                    [C.POINTER(_StepVec), _i, C.POINTER(_StepOp), _i, _i, C.POINTER(_StepAudit)])
_gguf_open = _decl("btf_hip_gguf_open", [C.c_char_p, _i, C.POINTER(C.c_void_p)])
_gguf_close = _decl("btf_hip_gguf_close", [_vp])
_gguf_info = _decl("btf_hip_gguf_info", [_vp, C.POINTER(_GgufHeader)])
_gguf_tensor = _decl("btf_hip_gguf_tensor", [_vp, _i64, C.POINTER(_GgufTensor)])
_gguf_find_tensor = _decl("btf_hip_gguf_find_tensor", [_vp, C.c_char_p], _i64)
_gguf_kv = _decl("btf_hip_gguf_kv", [_vp, _i64, C.POINTER(_GgufKv)])
_gguf_find_kv = _decl("btf_hip_gguf_find_kv", [_vp, C.c_char_p], _i64)
_gguf_kv_num = _decl("btf_hip_gguf_kv_num", [_vp, _i64, C.c_uint64, C.POINTER(C.c_int64), C.POINTER(C.c_double)])
_gguf_kv_str = _decl("btf_hip_gguf_kv_str", [_vp, _i64, C.c_uint64, C.POINTER(C.c_void_p), C.POINTER(C.c_uint64)])
_ggml_row_bytes = _decl("btf_hip_ggml_row_bytes", [C.c_uint32, _i64], _i64)
_gguf_plan = _decl("btf_hip_gguf_plan", [_vp, C.c_uint64, C.POINTER(_PackPlan)])
_loader_create = _decl("btf_hip_loader_create", [C.c_uint64, C.POINTER(C.c_void_p)])
_loader_upload = _decl("btf_hip_loader_upload_ptq1_0", [_vp, _vp, _i64, _i64, _vp, _vp, _vp])
_loader_finish = _decl("btf_hip_loader_finish", [_vp, C.POINTER(C.c_uint64)])
_loader_destroy = _decl("btf_hip_loader_destroy", [_vp])

#: Every symbol include/btf/hip_abi.h declares (checked by the CPU tests).
ABI_SYMBOLS = (
    "btf_hip_kernels_init", "btf_hip_gemv_max_nb", "btf_hip_launch_repack", "btf_hip_launch_prep",
    "btf_hip_launch_gemv", "btf_hip_launch_gemv_ex", "btf_hip_launch_gemv_ptq1_0", "btf_hip_launch_embed", "btf_hip_argmax_part_bytes",
    "btf_hip_launch_argmax", "btf_hip_launch_argmax_noalloc", "btf_hip_launch_pos_add", "btf_hip_last_error", "btf_hip_gemv_i32_dump", "btf_hip_gemv_set_policy",
    "btf_hip_gen_ptq1_0", "btf_hip_stream_read", "btf_hip_device_info", "btf_hip_device_count", "btf_hip_set_device", "btf_hip_malloc",
    "btf_hip_free", "btf_hip_host_alloc_mapped", "btf_hip_host_free", "btf_hip_memcpy_h2d", "btf_hip_memcpy_d2h",
    "btf_hip_memset", "btf_hip_device_synchronize", "btf_hip_stream_create", "btf_hip_stream_destroy",
    "btf_hip_stream_synchronize", "btf_hip_event_create", "btf_hip_event_destroy", "btf_hip_event_record",
    "btf_hip_event_elapsed_ms", "btf_hip_graph_begin", "btf_hip_graph_end", "btf_hip_graph_launch",
    "btf_hip_graph_destroy", "btf_hip_step_create", "btf_hip_step_launch", "btf_hip_step_error",
    "btf_hip_step_destroy", "btf_hip_step_set_spin_limit", "btf_hip_step_guards", "btf_hip_step_create_ops",
    "btf_hip_step_audit",
    "btf_hip_gguf_open",
    "btf_hip_gguf_close",
    "btf_hip_gguf_info", "btf_hip_gguf_tensor", "btf_hip_gguf_find_tensor", "btf_hip_gguf_kv",
    "btf_hip_gguf_find_kv", "btf_hip_gguf_kv_num", "btf_hip_gguf_kv_str", "btf_hip_ggml_row_bytes",
    "btf_hip_gguf_plan", "btf_hip_loader_create", "btf_hip_loader_upload_ptq1_0", "btf_hip_loader_finish",
    "btf_hip_loader_destroy",
)


class GemvMode(enum.IntEnum):
    """src/cuda/kernels.cuh:52"""
    kStore = 0
    kAdd = 1
    kSwiglu = 2


def _addr(p) -> int | None:
    if p is None:
        return None
    if isinstance(p, int):
        return p
    return p.data_ptr()


def _stream(st):
    if st is None:
        return None
    if isinstance(st, int):
        return st
    return st.cuda_stream  # torch.cuda.Stream


def _check(rc: int):
    if rc != BTF_OK:
        raise RuntimeError(_last_error().decode() or f"btf_hip error {rc}")


def _finalize(obj, _is_finalizing=sys.is_finalizing):
    """Release a handle from __del__, except at interpreter shutdown: then the
    HIP runtime (and a profiler attached to it) may already be torn down, and
    the process exit releases the device memory anyway. Owners that need a
    deterministic release call close() themselves. (The finalizers bind this
    function, and it binds sys.is_finalizing, as default arguments: at
    shutdown the module's globals may already be cleared.)"""
    if _is_finalizing():
        return
    obj.close()


@dataclass
class Q8Act:
    """Q8_0 activations of M rows of width K (src/cuda/kernels.cuh:26-31)."""
    q: object = None  # int8 [M][K]
    d: object = None  # f32 [M][K/32]
    s: object = None  # i32 [M][K/32]

    def _c(self):
        return _Q8Act(_addr(self.q), _addr(self.d), _addr(self.s))


@dataclass
class Hx:
    """Input transform of a folded weight, block 0 = none (src/cuda/kernels.cuh:33-38)."""
    block: int = 0
    perm_hd: int = 0
    perm_nk: int = 0
    perm_rep: int = 0
    signs: object = None  # f32 [n] or None

    def _c(self):
        return _Hx(self.block, self.perm_hd, self.perm_nk, self.perm_rep, _addr(self.signs))


@dataclass
class GemvSeg:
    """One packed matrix and its output (src/cuda/kernels.cuh:45-51)."""
    codes: object = None   # u8 [N][K/4]
    scales: object = None  # u16 [N][K/128]
    N: int = 0
    y: object = None       # f32 [M][ldy]
    ldy: int = 0

    def _c(self):
        return _GemvSeg(_addr(self.codes), _addr(self.scales), self.N, _addr(self.y), self.ldy)


def kernels_init(device: int = 0) -> None:
    """src/cuda/kernels.cuh:17"""
    _check(_kernels_init(device))


def gemv_max_nb(K: int) -> int:
    """src/cuda/kernels.cuh:20"""
    return _gemv_max_nb(K)


def launch_repack(src, nblocks: int, codes, scales, stream=None) -> None:
    """src/cuda/kernels.cuh:22-24: nblocks PTQ1_0 blocks -> T2 codes + scales."""
    _check(_launch_repack(_addr(src), nblocks, _addr(codes), _addr(scales), _stream(stream)))


def launch_prep(x, ldx: int, M: int, n: int, normw, eps: float, hx: Hx | None, xn_out, ldxn: int, a: Q8Act,
                stream=None) -> None:
    """src/cuda/kernels.cuh:40-43"""
    h = (hx or Hx())._c()
    q = a._c()
    _check(_launch_prep(_addr(x), ldx, M, n, _addr(normw), eps, C.byref(h), _addr(xn_out), ldxn, C.byref(q),
                        _stream(stream)))


def launch_gemv(segs, K: int, M: int, a: Q8Act, mode: GemvMode = GemvMode.kStore, stream=None) -> None:
    """src/cuda/kernels.cuh:53-56. `segs` is a list of 1..3 GemvSeg."""
    arr = (_GemvSeg * max(1, len(segs)))(*[s._c() for s in segs])
    q = a._c()
    _check(_launch_gemv(arr, len(segs), K, M, C.byref(q), int(mode), _stream(stream)))


def launch_embed(codes, scales, d_tok, M: int, E: int, inv: "Hx" = None, x=None, stream=None) -> None:
    """src/cuda/kernels.cuh:82-85."""
    h = (inv or Hx())._c()
    _check(_launch_embed(_addr(codes), _addr(scales), _addr(d_tok), M, E, C.byref(h), _addr(x), _stream(stream)))


def launch_embed_raw(codes, scales, d_tok, M, E, inv, x, stream=None) -> int:
    h = (inv or Hx())._c()
    return _launch_embed(_addr(codes), _addr(scales), _addr(d_tok), M, E, C.byref(h), _addr(x), _stream(stream))


def argmax_part_bytes(V: int) -> int:
    """src/cuda/kernels.cuh:89."""
    return int(_argmax_part_bytes(V))


def launch_argmax(logits, V: int, part, d_tok_out, stream=None) -> None:
    """src/cuda/kernels.cuh:87-90."""
    _check(_launch_argmax(_addr(logits), V, _addr(part), _addr(d_tok_out), _stream(stream)))


def launch_argmax_raw(logits, V, part, d_tok_out, stream=None) -> int:
    return _launch_argmax(_addr(logits), V, _addr(part), _addr(d_tok_out), _stream(stream))


def launch_argmax_noalloc(logits, V: int, d_tok_out, stream=None) -> None:
    """launch_argmax without a workspace: the library's static per-GPU scratch
    (concurrent calls on one GPU race)."""
    _check(_launch_argmax_noalloc(_addr(logits), V, _addr(d_tok_out), _stream(stream)))


def launch_argmax_noalloc_raw(logits, V, d_tok_out, stream=None) -> int:
    return _launch_argmax_noalloc(_addr(logits), V, _addr(d_tok_out), _stream(stream))


def launch_pos_add(d_pos, M: int, stream=None) -> None:
    """src/cuda/kernels.cuh:92."""
    _check(_launch_pos_add(_addr(d_pos), M, _stream(stream)))


def launch_gemv_ex(segs, K: int, M: int, a: Q8Act = None, x=None, ldx: int = 0,
                   mode: GemvMode = GemvMode.kStore, out: Q8Act = None, stream=None) -> None:
    """launch_gemv with the chain's quantizes fused in (no reference
    counterpart): input from Q8 rows `a` or fp32 rows `x` [M][ldx]; `out`
    (optional) receives the Q8 rows of the output."""
    _check(launch_gemv_ex_raw(segs, len(segs), K, M, a, x, ldx, int(mode), out, stream))


def launch_gemv_ex_raw(segs, nseg: int, K: int, M: int, a, x, ldx: int, mode: int, out=None, stream=None) -> int:
    arr = (_GemvSeg * max(1, len(segs)))(*[s._c() for s in segs]) if segs else None
    qa = C.byref(a._c()) if a is not None else None
    qo = C.byref(out._c()) if out is not None else None
    return _launch_gemv_ex(arr, nseg, K, M, qa, _addr(x), ldx, mode, qo, _stream(stream))


def launch_gemv_ptq1_0(segs, K: int, M: int, a: Q8Act, mode: GemvMode = GemvMode.kStore, stream=None) -> None:
    """launch_gemv on PTQ1_0 matrices read directly: each GemvSeg's codes are
    N rows of K/128 28-byte PTQ1_0 blocks and its scales None."""
    _check(launch_gemv_ptq1_0_raw(segs, len(segs), K, M, a, int(mode), stream))


def launch_gemv_ptq1_0_raw(segs, nseg: int, K: int, M: int, a: Q8Act, mode: int, stream=None) -> int:
    arr = (_GemvSeg * max(1, len(segs)))(*[s._c() for s in segs]) if segs else None
    q = a._c()
    return _launch_gemv_ptq1_0(arr, nseg, K, M, C.byref(q), mode, _stream(stream))


def launch_gemv_raw(segs, nseg: int, K: int, M: int, a: Q8Act, mode: int, stream=None) -> int:
    """Unchecked variant for tests of the argument validation: returns the status code."""
    arr = (_GemvSeg * max(1, len(segs)))(*[s._c() for s in segs]) if segs else None
    q = a._c()
    return _launch_gemv(arr, nseg, K, M, C.byref(q), mode, _stream(stream))


def launch_prep_raw(x, ldx, M, n, normw, eps, hx, xn_out, ldxn, a: Q8Act, stream=None) -> int:
    h = (hx or Hx())._c()
    q = a._c()
    return _launch_prep(_addr(x), ldx, M, n, _addr(normw), eps, C.byref(h), _addr(xn_out), ldxn, C.byref(q),
                        _stream(stream))


def launch_repack_raw(src, nblocks, codes, scales, stream=None) -> int:
    return _launch_repack(_addr(src), nblocks, _addr(codes), _addr(scales), _stream(stream))


def gemv_i32_dump(codes, N: int, K: int, M: int, a: Q8Act, I_out, stream=None) -> None:
    """Exact I[m][n][s] (int32 [M][N][K/32]) from the production GEMV kernels."""
    q = a._c()
    _check(_dump(_addr(codes), N, K, M, C.byref(q), _addr(I_out), _stream(stream)))


def gemv_set_policy(mfma_min_m: int) -> int:
    """Batches of M >= mfma_min_m use the int8-MFMA kernel; 0 = default. Returns the previous value."""
    return _set_policy(mfma_min_m)


def gen_ptq1_0(seed: int, mat: int, first_block: int, nblocks: int, dst, stream=None) -> None:
    """Seeded synthetic PTQ1_0 blocks on the device (benchmark weights)."""
    _check(_gen(seed, mat, first_block, nblocks, _addr(dst), _stream(stream)))


def stream_read(src, nbytes: int, sink, stream=None, never: int = 0x9E3779B9) -> None:
    """btf_hip_stream_read: a plain streaming read of nbytes at src (the
    practical HBM read ceiling); *sink is written only if the fold equals `never`."""
    _check(_stream_read(_addr(src), nbytes, never, _addr(sink), _stream(stream)))


@dataclass
class StepVec:
    """A vector slot of a step program: length n and optional device fp32 data."""
    n: int
    data: object = None


@dataclass
class StepGemv:
    """One GEMV of a step program (swiglu: codes/scales = gate, up_* = up).
    normw / eps / hx: the input's prep (launch_prep's RMSNorm and transform),
    for whole-token programs."""
    mode: int
    K: int
    N: int
    codes: object
    scales: object
    in_vec: int
    out_vec: int
    up_codes: object = None
    up_scales: object = None
    normw: object = None
    eps: float = 0.0
    hx: "Hx" = None

    def has_prep(self) -> bool:
        return self.normw is not None or (self.hx is not None and self.hx.block > 0)


@dataclass
class StepEmbed:
    """Embedding lookup of a whole-token program: vector `vec` = row *d_tok
    of the packed table, with the inverse transform `inv`."""
    vec: int
    table_codes: object
    table_scales: object
    d_tok: object
    inv: "Hx" = None


@dataclass
class StepArgmax:
    """Greedy pick over vector `vec` (directly after the GEMV that writes it)
    into *d_tok_out, then *d_pos += 1 if d_pos is given."""
    vec: int
    d_tok_out: object
    d_pos: object = None


STEP_GEMV, STEP_EMBED, STEP_ARGMAX = 0, 1, 2


def _step_gemv_c(g):
    return _StepGemv(int(g.mode), g.K, g.N, _addr(g.codes), _addr(g.scales), _addr(g.up_codes), _addr(g.up_scales),
                     g.in_vec, g.out_vec)


def _step_op_c(o):
    c = _StepOp()
    if isinstance(o, StepGemv):
        c.kind = STEP_GEMV
        c.gemv = _step_gemv_c(o)
        c.normw = _addr(o.normw)
        c.eps = o.eps
        c.hx = (o.hx or Hx())._c()
    elif isinstance(o, StepEmbed):
        c.kind = STEP_EMBED
        c.vec = o.vec
        c.table_codes, c.table_scales, c.d_tok = _addr(o.table_codes), _addr(o.table_scales), _addr(o.d_tok)
        c.hx = (o.inv or Hx())._c()
    elif isinstance(o, StepArgmax):
        c.kind = STEP_ARGMAX
        c.vec = o.vec
        c.d_tok_out, c.d_pos = _addr(o.d_tok_out), _addr(o.d_pos)
    else:
        c.kind = int(o)  # a raw kind (argument-check tests)
    return c


class StepProgram:
    """A decode step's GEMV chain run as one persistent launch
    (btf_hip_step_create / _launch / _error / _destroy). The vectors' data
    tensors must stay alive while the program exists."""

    def __init__(self, vecs, ops):
        """ops: StepGemv only (btf_hip_step_create), or with StepEmbed /
        StepArgmax / GEMV preps (btf_hip_step_create_ops)."""
        cv = (_StepVec * len(vecs))(*[_StepVec(v.n, _addr(v.data)) for v in vecs])
        h = C.c_void_p()
        if all(isinstance(o, StepGemv) and not o.has_prep() for o in ops):
            cg = (_StepGemv * len(ops))(*[_step_gemv_c(g) for g in ops])
            _check(_step_create(cv, len(vecs), cg, len(ops), C.byref(h)))
        else:
            co = (_StepOp * len(ops))(*[_step_op_c(o) for o in ops])
            _check(_step_create_ops(cv, len(vecs), co, len(ops), C.byref(h)))
        self.h = h.value
        self._keep = (vecs, ops)

    def launch(self, stream=None):
        _check(_step_launch(self.h, _stream(stream)))

    def launch_raw(self, stream=None) -> int:
        return _step_launch(self.h, _stream(stream))

    def error(self) -> int:
        """Device error flag of the launches since the last call (1 = a launch
        timed out waiting for data); clears it. Synchronise first."""
        e = C.c_int()
        _check(_step_error(self.h, C.byref(e)))
        return e.value

    def set_spin_limit(self, polls: int):
        _check(_step_spin(self.h, polls))

    def guards(self) -> int:
        """Ops that keep a write-after-read wait (test hook)."""
        g = C.c_int()
        _check(_step_guards(self.h, C.byref(g)))
        return g.value

    def close(self, _destroy=_step_destroy):
        if getattr(self, "h", None):
            _destroy(self.h)
            self.h = None

    def __del__(self, _fin=_finalize):
        _fin(self)


def step_audit(vecs, ops, G: int = 256) -> dict:
    """btf_hip_step_audit (host only, no device): the program for a grid of G
    workgroups, every global store of a launch replayed and checked against
    the buffers the program owns or was given. Pointers may be plain ints."""
    cv = (_StepVec * len(vecs))(*[_StepVec(v.n, _addr(v.data)) for v in vecs])
    co = (_StepOp * len(ops))(*[_step_op_c(o) for o in ops])
    r = _StepAudit()
    _check(_step_audit(cv, len(vecs), co, len(ops), G, C.byref(r)))
    return {"stores": r.stores, "outside": r.outside, "ops": r.ops, "guards": r.guards, "full": bool(r.full),
            "first_outside": r.first_outside.decode()}


def step_create_ops_raw(vecs, ops) -> int:
    """Status code of btf_hip_step_create_ops (the program is destroyed at once)."""
    cv = (_StepVec * max(1, len(vecs)))(*[_StepVec(v.n, _addr(v.data)) for v in vecs])
    co = (_StepOp * max(1, len(ops)))(*[_step_op_c(o) for o in ops])
    h = C.c_void_p()
    rc = _step_create_ops(cv, len(vecs), co, len(ops), C.byref(h))
    if rc == BTF_OK:
        _step_destroy(h.value)
    return rc


def step_create_raw(vecs, gemvs) -> int:
    """Status code of btf_hip_step_create (the program is destroyed at once)."""
    cv = (_StepVec * max(1, len(vecs)))(*[_StepVec(v.n, _addr(v.data)) for v in vecs])
    cg = (_StepGemv * max(1, len(gemvs)))(*[
        _StepGemv(int(g.mode), g.K, g.N, _addr(g.codes), _addr(g.scales), _addr(g.up_codes), _addr(g.up_scales),
                  g.in_vec, g.out_vec) for g in gemvs])
    h = C.c_void_p()
    rc = _step_create(cv, len(vecs), cg, len(gemvs), C.byref(h))
    if rc == BTF_OK:
        _step_destroy(h.value)
    return rc


def last_error() -> str:
    return _last_error().decode()


def device_info(device: int = 0) -> dict:
    info = _DeviceInfo()
    _check(_device_info(device, C.byref(info)))
    return {f: (getattr(info, f).decode() if isinstance(getattr(info, f), bytes) else getattr(info, f))
            for f, _ in _DeviceInfo._fields_}


class Graph:
    """A captured stream sequence, replayed with one launch (hipGraph)."""

    def __init__(self, stream):
        self.stream = _stream(stream)
        self.exec = None

    def __enter__(self):
        _check(_graph_begin(self.stream))
        return self

    def __exit__(self, et, ev, tb):
        h = C.c_void_p()
        rc = _graph_end(self.stream, C.byref(h))
        if et is None:
            _check(rc)
        self.exec = h.value

    def launch(self):
        _check(_graph_launch(self.exec, self.stream))

    def close(self, _destroy=_graph_destroy):
        if getattr(self, "exec", None):
            _destroy(self.exec)
            self.exec = None

    def __del__(self, _fin=_finalize):
        _fin(self)


class Event:
    """hipEvent on an explicit stream (timing of our own launches)."""

    def __init__(self):
        h = C.c_void_p()
        _check(_event_create(C.byref(h)))
        self.h = h.value

    def record(self, stream):
        _check(_event_record(self.h, _stream(stream)))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        _check(_event_elapsed(C.byref(ms), self.h, end.h))
        return ms.value

    def close(self, _destroy=_event_destroy):
        if getattr(self, "h", None):
            _destroy(self.h)
            self.h = None

    def __del__(self, _fin=_finalize):
        _fin(self)


class MappedHostBuffer:
    """Pinned, device-mapped host memory (launch_repack may read its source from it)."""

    def __init__(self, nbytes: int):
        host, dev = C.c_void_p(), C.c_void_p()
        _check(_host_alloc_mapped(C.byref(host), C.byref(dev), nbytes))
        self.host, self.dev, self.nbytes = host.value, dev.value, nbytes

    def view(self):
        import numpy as np
        return np.ctypeslib.as_array((C.c_uint8 * self.nbytes).from_address(self.host))

    def close(self, _free=_host_free):
        if getattr(self, "host", None):
            _free(self.host)
            self.host = None

    def __del__(self, _fin=_finalize):
        _fin(self)


GGUF_STRING, GGUF_ARRAY, GGUF_F32, GGUF_F64 = 8, 9, 6, 12
GGML_PTQ1_0 = 143


@dataclass
class GgufTensorInfo:
    name: str
    n_dims: int
    ne: tuple
    type: int
    offset: int
    bytes: int
    data: int | None  # host address inside the mapping (None: past the end of a header-only read)


class Gguf:
    """A GGUF v2/v3 file, memory-mapped (btf_hip_gguf_*): the reference's
    bd::Gguf interface (ref/bonsai-decoder/include/bd/gguf.hpp:49-85) over the
    C ABI. Raises RuntimeError with the reader's reason on a bad file."""

    def __init__(self, path: str, header_only: bool = False):
        h = C.c_void_p()
        _check(_gguf_open(os.fsencode(path), int(header_only), C.byref(h)))
        self.h = h.value
        hd = _GgufHeader()
        _check(_gguf_info(self.h, C.byref(hd)))
        self.version, self.alignment, self.data_offset = hd.version, hd.alignment, hd.data_offset
        self.file_bytes, self.n_tensors, self.n_kv = hd.file_bytes, hd.n_tensors, hd.n_kv

    def tensor_info(self, index: int) -> GgufTensorInfo:
        t = _GgufTensor()
        _check(_gguf_tensor(self.h, index, C.byref(t)))
        return GgufTensorInfo(t.name.decode("utf-8", "surrogateescape"), t.n_dims, tuple(t.ne[:t.n_dims]), t.type,
                              t.offset, t.bytes, t.data)

    @property
    def tensors(self):
        return [self.tensor_info(i) for i in range(self.n_tensors)]

    def tensor(self, name: str) -> GgufTensorInfo | None:
        i = _gguf_find_tensor(self.h, name.encode())
        return None if i < 0 else self.tensor_info(i)

    def kv_entry(self, index: int):
        """(key bytes, type, arr_type, values): numbers as (int, float)
        pairs, strings as bytes; a scalar's values hold one element."""
        k = _GgufKv()
        _check(_gguf_kv(self.h, index, C.byref(k)))
        key = C.string_at(k.key, k.key_len)
        et = k.arr_type if k.type == GGUF_ARRAY else k.type
        vals = []
        for e in range(k.len):
            if et == GGUF_STRING:
                sp, n = C.c_void_p(), C.c_uint64()
                _check(_gguf_kv_str(self.h, index, e, C.byref(sp), C.byref(n)))
                vals.append(C.string_at(sp.value, n.value) if n.value else b"")
            else:
                iv, fv = C.c_int64(), C.c_double()
                _check(_gguf_kv_num(self.h, index, e, C.byref(iv), C.byref(fv)))
                vals.append((iv.value, fv.value))
        return key, k.type, k.arr_type, vals

    def get(self, key: str, default=None):
        """A metadata value: int/float/str for a scalar, a list for an array."""
        i = _gguf_find_kv(self.h, key.encode())
        if i < 0:
            return default
        _, t, at, vals = self.kv_entry(i)
        conv = (lambda v: v.decode("utf-8", "surrogateescape")) if (at if t == GGUF_ARRAY else t) == GGUF_STRING \
            else (lambda v: v[1]) if (at if t == GGUF_ARRAY else t) in (GGUF_F32, GGUF_F64) else (lambda v: v[0])
        return [conv(v) for v in vals] if t == GGUF_ARRAY else conv(vals[0])

    def dump(self) -> str:
        """Canonical text of everything parsed (the format of the oracle's
        reference-reader dump: strings as length:hex, numbers as int and
        %.17g)."""
        def hx(b):
            return f"{len(b)}:{b.hex()}"

        def num(f):
            return ("%.17g" % f) if f == f else ("-nan" if str(f).startswith("-") else "nan")
        out = [f"version {self.version}", f"alignment {self.alignment}", f"data_offset {self.data_offset}",
               f"n_tensors {self.n_tensors}", f"n_kv {self.n_kv}"]
        for i in range(self.n_kv):
            key, t, at, vals = self.kv_entry(i)
            line = f"kv {hx(key)} {t}"
            if t == GGUF_ARRAY:
                line += f" {at} {len(vals)}"
                for v in vals:
                    line += " " + (hx(v) if at == GGUF_STRING else num(v[1]) if at in (GGUF_F32, GGUF_F64)
                                   else str(v[0]))
            elif t == GGUF_STRING:
                line += " " + hx(vals[0])
            else:
                line += f" {vals[0][0]} {num(vals[0][1])}"
            out.append(line)
        for i in range(self.n_tensors):
            t = _GgufTensor()
            _check(_gguf_tensor(self.h, i, C.byref(t)))
            out.append(f"tensor {hx(t.name)} {t.type} {t.n_dims} " + " ".join(str(x) for x in t.ne[:t.n_dims]) +
                       f" {t.offset} {t.bytes} {1 if t.data else 0}")
        return "\n".join(out) + "\n"

    def plan(self, staging_bytes: int) -> dict:
        p = _PackPlan()
        _check(_gguf_plan(self.h, staging_bytes, C.byref(p)))
        return {f: getattr(p, f) for f, _ in _PackPlan._fields_}

    def close(self, _close=_gguf_close):
        if getattr(self, "h", None):
            _close(self.h)
            self.h = None

    def __del__(self, _fin=_finalize):
        _fin(self)


def ggml_row_bytes(ggml_type: int, n: int) -> int:
    return _ggml_row_bytes(ggml_type, n)


def gguf_open_raw(path: str, header_only: bool = False) -> int:
    """Status code of btf_hip_gguf_open (the file is closed at once)."""
    h = C.c_void_p()
    rc = _gguf_open(os.fsencode(path), int(header_only), C.byref(h))
    if rc == BTF_OK:
        _gguf_close(h.value)
    return rc


class Loader:
    """Staged PTQ1_0 -> T2 upload through two pinned slots (btf_hip_loader_*)."""

    def __init__(self, staging_bytes: int):
        h = C.c_void_p()
        _check(_loader_create(staging_bytes, C.byref(h)))
        self.h = h.value

    def upload_ptq1_0(self, src, N: int, K: int, codes, scales, stream=None):
        """src: host address / numpy array of N*K/128*28 bytes; codes/scales: device."""
        if hasattr(src, "ctypes"):
            src = src.ctypes.data
        _check(_loader_upload(self.h, src, N, K, _addr(codes), _addr(scales), _stream(stream)))

    def upload_raw(self, src, N, K, codes, scales, stream=None) -> int:
        if hasattr(src, "ctypes"):
            src = src.ctypes.data
        return _loader_upload(self.h, src, N, K, _addr(codes), _addr(scales), _stream(stream))

    def finish(self) -> int:
        n = C.c_uint64()
        _check(_loader_finish(self.h, C.byref(n)))
        return n.value

    def close(self, _destroy=_loader_destroy):
        if getattr(self, "h", None):
            _destroy(self.h)
            self.h = None

    def __del__(self, _fin=_finalize):
        _fin(self)


def loader_create_raw(staging_bytes: int) -> int:
    h = C.c_void_p()
    rc = _loader_create(staging_bytes, C.byref(h))
    if rc == BTF_OK:
        _loader_destroy(h.value)
    return rc


def lib_path() -> str:
    return LIB_PATH
