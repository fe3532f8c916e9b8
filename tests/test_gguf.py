"""CPU tests of the load path's GGUF reader and memory plan (btf_hip_gguf_*,
csrc/gguf.cpp, csrc/loader.hip's plan).

The reader is pinned against the reference's own reader, bd::Gguf
(ref/bonsai-decoder/src/gguf.cpp:73-147, built into oracle/_ref): on files
written by the reference's writer and by tests/gguf_writer.py (every value
kind, v2 and v3, several alignments), both readers produce the same canonical
dump (header, every key/value in file order, every tensor info); on malformed
files both reject or accept alike -- including every truncation of a file,
in full and header-only mode. Tensor data pointers are checked against the
bytes written; the plan and the ggml row sizes against closed forms."""
import ctypes as C
import os
import struct

import numpy as np
import pytest

import gguf_writer as gw


@pytest.fixture(scope="module")
def lib():
    import btf_hip
    return btf_hip


def rich_writer(version=3, alignment=32, seed=3):
    rng = np.random.default_rng(seed)
    w = gw.Writer(version=version, alignment=alignment)
    w.add("general.architecture", gw.STRING, "qwen35")
    w.add("u8", gw.U8, 250).add("i8", gw.I8, -100).add("u16", gw.U16, 65000).add("i16", gw.I16, -30000)
    w.add("u32", gw.U32, 4000000000).add("i32", gw.I32, -2000000000).add("u64", gw.U64, (1 << 64) - 5)
    w.add("i64", gw.I64, -(1 << 62)).add("f32", gw.F32, 3.25e-7).add("f64", gw.F64, -1.0e300)
    w.add("neg_f32", gw.F32, -7.9).add("bool_t", gw.BOOL, 1).add("bool_raw", gw.BOOL, 7)
    w.add("empty_str", gw.STRING, "").add("bytes\x00key", gw.STRING, b"a\x00b\xff")
    w.add("arr_u8", gw.ARRAY, [0, 1, 255], gw.U8).add("arr_i64", gw.ARRAY, [-1, 1 << 40], gw.I64)
    w.add("arr_f32", gw.ARRAY, [0.5, -2.0, 1e-20], gw.F32).add("arr_f64", gw.ARRAY, [1.5, -0.25], gw.F64)
    w.add("arr_bool", gw.ARRAY, [1, 0, 9], gw.BOOL).add("arr_str", gw.ARRAY, ["x", "", "tok en"], gw.STRING)
    w.add("arr_empty", gw.ARRAY, [], gw.I32).add("u32", gw.U32, 5)  # a key present twice
    w.tensor("blk.0.ffn_gate.weight", (256, 12), 143, gw.ptq1_0_bytes(rng, 12, 256))
    w.tensor("blk.0.attn_norm.weight", (64,), 0, rng.integers(0, 256, 256, dtype=np.uint8))
    w.tensor("blk.0.q8", (64, 3), 8, rng.integers(0, 256, 2 * 3 * 34, dtype=np.uint8))
    w.tensor("blk.0.emb", (32, 2, 3), 1, rng.integers(0, 256, 32 * 6 * 2, dtype=np.uint8))
    w.tensor("output.weight", (384, 7), 143, gw.ptq1_0_bytes(rng, 7, 384))
    w.tensor("x4d", (2, 1, 3, 1), 30, rng.integers(0, 256, 12, dtype=np.uint8))
    return w


def test_reads_reference_written_files(lib, ref, tmp_path):
    for a in (32, 64, 256):
        p = str(tmp_path / f"ex{a}.gguf")
        ref.gguf_write_example(p, alignment=a, seed=a)
        ok, text = ref.gguf_dump(p)
        assert ok, text
        g = lib.Gguf(p)
        assert g.dump() == text
        assert g.get("general.architecture") == "qwen35" and g.get("qwen35.block_count") == 2
        assert g.get("test.strings") == ["a", "", "bonsai ternary", "line\nbreak"]
        assert g.alignment == a and g.n_tensors == 5


@pytest.mark.parametrize("version,alignment", [(3, 32), (2, 32), (3, 16), (3, 1024)])
def test_same_parse_as_reference_reader(lib, ref, tmp_path, version, alignment):
    p = str(tmp_path / "rich.gguf")
    img = rich_writer(version, alignment).write(p)
    ok, text = ref.gguf_dump(p)
    assert ok, text
    g = lib.Gguf(p)
    assert g.dump() == text
    assert g.version == version and g.alignment == alignment and g.file_bytes == len(img)
    # typed access; the repeated key resolves to its last value
    assert g.get("u32") == 5 and g.get("i8") == -100 and g.get("bool_raw") == 1
    assert g.get("f32") == pytest.approx(3.25e-7) and g.get("arr_str") == ["x", "", "tok en"]
    assert g.get("missing", "dflt") == "dflt"
    # tensor data are the written bytes, in the mapping
    rng = np.random.default_rng(3)
    want = gw.ptq1_0_bytes(rng, 12, 256)
    t = g.tensor("blk.0.ffn_gate.weight")
    assert t.ne == (256, 12) and t.type == 143 and t.bytes == 12 * 2 * 28
    assert C.string_at(t.data, t.bytes) == want.tobytes()
    assert t.data == _map_base(g) + g.data_offset + t.offset
    assert g.tensor("nope") is None


def _map_base(g):
    t0 = g.tensor_info(0)
    return t0.data - g.data_offset - t0.offset


def test_every_truncation_like_the_reference(lib, ref, tmp_path):
    """Each prefix of a small file: both readers reject it, or both read the
    same header (header-only mode accepts tensors past the end)."""
    w = gw.Writer(alignment=32)
    w.add("general.architecture", gw.STRING, "t").add("arr", gw.ARRAY, [1, 2, 3], gw.U16)
    w.tensor("a", (128, 2), 143, bytes(range(56)))
    w.tensor("b", (4,), 0, bytes(16))
    img = w.build()
    p = str(tmp_path / "t.gguf")
    for n in list(range(1, len(img) + 1)):
        with open(p, "wb") as f:
            f.write(img[:n])
        for header_only in (False, True):
            ok, text = ref.gguf_dump(p, header_only)
            rc = lib.gguf_open_raw(p, header_only)
            assert (rc == 0) == ok, (n, header_only, text, lib.last_error())
            if ok:
                assert lib.Gguf(p, header_only).dump() == text, (n, header_only)


def _bad(lib, ref, path, img, reason):
    with open(path, "wb") as f:
        f.write(img)
    ok, text = ref.gguf_dump(path)
    assert not ok, "the reference reader accepted it"
    assert lib.gguf_open_raw(path) != 0
    assert reason in lib.last_error(), (lib.last_error(), text)


def test_malformed_files_rejected_like_the_reference(lib, ref, tmp_path):
    p = str(tmp_path / "bad.gguf")
    good = gw.Writer().add("k", gw.U32, 1).tensor("t", (128, 1), 143, bytes(28)).build()
    _bad(lib, ref, p, b"GGUX" + good[4:], "bad magic")
    _bad(lib, ref, p, good[:4] + struct.pack("<I", 1) + good[8:], "unsupported version")
    _bad(lib, ref, p, good[:4] + struct.pack("<I", 4) + good[8:], "unsupported version")
    _bad(lib, ref, p, good[:8] + struct.pack("<Q", 1 << 25) + good[16:], "implausible counts")
    _bad(lib, ref, p, gw.Writer(alignment=24).tensor("t", (128, 1), 143, bytes(28)).build(), "bad alignment")
    w = gw.Writer(write_alignment_key=False).add("general.alignment", gw.STRING, "32")
    _bad(lib, ref, p, w.build(), "bad alignment")
    _bad(lib, ref, p, gw.Writer().tensor("t", (100, 1), 143, bytes(28)).build(), "row not whole blocks")
    _bad(lib, ref, p, gw.Writer().tensor("t", (128, 1), 77, bytes(28)).build(), "unknown ggml type")
    _bad(lib, ref, p, gw.Writer().tensor("t", (128, 1), 143, bytes(28), offset=8).build(), "misaligned")
    _bad(lib, ref, p, gw.Writer().tensor("t", (), 0, b"").build(), "bad n_dims")
    _bad(lib, ref, p, gw.Writer().tensor("t", (1, 1, 1, 1, 1), 0, bytes(4)).build(), "bad n_dims")
    w = gw.Writer()
    w.kv.append(struct.pack("<Q", 1) + b"k" + struct.pack("<IQ", gw.STRING, (1 << 30) + 1))
    _bad(lib, ref, p, w.build(), "string too long")
    w = gw.Writer()
    w.kv.append(struct.pack("<Q", 1) + b"k" + struct.pack("<IIQ", gw.ARRAY, gw.U8, (1 << 32) + 1))
    _bad(lib, ref, p, w.build(), "array too large")
    w = gw.Writer()
    w.kv.append(struct.pack("<Q", 1) + b"k" + struct.pack("<I", 13) + bytes(8))
    _bad(lib, ref, p, w.build(), "bad value type")
    # tensor data past the end: rejected, accepted header-only (data NULL)
    img = gw.Writer().tensor("t", (128, 4), 143, bytes(112)).build()
    _bad(lib, ref, p, img[:-40], "past end")
    ok, text = ref.gguf_dump(p, True)
    assert ok and lib.Gguf(p, True).dump() == text
    assert lib.Gguf(p, True).tensor("t").data is None
    assert lib.gguf_open_raw(str(tmp_path / "absent.gguf")) != 0


def test_ggml_row_bytes(lib):
    for ty, (blk, nb) in gw.GGML.items():
        assert lib.ggml_row_bytes(ty, 4 * blk) == 4 * nb
        if blk > 1:
            assert lib.ggml_row_bytes(ty, blk + 1) == -1
    assert lib.ggml_row_bytes(143, 5120) == 40 * 28
    assert lib.ggml_row_bytes(99, 32) == -1


def test_plan_closed_form(lib, tmp_path):
    rng = np.random.default_rng(9)
    w = gw.Writer(alignment=64)
    shapes = [(5120, 7), (1024, 33), (128, 1)]
    for i, (K, N) in enumerate(shapes):
        w.tensor(f"m{i}", (K, N), 143, gw.ptq1_0_bytes(rng, N, K))
    w.tensor("norm", (96,), 0, bytes(384))
    w.tensor("pq", (128, 2), 142, bytes(68))        # a different packed type: not a T2 matrix
    w.tensor("vec3d", (128, 2, 2), 143, bytes(112))  # PTQ1_0 but not 2-D
    p = str(tmp_path / "plan.gguf")
    w.write(p)
    plan = lib.Gguf(p).plan(1 << 20)
    cb = sum(N * K // 4 for K, N in shapes)
    sb = sum(N * K // 64 for K, N in shapes)
    up = lambda x: (x + 255) // 256 * 256
    assert plan["n_matrices"] == 3
    assert plan["codes_bytes"] == cb and plan["scales_bytes"] == sb
    assert plan["arena_bytes"] == sum(up(N * K // 4) + up(N * K // 64) for K, N in shapes)
    assert plan["source_bytes"] == sum(N * K // 128 * 28 for K, N in shapes)
    assert plan["other_bytes"] == 384 + 68 + 112
    assert plan["staging_host_bytes"] == plan["staging_device_bytes"] == 2 << 20


def test_loader_argument_checks_without_device(lib):
    # no device in this process: creation needs kernels_init on a device
    assert lib.loader_create_raw(1 << 20) != 0
    assert lib.loader_create_raw(4) != 0  # slot smaller than one PTQ1_0 block
