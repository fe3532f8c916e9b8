"""GPU tests of the load path: GGUF file -> staged upload -> T2 layout
(btf_hip_gguf_*, btf_hip_loader_*), byte-exact against the oracle's host
repack (oracle/btf_oracle.c, pinned to the reference's src/repack.cpp:16-27).

The loader's staging slots are sized so a matrix crosses many slices (both
slots in turn, a last slice shorter than the others, one row per slice),
and every matrix of a GGUF written with tests/gguf_writer.py is uploaded
from the file's mapping into one device arena laid out by the plan."""
import numpy as np
import pytest

import gguf_writer as gw

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def stream():
    return _torch().cuda.current_stream().cuda_stream


def oracle_repack(oracle, src, N, K):
    return oracle.repack_rows(np.ascontiguousarray(src, np.uint8).reshape(N, K // 128 * 28), N, K)


def test_loader_slices_byte_exact(hip, oracle):
    torch = _torch()
    rng = np.random.default_rng(41)
    # small slots (many slices, both slots, a short last slice, one row per
    # slice) and large ones (the host copy of a slice split over threads)
    for N, K, staging in [(37, 1024, 3 * 8 * 28 + 5), (64, 5120, 40 * 28), (5, 128, 28), (300, 2048, 1 << 20),
                          (8192, 5120, 16 << 20), (20000, 5120, 12 << 20)]:
        src = gw.ptq1_0_bytes(rng, N, K)
        codes = torch.full((N * K // 4,), 0xEE, dtype=torch.uint8, device="cuda")
        scales = torch.full((N * K // 128,), -1, dtype=torch.int16, device="cuda")
        L = hip.Loader(staging)
        L.upload_ptq1_0(src, N, K, codes, scales, stream())
        assert L.finish() == src.size
        L.close()
        torch.cuda.synchronize()
        wc, ws = oracle_repack(oracle, src, N, K)
        assert np.array_equal(codes.cpu().numpy(), wc.reshape(-1)), (N, K, staging)
        assert np.array_equal(scales.cpu().numpy().view(np.uint16), ws.reshape(-1)), (N, K, staging)


def test_loader_rejects_bad_arguments(hip):
    torch = _torch()
    L = hip.Loader(1024)
    codes = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    scales = torch.zeros(1 << 12, dtype=torch.int16, device="cuda")
    src = np.zeros(1 << 16, np.uint8)
    assert L.upload_raw(src, 4, 100, codes, scales, stream()) != 0       # K % 128
    assert L.upload_raw(src, 4, 8192, codes, scales, stream()) != 0      # a row (1792 B) > slot
    assert L.upload_raw(src, 4, 128, codes.data_ptr() + 4, scales, stream()) != 0  # codes alignment
    assert L.upload_raw(src, 0, 128, codes, scales, stream()) == 0       # N = 0: nothing
    assert L.upload_raw(None, 4, 128, codes, scales, stream()) != 0
    L.close()
    assert hip.loader_create_raw(16) != 0


def test_gguf_to_device_arena(hip, oracle, tmp_path):
    """Every PTQ1_0 matrix of a file, uploaded from the mapping into one
    arena at the plan's offsets, equals the host repack of the file's bytes."""
    torch = _torch()
    rng = np.random.default_rng(43)
    shapes = {"blk.0.ffn_gate.weight": (1024, 96), "blk.0.ffn_down.weight": (3072, 40),
              "output.weight": (1024, 333), "blk.0.attn_q.weight": (2048, 1)}
    w = gw.Writer(alignment=64)
    data = {}
    for name, (K, N) in shapes.items():
        data[name] = gw.ptq1_0_bytes(rng, N, K)
        w.tensor(name, (K, N), 143, data[name])
    w.tensor("blk.0.attn_norm.weight", (1024,), 0, rng.integers(0, 256, 4096, dtype=np.uint8))
    p = str(tmp_path / "model.gguf")
    w.write(p)
    g = hip.Gguf(p)
    plan = g.plan(1 << 16)
    assert plan["n_matrices"] == len(shapes)
    arena = torch.zeros(plan["arena_bytes"], dtype=torch.uint8, device="cuda")
    base = arena.data_ptr()
    L = hip.Loader(1 << 16)
    off, placed = 0, {}
    for t in g.tensors:
        if t.type != 143 or t.n_dims != 2:
            continue
        K, N = t.ne
        co, so = off, off + (N * K // 4 + 255) // 256 * 256
        off = so + (N * K // 64 + 255) // 256 * 256
        L.upload_ptq1_0(t.data, N, K, base + co, base + so, stream())
        placed[t.name] = (N, K, co, so)
    assert off == plan["arena_bytes"]
    assert L.finish() == plan["source_bytes"]
    L.close()
    torch.cuda.synchronize()
    host = arena.cpu().numpy()
    for name, (N, K, co, so) in placed.items():
        wc, ws = oracle_repack(oracle, data[name], N, K)
        assert np.array_equal(host[co:co + N * K // 4], wc.reshape(-1)), name
        assert np.array_equal(host[so:so + N * K // 64].view(np.uint16), ws.reshape(-1)), name
    g.close()
