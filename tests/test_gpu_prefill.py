"""GPU parity of the prefill GEMM (M = 512 activation rows) at the 27B layer
shapes, on the seeded generator's weights: QKV 5120->7168 store, o
5120->5120 add, gate+up 5120->2x17408 swiglu, down 17408->5120 add.

  * y (the whole output, as launch_gemv writes it) within rel-RMS 1e-3 and
    max error 1e-3 of max |ref| of the emulator GEMV (src/emu_decoder.cpp:
    143-165) on sampled output rows (the first, a middle and the last weight
    tiles), for every activation row;
  * the int32 sub-block accumulators I[m][n][s] bit-exact against the
    oracle's brute-force sum of (code - 1) * q on the same sampled rows, read
    from btf_hip_gemv_i32_dump of the FULL matrix, which runs the prefill
    tile that launch_gemv runs at this shape (the same kernel and grid, with
    I written instead of y).
The reference's own kernel cases reach K = 17408 (tests/test_gpu_kernels.cpp:
562-564); its test compares y only (:203-276).
"""
import numpy as np
import pytest

from helpers import assert_close_1e3, random_act

pytestmark = pytest.mark.gpu

M = 512
SHAPES = [("qkv", 5120, 7168, "store"), ("o", 5120, 5120, "add"), ("gateup", 5120, 17408, "swiglu"),
          ("down", 17408, 5120, "add")]


def _torch():
    import torch
    return torch


def dev(a):
    torch = _torch()
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a.copy()).cuda()


def stream():
    return _torch().cuda.current_stream().cuda_stream


def gen_matrix(hip, N, K, mat_id):
    """The benchmark's seeded generator + the device repack (both bit-exact
    with the oracle: test_gpu_parity)."""
    torch = _torch()
    nb = N * K // 128
    src = torch.empty(nb * 28, dtype=torch.uint8, device="cuda")
    codes = torch.empty((N, K // 4), dtype=torch.uint8, device="cuda")
    scales = torch.empty((N, K // 128), dtype=torch.int16, device="cuda")
    hip.gen_ptq1_0(0, mat_id, 0, nb, src, stream())
    hip.launch_repack(src, nb, codes, scales, stream())
    torch.cuda.synchronize()
    return codes, scales


def rows_of(t, sel):
    """Host copy of rows `sel` of a device matrix."""
    _torch().cuda.synchronize()
    return np.ascontiguousarray(t[dev(sel).long()].cpu().numpy())


@pytest.mark.parametrize("name,K,N,mode", SHAPES, ids=[s[0] for s in SHAPES])
def test_prefill_27b_layer_shape(hip, oracle, name, K, N, mode):
    torch = _torch()
    G = hip.GemvMode
    rng = np.random.default_rng(K + N)
    _, q, d, s = random_act(oracle, rng, M, K)
    act = hip.Q8Act(dev(q), dev(d), dev(s))
    ids = {"qkv": (0,), "o": (1,), "gateup": (2, 3), "down": (4,)}[name]
    mats = [gen_matrix(hip, N, K, 500 + i) for i in ids]
    sel = np.unique(np.r_[0:70, N // 2 - 40:N // 2 + 40, N - 37:N]).astype(np.int64)
    host_rows = [(rows_of(c, sel), rows_of(sc, sel).view(np.uint16)) for c, sc in mats]

    # y at the full shape
    y0 = rng.standard_normal((M, N)).astype(np.float32) if mode == "add" else np.zeros((M, N), np.float32)
    y = dev(y0)
    segs = [hip.GemvSeg(mats[0][0], mats[0][1], N, y, N)]
    if mode == "swiglu":
        segs.append(hip.GemvSeg(mats[1][0], mats[1][1], N, None, 0))
    hip.launch_gemv(segs, K, M, act, {"store": G.kStore, "add": G.kAdd, "swiglu": G.kSwiglu}[mode], stream())
    torch.cuda.synchronize()
    got = y[:, dev(sel).long()].cpu().numpy()
    if mode == "swiglu":
        ref = oracle.swiglu(*[oracle.gemv(c, sc, K, q, d, s) for c, sc in host_rows])
    else:
        ref = oracle.gemv(*host_rows[0], K, q, d, s, y=np.ascontiguousarray(y0[:, sel]), add=mode == "add")
    assert_close_1e3(got, ref, f"{name} M={M} y")
    del y

    # I of every matrix, dumped at the full shape
    I = torch.empty((M, N, K // 32), dtype=torch.int32, device="cuda")
    for (c, _), (hc, _) in zip(mats, host_rows):
        I.fill_(-(1 << 30))
        hip.gemv_i32_dump(c, N, K, M, act, I, stream())
        torch.cuda.synchronize()
        got_i = I[:, dev(sel).long(), :].cpu().numpy()
        want_i = oracle.gemv_i32(hc, K, q, s)
        bad = np.argwhere(got_i != want_i)
        assert bad.size == 0, f"{name}: I differs at {len(bad)} places, first (m, row, s) = {bad[0]}"
    del I
