"""GPU tests of the GEMV that reads PTQ1_0 blocks directly
(btf_hip_launch_gemv_ptq1_0, csrc/gemv_b3.hip).

Its outputs must equal, bit for bit, those of launch_gemv's v_dot4 path on
the same matrices repacked to T2 (the kernels form every sum in the same
floating-point order), and be within the path's 1e-3 bar of the oracle GEMV
on the oracle's repack (oracle/btf_oracle.c, pinned to the reference's
src/repack.cpp:16-27 and the reference GEMV). The repack decodes each digit
with the reference's ptq1_0_trit (src/types.hpp:70-78), so bit equality
with the T2 path also pins the direct kernel's digit layout: every element
position of the block, every byte value (bytes above 242 included, which the
encoder never writes), every sub-block boundary."""
import numpy as np
import pytest

from helpers import assert_close_1e3, random_act, random_ptq

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def dev(a):
    torch = _torch()
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a.copy()).cuda()


def host(t):
    _torch().cuda.synchronize()
    return t.cpu().numpy()


def stream():
    return _torch().cuda.current_stream().cuda_stream


def any_bytes_ptq(rng, N, K):
    """PTQ1_0 rows whose digit bytes take every value 0..255 and whose fp16
    scales are finite, of both signs, normal and subnormal."""
    blk = rng.integers(0, 256, size=(N, K // 128, 28), dtype=np.uint8)
    mag = rng.uniform(1e-6, 4.0, size=(N, K // 128)).astype(np.float16)
    sign = np.where(rng.random((N, K // 128)) < 0.3, -1, 1).astype(np.float16)
    blk[:, :, 26:28] = (mag * sign).view(np.uint8).reshape(N, K // 128, 2)
    return blk.reshape(N, K // 128 * 28)


def t2_of(oracle, src, N, K):
    codes, scales = oracle.repack_rows(src, N, K)
    return dev(codes), dev(scales)


def both(hip, oracle, srcs, Ns, K, M, act, mode, ys_b3, ys_t2, ldys):
    """Run the direct kernel and the T2 path on the same matrices."""
    segs_b3, segs_t2 = [], []
    for i, (src, n) in enumerate(zip(srcs, Ns)):
        c, s = t2_of(oracle, src, n, K)
        segs_b3.append(hip.GemvSeg(dev(src), None, n, ys_b3[i], ldys[i]))
        segs_t2.append(hip.GemvSeg(c, s, n, ys_t2[i], ldys[i]))
    old = hip.gemv_set_policy(1 << 20)  # every M on the v_dot4 path
    try:
        hip.launch_gemv_ptq1_0(segs_b3, K, M, act, mode, stream())
        hip.launch_gemv(segs_t2, K, M, act, mode, stream())
    finally:
        hip.gemv_set_policy(old)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("K,M", [(128, 1), (1024, 1), (1152, 2), (3200, 3), (5120, 1), (5120, 5), (16384, 1),
                                 (17408, 2), (20480, 1), (32768, 1)])
def test_store_three_segments_bit_exact(hip, oracle, K, M):
    """Three outputs with ldy = N + 3 (rows past N untouched); ragged K (not
    a multiple of 1024: a slice with dead lanes); K past 16384 (four rows per
    step, and the T2 kernel's extra slice); M > 2 (passes of two rows)."""
    torch = _torch()
    rng = np.random.default_rng(K * 7 + M)
    Ns = [37, 64, 9]
    srcs = [any_bytes_ptq(rng, n, K) for n in Ns]
    _, q, d, s = random_act(oracle, rng, M, K, 3.0)
    act = hip.Q8Act(dev(q), dev(d), dev(s))
    yb = [torch.full((M, n + 3), 7.0, dtype=torch.float32, device="cuda") for n in Ns]
    yt = [torch.full((M, n + 3), 7.0, dtype=torch.float32, device="cuda") for n in Ns]
    both(hip, oracle, srcs, Ns, K, M, act, hip.GemvMode.kStore, yb, yt, [n + 3 for n in Ns])
    for i, n in enumerate(Ns):
        gb, gt = host(yb[i]), host(yt[i])
        assert np.array_equal(bits(gb), bits(gt)), (K, M, n)
        assert np.all(gb[:, n:] == 7.0), "wrote past N"
        codes, scales = oracle.repack_rows(srcs[i], n, K)
        assert_close_1e3(gb[:, :n], oracle.gemv(codes, scales, K, q, d, s), f"K={K} N={n}")


@pytest.mark.parametrize("K,M", [(1024, 1), (5120, 2), (17408, 1)])
def test_add_and_swiglu_bit_exact(hip, oracle, K, M):
    torch = _torch()
    rng = np.random.default_rng(K + 100 * M)
    _, q, d, s = random_act(oracle, rng, M, K)
    act = hip.Q8Act(dev(q), dev(d), dev(s))
    # add: y = y0 + W x
    N = 200
    src = random_ptq(oracle, rng, N, K)
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    yb, yt = dev(y0), dev(y0)
    both(hip, oracle, [src], [N], K, M, act, hip.GemvMode.kAdd, [yb], [yt], [N])
    assert np.array_equal(bits(host(yb)), bits(host(yt)))
    codes, scales = oracle.repack_rows(src, N, K)
    assert_close_1e3(host(yb), oracle.gemv(codes, scales, K, q, d, s, y=y0.copy(), add=True), "add")
    # swiglu: gate and up interleaved within a workgroup
    N = 333
    g, u = random_ptq(oracle, rng, N, K), any_bytes_ptq(rng, N, K)
    yb = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    yt = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    both(hip, oracle, [g, u], [N, N], K, M, act, hip.GemvMode.kSwiglu, [yb, None], [yt, None], [N, 0])
    assert np.array_equal(bits(host(yb)), bits(host(yt)))
    gc, gs = oracle.repack_rows(g, N, K)
    uc, us = oracle.repack_rows(u, N, K)
    ref = oracle.swiglu(oracle.gemv(gc, gs, K, q, d, s), oracle.gemv(uc, us, K, q, d, s))
    assert_close_1e3(host(yb), ref, "swiglu")


@pytest.mark.parametrize("K,N,mode", [(5120, 7168, "store"), (5120, 17408, "swiglu"), (17408, 5120, "add")])
def test_27b_shapes_batch1(hip, oracle, K, N, mode):
    """The 27B layer shapes at M = 1 on the seeded generator's blocks."""
    torch = _torch()
    G = hip.GemvMode
    m = {"store": G.kStore, "add": G.kAdd, "swiglu": G.kSwiglu}[mode]
    nmat = 2 if mode == "swiglu" else 1
    srcs = [oracle.gen_ptq1_0(3, N + K + i, N * K // 128).reshape(N, K // 128 * 28) for i in range(nmat)]
    rng = np.random.default_rng(N)
    _, q, d, s = random_act(oracle, rng, 1, K)
    act = hip.Q8Act(dev(q), dev(d), dev(s))
    y0 = rng.standard_normal((1, N)).astype(np.float32)
    yb, yt = dev(y0), dev(y0)
    both(hip, oracle, srcs, [N] * nmat, K, 1, act, m, [yb] + [None] * (nmat - 1), [yt] + [None] * (nmat - 1),
         [N] + [0] * (nmat - 1))
    assert np.array_equal(bits(host(yb)), bits(host(yt)))
    mats = [oracle.repack_rows(x, N, K) for x in srcs]
    refs = [oracle.gemv(c, sc, K, q, d, s) for c, sc in mats]
    ref = oracle.swiglu(*refs) if mode == "swiglu" else (y0 + refs[0] if mode == "add" else refs[0])
    assert_close_1e3(host(yb), ref, f"{K}->{N} {mode}")


def test_zero_activation_and_unaligned_rows(hip, oracle):
    """All-zero activation blocks (d = +-0) give +0 like the T2 path; a matrix
    at a 4-byte (not 16-byte) aligned address; N = 1."""
    torch = _torch()
    rng = np.random.default_rng(5)
    K, M = 2048, 2
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[0] = 0.0
    x[1, 512:1024] = -0.0
    q, d, s = oracle.quantize_rows(x)
    act = hip.Q8Act(dev(q), dev(d), dev(s))
    for N in (1, 45):
        src = any_bytes_ptq(rng, N, K)
        buf = torch.zeros(src.size + 4, dtype=torch.uint8, device="cuda")
        buf[4:] = dev(src.reshape(-1))
        c, sc = t2_of(oracle, src, N, K)
        yb = torch.full((M, N), 3.0, dtype=torch.float32, device="cuda")
        yt = torch.full((M, N), 3.0, dtype=torch.float32, device="cuda")
        hip.launch_gemv_ptq1_0([hip.GemvSeg(buf.data_ptr() + 4, None, N, yb, N)], K, M, act,
                               hip.GemvMode.kStore, stream())
        hip.launch_gemv([hip.GemvSeg(c, sc, N, yt, N)], K, M, act, hip.GemvMode.kStore, stream())
        gb = host(yb)
        assert np.array_equal(bits(gb), bits(host(yt)))
        assert np.all(bits(gb[0]) == 0), "zero input: +0"


def test_rejects_t2_arguments(hip):
    torch = _torch()
    a = hip.Q8Act(torch.zeros((1, 1024), dtype=torch.int8, device="cuda"),
                  torch.zeros((1, 32), dtype=torch.float32, device="cuda"),
                  torch.zeros((1, 32), dtype=torch.int32, device="cuda"))
    y = torch.zeros((1, 4), dtype=torch.float32, device="cuda")
    blocks = torch.zeros(4 * 8 * 28, dtype=torch.uint8, device="cuda")
    sc = torch.zeros(32, dtype=torch.int16, device="cuda")
    with pytest.raises(RuntimeError, match="NULL"):
        hip.launch_gemv_ptq1_0([hip.GemvSeg(blocks, sc, 4, y, 4)], 1024, 1, a, hip.GemvMode.kStore, stream())
    with pytest.raises(RuntimeError, match="32768"):
        hip.launch_gemv_ptq1_0([hip.GemvSeg(blocks, None, 4, y, 4)], 40960, 1, a, hip.GemvMode.kStore, stream())
