"""GPU parity tests: every HIP kernel of the path, called through the C ABI,
against the oracle on the same seeded inputs.

Bars: bit-exact for repack (bytes), Q8 (q, d bits, s) and the int32
sub-block accumulators I[m][n][s]; GEMV outputs within rel-RMS 1e-3 and
max |err| <= 1e-3 * max |ref| of the emulator (src/emu_decoder.cpp:143-165).
The shapes follow the reference's kernel tests
(tests/test_gpu_kernels.cpp:556-564) plus the 27B layer shapes.
"""
import numpy as np
import pytest

from helpers import assert_close_1e3, gen_mat, random_act, random_mat, random_ptq, rel_rms

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def dev(a):
    """numpy -> device tensor with the same bytes."""
    torch = _torch()
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    elif a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a.copy()).cuda()


def host(t, dtype=None):
    torch = _torch()
    torch.cuda.synchronize()
    a = t.cpu().numpy()
    return a.view(dtype) if dtype is not None else a


def zeros(shape, dtype):
    torch = _torch()
    return torch.zeros(shape, dtype=dtype, device="cuda")


def stream():
    return _torch().cuda.current_stream().cuda_stream


def q8_dev(q, d, s, hip):
    return hip.Q8Act(dev(q), dev(d), dev(s))


# ---------------------------------------------------------------- repack
@pytest.mark.parametrize("kind", ["encoder", "random_bytes"])
def test_repack_device_source(hip, oracle, kind):
    rng = np.random.default_rng(1234)
    N, K = 41, 1024
    if kind == "encoder":
        src = random_ptq(oracle, rng, N, K)
    else:  # every byte value, including ones the encoder never emits
        src = rng.integers(0, 256, (N, K // 128 * 28), dtype=np.uint8)
    codes_ref, scales_ref = oracle.repack_rows(src, N, K)
    torch = _torch()
    codes = zeros((N, K // 4), torch.uint8)
    scales = zeros((N, K // 128), torch.int16)
    hip.launch_repack(dev(src), N * K // 128, codes, scales, stream())
    assert np.array_equal(host(codes), codes_ref)
    assert np.array_equal(host(scales, np.uint16), scales_ref)


def test_repack_mapped_host_source(hip, oracle):
    """The source may be pinned, mapped host memory (as at model load)."""
    rng = np.random.default_rng(7)
    N, K = 33, 2048
    src = random_ptq(oracle, rng, N, K)
    buf = hip.MappedHostBuffer(src.size)
    buf.view()[:] = src.reshape(-1)
    codes_ref, scales_ref = oracle.repack_rows(src, N, K)
    torch = _torch()
    codes = zeros((N, K // 4), torch.uint8)
    scales = zeros((N, K // 128), torch.int16)
    hip.launch_repack(buf.dev, N * K // 128, codes, scales, stream())
    assert np.array_equal(host(codes), codes_ref)
    assert np.array_equal(host(scales, np.uint16), scales_ref)
    buf.close()


def test_repack_many_blocks_ragged(hip, oracle):
    """Grid-stride path: more blocks than one grid covers, ragged tail."""
    nb = 1_000_003
    src = oracle.gen_ptq1_0(3, 11, nb)
    codes_ref, scales_ref = oracle.repack_blocks(src, nb)
    torch = _torch()
    codes = zeros((nb, 32), torch.uint8)
    scales = zeros((nb,), torch.int16)
    hip.launch_repack(dev(src), nb, codes, scales, stream())
    assert np.array_equal(host(codes), codes_ref)
    assert np.array_equal(host(scales, np.uint16), scales_ref)


def test_generator_matches_oracle(hip, oracle):
    torch = _torch()
    for first, nb in [(0, 1000), (123_457, 777)]:
        ref = oracle.gen_ptq1_0(0, 5, nb, first_block=first)
        out = zeros((nb, 28), torch.uint8)
        hip.gen_ptq1_0(0, 5, first, nb, out, stream())
        assert np.array_equal(host(out), ref)


# ---------------------------------------------------------------- Q8 prep
def _special_rows(K):
    """Rows that hit the Q8 edge cases: zero blocks (+0 / -0 last), exact .5
    ties, +-amax, tiny values (subnormal fp16 d), large values."""
    x = np.zeros((6, K), np.float32)
    x[0, :32] = 0.0
    x[0, 32:64] = -0.0
    x[0, 64:96] = np.linspace(-1, 1, 32)
    x[0, 95] = -0.0  # non-zero block ending in -0
    b = np.arange(32, dtype=np.float32)
    x[1, :32] = b - 15.5  # amax 16 -> id = 127/16, q = x*id
    x[1, 32:64] = np.where(b % 2 == 0, 2.5, -3.5)  # with amax 127 below: id = 1 -> ties
    x[1, 63] = 127.0
    x[1, 64:96] = -127.0
    x[1, 96:128] = 1e-7 * (b - 16)  # tiny: fp16 d is subnormal
    x[2] = 1e4 * np.sin(np.arange(K, dtype=np.float32))
    x[3] = 1e-30 * np.cos(np.arange(K, dtype=np.float32))
    x[4, ::7] = -3.0
    x[5] = np.float32(0.5) * (np.arange(K) % 5 - 2)
    return x


@pytest.mark.parametrize("K", [256, 1024, 5120, 17408])
def test_q8_bit_exact(hip, oracle, K):
    rng = np.random.default_rng(K)
    M = 13
    x = (rng.standard_normal((M, K)) * 3).astype(np.float32)
    x = np.concatenate([x, _special_rows(K)], axis=0)
    M = x.shape[0]
    ldx = K + 8  # row stride wider than the row
    xp = np.zeros((M, ldx), np.float32)
    xp[:, :K] = x
    q_ref, d_ref, s_ref = oracle.quantize_rows(x)
    torch = _torch()
    a = hip.Q8Act(zeros((M, K), torch.int8), zeros((M, K // 32), torch.float32), zeros((M, K // 32), torch.int32))
    hip.launch_prep(dev(xp), ldx, M, K, None, 0.0, None, None, 0, a, stream())
    assert np.array_equal(host(a.q), q_ref)
    assert np.array_equal(host(a.d).view(np.uint32), d_ref.view(np.uint32))
    assert np.array_equal(host(a.s), s_ref)


def test_q8_unaligned_rows(hip, oracle):
    """Scalar-load variant: a row stride that is not a multiple of 4 floats."""
    rng = np.random.default_rng(5)
    M, K, ldx = 5, 1024, 1027
    xp = (rng.standard_normal((M, ldx)) * 2).astype(np.float32)
    q_ref, d_ref, s_ref = oracle.quantize_rows(np.ascontiguousarray(xp[:, :K]))
    torch = _torch()
    a = hip.Q8Act(zeros((M, K), torch.int8), zeros((M, K // 32), torch.float32), zeros((M, K // 32), torch.int32))
    hip.launch_prep(dev(xp), ldx, M, K, None, 0.0, None, None, 0, a, stream())
    assert np.array_equal(host(a.q), q_ref)
    assert np.array_equal(host(a.d).view(np.uint32), d_ref.view(np.uint32))
    assert np.array_equal(host(a.s), s_ref)


# The reference's prep cases (tests/test_gpu_kernels.cpp:557-561):
# (n, hadamard block, norm, perm, signs, M)
PREP_CASES = [(1024, 64, True, False, True, 1), (5120, 1024, True, False, True, 3),
              (2048, 128, False, True, True, 8), (256, 0, True, False, False, 2),
              (17408, 1024, False, False, True, 1),
              # beyond the reference's cases: a tail slice (1056 = 1024 + 32, span 32),
              # blocks below one lane's 16 values, 17 slices with the norm (more
              # slices than waves), the perm under the norm, a 3-slice row
              (1056, 32, True, False, True, 2), (1056, 16, False, False, False, 3), (2048, 2, True, False, True, 1),
              (17408, 1024, True, False, True, 2), (4096, 512, True, True, False, 5), (3072, 1024, False, False, True, 4),
              (5120, 1, True, False, True, 1), (96, 32, False, False, True, 1)]


@pytest.mark.parametrize("n,block,norm,perm,signs,M", PREP_CASES)
def test_prep_full(hip, oracle, n, block, norm, perm, signs, M):
    rng = np.random.default_rng(1234 + n)
    eps = 1e-6
    x = (rng.standard_normal((M, n)) * 3).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    sg = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float32)
    hd, nk, rep = (32, n // 64, 2) if perm else (0, 0, 0)
    q_ref, d_ref, s_ref, xn_ref = oracle.prep(x, w if norm else None, eps, block, hd, nk, rep,
                                              sg if signs else None)
    torch = _torch()
    a = hip.Q8Act(zeros((M, n), torch.int8), zeros((M, n // 32), torch.float32), zeros((M, n // 32), torch.int32))
    xn = zeros((M, n), torch.float32)
    hx = hip.Hx(block, hd, nk, rep, dev(sg) if signs else None)
    hip.launch_prep(dev(x), n, M, n, dev(w) if norm else None, eps, hx, xn, n, a, stream())
    gq, gd, gs, gxn = host(a.q), host(a.d), host(a.s), host(xn)
    assert np.isfinite(gd).all()
    # The reference's bars (tests/test_gpu_kernels.cpp:152-158). Without the
    # norm every stage is order-identical, so the result is bit-exact.
    dq = np.abs(gq.astype(np.int32) - q_ref.astype(np.int32))
    assert dq.max() <= 1 and (dq != 0).mean() <= 1e-3
    assert rel_rms(gd, d_ref) <= 1e-4
    assert rel_rms(gxn, xn_ref) <= 1e-6
    if not norm:
        assert np.array_equal(gq, q_ref)
        assert np.array_equal(gd.view(np.uint32), d_ref.view(np.uint32))
        assert np.array_equal(gs, s_ref)
        assert np.array_equal(gxn, xn_ref)


def test_prep_zero_rows_and_blocks(hip, oracle):
    """All-zero rows (norm scale 1/sqrt(eps)) and zero blocks (d = +-0 with
    the sign of the block's last value) through the full prep, bit-exact
    without the norm, within the reference's bars with it."""
    rng = np.random.default_rng(99)
    n, M = 2048, 3
    x = (rng.standard_normal((M, n)) * 2).astype(np.float32)
    x[0] = 0.0
    x[1, 64:96] = 0.0
    x[1, 127] = -0.0
    x[2, 1024:1056] = -0.0
    w = rng.standard_normal(n).astype(np.float32)
    sg = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float32)
    torch = _torch()
    for norm, block in ((False, 0), (False, 64), (True, 256)):
        q_ref, d_ref, s_ref, _ = oracle.prep(x, w if norm else None, 1e-6, block, 0, 0, 0, sg if block else None)
        a = hip.Q8Act(zeros((M, n), torch.int8), zeros((M, n // 32), torch.float32), zeros((M, n // 32), torch.int32))
        xn = zeros((M, n), torch.float32)  # forces the full prep kernel even without norm and transform
        hip.launch_prep(dev(x), n, M, n, dev(w) if norm else None, 1e-6, hip.Hx(block, 0, 0, 0, dev(sg) if block else None),
                        xn, n, a, stream())
        gq, gd, gs = host(a.q), host(a.d), host(a.s)
        if norm:
            dq = np.abs(gq.astype(np.int32) - q_ref.astype(np.int32))
            assert dq.max() <= 1 and (dq != 0).mean() <= 1e-3
            assert rel_rms(gd, d_ref) <= 1e-4
        else:
            assert np.array_equal(gq, q_ref)
            assert np.array_equal(gd.view(np.uint32), d_ref.view(np.uint32)), f"block {block}: d bits"
            assert np.array_equal(gs, s_ref)


# ---------------------------------------------------------------- GEMV / GEMM
PATHS = {"dot4": 1 << 20, "mfma": 1}  # policy: M >= value uses MFMA


@pytest.fixture(params=list(PATHS))
def path(request, hip):
    hip.gemv_set_policy(PATHS[request.param])
    yield request.param
    hip.gemv_set_policy(0)


@pytest.mark.parametrize("K,M", [(1024, 1), (1024, 3), (1024, 8), (1024, 13), (5120, 1), (5120, 4),
                                 (17408, 1), (17408, 2), (2048, 32), (1024, 40)])
def test_gemv_i32_bit_exact(hip, oracle, path, K, M):
    """The int32 sub-block accumulators are bit-exact on both kernel paths
    (MFMA: the K-split tile up to 32 rows, the 64-row tile above)."""
    rng = np.random.default_rng(K * 31 + M)
    N = 37
    codes, scales = random_mat(oracle, rng, N, K)
    _, q, d, s = random_act(oracle, rng, M, K, 3.0)
    I_ref = oracle.gemv_i32(codes, K, q, s)
    torch = _torch()
    out = zeros((M, N, K // 32), torch.int32)
    hip.gemv_i32_dump(dev(codes), N, K, M, q8_dev(q, d, s, hip), out, stream())
    assert np.array_equal(host(out), I_ref)


@pytest.mark.parametrize("K,M", [(1024, 1), (1024, 3), (1024, 8), (1024, 13), (5120, 1), (17408, 2)])
def test_gemv_modes_three_segments(hip, oracle, path, K, M):
    """store into three outputs with ldy = N + 3, add, and swiglu
    (tests/test_gpu_kernels.cpp:203-276), against the emulator GEMV."""
    rng = np.random.default_rng(4321 + K + M)
    Ns = [37, 64, 9]
    mats = [random_mat(oracle, rng, n, K) for n in Ns]
    _, q, d, s = random_act(oracle, rng, M, K, 3.0)
    act = q8_dev(q, d, s, hip)
    torch = _torch()
    # store
    ys = [zeros((M, n + 3), torch.float32) for n in Ns]
    segs = [hip.GemvSeg(dev(c), dev(sc), n, y, n + 3) for (c, sc), n, y in zip(mats, Ns, ys)]
    hip.launch_gemv(segs, K, M, act, hip.GemvMode.kStore, stream())
    for (c, sc), n, y in zip(mats, Ns, ys):
        ref = oracle.gemv(c, sc, K, q, d, s)
        got = host(y)
        assert_close_1e3(got[:, :n], ref, f"store N={n}")
        assert np.all(got[:, n:] == 0), "wrote past N"
    # add: y = y0 + W x
    y0 = rng.standard_normal((M, Ns[0])).astype(np.float32)
    yd = dev(y0)
    hip.launch_gemv([hip.GemvSeg(dev(mats[0][0]), dev(mats[0][1]), Ns[0], yd, Ns[0])], K, M, act,
                    hip.GemvMode.kAdd, stream())
    ref = oracle.gemv(mats[0][0], mats[0][1], K, q, d, s, y=y0.copy(), add=True)
    assert_close_1e3(host(yd), ref, "add")
    # swiglu: gate = mats[1], up = a fresh N=64 matrix; segs[1].y unused (None)
    up = random_mat(oracle, rng, Ns[1], K)
    g = zeros((M, Ns[1]), torch.float32)
    sw = [hip.GemvSeg(dev(mats[1][0]), dev(mats[1][1]), Ns[1], g, Ns[1]),
          hip.GemvSeg(dev(up[0]), dev(up[1]), Ns[1], None, 0)]
    hip.launch_gemv(sw, K, M, act, hip.GemvMode.kSwiglu, stream())
    gref = oracle.gemv(mats[1][0], mats[1][1], K, q, d, s)
    uref = oracle.gemv(up[0], up[1], K, q, d, s)
    assert_close_1e3(host(g), oracle.swiglu(gref, uref), "swiglu")


@pytest.mark.parametrize("K,N", [(5120, 5120), (5120, 7168), (17408, 5120)])
def test_gemv_27b_shapes_batch1(hip, oracle, K, N):
    """Config shapes at M = 1 on the seeded generator's weights."""
    codes, scales = gen_mat(oracle, 0, N + K, N, K)
    rng = np.random.default_rng(0)
    _, q, d, s = random_act(oracle, rng, 1, K)
    ref = oracle.gemv(codes, scales, K, q, d, s)
    torch = _torch()
    y = zeros((1, N), torch.float32)
    hip.launch_gemv([hip.GemvSeg(dev(codes), dev(scales), N, y, N)], K, 1, q8_dev(q, d, s, hip),
                    hip.GemvMode.kStore, stream())
    assert_close_1e3(host(y), ref, f"{K}->{N}")
    I_ref = oracle.gemv_i32(codes[:64], K, q, s)
    out = zeros((1, 64, K // 32), torch.int32)
    hip.gemv_i32_dump(dev(codes[:64].copy()), 64, K, 1, q8_dev(q, d, s, hip), out, stream())
    assert np.array_equal(host(out), I_ref)


def test_gemv_27b_gate_up_swiglu_batch1(hip, oracle):
    """Config 2's gate/up pair at full shape (5120 -> 2 x 17408) as one
    swiglu launch at M = 1, on the seeded generator's weights: silu(g) * u
    within 1e-3 of the oracle; I bit-exact on the first and last 64 rows of
    both matrices."""
    K, N = 5120, 17408
    gate = gen_mat(oracle, 0, 5 * 7 + 2, N, K)
    up = gen_mat(oracle, 0, 5 * 7 + 3, N, K)
    rng = np.random.default_rng(11)
    _, q, d, s = random_act(oracle, rng, 1, K)
    ref = oracle.swiglu(oracle.gemv(gate[0], gate[1], K, q, d, s), oracle.gemv(up[0], up[1], K, q, d, s))
    torch = _torch()
    h = zeros((1, N), torch.float32)
    act = q8_dev(q, d, s, hip)
    hip.launch_gemv([hip.GemvSeg(dev(gate[0]), dev(gate[1]), N, h, N), hip.GemvSeg(dev(up[0]), dev(up[1]), N, None, 0)],
                    K, 1, act, hip.GemvMode.kSwiglu, stream())
    assert_close_1e3(host(h), ref, "gate/up swiglu 5120->17408")
    for codes in (gate[0], up[0]):
        for rows in (slice(0, 64), slice(N - 64, N)):
            sub = np.ascontiguousarray(codes[rows])
            out = zeros((1, 64, K // 32), torch.int32)
            hip.gemv_i32_dump(dev(sub), 64, K, 1, act, out, stream())
            assert np.array_equal(host(out), oracle.gemv_i32(sub, K, q, s))


# The layer's projections at full shape (config 3): (kind, K, N, mode)
LAYER_KINDS = [("qkv", 5120, 7168, "store"), ("o", 5120, 5120, "add"), ("gateup", 5120, 17408, "swiglu"),
               ("down", 17408, 5120, "add")]


@pytest.mark.parametrize("M", [8, 32])
@pytest.mark.parametrize("kind,K,N,mode", LAYER_KINDS)
def test_gemm_27b_layer_shapes_batched(hip, oracle, kind, K, N, mode, M):
    """Batched decode on every projection of a 27B layer at full shape, on
    the seeded generator's weights, against the oracle (add mode onto a
    random residual; swiglu as one gate+up launch)."""
    mid = 1000 + LAYER_KINDS.index((kind, K, N, mode)) * 2
    W = gen_mat(oracle, 0, mid, N, K)
    rng = np.random.default_rng(M * 31 + K)
    _, q, d, s = random_act(oracle, rng, M, K)
    torch = _torch()
    act = q8_dev(q, d, s, hip)
    G = hip.GemvMode
    if mode == "swiglu":
        U = gen_mat(oracle, 0, mid + 1, N, K)
        ref = oracle.swiglu(oracle.gemv(W[0], W[1], K, q, d, s), oracle.gemv(U[0], U[1], K, q, d, s))
        y = zeros((M, N), torch.float32)
        hip.launch_gemv([hip.GemvSeg(dev(W[0]), dev(W[1]), N, y, N), hip.GemvSeg(dev(U[0]), dev(U[1]), N, None, 0)],
                        K, M, act, G.kSwiglu, stream())
    else:
        y0 = rng.standard_normal((M, N)).astype(np.float32) if mode == "add" else np.zeros((M, N), np.float32)
        ref = oracle.gemv(W[0], W[1], K, q, d, s, y=y0.copy(), add=mode == "add")
        y = dev(y0)
        hip.launch_gemv([hip.GemvSeg(dev(W[0]), dev(W[1]), N, y, N)], K, M, act,
                        G.kAdd if mode == "add" else G.kStore, stream())
    assert_close_1e3(host(y), ref, f"{kind} M={M}")


@pytest.mark.parametrize("M", [4, 8, 16, 32, 512])
def test_gemm_batched_and_prefill(hip, oracle, M):
    """Config-3/4 batch sizes on a 5120-wide layer slice (N = 256)."""
    K, N = 5120, 256
    codes, scales = gen_mat(oracle, 1, 77, N, K)
    rng = np.random.default_rng(M)
    _, q, d, s = random_act(oracle, rng, M, K)
    ref = oracle.gemv(codes, scales, K, q, d, s)
    torch = _torch()
    y = zeros((M, N), torch.float32)
    hip.launch_gemv([hip.GemvSeg(dev(codes), dev(scales), N, y, N)], K, M, q8_dev(q, d, s, hip),
                    hip.GemvMode.kStore, stream())
    assert_close_1e3(host(y), ref, f"M={M}")


@pytest.mark.parametrize("K,M", [(128, 3), (384, 17), (1152, 5), (3200, 32), (17536, 9), (6144, 5), (10240, 6),
                                 (20608, 4)])
def test_gemm_k_split_tile_edges(hip, oracle, K, M):
    """Batches of 3..32 rows run on the K-split 16-row tiles (each wave a
    contiguous share of the 128-column blocks: the packed tile up to 16 rows,
    two blocks per ring stage, the register-staged tile above): block counts
    that do not split evenly (1 block: the other waves idle; 3, 9, 25, 137
    blocks: odd shares), one and two groups of activation rows with dead rows,
    16-row weight tiles with dead rows (N = 37, 9), and the three modes,
    against the emulator GEMV. Up to 8 rows the packed tile loads each wave's
    weight scales once: swiglu there takes 4 waves past 40 blocks (48 blocks:
    K = 6144) and 8 past 64 (80 blocks: K = 10240), and shapes past 160
    blocks (161: K = 20608) take the register-staged tile."""
    rng = np.random.default_rng(K + 1000 * M)
    _, q, d, s = random_act(oracle, rng, M, K, 3.0)
    act = q8_dev(q, d, s, hip)
    torch = _torch()
    G = hip.GemvMode
    Ns = [37, 9]
    mats = [random_mat(oracle, rng, n, K) for n in Ns]
    ys = [zeros((M, n + 1), torch.float32) for n in Ns]
    segs = [hip.GemvSeg(dev(c), dev(sc), n, y, n + 1) for (c, sc), n, y in zip(mats, Ns, ys)]
    hip.launch_gemv(segs, K, M, act, G.kStore, stream())
    for (c, sc), n, y in zip(mats, Ns, ys):
        got = host(y)
        assert_close_1e3(got[:, :n], oracle.gemv(c, sc, K, q, d, s), f"store K={K} M={M} N={n}")
        assert np.all(got[:, n:] == 0), "wrote past N"
    y0 = rng.standard_normal((M, Ns[0])).astype(np.float32)
    yd = dev(y0)
    hip.launch_gemv([hip.GemvSeg(dev(mats[0][0]), dev(mats[0][1]), Ns[0], yd, Ns[0])], K, M, act, G.kAdd,
                    stream())
    assert_close_1e3(host(yd), oracle.gemv(mats[0][0], mats[0][1], K, q, d, s, y=y0.copy(), add=True), "add")
    up = random_mat(oracle, rng, Ns[0], K)
    g = zeros((M, Ns[0]), torch.float32)
    hip.launch_gemv([hip.GemvSeg(dev(mats[0][0]), dev(mats[0][1]), Ns[0], g, Ns[0]),
                     hip.GemvSeg(dev(up[0]), dev(up[1]), Ns[0], None, 0)], K, M, act, G.kSwiglu, stream())
    ref = oracle.swiglu(oracle.gemv(mats[0][0], mats[0][1], K, q, d, s), oracle.gemv(up[0], up[1], K, q, d, s))
    assert_close_1e3(host(g), ref, "swiglu")
    I_ref = oracle.gemv_i32(mats[1][0], K, q, s)
    out = zeros((M, Ns[1], K // 32), torch.int32)
    hip.gemv_i32_dump(dev(mats[1][0]), Ns[1], K, M, act, out, stream())
    assert np.array_equal(host(out), I_ref)


@pytest.mark.parametrize("K,M", [(1024, 33), (5120, 200), (2048, 512)])
def test_gemm_prefill_tile_modes(hip, oracle, K, M):
    """More than 32 rows run on the prefill tile (64 staged weight rows x 128
    activation rows, 2 x 4 MFMA tiles per wave): three store segments with
    dead weight rows (N = 37, 70, 9), a dead activation tail (M = 33, 200),
    add, and swiglu (gate and up of the same outputs in one wave), against
    the emulator GEMV."""
    rng = np.random.default_rng(K + M)
    _, q, d, s = random_act(oracle, rng, M, K, 3.0)
    act = q8_dev(q, d, s, hip)
    torch = _torch()
    G = hip.GemvMode
    Ns = [37, 70, 9]
    mats = [random_mat(oracle, rng, n, K) for n in Ns]
    ys = [zeros((M, n + 3), torch.float32) for n in Ns]
    segs = [hip.GemvSeg(dev(c), dev(sc), n, y, n + 3) for (c, sc), n, y in zip(mats, Ns, ys)]
    hip.launch_gemv(segs, K, M, act, G.kStore, stream())
    for (c, sc), n, y in zip(mats, Ns, ys):
        got = host(y)
        assert_close_1e3(got[:, :n], oracle.gemv(c, sc, K, q, d, s), f"store K={K} M={M} N={n}")
        assert np.all(got[:, n:] == 0), "wrote past N"
    y0 = rng.standard_normal((M, Ns[1])).astype(np.float32)
    yd = dev(y0)
    hip.launch_gemv([hip.GemvSeg(dev(mats[1][0]), dev(mats[1][1]), Ns[1], yd, Ns[1])], K, M, act, G.kAdd,
                    stream())
    assert_close_1e3(host(yd), oracle.gemv(mats[1][0], mats[1][1], K, q, d, s, y=y0.copy(), add=True), "add")
    up = random_mat(oracle, rng, Ns[1], K)
    g = zeros((M, Ns[1]), torch.float32)
    hip.launch_gemv([hip.GemvSeg(dev(mats[1][0]), dev(mats[1][1]), Ns[1], g, Ns[1]),
                     hip.GemvSeg(dev(up[0]), dev(up[1]), Ns[1], None, 0)], K, M, act, G.kSwiglu, stream())
    ref = oracle.swiglu(oracle.gemv(mats[1][0], mats[1][1], K, q, d, s), oracle.gemv(up[0], up[1], K, q, d, s))
    assert_close_1e3(host(g), ref, "swiglu")


def test_gemm_prefill_wide_tile(hip, oracle):
    """Grids of at least two workgroups per CU take the 128-row activation
    tile: M = 400 (a dead tail of 112 rows in the last tile), store on
    N = 16421 and swiglu on N = 8197, checked on sampled output columns (the
    first, a middle and the last weight tiles) against the emulator GEMV."""
    K, M = 1024, 400
    rng = np.random.default_rng(400)
    _, q, d, s = random_act(oracle, rng, M, K, 3.0)
    act = q8_dev(q, d, s, hip)
    torch = _torch()
    G = hip.GemvMode
    for mode, N in ((G.kStore, 16421), (G.kSwiglu, 8197)):
        sel = np.r_[0:70, N // 2 - 40:N // 2 + 40, N - 37:N]
        mats = [random_mat(oracle, rng, N, K) for _ in range(2 if mode == G.kSwiglu else 1)]
        y = zeros((M, N), torch.float32)
        segs = [hip.GemvSeg(dev(mats[0][0]), dev(mats[0][1]), N, y, N)]
        if mode == G.kSwiglu:
            segs.append(hip.GemvSeg(dev(mats[1][0]), dev(mats[1][1]), N, None, 0))
        hip.launch_gemv(segs, K, M, act, mode, stream())
        refs = [oracle.gemv(np.ascontiguousarray(c[sel]), np.ascontiguousarray(sc[sel]), K, q, d, s)
                for c, sc in mats]
        ref = oracle.swiglu(*refs) if mode == G.kSwiglu else refs[0]
        assert_close_1e3(host(y)[:, sel], ref, f"mode={mode} N={N}")


def test_gemm_prefill_unaligned_scales(hip, oracle):
    """The prefill ring loads the activation scales d in 16-byte pieces; a d
    array at an 8-byte (not 16-byte) aligned address takes the register-staged
    prefill tile instead. Both against the emulator GEMV."""
    K, M, N = 1024, 40, 45
    rng = np.random.default_rng(41)
    _, q, d, s = random_act(oracle, rng, M, K, 3.0)
    codes, scales = random_mat(oracle, rng, N, K)
    ref = oracle.gemv(codes, scales, K, q, d, s)
    torch = _torch()
    dbuf = zeros(d.size + 2, torch.float32)
    dbuf[2:] = dev(d.reshape(-1))
    for dptr in (dev(d), dbuf.data_ptr() + 8):
        y = zeros((M, N), torch.float32)
        act = hip.Q8Act(dev(q), dptr, dev(s))
        hip.launch_gemv([hip.GemvSeg(dev(codes), dev(scales), N, y, N)], K, M, act, hip.GemvMode.kStore, stream())
        assert_close_1e3(host(y), ref, "prefill d alignment")


@pytest.mark.parametrize("M", [5, 8, 13])
def test_gemm_batched_unaligned_scales(hip, oracle, M):
    """Up to 16 rows run on the packed tile, whose LDS-direct ring loads d and
    s in 16-byte pieces; d or s at an 8-byte (not 16-byte) aligned address
    take the register-staged K-split tile. Every combination against the
    emulator GEMV (swiglu too), and I of the misaligned case bit-exact."""
    K, N = 1152, 45  # 9 blocks: the waves' ranges are odd and uneven
    rng = np.random.default_rng(43 + M)
    _, q, d, s = random_act(oracle, rng, M, K, 3.0)
    g, gs = random_mat(oracle, rng, N, K)
    u, us = random_mat(oracle, rng, N, K)
    ref = oracle.swiglu(oracle.gemv(g, gs, K, q, d, s), oracle.gemv(u, us, K, q, d, s))
    torch = _torch()
    dbuf, sbuf = zeros(d.size + 2, torch.float32), zeros(s.size + 2, torch.int32)
    dbuf[2:] = dev(d.reshape(-1))
    sbuf[2:] = dev(s.reshape(-1))
    G = hip.GemvMode
    for dptr, sptr in ((dev(d), dev(s)), (dbuf.data_ptr() + 8, dev(s)), (dev(d), sbuf.data_ptr() + 8)):
        act = hip.Q8Act(dev(q), dptr, sptr)
        y = zeros((M, N), torch.float32)
        hip.launch_gemv([hip.GemvSeg(dev(g), dev(gs), N, y, N), hip.GemvSeg(dev(u), dev(us), N, None, 0)], K, M, act,
                        G.kSwiglu, stream())
        assert_close_1e3(host(y), ref, f"M={M} swiglu, d/s alignment")
        out = zeros((M, N, K // 32), torch.int32)
        hip.gemv_i32_dump(dev(g), N, K, M, act, out, stream())
        assert np.array_equal(host(out), oracle.gemv_i32(g, K, q, s)), f"M={M} I"


def test_prep_then_gemv_end_to_end(hip, oracle):
    """GPU quantize feeding the GPU GEMV equals oracle quantize + emulator GEMV."""
    rng = np.random.default_rng(99)
    K, N, M = 5120, 300, 2
    codes, scales = random_mat(oracle, rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    q, d, s = oracle.quantize_rows(x)
    ref = oracle.gemv(codes, scales, K, q, d, s)
    torch = _torch()
    a = hip.Q8Act(zeros((M, K), torch.int8), zeros((M, K // 32), torch.float32), zeros((M, K // 32), torch.int32))
    hip.launch_prep(dev(x), K, M, K, None, 0.0, None, None, 0, a, stream())
    y = zeros((M, N), torch.float32)
    hip.launch_gemv([hip.GemvSeg(dev(codes), dev(scales), N, y, N)], K, M, a, hip.GemvMode.kStore, stream())
    assert_close_1e3(host(y), ref, "prep+gemv")


@pytest.mark.parametrize("K,M", [(1024, 1), (5120, 1), (5120, 3), (17408, 1), (20480, 2)])
def test_gemv_fused_input_quantize(hip, oracle, K, M):
    """launch_gemv_ex from fp32 rows (the Q8 quantize inside the GEMV launch)
    equals launch_prep + launch_gemv (v_dot4 path) bit for bit in every mode,
    and the emulator's quantize + GEMV to the float bar; inputs include the
    quantizer's edge rows (zero blocks with +-0 ends, ties, subnormal d) and
    ldx > K."""
    rng = np.random.default_rng(777 + K + M)
    N = 96
    x = (rng.standard_normal((M, K)) * 3).astype(np.float32)
    x[0, :] = _special_rows(K)[M % 6] if M > 1 else x[0, :]
    if M == 1:
        x[0, :128] = _special_rows(K)[0, :128]
    ldx = K + 4
    xp = np.zeros((M, ldx), np.float32)
    xp[:, :K] = x
    xd = dev(xp)
    q, d, s = oracle.quantize_rows(x)
    gate, up, mat = (random_mat(oracle, rng, N, K) for _ in range(3))
    torch = _torch()
    a = hip.Q8Act(zeros((M, K), torch.int8), zeros((M, K // 32), torch.float32), zeros((M, K // 32), torch.int32))
    hip.launch_prep(xd, ldx, M, K, None, 0.0, None, None, 0, a, stream())
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    for mode in (hip.GemvMode.kStore, hip.GemvMode.kAdd, hip.GemvMode.kSwiglu):
        outs = []
        for fused in (False, True):
            y = dev(y0.copy())
            if mode == hip.GemvMode.kSwiglu:
                segs = [hip.GemvSeg(dev(gate[0]), dev(gate[1]), N, y, N), hip.GemvSeg(dev(up[0]), dev(up[1]), N, None, 0)]
            else:
                segs = [hip.GemvSeg(dev(mat[0]), dev(mat[1]), N, y, N)]
            if fused:
                hip.launch_gemv_ex(segs, K, M, x=xd, ldx=ldx, mode=mode, stream=stream())
            else:  # on the v_dot4 path too (larger M takes the MFMA kernel, another float order)
                prev = hip.gemv_set_policy(1 << 20)
                try:
                    hip.launch_gemv(segs, K, M, a, mode, stream())
                finally:
                    hip.gemv_set_policy(prev)
            outs.append(host(y))
        assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), f"mode {mode}"
        if mode == hip.GemvMode.kSwiglu:
            ref = oracle.swiglu(oracle.gemv(gate[0], gate[1], K, q, d, s), oracle.gemv(up[0], up[1], K, q, d, s))
        else:
            ref = oracle.gemv(mat[0], mat[1], K, q, d, s, y=y0.copy(), add=mode == hip.GemvMode.kAdd)
        assert_close_1e3(outs[1], ref, f"fused mode {mode}")


@pytest.mark.parametrize("K,N,M,xin", [(1024, 64, 1, False), (5120, 160, 2, False), (5120, 96, 1, True),
                                       (17408, 64, 1, False), (20480, 32, 1, True)])
def test_gemv_fused_output_quantize(hip, oracle, K, N, M, xin):
    """launch_gemv_ex with a Q8 output: y equals launch_gemv's (v_dot4 path)
    bit for bit and the Q8 rows equal launch_prep of that y (and the
    oracle's quantize) bit for bit, in every mode (swiglu only where
    K <= 10240), from Q8 or fp32 input."""
    rng = np.random.default_rng(99 + K + N + M)
    x = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    xd = dev(x)
    q, d, s = oracle.quantize_rows(x)
    torch = _torch()
    a = q8_dev(q, d, s, hip)
    mat, gate, up = (random_mat(oracle, rng, N, K) for _ in range(3))
    mat[0][:32] = 0x55  # rows 0..31 all trit 0: an all-zero output block (store; add onto zeros)
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    y0[:, :32] = 0.0
    modes = [hip.GemvMode.kStore, hip.GemvMode.kAdd] + ([hip.GemvMode.kSwiglu] if K <= 10240 else [])
    for mode in modes:
        if mode == hip.GemvMode.kSwiglu:
            mk = lambda y: [hip.GemvSeg(dev(gate[0]), dev(gate[1]), N, y, N),
                            hip.GemvSeg(dev(up[0]), dev(up[1]), N, None, 0)]
        else:
            mk = lambda y: [hip.GemvSeg(dev(mat[0]), dev(mat[1]), N, y, N)]
        y_ref = dev(y0.copy())
        prev = hip.gemv_set_policy(1 << 20)
        try:
            hip.launch_gemv(mk(y_ref), K, M, a, mode, stream())
        finally:
            hip.gemv_set_policy(prev)
        y = dev(y0.copy())
        out = hip.Q8Act(zeros((M, N), torch.int8), zeros((M, N // 32), torch.float32), zeros((M, N // 32), torch.int32))
        if xin:
            hip.launch_gemv_ex(mk(y), K, M, x=xd, ldx=K, mode=mode, out=out, stream=stream())
        else:
            hip.launch_gemv_ex(mk(y), K, M, a=a, mode=mode, out=out, stream=stream())
        yh = host(y)
        assert np.array_equal(yh.view(np.uint32), host(y_ref).view(np.uint32)), f"y, mode {mode}"
        rq, rd, rs = oracle.quantize_rows(yh)
        assert np.array_equal(host(out.q), rq), f"q, mode {mode}"
        assert np.array_equal(host(out.d).view(np.uint32), rd.view(np.uint32)), f"d, mode {mode}"
        assert np.array_equal(host(out.s), rs), f"s, mode {mode}"


@pytest.mark.parametrize("K,N,M", [(5120, 160, 3), (5120, 96, 8), (17408, 64, 8), (5120, 128, 16),
                                   (1024, 96, 20), (17408, 64, 32)])
def test_gemm_fused_output_quantize_batched(hip, oracle, K, N, M):
    """launch_gemv_ex with Q8 rows in and out for a batch (the int8-MFMA
    K-split kernel with 32-row output tiles, one launch): y equals
    launch_gemv's bit for bit, the Q8 rows equal the oracle's quantize of that
    y bit for bit, and y is within the bars of the oracle GEMV, in every mode;
    rows 0..31 of the plain matrix are all trit 0 (an all-zero output block)."""
    rng = np.random.default_rng(7 + K + N + M)
    x = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    q, d, s = oracle.quantize_rows(x)
    torch = _torch()
    a = q8_dev(q, d, s, hip)
    mat, gate, up = (random_mat(oracle, rng, N, K) for _ in range(3))
    mat[0][:32] = 0x55
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    y0[:, :32] = 0.0
    for mode in (hip.GemvMode.kStore, hip.GemvMode.kAdd, hip.GemvMode.kSwiglu):
        if mode == hip.GemvMode.kSwiglu:
            mk = lambda y: [hip.GemvSeg(dev(gate[0]), dev(gate[1]), N, y, N),
                            hip.GemvSeg(dev(up[0]), dev(up[1]), N, None, 0)]
        else:
            mk = lambda y: [hip.GemvSeg(dev(mat[0]), dev(mat[1]), N, y, N)]
        y_ref = dev(y0.copy())
        hip.launch_gemv(mk(y_ref), K, M, a, mode, stream())
        y = dev(y0.copy())
        out = hip.Q8Act(zeros((M, N), torch.int8), zeros((M, N // 32), torch.float32), zeros((M, N // 32), torch.int32))
        hip.launch_gemv_ex(mk(y), K, M, a=a, mode=mode, out=out, stream=stream())
        yh = host(y)
        assert np.array_equal(yh.view(np.uint32), host(y_ref).view(np.uint32)), f"y, mode {mode}"
        rq, rd, rs = oracle.quantize_rows(yh)
        assert np.array_equal(host(out.q), rq), f"q, mode {mode}"
        assert np.array_equal(host(out.d).view(np.uint32), rd.view(np.uint32)), f"d, mode {mode}"
        assert np.array_equal(host(out.s), rs), f"s, mode {mode}"
        if mode == hip.GemvMode.kSwiglu:
            ref = oracle.swiglu(oracle.gemv(gate[0], gate[1], K, q, d, s), oracle.gemv(up[0], up[1], K, q, d, s))
        else:
            ref = oracle.gemv(mat[0], mat[1], K, q, d, s, y=y0.copy(), add=mode == hip.GemvMode.kAdd)
        assert_close_1e3(yh, ref, f"fused batched mode {mode}")


def test_gemm_fused_batched_chain_matches_prep_chain(hip, oracle):
    """Batched decode (M = 8) through a 3-GEMM chain whose quantizes ride in
    the producers' epilogues equals the chain of launch_prep + launch_gemv
    pairs bit for bit, y and the Q8 rows handed on."""
    rng = np.random.default_rng(515)
    M, K0, K1, K2 = 8, 2048, 4096, 1024
    m0, m1, m2 = random_mat(oracle, rng, K1, K0), random_mat(oracle, rng, K2, K1), random_mat(oracle, rng, 96, K2)
    x = rng.standard_normal((M, K0)).astype(np.float32)
    torch = _torch()

    def q8(n):
        return hip.Q8Act(zeros((M, n), torch.int8), zeros((M, n // 32), torch.float32), zeros((M, n // 32), torch.int32))
    res = []
    for fused in (False, True):
        xd = dev(x)
        y1, y2, y3 = zeros((M, K1), torch.float32), zeros((M, K2), torch.float32), zeros((M, 96), torch.float32)
        a0, a1, a2 = q8(K0), q8(K1), q8(K2)
        hip.launch_prep(xd, K0, M, K0, None, 0.0, None, None, 0, a0, stream())
        if fused:
            hip.launch_gemv_ex([hip.GemvSeg(dev(m0[0]), dev(m0[1]), K1, y1, K1)], K0, M, a=a0, out=a1, stream=stream())
            hip.launch_gemv_ex([hip.GemvSeg(dev(m1[0]), dev(m1[1]), K2, y2, K2)], K1, M, a=a1, out=a2, stream=stream())
        else:
            hip.launch_gemv([hip.GemvSeg(dev(m0[0]), dev(m0[1]), K1, y1, K1)], K0, M, a0, hip.GemvMode.kStore, stream())
            hip.launch_prep(y1, K1, M, K1, None, 0.0, None, None, 0, a1, stream())
            hip.launch_gemv([hip.GemvSeg(dev(m1[0]), dev(m1[1]), K2, y2, K2)], K1, M, a1, hip.GemvMode.kStore, stream())
            hip.launch_prep(y2, K2, M, K2, None, 0.0, None, None, 0, a2, stream())
        hip.launch_gemv([hip.GemvSeg(dev(m2[0]), dev(m2[1]), 96, y3, 96)], K2, M, a2, hip.GemvMode.kStore, stream())
        res.append([host(t) for t in (y1, y2, y3, a1.q, a1.d, a1.s, a2.q, a2.d, a2.s)])
    for u, v in zip(*res):
        assert np.array_equal(u.view(np.uint8), v.view(np.uint8))


def test_gemv_fused_chain_matches_prep_chain(hip, oracle):
    """A 3-GEMV chain whose quantizes ride in the GEMV launches (fp32 input
    quantized by the first, Q8 outputs feeding the next) equals the chain of
    launch_prep + launch_gemv pairs bit for bit."""
    rng = np.random.default_rng(4242)
    K0, K1, K2 = 5120, 2048, 1024
    m0, m1, m2 = random_mat(oracle, rng, K1, K0), random_mat(oracle, rng, K2, K1), random_mat(oracle, rng, 96, K2)
    x = rng.standard_normal((1, K0)).astype(np.float32)
    torch = _torch()
    def q8(n):
        return hip.Q8Act(zeros((1, n), torch.int8), zeros((1, n // 32), torch.float32), zeros((1, n // 32), torch.int32))
    res = []
    for fused in (False, True):
        xd = dev(x)
        y1, y2, y3 = zeros((1, K1), torch.float32), zeros((1, K2), torch.float32), zeros((1, 96), torch.float32)
        a1, a2 = q8(K1), q8(K2)
        if fused:
            hip.launch_gemv_ex([hip.GemvSeg(dev(m0[0]), dev(m0[1]), K1, y1, K1)], K0, 1, x=xd, ldx=K0, out=a1,
                               stream=stream())
            hip.launch_gemv_ex([hip.GemvSeg(dev(m1[0]), dev(m1[1]), K2, y2, K2)], K1, 1, a=a1, out=a2, stream=stream())
            hip.launch_gemv([hip.GemvSeg(dev(m2[0]), dev(m2[1]), 96, y3, 96)], K2, 1, a2, hip.GemvMode.kStore, stream())
        else:
            a0 = q8(K0)
            hip.launch_prep(xd, K0, 1, K0, None, 0.0, None, None, 0, a0, stream())
            hip.launch_gemv([hip.GemvSeg(dev(m0[0]), dev(m0[1]), K1, y1, K1)], K0, 1, a0, hip.GemvMode.kStore, stream())
            hip.launch_prep(y1, K1, 1, K1, None, 0.0, None, None, 0, a1, stream())
            hip.launch_gemv([hip.GemvSeg(dev(m1[0]), dev(m1[1]), K2, y2, K2)], K1, 1, a1, hip.GemvMode.kStore, stream())
            hip.launch_prep(y2, K2, 1, K2, None, 0.0, None, None, 0, a2, stream())
            hip.launch_gemv([hip.GemvSeg(dev(m2[0]), dev(m2[1]), 96, y3, 96)], K2, 1, a2, hip.GemvMode.kStore, stream())
        res.append([host(t) for t in (y1, y2, y3)])
    for u, v in zip(*res):
        assert np.array_equal(u.view(np.uint32), v.view(np.uint32))


@pytest.mark.parametrize("E,block,mapped", [(1024, 0, False), (5120, 1024, False), (5120, 128, True),
                                             (2048, 1024, False), (17408, 256, False),
                                             (1152, 128, False), (1152, 16, True), (3072, 1024, False),
                                             (5120, 2, False), (128, 128, False)])
def test_embed_bit_exact(hip, oracle, E, block, mapped):
    """Embedding rows of a packed table (device or mapped host memory) with
    the inverse transform equal the emulator's lookup (oracle) bit for bit;
    tokens include the table's first and last rows."""
    rng = np.random.default_rng(E + block)
    V = 300
    codes, scales = random_mat(oracle, rng, V, E)
    toks = np.array([0, V - 1, 17, 17, 123], np.int32)
    sg = np.where(rng.random(E) < 0.5, -1.0, 1.0).astype(np.float32) if block else None
    ref = oracle.embed(codes, scales, toks, E, V, block, sg)
    torch = _torch()
    x = zeros((toks.size, E), torch.float32)
    bufs = []
    if mapped:
        for a in (codes, scales):
            b = hip.MappedHostBuffer(a.nbytes)
            b.view()[:] = np.ascontiguousarray(a).view(np.uint8).ravel()
            bufs.append(b)
        cptr, sptr = bufs[0].dev, bufs[1].dev
    else:
        cd, sd = dev(codes), dev(scales)
        cptr, sptr = cd, sd
    hip.launch_embed(cptr, sptr, dev(toks), toks.size, E, hip.Hx(block=block, signs=dev(sg) if sg is not None else None),
                     x, stream())
    torch.cuda.synchronize()
    got = host(x)
    for b in bufs:
        b.close()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_embed_block_wider_than_the_span_is_rejected(hip, oracle):
    """As the reference launcher (src/cuda/kernels.cu:889-891): a transform
    block must divide the span (at most 1024 columns)."""
    rng = np.random.default_rng(5)
    codes, scales = random_mat(oracle, rng, 8, 2048)
    torch = _torch()
    x = zeros((1, 2048), torch.float32)
    with pytest.raises(RuntimeError, match="span"):
        hip.launch_embed(dev(codes), dev(scales), dev(np.array([1], np.int32)), 1, 2048, hip.Hx(block=2048), x,
                         stream())


@pytest.mark.parametrize("V", [1, 100, 4097, 248320, 2048 * 256 + 77])
def test_argmax_matches_oracle(hip, oracle, V):
    """Greedy pick over the logits: random values, a planted tie (the smaller
    index wins), all -inf but two, an interior NaN (never wins), all equal."""
    rng = np.random.default_rng(V)
    torch = _torch()
    part = zeros((hip.argmax_part_bytes(V) // 4,), torch.int32)
    out = zeros((1,), torch.int32)
    cases = [rng.standard_normal(V).astype(np.float32)]
    if V > 10:
        t = rng.standard_normal(V).astype(np.float32)
        t[[V // 3, V - 2]] = t.max() + 2
        cases.append(t)
        t = np.full(V, -np.inf, np.float32)
        t[[5, V - 1]] = -7.0
        cases.append(t)
        t = rng.standard_normal(V).astype(np.float32)
        t[V // 2] = np.nan
        cases.append(t)
        cases.append(np.full(V, 0.5, np.float32))
        t = np.full(V, -1.0, np.float32)
        t[[3, V - 3]] = -0.0  # -0 == +0: the first one wins
        t[V // 2] = 0.0
        cases.append(t)
        cases.append(np.full(V, np.nan, np.float32))
    for l in cases:
        hip.launch_argmax(dev(l), V, part, out, stream())
        assert int(host(out)[0]) == oracle.argmax(l)


def test_pos_add_eager_and_in_a_graph(hip):
    """pos_add adds M to the device counter, eagerly and on every replay of a
    captured graph (with eager work and syncs between the replays)."""
    torch = _torch()
    pos = dev(np.array([5], np.int32))
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        hip.launch_pos_add(pos, 3, s.cuda_stream)
        s.synchronize()
        assert int(host(pos)[0]) == 8
        g = hip.Graph(s.cuda_stream)
        with g:
            hip.launch_pos_add(pos, 1, s.cuda_stream)
        want = 8
        for _ in range(3):
            g.launch()
            s.synchronize()
            want += 1
            assert int(host(pos)[0]) == want
            hip.launch_pos_add(pos, 10, s.cuda_stream)
            s.synchronize()
            want += 10
            assert int(host(pos)[0]) == want


def test_graph_replay_matches_eager(hip, oracle):
    """A captured quantize + GEMV + add sequence replays identically (several
    replays with eager work and syncs between them)."""
    torch = _torch()
    rng = np.random.default_rng(2024)
    K, N = 1024, 200
    codes, scales = random_mat(oracle, rng, N, K)
    x = dev(rng.standard_normal((1, K)).astype(np.float32))
    a = hip.Q8Act(zeros((1, K), torch.int8), zeros((1, K // 32), torch.float32), zeros((1, K // 32), torch.int32))
    cd, sd = dev(codes), dev(scales)
    y = zeros((1, N), torch.float32)
    s = torch.cuda.Stream()  # the null stream cannot be captured
    with torch.cuda.stream(s):
        def seq():
            hip.launch_prep(x, K, 1, K, None, 0.0, None, None, 0, a, s.cuda_stream)
            hip.launch_gemv([hip.GemvSeg(cd, sd, N, y, N)], K, 1, a, hip.GemvMode.kAdd, s.cuda_stream)
        seq()
        s.synchronize()
        eager1 = host(y).copy()
        seq()
        s.synchronize()
        eager2 = host(y).copy()
        y.zero_()
        s.synchronize()
        g = hip.Graph(s)
        with g:
            seq()
        for rep in range(3):
            y.zero_()
            s.synchronize()
            g.launch()
            s.synchronize()
            assert np.array_equal(host(y), eager1), f"replay {rep}"
            g.launch()
            s.synchronize()
            assert np.array_equal(host(y), eager2), f"double replay {rep}"
            _ = (x * 2).sum().item()  # unrelated eager work between replays


def test_invalid_arguments_raise(hip):
    torch = _torch()
    a = hip.Q8Act(zeros((1, 1024), torch.int8), zeros((1, 32), torch.float32), zeros((1, 32), torch.int32))
    seg = hip.GemvSeg(zeros((4, 256), torch.uint8), zeros((4, 8), torch.int16), 4, zeros((1, 4), torch.float32), 4)
    with pytest.raises(RuntimeError, match="multiple of 128"):
        hip.launch_gemv([seg], 1000, 1, a, hip.GemvMode.kStore, stream())
    with pytest.raises(RuntimeError, match="swiglu"):
        hip.launch_gemv([seg], 1024, 1, a, hip.GemvMode.kSwiglu, stream())
    with pytest.raises(RuntimeError, match="multiple of 32"):
        hip.launch_prep(zeros((1, 1024), torch.float32), 1024, 1, 1000, None, 0.0, None, None, 0, a, stream())
