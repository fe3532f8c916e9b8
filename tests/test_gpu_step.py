"""GPU tests of the decode-step program (btf_hip_step_*): a chain of GEMVs,
each with the Q8 quantize of its input, run as one persistent launch.

Bars:
  * bit-exact against the same chain launched op by op (launch_prep without
    norm/transform + launch_gemv, batch 1): the step kernel uses the same
    dot products, the same per-1024-column-slice DPP reduction and the same
    slice order, and its producer-side Q8 is the q8 kernel's arithmetic;
  * each op within rel-RMS 1e-3 (and max error 1e-3 of max |ref|) of the
    oracle (oracle Q8 + emulator GEMV of src/emu_decoder.cpp:143-165, SwiGLU)
    applied to the step's own input vector.
The chain mirrors a decoder layer's GEMVs (src/cuda/gpu_decoder.cu:452-486):
QKV (store) reading the residual stream written by the layer before, o
(+= residual), gate/up (swiglu) and down (+= residual). Gate/up read a fixed
normed-input stand-in: without the model's RMSNorm a residual feeding them
would grow quadratically and overflow within a few layers.
"""
import numpy as np
import pytest

from helpers import assert_close_1e3, random_mat

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


class Mat:
    """A packed matrix on the device (codes [N][K/4], scales [N][K/128])."""

    def __init__(self, codes, scales, N, K, host_codes=None, host_scales=None):
        self.codes, self.scales, self.N, self.K = codes, scales, N, K
        self.host_codes, self.host_scales = host_codes, host_scales


def host_mat(oracle, rng, N, K):
    """Random weights with block scales ~0.03 (a GEMV then keeps the input's
    magnitude order over a chain; with unit scales every op multiplies it by
    ~20 and a few ops overflow the fp16 Q8 scale on the CPU and GPU alike)."""
    c, s = random_mat(oracle, rng, N, K, scale=0.03)
    return Mat(dev(c), dev(s), N, K, c, s)


def gen_dev_mat(hip, N, K, mat_id, seed=7):
    """Seeded generator + repack on the device (both bit-exact with the
    oracle, see test_gpu_parity)."""
    torch = _torch()
    nb = N * K // 128
    src = torch.empty(nb * 28, dtype=torch.uint8, device="cuda")
    codes = torch.empty(N * K // 4, dtype=torch.uint8, device="cuda")
    scales = torch.empty(N * K // 128, dtype=torch.int16, device="cuda")
    hip.gen_ptq1_0(seed, mat_id, 0, nb, src, stream())
    hip.launch_repack(src, nb, codes, scales, stream())
    torch.cuda.synchronize()
    return Mat(codes, scales, N, K)


def layer_ops(hip, mats, RES, QKV, ATT, H, X):
    """The four GEMVs of one layer over vector slots RES, QKV, ATT, H, X."""
    G = hip.GemvMode
    qkv, o, gate, up, down = mats
    return [
        hip.StepGemv(G.kStore, qkv.K, qkv.N, qkv.codes, qkv.scales, RES, QKV),
        hip.StepGemv(G.kAdd, o.K, o.N, o.codes, o.scales, ATT, RES),
        hip.StepGemv(G.kSwiglu, gate.K, gate.N, gate.codes, gate.scales, X, H, up.codes, up.scales),
        hip.StepGemv(G.kAdd, down.K, down.N, down.codes, down.scales, H, RES),
    ]


def run_sequential(hip, ops, vecs):
    """The same chain launched op by op on torch tensors `vecs` (updated)."""
    torch = _torch()
    G = hip.GemvMode
    for op in ops:
        K = op.K
        act = hip.Q8Act(torch.empty(K, dtype=torch.int8, device="cuda"),
                        torch.empty(K // 32, dtype=torch.float32, device="cuda"),
                        torch.empty(K // 32, dtype=torch.int32, device="cuda"))
        hip.launch_prep(vecs[op.in_vec], K, 1, K, None, 0.0, None, None, 0, act, stream())
        y = vecs[op.out_vec]
        if op.mode == G.kSwiglu:
            segs = [hip.GemvSeg(op.codes, op.scales, op.N, y, op.N), hip.GemvSeg(op.up_codes, op.up_scales, op.N, None, 0)]
        else:
            segs = [hip.GemvSeg(op.codes, op.scales, op.N, y, op.N)]
        hip.launch_gemv(segs, K, 1, act, op.mode, stream())
    torch.cuda.synchronize()


def small_chain(hip, oracle, layers, H=1024, NQ=1000, F=3072, seed=5):
    """Vectors: 0 = residual (input, += target), 1 = qkv output (N = 1000, not
    a multiple of 32: a partial last unit), 2 = attention-output stand-in,
    3 = MLP hidden, 4 = the normed-input stand-in. Random encoder-quantized
    weights. (Step programs take K % 1024 == 0 and N % 4 == 0.)"""
    rng = np.random.default_rng(seed)
    res0 = rng.standard_normal(H).astype(np.float32)
    att = (rng.standard_normal(H) * 2).astype(np.float32)
    xin = rng.standard_normal(H).astype(np.float32)
    ops, hm = [], []
    for _ in range(layers):
        mats = [host_mat(oracle, rng, NQ, H), host_mat(oracle, rng, H, H), host_mat(oracle, rng, F, H),
                host_mat(oracle, rng, F, H), host_mat(oracle, rng, H, F)]
        ops += layer_ops(hip, mats, 0, 1, 2, 3, 4)
    return ops, (res0, att, xin), (H, NQ, F)


def make_vectors(hip, inputs, dims, with_h_data=False):
    torch = _torch()
    res0, att, xin = inputs
    H, NQ, F = dims
    t = [dev(res0), torch.zeros(NQ, dtype=torch.float32, device="cuda"), dev(att),
         torch.zeros(F, dtype=torch.float32, device="cuda"), dev(xin)]
    vecs = [hip.StepVec(H, t[0]), hip.StepVec(NQ, t[1]), hip.StepVec(H, t[2]),
            hip.StepVec(F, t[3] if with_h_data else None), hip.StepVec(H, t[4])]
    return vecs, t


@pytest.mark.parametrize("layers", [1, 3])
def test_step_matches_sequential_small(hip, oracle, layers):
    ops, inputs, dims = small_chain(hip, oracle, layers)
    vecs, t = make_vectors(hip, inputs, dims, with_h_data=True)
    prog = hip.StepProgram(vecs, ops)
    prog.launch(stream())
    _torch().cuda.synchronize()
    assert prog.error() == 0
    # sequential launches on fresh copies
    _, s = make_vectors(hip, inputs, dims, with_h_data=True)
    run_sequential(hip, ops, s)
    for name, a, b in zip(("res", "qkv", "att", "h", "x"), t, s):
        ga, gb = host(a), host(b)
        assert np.isfinite(ga).all(), name
        assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32)), \
            f"{name}: step != sequential (max diff {np.max(np.abs(ga - gb)):.3e})"
    prog.close()


def test_step_reordered_chain_and_war(hip, oracle):
    """The bench's program order (gate/up, QKV, o, down per layer: each op's
    input produced two or three ops earlier, versions double-buffered) equals
    the op-by-op launches; plus a vector read through the launch's quantize
    prologue and then overwritten by a STORE as its final writer (the plain
    store must wait for every read of the user's data)."""
    torch = _torch()
    G = hip.GemvMode
    rng = np.random.default_rng(31)
    H, NQ, F = 1024, 1000, 3072
    ops = []
    for _ in range(3):
        qkv, o, gate, up, down = (host_mat(oracle, rng, NQ, H), host_mat(oracle, rng, H, H), host_mat(oracle, rng, F, H),
                                  host_mat(oracle, rng, F, H), host_mat(oracle, rng, H, F))
        ops += [hip.StepGemv(G.kSwiglu, H, F, gate.codes, gate.scales, 4, 3, up.codes, up.scales),
                hip.StepGemv(G.kStore, H, NQ, qkv.codes, qkv.scales, 0, 1),
                hip.StepGemv(G.kAdd, H, H, o.codes, o.scales, 2, 0),
                hip.StepGemv(G.kAdd, F, H, down.codes, down.scales, 3, 0)]
    # vector 5 (data) is read by an op, then overwritten by a STORE (version 1, final)
    w5a, w5b = host_mat(oracle, rng, H, H), host_mat(oracle, rng, H, H)
    ops += [hip.StepGemv(G.kStore, H, H, w5a.codes, w5a.scales, 5, 6),
            hip.StepGemv(G.kStore, H, H, w5b.codes, w5b.scales, 4, 5)]
    inputs = [rng.standard_normal(n).astype(np.float32) for n in (H, NQ, H, F, H, H, H)]

    def vectors():
        t = [dev(a) for a in inputs]
        return [hip.StepVec(int(x.numel()), x) for x in t], t

    vecs, t = vectors()
    prog = hip.StepProgram(vecs, ops)
    # the final STORE into vector 5's user buffer keeps its wait for the read
    # of that data: the data flow before it does not order every read
    assert prog.guards() >= 1
    for rep in range(2):
        if rep:
            for x, a in zip(t, inputs):
                x.copy_(dev(a))
        prog.launch(stream())
        torch.cuda.synchronize()
        assert prog.error() == 0
        _, s = vectors()
        run_sequential(hip, ops, s)
        for k, (a, b) in enumerate(zip(t, s)):
            ga, gb = host(a), host(b)
            assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32)), f"launch {rep} vector {k}"
    prog.close()


def test_step_prefix_reader_keeps_its_guard(hip, oracle):
    """An op reading the first 1024 values of a vector that every workgroup
    wrote (8192 values) overwrites a Q8 buffer whose earlier version other
    workgroups may still be reading: the program keeps that write-after-read
    wait (the host analysis credits only the writers of the prefix) and the
    launch equals the op-by-op launches, twice in a row."""
    torch = _torch()
    G = hip.GemvMode
    rng = np.random.default_rng(41)
    m = lambda N, K: host_mat(oracle, rng, N, K)
    spec = [(1024, 1024, 1, 2, G.kStore), (1024, 1024, 4, 1, G.kStore), (1024, 1024, 1, 2, G.kStore),
            (1024, 1024, 4, 1, G.kStore), (1024, 1024, 1, 2, G.kStore), (1024, 8192, 4, 0, G.kStore),
            (1024, 1024, 0, 1, G.kStore), (1024, 1024, 1, 3, G.kStore)]
    ops = []
    for K, N, i, o, mode in spec:
        w = m(N, K)
        ops.append(hip.StepGemv(mode, K, N, w.codes, w.scales, i, o))
    lengths = (8192, 1024, 1024, 1024, 1024)
    inputs = [rng.standard_normal(n).astype(np.float32) for n in lengths]

    def vectors():
        t = [dev(a) for a in inputs]
        return [hip.StepVec(int(x.numel()), x) for x in t], t

    vecs, t = vectors()
    prog = hip.StepProgram(vecs, ops)
    full_ops = list(ops)
    full_ops[6] = hip.StepGemv(G.kStore, 8192, 1024, *(lambda w: (w.codes, w.scales))(m(1024, 8192)), 0, 1)
    assert prog.guards() == hip.step_audit(vecs, ops)["guards"] >= 1
    assert hip.step_audit(vecs, full_ops)["guards"] == prog.guards() - 1
    for rep in range(2):
        if rep:
            for x, a in zip(t, inputs):
                x.copy_(dev(a))
        prog.launch(stream())
        torch.cuda.synchronize()
        assert prog.error() == 0
        _, s = vectors()
        run_sequential(hip, ops, s)
        for k, (a, b) in enumerate(zip(t, s)):
            ga, gb = host(a), host(b)
            assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32)), f"launch {rep} vector {k}"
    prog.close()


def test_step_each_op_vs_oracle(hip, oracle):
    """Every op against the oracle on the step's own input vector: a chain in
    which each op writes a vector of its own (all observable), so a Q8 input
    that differs in the last float bit between GPU and CPU (and would round
    one q the other way) cannot compound across ops."""
    torch = _torch()
    G = hip.GemvMode
    rng = np.random.default_rng(23)
    H, F, N0 = 1024, 3072, 2048
    W = [host_mat(oracle, rng, N0, H), host_mat(oracle, rng, H, N0), host_mat(oracle, rng, F, H),
         host_mat(oracle, rng, F, H), host_mat(oracle, rng, H, F)]
    x0 = rng.standard_normal(H).astype(np.float32)
    r0 = rng.standard_normal(H).astype(np.float32)
    r1 = rng.standard_normal(H).astype(np.float32)
    # vectors: 0 = x (input), 1 = a (N0), 2 = r (+= target, H), 3 = h (F), 4 = out (+= target, H)
    t = [dev(x0), torch.zeros(N0, dtype=torch.float32, device="cuda"), dev(r0),
         torch.zeros(F, dtype=torch.float32, device="cuda"), dev(r1)]
    vecs = [hip.StepVec(int(v.numel()), v) for v in t]
    ops = [hip.StepGemv(G.kStore, H, N0, W[0].codes, W[0].scales, 0, 1),
           hip.StepGemv(G.kAdd, N0, H, W[1].codes, W[1].scales, 1, 2),
           hip.StepGemv(G.kSwiglu, H, F, W[2].codes, W[2].scales, 2, 3, W[3].codes, W[3].scales),
           hip.StepGemv(G.kAdd, F, H, W[4].codes, W[4].scales, 3, 4)]
    prog = hip.StepProgram(vecs, ops)
    prog.launch(stream())
    torch.cuda.synchronize()
    assert prog.error() == 0
    a, r, h, out = host(t[1]), host(t[2]), host(t[3]), host(t[4])

    def q8(v):
        return oracle.quantize_rows(np.ascontiguousarray(v[None, :]))

    q, d, s = q8(x0)
    assert_close_1e3(a, oracle.gemv(W[0].host_codes, W[0].host_scales, H, q, d, s)[0], "store")
    q, d, s = q8(a)
    assert_close_1e3(r, oracle.gemv(W[1].host_codes, W[1].host_scales, N0, q, d, s, y=r0[None, :].copy(),
                                    add=True)[0], "add")
    q, d, s = q8(r)
    g = oracle.gemv(W[2].host_codes, W[2].host_scales, H, q, d, s)
    u = oracle.gemv(W[3].host_codes, W[3].host_scales, H, q, d, s)
    assert_close_1e3(h, oracle.swiglu(g, u)[0], "swiglu")
    q, d, s = q8(h)
    assert_close_1e3(out, oracle.gemv(W[4].host_codes, W[4].host_scales, F, q, d, s, y=r1[None, :].copy(),
                                      add=True)[0], "add K=3072")
    prog.close()


@pytest.mark.parametrize("nops", [1, 2])
def test_step_one_and_two_ops(hip, oracle, nops):
    """The shortest programs (the work records staged for ops past the end),
    launched twice, bit-exact against the op-by-op launches."""
    torch = _torch()
    G = hip.GemvMode
    rng = np.random.default_rng(50 + nops)
    W = [host_mat(oracle, rng, 2048, 1024), host_mat(oracle, rng, 1024, 2048)]
    x0 = rng.standard_normal(1024).astype(np.float32)
    r0 = rng.standard_normal(1024).astype(np.float32)
    ops = [hip.StepGemv(G.kStore, 1024, 2048, W[0].codes, W[0].scales, 0, 1),
           hip.StepGemv(G.kAdd, 2048, 1024, W[1].codes, W[1].scales, 1, 2)][:nops]

    def vectors():
        t = [dev(x0), torch.zeros(2048, dtype=torch.float32, device="cuda"), dev(r0)]
        return [hip.StepVec(int(v.numel()), v) for v in t], t

    vecs, t = vectors()
    prog = hip.StepProgram(vecs, ops)
    _, s = vectors()
    for rep in range(2):
        prog.launch(stream())
        run_sequential(hip, ops, s)
        _torch().cuda.synchronize()
        assert prog.error() == 0
        for name, a, b in zip(("x", "a", "r"), t, s):
            assert np.array_equal(host(a).view(np.uint32), host(b).view(np.uint32)), f"launch {rep}: {name}"
    prog.close()


def test_step_repeated_launches(hip, oracle):
    """Three launches in a row continue the residual stream (the program's
    epoch/tag progression): equal to three sequential passes."""
    ops, inputs, dims = small_chain(hip, oracle, 2, seed=11)
    vecs, t = make_vectors(hip, inputs, dims)
    prog = hip.StepProgram(vecs, ops)
    _, s = make_vectors(hip, inputs, dims, with_h_data=True)
    for rep in range(3):
        prog.launch(stream())
        run_sequential(hip, ops, s)
        _torch().cuda.synchronize()
        assert prog.error() == 0
        for name, i in (("res", 0), ("qkv", 1)):
            assert np.array_equal(host(t[i]).view(np.uint32), host(s[i]).view(np.uint32)), f"launch {rep}: {name}"
    prog.close()


def test_step_27b_layer_and_output(hip):
    """One 27B layer (QKV 5120->7168, o 5120->5120, gate/up 5120->17408,
    down 17408->5120) plus the output projection 5120->248320 in one launch,
    bit-exact against the op-by-op launches."""
    torch = _torch()
    E, F, QKV, V = 5120, 17408, 7168, 248320
    mats = [gen_dev_mat(hip, QKV, E, 1), gen_dev_mat(hip, E, E, 2), gen_dev_mat(hip, F, E, 3),
            gen_dev_mat(hip, F, E, 4), gen_dev_mat(hip, E, F, 5)]
    out = gen_dev_mat(hip, V, E, 6)
    ops = layer_ops(hip, mats, 0, 1, 2, 3, 5)
    ops.append(hip.StepGemv(hip.GemvMode.kStore, E, V, out.codes, out.scales, 0, 4))
    rng = np.random.default_rng(3)
    res0 = rng.standard_normal(E).astype(np.float32)
    att = rng.standard_normal(E).astype(np.float32)
    xin = rng.standard_normal(E).astype(np.float32)

    def vectors():
        t = [dev(res0), torch.zeros(QKV, dtype=torch.float32, device="cuda"), dev(att),
             torch.zeros(F, dtype=torch.float32, device="cuda"), torch.zeros(V, dtype=torch.float32, device="cuda"),
             dev(xin)]
        return [hip.StepVec(E, t[0]), hip.StepVec(QKV, t[1]), hip.StepVec(E, t[2]), hip.StepVec(F, t[3]),
                hip.StepVec(V, t[4]), hip.StepVec(E, t[5])], t

    vecs, t = vectors()
    prog = hip.StepProgram(vecs, ops)
    prog.launch(stream())
    torch.cuda.synchronize()
    assert prog.error() == 0
    _, s = vectors()
    run_sequential(hip, ops, s)
    for name, a, b in zip(("res", "qkv", "att", "h", "logits", "x"), t, s):
        ga, gb = host(a), host(b)
        assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32)), \
            f"{name}: step != sequential (max diff {np.max(np.abs(ga - gb)):.3e})"
    assert np.isfinite(host(t[4])).all() and np.abs(host(t[4])).max() > 0
    prog.close()


class Sweep27B:
    """Every matrix of the 27B-shape decode-step sweep (64 layers of QKV
    5120->7168, o 5120->5120, gate/up 5120->17408, down 17408->5120, and the
    output projection 5120->248320; 5.95 GB) in one device arena, from the
    seeded generator (seed 0, matrix id 5 l + k, output 320) repacked on the
    device. Both steps are bit-exact with the oracle (test_gpu_parity)."""

    E, F, QKV, V, L = 5120, 17408, 7168, 248320, 64

    def __init__(self, hip):
        torch = _torch()
        shapes = []
        for l in range(self.L):
            shapes += [(("qkv", l), self.QKV, self.E, 5 * l), (("o", l), self.E, self.E, 5 * l + 1),
                       (("gate", l), self.F, self.E, 5 * l + 2), (("up", l), self.F, self.E, 5 * l + 3),
                       (("down", l), self.E, self.F, 5 * l + 4)]
        shapes.append((("output", self.L), self.V, self.E, 5 * 64))
        off, self.mats = 0, {}
        al = lambda n: (n + 255) // 256 * 256
        for key, N, K, mid in shapes:
            co = off
            off = al(off + N * K // 4)
            so = off
            off = al(off + N * K // 64)
            self.mats[key] = (N, K, mid, co, so)
        self.arena = torch.empty(off, dtype=torch.uint8, device="cuda")
        stage = torch.empty(max(N * K // 128 for N, K, _, _, _ in self.mats.values()) * 28, dtype=torch.uint8,
                            device="cuda")
        base = self.arena.data_ptr()
        for (N, K, mid, co, so) in self.mats.values():
            hip.gen_ptq1_0(0, mid, 0, N * K // 128, stage, stream())
            hip.launch_repack(stage, N * K // 128, base + co, base + so, stream())
        torch.cuda.synchronize()
        del stage

    def w(self, key):
        N, K, _, co, so = self.mats[key]
        base = self.arena.data_ptr()
        return base + co, base + so

    def host(self, key, rows=None):
        N, K, _, co, so = self.mats[key]
        codes = self.arena[co:co + N * K // 4].cpu().numpy().reshape(N, K // 4)
        scales = self.arena[so:so + N * K // 64].cpu().numpy().view(np.uint16).reshape(N, K // 128)
        if rows is not None:
            codes, scales = codes[rows], scales[rows]
        return np.ascontiguousarray(codes), np.ascontiguousarray(scales)


@pytest.mark.parametrize("NF", [4096, 9216, 17408])
def test_step_work_orders_bit_exact(hip, NF):
    """The plain kernel's work orders, at 5120 columns: a swiglu op of NF
    outputs (128, 288 or 544 units over 256 workgroups: 0-1, 1-2 or 2-3
    units per workgroup) runs the unit-interleaved order rebalanced over the
    SIMDs (in odd units waves 2 and 3 take the batches of positions 8 and 9,
    waves 8 and 9 skip them; with one unit there is no odd unit), then an
    add op of K = NF and two store ops of 5 and 7 batches per unit-owning
    workgroup (the extra batches on the lowest waves, the waves without
    items pacing their refills). Two layers, every vector bit-exact against
    the same chain launched op by op."""
    torch = _torch()
    G = hip.GemvMode
    E, N2 = 5120, 7168
    rng = np.random.default_rng(NF)
    res0 = rng.standard_normal(E).astype(np.float32)
    mats = {}
    mid = 0
    for l in range(2):
        for name, N, K in (("gate", NF, E), ("up", NF, E), ("down", E, NF), ("s5", N2, E), ("s7", 1792, 7 * 1024)):
            mats[(name, l)] = gen_dev_mat(hip, N, K, 900 + mid, seed=NF)
            mid += 1
    ops = []
    for l in range(2):
        g, u, d, a, b = (mats[(n, l)] for n in ("gate", "up", "down", "s5", "s7"))
        ops += [hip.StepGemv(G.kSwiglu, E, NF, g.codes, g.scales, 0, 1, u.codes, u.scales),
                hip.StepGemv(G.kAdd, NF, E, d.codes, d.scales, 1, 0),
                hip.StepGemv(G.kStore, E, N2, a.codes, a.scales, 0, 2),
                hip.StepGemv(G.kStore, 7 * 1024, 1792, b.codes, b.scales, 2, 3)]

    def vectors():
        t = [dev(res0), torch.zeros(NF, dtype=torch.float32, device="cuda"),
             torch.zeros(N2, dtype=torch.float32, device="cuda"), torch.zeros(1792, dtype=torch.float32, device="cuda")]
        return [hip.StepVec(int(v.numel()), v) for v in t], t

    vecs, t = vectors()
    prog = hip.StepProgram(vecs, ops)
    prog.launch(stream())
    torch.cuda.synchronize()
    assert prog.error() == 0
    _, s = vectors()
    run_sequential(hip, ops, s)
    for k, (a, b) in enumerate(zip(t, s)):
        ga, gb = host(a), host(b)
        assert np.isfinite(ga).all(), k
        assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32)), \
            f"vector {k}: step != sequential (max diff {np.max(np.abs(ga - gb)):.3e})"
    prog.close()


def test_step_27b_full_sweep_and_output_head(hip, oracle):
    """The benchmark's full decode-step program (config 5): 64 layers of the
    27B shapes plus the 5120->248320 output projection, 257 GEMVs in one
    launch, on the seeded generator's weights. The data flow is the
    benchmark's: QKV reads the residual, o stores W_o * (attention-output
    stand-in) into x, gate/up read x, down adds into the residual, the output
    projection reads the final residual.
      * Every vector's final value is bit-exact against the same chain
        launched op by op (launch_prep + launch_gemv).
      * Sampled ops of the op-by-op run -- layers 0, 31 and 63 (QKV, o,
        gate+up, down) and every 16th row of the output projection -- are
        within 1e-3 of the oracle applied to their own input vectors, so the
        step, bit-exact with that run, is pinned to the oracle along the
        whole chain."""
    torch = _torch()
    G = hip.GemvMode
    W = Sweep27B(hip)
    E, F, QKV, V, L = W.E, W.F, W.QKV, W.V, W.L
    rng = np.random.default_rng(0)
    res0 = rng.standard_normal(E).astype(np.float32)
    att = rng.standard_normal(E).astype(np.float32)

    def vectors():
        t = [dev(res0), torch.zeros(QKV, dtype=torch.float32, device="cuda"), dev(att),
             torch.zeros(E, dtype=torch.float32, device="cuda"), torch.zeros(F, dtype=torch.float32, device="cuda"),
             torch.zeros(V, dtype=torch.float32, device="cuda")]
        return [hip.StepVec(int(v.numel()), v) for v in t], t

    ops = []
    for l in range(L):
        gc, gs = W.w(("gate", l))
        uc, us = W.w(("up", l))
        ops += [hip.StepGemv(G.kStore, E, QKV, *W.w(("qkv", l)), 0, 1),
                hip.StepGemv(G.kStore, E, E, *W.w(("o", l)), 2, 3),
                hip.StepGemv(G.kSwiglu, E, F, gc, gs, 3, 4, uc, us),
                hip.StepGemv(G.kAdd, F, E, *W.w(("down", l)), 4, 0)]
    ops.append(hip.StepGemv(G.kStore, E, V, *W.w(("output", L)), 0, 5))
    vecs, t = vectors()
    prog = hip.StepProgram(vecs, ops)
    prog.launch(stream())
    torch.cuda.synchronize()
    assert prog.error() == 0
    prog.close()

    # the same chain op by op, keeping the sampled ops' inputs and outputs
    _, s = vectors()
    sample, seen = (0, 31, 63), {}
    for i, op in enumerate(ops):
        l, k = divmod(i, 4)
        keep = l in sample or l == L
        if keep:
            seen[(l, k, "in")] = host(s[op.in_vec]).copy()
            if op.mode == G.kAdd:
                seen[(l, k, "old")] = host(s[op.out_vec]).copy()
        run_sequential(hip, [op], s)
        if keep:
            seen[(l, k, "out")] = host(s[op.out_vec]).copy()
    for name, a, b in zip(("res", "qkv", "att", "x", "h", "logits"), t, s):
        ga, gb = host(a), host(b)
        assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32)), \
            f"{name}: step != op-by-op (max diff {np.max(np.abs(ga - gb)):.3e})"
    assert np.isfinite(host(t[5])).all() and np.abs(host(t[5])).max() > 0

    names = ("qkv", "o", "gate", "down")
    for l in sample:
        for k, name in enumerate(names):
            x = seen[(l, k, "in")]
            q, d, s_ = oracle.quantize_rows(x[None, :])
            K = x.size
            if name == "gate":
                g = oracle.gemv(*W.host(("gate", l)), K, q, d, s_)
                u = oracle.gemv(*W.host(("up", l)), K, q, d, s_)
                want = oracle.swiglu(g, u)[0]
            elif name == "down":
                want = oracle.gemv(*W.host(("down", l)), K, q, d, s_, y=seen[(l, k, "old")][None, :].copy(),
                                   add=True)[0]
            else:
                want = oracle.gemv(*W.host((name, l)), K, q, d, s_)[0]
            assert_close_1e3(seen[(l, k, "out")], want, f"layer {l} {name}")
    rows = np.arange(0, V, 16)
    x = seen[(L, 0, "in")]
    q, d, s_ = oracle.quantize_rows(x[None, :])
    want = oracle.gemv(*W.host(("output", L), rows), E, q, d, s_)[0]
    assert_close_1e3(seen[(L, 0, "out")][rows], want, "output projection (every 16th row)")


def test_step_timeout_sets_error_and_recovers(hip, oracle):
    """A poll bound of 1 makes waiting workgroups give up (forced from the
    host: every wait is bounded, every wave still exits). The program is
    built so that a wait must outlast two polls: op 0 (K = 20480, 32 units)
    runs on 32 workgroups, each waiting for its quantized input and then
    streaming 160 KB of weights in two ring rounds, while op 1's units sit
    on workgroups that own none of op 0's and poll op 0's output at once.
    The launch reports the error; with the default bound restored the next
    launch is exact."""
    torch = _torch()
    G = hip.GemvMode
    rng = np.random.default_rng(17)
    W0 = host_mat(oracle, rng, 1024, 20480)
    W1 = host_mat(oracle, rng, 1024, 1024)
    x0 = rng.standard_normal(20480).astype(np.float32)
    ops = [hip.StepGemv(G.kStore, 20480, 1024, W0.codes, W0.scales, 0, 1),
           hip.StepGemv(G.kStore, 1024, 1024, W1.codes, W1.scales, 1, 2)]

    def vectors():
        t = [dev(x0), torch.zeros(1024, dtype=torch.float32, device="cuda"),
             torch.zeros(1024, dtype=torch.float32, device="cuda")]
        return [hip.StepVec(int(v.numel()), v) for v in t], t

    vecs, t = vectors()
    prog = hip.StepProgram(vecs, ops)
    prog.set_spin_limit(1)
    prog.launch(stream())
    torch.cuda.synchronize()
    assert prog.error() == 1, "a one-poll bound must time out"
    assert prog.error() == 0, "error() clears the flag"
    prog.set_spin_limit(0)
    prog.launch(stream())
    _, s = vectors()
    run_sequential(hip, ops, s)
    torch.cuda.synchronize()
    assert prog.error() == 0
    for i in (1, 2):
        assert np.array_equal(host(t[i]).view(np.uint32), host(s[i]).view(np.uint32))
    prog.close()


def test_step_add_after_swiglu_into_the_same_vector(hip, oracle):
    """v1 = silu(Wg v0) * (Wu v0); v1 += W v2: the add takes the swiglu's
    output rows as its old values (same units and placement). Bit-exact
    against the op-by-op launches, and within 1e-3 of the oracle."""
    torch = _torch()
    G = hip.GemvMode
    rng = np.random.default_rng(23)
    Wg, Wu, Wa = (host_mat(oracle, rng, 256, 1024) for _ in range(3))
    x0 = rng.standard_normal(1024).astype(np.float32)
    x2 = rng.standard_normal(1024).astype(np.float32)
    ops = [hip.StepGemv(G.kSwiglu, 1024, 256, Wg.codes, Wg.scales, 0, 1, Wu.codes, Wu.scales),
           hip.StepGemv(G.kAdd, 1024, 256, Wa.codes, Wa.scales, 2, 1)]

    def vectors():
        t = [dev(x0), torch.zeros(256, dtype=torch.float32, device="cuda"), dev(x2)]
        return [hip.StepVec(int(v.numel()), v) for v in t], t

    vecs, t = vectors()
    prog = hip.StepProgram(vecs, ops)
    _, s = vectors()
    for rep in range(2):  # the swiglu overwrites v1, so every launch gives the same result
        prog.launch(stream())
        torch.cuda.synchronize()
        assert prog.error() == 0
        run_sequential(hip, ops, s)
        assert np.array_equal(host(t[1]).view(np.uint32), host(s[1]).view(np.uint32)), f"launch {rep}"
    q0, d0, s0 = oracle.quantize_rows(x0[None, :])
    g = oracle.gemv(Wg.host_codes, Wg.host_scales, 1024, q0, d0, s0)
    u = oracle.gemv(Wu.host_codes, Wu.host_scales, 1024, q0, d0, s0)
    h = oracle.swiglu(g, u)
    q2, d2, s2 = oracle.quantize_rows(x2[None, :])
    want = oracle.gemv(Wa.host_codes, Wa.host_scales, 1024, q2, d2, s2, y=h.copy(), add=True)[0]
    assert_close_1e3(host(t[1]), want, "swiglu then add")
    prog.close()


def test_step_nan_values_quantize_as_the_q8_kernel(hip, oracle):
    """NaN values in a GEMV input: the Q8 of a block drops them (its running
    max starts at 0, as in the q8 kernel and on the CPU, so a NaN never
    becomes the amax; an all-NaN block is an all-zero one). Both of the step
    program's producer-side quantizes: a user vector with NaNs (the
    prologue's), and the NaN outputs of GEMV rows with NaN scales that the
    next GEMV reads (the epilogue's). Bit-exact against the op-by-op
    launches, and the second GEMV's outputs finite."""
    torch = _torch()
    G = hip.GemvMode
    rng = np.random.default_rng(91)
    K0, N0, N1 = 1024, 2048, 1024
    x0 = rng.standard_normal(K0).astype(np.float32)
    x0[0:32] = np.nan  # an all-NaN block
    x0[100] = np.nan   # one NaN among finite values
    c0, s0 = random_mat(oracle, rng, N0, K0, scale=0.03)
    s0 = s0.copy()
    s0[64:96] = 0x7E00  # one whole output block of NaN rows
    s0[200, 3] = 0x7E00  # and one NaN row among finite ones
    W0 = Mat(dev(c0), dev(s0), N0, K0, c0, s0)
    W1 = host_mat(oracle, rng, N1, N0)
    ops = [hip.StepGemv(G.kStore, K0, N0, W0.codes, W0.scales, 0, 1),
           hip.StepGemv(G.kStore, N0, N1, W1.codes, W1.scales, 1, 2)]

    def vectors():
        t = [dev(x0), torch.zeros(N0, dtype=torch.float32, device="cuda"),
             torch.zeros(N1, dtype=torch.float32, device="cuda")]
        return [hip.StepVec(int(v.numel()), v) for v in t], t

    vecs, t = vectors()
    prog = hip.StepProgram(vecs, ops)
    prog.launch(stream())
    _torch().cuda.synchronize()
    assert prog.error() == 0
    prog.close()
    _, s = vectors()
    run_sequential(hip, ops, s)
    h1 = host(s[1])
    assert np.isnan(h1[64:96]).all() and np.isnan(h1[200]) and np.isfinite(h1[96:200]).all()
    for name, a, b in zip(("x", "a", "y"), t, s):
        assert np.array_equal(host(a).view(np.uint32), host(b).view(np.uint32)), name
    assert np.isfinite(host(t[2])).all()


def test_step_invalid_programs(hip):
    torch = _torch()
    G = hip.GemvMode
    codes = torch.zeros(1024 * 1024 // 4, dtype=torch.uint8, device="cuda")
    scales = torch.zeros(1024 * 1024 // 128, dtype=torch.int16, device="cuda")
    x = torch.zeros(1024, dtype=torch.float32, device="cuda")
    v = [hip.StepVec(1024, x), hip.StepVec(1024, None)]
    ok = hip.StepGemv(G.kStore, 1024, 1024, codes, scales, 0, 1)
    assert hip.step_create_raw(v, [ok]) == hip.BTF_OK
    bad = [
        hip.StepGemv(G.kStore, 1024, 1024, codes, scales, 0, 0),           # reads its own output
        hip.StepGemv(G.kStore, 1000, 1024, codes, scales, 0, 1),           # K % 128
        hip.StepGemv(G.kStore, 1152, 1024, codes, scales, 0, 1),           # K % 1024
        hip.StepGemv(G.kStore, 1024, 1022, codes, scales, 0, 1),           # N % 4 (and != length)
        hip.StepGemv(G.kStore, 1024, 512, codes, scales, 0, 1),            # N != output length
        hip.StepGemv(G.kStore, 1024, 1024, codes, scales, 0, 2),           # vector index
        hip.StepGemv(7, 1024, 1024, codes, scales, 0, 1),                  # mode
        hip.StepGemv(G.kStore, 1024, 1024, codes.data_ptr() + 4, scales, 0, 1),  # codes alignment
        hip.StepGemv(G.kSwiglu, 1024, 1024, codes, scales, 0, 1),          # swiglu without up
        hip.StepGemv(G.kStore, 1024, 1024, codes, scales, 1, 0),           # reads vector 1 before any write (no data)
    ]
    for b in bad:
        assert hip.step_create_raw(v, [b]) == hip.BTF_ERR_ARGS, b
        assert hip.last_error()
    # quantized vector of a length that is not a multiple of 32
    v2 = [hip.StepVec(1000, x), hip.StepVec(1024, None)]
    assert hip.step_create_raw(v2, [hip.StepGemv(G.kStore, 896, 1024, codes, scales, 0, 1)]) == hip.BTF_ERR_ARGS
    # K beyond the widest supported input
    big = [hip.StepVec(24576, x), hip.StepVec(1024, None)]
    assert hip.step_create_raw(big, [hip.StepGemv(G.kStore, 24576, 1024, codes, scales, 0, 1)]) == hip.BTF_ERR_ARGS
    # output too tall for the per-workgroup partial buffer (nothing is launched)
    tall = [hip.StepVec(20480, x), hip.StepVec(131072, None)]
    assert hip.step_create_raw(tall, [hip.StepGemv(G.kStore, 20480, 131072, codes, scales, 0, 1)]) == \
        hip.BTF_ERR_ARGS
