"""GPU tests of whole-token step programs (btf_hip_step_create_ops): the
embedding lookup, every GEMV's full input prep (RMSNorm, tiled -> grouped
perm, signs, blockwise FWHT, Q8), the GEMV chain, the greedy pick and the
position counter, all in one launch.

Bars:
  * bit-exact against the same step launched op by op through the C ABI
    (launch_embed, launch_prep + launch_gemv per GEMV, launch_argmax,
    launch_pos_add -- the reference decoder's sequence,
    src/cuda/gpu_decoder.cu:401-421, 452-486): every vector, the token and
    the position;
  * the pieces within the oracle's bars: the embedding bit-exact, each
    sampled GEMV within rel-RMS 1e-3 (and max error 1e-3 of max |ref|) of the
    oracle's prep + emulator GEMV applied to the op's own fp32 input, and the
    token equal to the oracle's greedy pick over the logits.
The chain follows the reference decoder's attention layer and FFN: QKV reads
the residual through the attention norm; o adds W_o * (attention-output
stand-in) into the residual; gate/up read the residual through the FFN norm;
down adds into the residual; the output projection reads it through the
output norm.
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


def run_ops_sequential(hip, ops, vecs):
    """The program op by op through the C ABI, on torch tensors `vecs`."""
    torch = _torch()
    G = hip.GemvMode
    for op in ops:
        if isinstance(op, hip.StepEmbed):
            y = vecs[op.vec]
            hip.launch_embed(op.table_codes, op.table_scales, op.d_tok, 1, int(y.numel()), op.inv, y, stream())
        elif isinstance(op, hip.StepGemv):
            K = op.K
            act = hip.Q8Act(torch.empty(K, dtype=torch.int8, device="cuda"),
                            torch.empty(K // 32, dtype=torch.float32, device="cuda"),
                            torch.empty(K // 32, dtype=torch.int32, device="cuda"))
            hip.launch_prep(vecs[op.in_vec], K, 1, K, op.normw, op.eps, op.hx, None, 0, act, stream())
            y = vecs[op.out_vec]
            segs = [hip.GemvSeg(op.codes, op.scales, op.N, y, op.N)]
            if op.mode == G.kSwiglu:
                segs.append(hip.GemvSeg(op.up_codes, op.up_scales, op.N, None, 0))
            hip.launch_gemv(segs, K, 1, act, op.mode, stream())
        else:
            V = int(vecs[op.vec].numel())
            part = torch.empty(hip.argmax_part_bytes(V) // 4, dtype=torch.int32, device="cuda")
            hip.launch_argmax(vecs[op.vec], V, part, op.d_tok_out, stream())
            if op.d_pos is not None:
                hip.launch_pos_add(op.d_pos, 1, stream())
    torch.cuda.synchronize()


class Chain:
    """A small whole-token chain: embedding (inverse FWHT 1024 + signs),
    `layers` x (QKV with norm + FWHT 256 + signs; o += with FWHT 1024, the
    tiled -> grouped perm and signs; gate/up swiglu with norm + FWHT 1024;
    down += with FWHT 512 + signs), the output projection with norm + FWHT
    1024 + signs, the greedy pick and the position counter. The token the
    pick writes is the one the next launch embeds."""

    def __init__(self, hip, oracle, layers=2, E=2048, F=3072, NQ=1000, V=4000, seed=3):
        rng = np.random.default_rng(seed)
        # the embedding table has a row for every logit: the picked token is
        # the next launch's embedding row
        VT = V
        self.E, self.F, self.NQ, self.V, self.VT = E, F, NQ, V, VT
        mat = lambda N, K: random_mat(oracle, rng, N, K, scale=0.03)
        self.table = random_mat(oracle, rng, VT, E, scale=1.0)
        sgn = lambda n: np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float32)
        nrm = lambda n: (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        self.host = {"emb_signs": sgn(E), "out_norm": nrm(E), "out_signs": sgn(E)}
        self.att0 = (rng.standard_normal(E) * 2).astype(np.float32)
        self.layers = []
        for _ in range(layers):
            L = {"qkv": mat(NQ, E), "o": mat(E, E), "gate": mat(F, E), "up": mat(F, E), "down": mat(E, F),
                 "attn_norm": nrm(E), "ffn_norm": nrm(E), "qkv_signs": sgn(E), "o_signs": sgn(E),
                 "down_signs": sgn(F)}
            self.layers.append(L)
        self.out = mat(V, E)
        # device copies
        keep = []
        D = lambda a: keep.append(dev(a)) or keep[-1]
        self.tc, self.ts = D(self.table[0]), D(self.table[1])
        self.emb_inv = hip.Hx(block=1024, signs=D(self.host["emb_signs"]))
        self.dl = []
        for L in self.layers:
            d = {k: (D(v[0]), D(v[1])) if isinstance(v, tuple) else D(v) for k, v in L.items()}
            self.dl.append(d)
        self.dout = (D(self.out[0]), D(self.out[1]))
        self.dout_norm, self.dout_signs = D(self.host["out_norm"]), D(self.host["out_signs"])
        self._keep = keep
        self.hip = hip

    def ops(self, tok, tok_out, pos):
        """Vector slots: 0 residual, 1 qkv, 2 attention-output stand-in, 3 h, 4 logits."""
        hip, E, F, NQ, V = self.hip, self.E, self.F, self.NQ, self.V
        G = hip.GemvMode
        ops = [hip.StepEmbed(0, self.tc, self.ts, tok, self.emb_inv)]
        for d in self.dl:
            ops += [
                hip.StepGemv(G.kStore, E, NQ, *d["qkv"], 0, 1, normw=d["attn_norm"], eps=1e-6,
                             hx=hip.Hx(block=256, signs=d["qkv_signs"])),
                hip.StepGemv(G.kAdd, E, E, *d["o"], 2, 0, hx=hip.Hx(1024, 64, E // 128, 2, d["o_signs"])),
                hip.StepGemv(G.kSwiglu, E, F, *d["gate"], 0, 3, *d["up"], normw=d["ffn_norm"], eps=1e-6,
                             hx=hip.Hx(block=1024)),
                hip.StepGemv(G.kAdd, F, E, *d["down"], 3, 0, hx=hip.Hx(block=512, signs=d["down_signs"])),
            ]
        ops.append(hip.StepGemv(G.kStore, E, V, *self.dout, 0, 4, normw=self.dout_norm, eps=1e-6,
                                hx=hip.Hx(block=1024, signs=self.dout_signs)))
        ops.append(hip.StepArgmax(4, tok_out, pos))
        return ops

    def vectors(self):
        torch = _torch()
        z = lambda n: torch.zeros(n, dtype=torch.float32, device="cuda")
        t = [z(self.E), z(self.NQ), dev(self.att0), z(self.F), z(self.V)]
        return [self.hip.StepVec(int(v.numel()), v) for v in t], t


def test_whole_token_small_chain_matches_op_by_op_and_oracle(hip, oracle):
    """Three launches of a two-layer whole-token program, each decoding the
    token the previous one picked, bit-exact against the op-by-op launches
    (vectors, token, position); each launch's output projection within the
    oracle's bars and its token equal to the oracle's pick over the logits."""
    torch = _torch()
    C = Chain(hip, oracle)
    tok = dev(np.array([17], np.int32))
    pos = dev(np.array([5], np.int32))
    vecs, t = C.vectors()
    prog = hip.StepProgram(vecs, C.ops(tok, tok, pos))
    tok_s = dev(np.array([17], np.int32))
    pos_s = dev(np.array([5], np.int32))
    _, s = C.vectors()
    ops_s = C.ops(tok_s, tok_s, pos_s)
    toks = []
    for rep in range(3):
        t0 = int(host(tok)[0])
        prog.launch(stream())
        torch.cuda.synchronize()
        assert prog.error() == 0
        run_ops_sequential(hip, ops_s, s)
        for name, a, b in zip(("res", "qkv", "att", "h", "logits"), t, s):
            assert np.array_equal(host(a).view(np.uint32), host(b).view(np.uint32)), f"launch {rep}: {name}"
        assert int(host(tok)[0]) == int(host(tok_s)[0]), f"launch {rep}: token"
        assert int(host(pos)[0]) == 6 + rep == int(host(pos_s)[0])
        logits = host(t[4])
        assert np.isfinite(logits).all()
        assert int(host(tok)[0]) == oracle.argmax(logits)
        toks.append((t0, int(host(tok)[0])))
        # the output projection within the oracle's bars on the final residual
        res = host(t[0])
        q, d, s_, _ = oracle.prep(res[None, :], C.host["out_norm"], 1e-6, 1024, 0, 0, 0, C.host["out_signs"])
        assert_close_1e3(logits, oracle.gemv(C.out[0], C.out[1], C.E, q, d, s_)[0], f"launch {rep}: output projection")
    assert toks[1][0] == toks[0][1] and toks[2][0] == toks[1][1], "each launch embeds the previous pick"
    prog.close()


def test_whole_token_one_layer_pieces_vs_oracle(hip, oracle):
    """A one-layer whole-token program: the embedding bit-exact with the
    oracle, and QKV (norm + FWHT 256 + signs), o (FWHT + perm + signs, +=),
    gate/up (norm + FWHT, swiglu), down (FWHT 512 + signs, +=) and the output
    projection each within 1e-3 of the oracle applied to the op-by-op run's
    own inputs (bit-exact with the step's)."""
    torch = _torch()
    C = Chain(hip, oracle, layers=1, seed=9)
    tok = dev(np.array([123], np.int32))
    vecs, t = C.vectors()
    prog = hip.StepProgram(vecs, C.ops(tok, dev(np.array([0], np.int32)), None))
    prog.launch(stream())
    torch.cuda.synchronize()
    assert prog.error() == 0
    prog.close()
    # op by op, keeping each GEMV's fp32 input and old value
    _, s = C.vectors()
    ops = C.ops(dev(np.array([123], np.int32)), dev(np.array([0], np.int32)), None)
    seen = []
    for op in ops:
        if isinstance(op, hip.StepGemv):
            seen.append((host(s[op.in_vec]).copy(), host(s[op.out_vec]).copy()))
        run_ops_sequential(hip, [op], s)
        if isinstance(op, hip.StepGemv):
            seen[-1] += (host(s[op.out_vec]).copy(),)
    for name, a, b in zip(("res", "qkv", "att", "h", "logits"), t, s):
        assert np.array_equal(host(a).view(np.uint32), host(b).view(np.uint32)), name
    E, F = C.E, C.F
    L0 = C.layers[0]
    x0 = oracle.embed(C.table[0], C.table[1], np.array([123], np.int32), E, C.VT, 1024, C.host["emb_signs"])[0]
    assert np.array_equal(seen[0][0].view(np.uint32), x0.view(np.uint32)), "embedding"
    h = C.host
    specs = [  # (normw, block, perm (hd, nk, rep), signs, matrix, K, mode)
        (L0["attn_norm"], 256, (0, 0, 0), L0["qkv_signs"], L0["qkv"], E, "store"),
        (None, 1024, (64, E // 128, 2), L0["o_signs"], L0["o"], E, "add"),
        (L0["ffn_norm"], 1024, (0, 0, 0), None, (L0["gate"], L0["up"]), E, "swiglu"),
        (None, 512, (0, 0, 0), L0["down_signs"], L0["down"], F, "add"),
        (h["out_norm"], 1024, (0, 0, 0), h["out_signs"], C.out, E, "store"),
    ]
    for k, (normw, block, (hd, nk, rep), sg, W, K, mode) in enumerate(specs):
        xin, old, got = seen[k]
        q, d, s_, _ = oracle.prep(xin[None, :], normw, 1e-6, block, hd, nk, rep, sg)
        if mode == "swiglu":
            want = oracle.swiglu(oracle.gemv(W[0][0], W[0][1], K, q, d, s_), oracle.gemv(W[1][0], W[1][1], K, q, d, s_))[0]
        else:
            want = oracle.gemv(W[0], W[1], K, q, d, s_, y=old[None, :].copy() if mode == "add" else None,
                               add=mode == "add")[0]
        assert_close_1e3(got, want, f"op {k}")


def test_step_prep_nan_input_quantizes_as_launch_prep(hip, oracle):
    """A NaN in a prepped GEMV's input: the transform spreads it over its
    1024-value block, whose Q8 blocks are then all NaN and quantize to zero
    (the running max starts at 0, as in launch_prep). With the RMSNorm the
    whole input is NaN (the scale is). Bit-exact against launch_prep +
    launch_gemv, with finite outputs."""
    torch = _torch()
    G = hip.GemvMode
    rng = np.random.default_rng(92)
    K, N = 3072, 1024
    x = rng.standard_normal(K).astype(np.float32)
    x[1500] = np.nan
    W = random_mat(oracle, rng, N, K, scale=0.03)
    Wd = (dev(W[0]), dev(W[1]))
    signs = dev(np.where(rng.random(K) < 0.5, -1.0, 1.0).astype(np.float32))
    normw = dev((1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    for norm in (None, normw):
        ops = [hip.StepGemv(G.kStore, K, N, *Wd, 0, 1, normw=norm, eps=1e-6, hx=hip.Hx(block=1024, signs=signs))]
        vec = lambda: [dev(x), torch.zeros(N, dtype=torch.float32, device="cuda")]
        t = vec()
        prog = hip.StepProgram([hip.StepVec(int(v.numel()), v) for v in t], ops)
        prog.launch(stream())
        torch.cuda.synchronize()
        assert prog.error() == 0
        prog.close()
        s = vec()
        run_ops_sequential(hip, ops, s)
        got, want = host(t[1]), host(s[1])
        assert np.isfinite(got).all(), f"norm={norm is not None}"
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"norm={norm is not None}"


@pytest.mark.parametrize("block", [2, 4, 8, 16, 32, 64, 128, 256, 512, 1024])
def test_step_prep_every_transform_block(hip, oracle, block):
    """Each transform block size through the step program's prep (the
    strided slice layout puts stages len = 1..32 across lanes and 64..512 in
    the lane, so small blocks use only the cross-lane stages): a two-GEMV
    program -- the first with RMSNorm + signs + FWHT, the second with the
    tiled -> grouped gather + FWHT, over a 3-slice input (K = 3072) so that
    the slices land on different waves -- bit-exact with launch_prep +
    launch_gemv, and each GEMV within the oracle's bars."""
    torch = _torch()
    rng = np.random.default_rng(100 + block)
    K, N1, N2 = 3072, 3072, 640
    G = hip.GemvMode
    W1 = random_mat(oracle, rng, N1, K, scale=0.03)
    W2 = random_mat(oracle, rng, N2, N1, scale=0.03)
    normw = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    sg = np.where(rng.random(K) < 0.5, -1.0, 1.0).astype(np.float32)
    x0 = rng.standard_normal(K).astype(np.float32)
    keep = [dev(a) for a in (W1[0], W1[1], W2[0], W2[1], normw, sg)]
    c1, s1, c2, s2, dnw, dsg = keep
    hx1 = hip.Hx(block=block, signs=dsg)
    hx2 = hip.Hx(block, 64, 12, 4)  # gather: hd 64, nk 12, rep 4 -> 3072
    ops = [hip.StepGemv(G.kStore, K, N1, c1.data_ptr(), s1.data_ptr(), 0, 1, normw=dnw, eps=1e-6, hx=hx1),
           hip.StepGemv(G.kStore, N1, N2, c2.data_ptr(), s2.data_ptr(), 1, 2, hx=hx2)]

    def vectors():
        return [dev(x0), torch.zeros(N1, dtype=torch.float32, device="cuda"),
                torch.zeros(N2, dtype=torch.float32, device="cuda")]

    t = vectors()
    prog = hip.StepProgram([hip.StepVec(K, t[0]), hip.StepVec(N1, t[1]), hip.StepVec(N2, t[2])], ops)
    prog.launch(stream())
    torch.cuda.synchronize()
    assert prog.error() == 0
    prog.close()
    s = vectors()
    run_ops_sequential(hip, ops, s)
    for name, a, b in zip(("x", "y1", "y2"), t, s):
        assert np.array_equal(host(a).view(np.uint32), host(b).view(np.uint32)), f"block {block}: {name}"
    q, d, s_, _ = oracle.prep(x0[None, :], normw, 1e-6, block, 0, 0, 0, sg)
    assert_close_1e3(host(t[1]), oracle.gemv(W1[0], W1[1], K, q, d, s_)[0], f"block {block}: GEMV 1")
    q, d, s_, _ = oracle.prep(host(t[1])[None, :], None, 0.0, block, 64, 12, 4, None)
    assert_close_1e3(host(t[2]), oracle.gemv(W2[0], W2[1], N1, q, d, s_)[0], f"block {block}: GEMV 2")


def test_whole_token_27b_bench_program(hip, oracle):
    """The benchmark's whole-token program at the 27B shapes (the bench's own
    Setup and token_ops): the embedding (inverse FWHT 1024 + signs), 64 x
    (QKV with RMSNorm + FWHT 1024 + signs, o += with FWHT + signs, gate+up
    swiglu with RMSNorm + FWHT + signs, down += with FWHT + signs), the
    5120->248320 output projection with RMSNorm + FWHT + signs, the greedy
    pick and the position counter, in one launch.
      * Every vector, the token and the position are bit-exact against the
        same ops launched one by one (launch_embed, launch_prep + launch_gemv,
        launch_argmax, launch_pos_add: src/cuda/gpu_decoder.cu:401-421,
        452-486), over two launches (the second decodes the first's pick).
      * Sampled prepped ops of the op-by-op run -- layers 0, 31 and 63 and
        every 16th row of the output projection -- are within 1e-3 of the
        oracle's prep + emulator GEMV on their own fp32 inputs, and each
        launch's token is the oracle's greedy pick over its logits."""
    import os
    import sys
    torch = _torch()
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    if root not in sys.path:
        sys.path.insert(0, root)
    import bench
    L, E, F, V = bench.LAYERS, bench.E, bench.F, bench.V
    S = bench.Setup(hip, torch, L, with_embed=True)
    T = bench.Token(S, L)
    # the op-by-op twin: its own token, position and vectors
    z = lambda n: torch.zeros(n, dtype=torch.float32, device="cuda")
    tok2, pos2 = dev(np.array([T.tok0], np.int32)), torch.zeros(1, dtype=torch.int32, device="cuda")
    twin = [z(E), z(bench.QKV), T.att.clone(), z(F), z(V)]
    ops = T.ops()
    T.tok.fill_(T.tok0)
    T.pos.zero_()
    prog = hip.StepProgram(T.vecs(), ops)
    sample = (0, 31, 63)
    G = hip.GemvMode
    try:
        for launch in range(2):
            prog.launch(stream())
            torch.cuda.synchronize()
            assert prog.error() == 0
            seen = {}
            tops = bench.token_ops(hip, S.weights, L, tok2, pos2, T.hx,
                                   [tuple(T.nw(w) for w in ln) for ln in T.norm], T.signs,
                                   T.nw(T.out_norm), T.out_signs, T.emb_signs)
            gi = 0
            for op in tops:
                keep = isinstance(op, hip.StepGemv) and (gi // 4 in sample or gi == 4 * L)
                if keep:
                    seen[gi] = [host(twin[op.in_vec]).copy(), host(twin[op.out_vec]).copy()]
                run_ops_sequential(hip, [op], twin)
                if keep:
                    seen[gi].append(host(twin[op.out_vec]).copy())
                gi += isinstance(op, hip.StepGemv)
            for name, a, b in zip(("res", "qkv", "att", "h", "logits"), T.vecs(), twin):
                ga, gb = host(a.data), host(b)
                assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32)), \
                    f"launch {launch} {name}: step != op-by-op (max diff {np.max(np.abs(ga - gb)):.3e})"
            tok_step, tok_seq = int(host(T.tok)[0]), int(host(tok2)[0])
            assert tok_step == tok_seq and int(host(T.pos)[0]) == int(host(pos2)[0]) == launch + 1
            logits = host(T.logits)
            assert np.isfinite(logits).all()
            assert tok_step == oracle.argmax(logits)
            # sampled ops against the oracle
            for gi, (xin, old, got) in sorted(seen.items()):
                l, k = divmod(gi, 4)
                if gi == 4 * L:
                    normw, sg, key, K, mode = T.out_norm, T.out_signs, ("output", L), E, "store"
                else:
                    na, nf = T.norm[l]
                    sq, so_, sgu, sd = T.signs[l]
                    normw, sg, key, K, mode = [(na, sq, ("qkv", l), E, "store"), (None, so_, ("o", l), E, "add"),
                                               (nf, sgu, ("gate", l), E, "swiglu"),
                                               (None, sd, ("down", l), F, "add")][k]
                hn = host(normw) if normw is not None else None
                q, d, s_, _ = oracle.prep(xin[None, :], hn, 1e-6, 1024, 0, 0, 0, host(sg))
                if mode == "swiglu":
                    want = oracle.swiglu(oracle.gemv(*S.host_mat("gate", l), K, q, d, s_),
                                         oracle.gemv(*S.host_mat("up", l), K, q, d, s_))[0]
                    assert_close_1e3(got, want, f"launch {launch} layer {l} gate+up")
                elif gi == 4 * L:
                    rows = np.arange(0, V, 16)
                    c, sc = S.host_mat("output", L)
                    want = oracle.gemv(np.ascontiguousarray(c[rows]), np.ascontiguousarray(sc[rows]), K, q, d, s_)[0]
                    assert_close_1e3(got[rows], want, f"launch {launch} output projection (every 16th row)")
                else:
                    want = oracle.gemv(*S.host_mat(*key), K, q, d, s_, y=old[None, :].copy() if mode == "add" else None,
                                       add=mode == "add")[0]
                    assert_close_1e3(got, want, f"launch {launch} layer {l} {key[0]}")
    finally:
        prog.close()
