#!/usr/bin/env python3
"""Benchmark of the fused ternary matmul path on one MI355X.

Default workload: the 27B-scale decode-step weight sweep at batch 1 --
64 layers x (QKV 5120->7168, o 5120->5120, gate+up 5120->17408 as one
swiglu GEMV, down 17408->5120 (+= residual)) plus the
untied output projection 5120->248,320, every GEMV fed by the Q8 quantize of
its input. 5,952,839,680 B of packed codes + scales per step, seeded
synthetic weights (trits p = 0.3/0.4/0.3, fp16 scales U[0.01, 0.05]) and
N(0,1) activations.

Data flow of a layer (the same for both engines): QKV reads the residual
stream (written by the previous layer's down), o writes W_o * (attention-
output stand-in) to x, gate/up read x, down adds W_down * h into the
residual; the output projection reads the final residual. Every GEMV but o
waits for the one before it, as in the decoder; o's input stands in for
the attention output, which is outside this path. (Without the model's
RMSNorm, o adding into the residual that gate/up read would grow
quadratically and overflow; o storing into x keeps every value finite.)

Engines (at batch 1 all three are timed; the fastest gives `value`):
  step : the whole GEMV chain as ONE persistent launch (btf_hip_step_*),
         each op's Q8 input produced by its producer;
  chain: one hipGraph of GEMV launches with most quantizes fused in
         (btf_hip_launch_gemv_ex: QKV, o and gate/up quantize their own fp32
         inputs; down and the output projection keep a quantize launch);
  graph: one hipGraph of quantize + GEMV launches (2 per GEMV), as the
         reference decoder captures its step.
The step and chain engines' outputs are checked bit-exact against the graph
engine's before timing ("verified" in the JSON line). All engines are rated
on the same algorithmic bytes of the workload.

`value` = algorithmic bytes of one step / measured step time (weights,
activations and outputs already resident in HBM), in GB/s.
`roofline` = the dominant kernel's algorithmic bytes per launch over its
average launch time from HIP events on the stream it runs on (the step
engine: the step kernel itself, one launch per step).
`cpu_baseline` = the reference's CPU emulator GEMV (oracle/_ref, built from
the reference sources) or the oracle port, timed on this host on a bounded
sample of the same workload (about --cpu-budget seconds).

Other workloads (--workload layer|batched|prefill) report the other
configurations the same way; they are measurement aids, the default line is
the sweep.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "bonsai-ternary-fast_amd")
ORACLE = os.path.join(ROOT, "oracle")

METRIC = "ternary GEMV HBM GB/s (% of 8 TB/s) at 27B shapes; implied batch-1 tok/s"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
E, F, QKV, V, LAYERS = 5120, 17408, 7168, 248320, 64


def under_profiler() -> bool:
    """Is this process running under rocprofv3 (its tool library preloaded)?"""
    return bool(os.environ.get("ROCPROFILER_LIBRARY_CTOR")) or "rocprofiler" in os.environ.get("LD_PRELOAD", "")


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def align(n, a=256):
    return (n + a - 1) // a * a


def gemv_bytes(N, K, M, out_rw=1, nmat=1):
    """Algorithmic bytes of one GEMV launch: weights (codes + scales) of every
    matrix, the Q8 rows (q + d + s), the outputs (read too when added)."""
    return nmat * (N * K // 4 + N * K // 64) + M * (K + K // 4) + 4 * M * N * out_rw


def b3_bytes(N, K, M, out_rw=1, nmat=1):
    """The same GEMV reading PTQ1_0 blocks directly: 28 B per 128 weights."""
    return nmat * (N * K // 128 * 28) + M * (K + K // 4) + 4 * M * N * out_rw


def prep_bytes(K, M):
    return M * (4 * K + K + K // 4)


SWEEP_VECS = (E, QKV, E, E, F, V)  # the sweep program's vector slots (the logits only with the output)
TOKEN_VECS = (E, QKV, E, F, V)     # the whole-token program's vector slots


def sweep_ops(hip, w, layers, with_output=True):
    """The sweep's step program (batch 1), in the op-by-op order: every op
    waits for the one before it, except o, whose input stands in for the
    attention output. w(name, layer) -> (codes, scales) addresses. Vector
    slots: 0 residual, 1 qkv, 2 attention-output stand-in, 3 x, 4 h, 5 logits."""
    G = hip.GemvMode
    ops = []
    for l in range(layers):
        gc, gs = w("gate", l)
        uc, us = w("up", l)
        ops.append(hip.StepGemv(G.kStore, E, QKV, *w("qkv", l), 0, 1))
        ops.append(hip.StepGemv(G.kStore, E, E, *w("o", l), 2, 3))
        ops.append(hip.StepGemv(G.kSwiglu, E, F, gc, gs, 3, 4, uc, us))
        ops.append(hip.StepGemv(G.kAdd, F, E, *w("down", l), 4, 0))
    if with_output:
        ops.append(hip.StepGemv(G.kStore, E, V, *w("output", layers), 0, 5))
    return ops


def token_ops(hip, w, layers, tok, pos, hx, norms, signs, out_norm, out_signs, emb_signs):
    """The whole-token step program: embedding, 64 x (QKV, o, gate+up, down)
    each with its prep, the output projection and the greedy pick.
    hx(signs) -> the transform (or None); norms[l] = (attention, FFN) RMSNorm
    weights (or None); signs[l] = the qkv, o, gate/up and down inputs' signs.
    Vector slots: 0 residual, 1 qkv, 2 attention-output stand-in, 3 h, 4 logits."""
    G = hip.GemvMode
    ops = [hip.StepEmbed(0, *w("embed", layers), tok, hx(emb_signs))]
    for l in range(layers):
        na, nf = norms[l]
        sq, so_, sgu, sd = signs[l]
        ops += [hip.StepGemv(G.kStore, E, QKV, *w("qkv", l), 0, 1, normw=na, eps=1e-6, hx=hx(sq)),
                hip.StepGemv(G.kAdd, E, E, *w("o", l), 2, 0, hx=hx(so_)),
                hip.StepGemv(G.kSwiglu, E, F, *w("gate", l), 0, 3, *w("up", l), normw=nf, eps=1e-6, hx=hx(sgu)),
                hip.StepGemv(G.kAdd, F, E, *w("down", l), 3, 0, hx=hx(sd))]
    ops.append(hip.StepGemv(G.kStore, E, V, *w("output", layers), 0, 4, normw=out_norm, eps=1e-6, hx=hx(out_signs)))
    ops.append(hip.StepArgmax(4, tok, pos))
    return ops


class Setup:
    """Weights of every matrix of the sweep, resident in one device arena."""

    def __init__(self, hip, torch, layers, seed=0, keep_src=False, with_embed=False):
        """keep_src: also keep every matrix's PTQ1_0 rows resident (for the
        GEMV that reads them directly). with_embed: also a packed embedding
        table of the output projection's shape (V x 5120, matrix id 321)."""
        self.hip, self.torch = hip, torch
        shapes = []  # (name, layer, N, K, matrix id)
        for l in range(layers):
            shapes += [("qkv", l, QKV, E, 5 * l), ("o", l, E, E, 5 * l + 1), ("gate", l, F, E, 5 * l + 2),
                       ("up", l, F, E, 5 * l + 3), ("down", l, E, F, 5 * l + 4)]
        shapes.append(("output", layers, V, E, 5 * 64))
        if with_embed:
            shapes.append(("embed", layers, V, E, 5 * 64 + 1))
        off, self.mats = 0, {}
        for name, l, N, K, mid in shapes:
            co = off
            off = align(off + N * K // 4)
            so = off
            off = align(off + N * K // 64)
            self.mats[(name, l)] = (N, K, mid, co, so)
        self.arena_bytes = off
        self.arena = torch.empty(off, dtype=torch.uint8, device="cuda")
        base = self.arena.data_ptr()
        self.src_off, soff = {}, 0
        for key, (N, K, _, _, _) in self.mats.items():
            if key[0] == "embed":
                continue
            self.src_off[key] = soff
            soff = align(soff + N * K // 128 * 28)
        self.src = torch.empty(soff if keep_src else 0, dtype=torch.uint8, device="cuda")
        maxblk = max(N * K // 128 for N, K, _, _, _ in self.mats.values())
        stage = torch.empty(maxblk * 28 if (not keep_src or with_embed) else 0, dtype=torch.uint8, device="cuda")
        st = torch.cuda.current_stream().cuda_stream
        t0 = time.time()
        for (name, l), (N, K, mid, co, so) in self.mats.items():
            nb = N * K // 128
            src = self.src.data_ptr() + self.src_off[(name, l)] if keep_src and name != "embed" else stage.data_ptr()
            hip.gen_ptq1_0(seed, mid, 0, nb, src, st)
            hip.launch_repack(src, nb, base + co, base + so, st)
        torch.cuda.synchronize()
        self.setup_s = time.time() - t0
        self.weight_bytes = sum(N * K // 4 + N * K // 64 for (name, _), (N, K, _, _, _) in self.mats.items()
                                if name != "embed")
        del stage

    def weights(self, name, l):
        """(codes, scales) device addresses of one matrix."""
        N, K, mid, co, so = self.mats[(name, l)]
        base = self.arena.data_ptr()
        return base + co, base + so

    def seg(self, name, l, y, ldy):
        N, K, mid, co, so = self.mats[(name, l)]
        base = self.arena.data_ptr()
        return self.hip.GemvSeg(base + co, base + so, N, y, ldy)

    def src_seg(self, name, l, y, ldy):
        """The matrix as PTQ1_0 rows (Setup(keep_src=True))."""
        N, K, mid, co, so = self.mats[(name, l)]
        return self.hip.GemvSeg(self.src.data_ptr() + self.src_off[(name, l)], None, N, y, ldy)

    def host_mat(self, name, l):
        """(codes, scales) numpy copies of one matrix."""
        import numpy as np
        N, K, mid, co, so = self.mats[(name, l)]
        codes = self.arena[co:co + N * K // 4].cpu().numpy().reshape(N, K // 4)
        scales = self.arena[so:so + N * K // 64].cpu().numpy().view(np.uint16).reshape(N, K // 128)
        return codes, scales


class Step:
    """One decode step (or M-row batch) of quantize + GEMV launches."""

    def __init__(self, S: Setup, M, layers, with_output=True):
        import numpy as np
        hip, torch = S.hip, S.torch
        self.S, self.M, self.layers = S, M, layers
        rng = np.random.default_rng(0)
        dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
        self.x = torch.zeros((M, E), dtype=torch.float32, device="cuda")  # FFN input (o-proj output)
        self.xo = dev(rng.standard_normal((M, E)).astype(np.float32))    # attention-output stand-in
        self.res0 = rng.standard_normal((M, E)).astype(np.float32)       # residual stream at step start
        self.res = dev(self.res0)
        self.qkv = torch.zeros((M, QKV), dtype=torch.float32, device="cuda")
        self.h = torch.zeros((M, F), dtype=torch.float32, device="cuda")
        self.logits = torch.zeros((1, V), dtype=torch.float32, device="cuda") if with_output else None
        Kmax = F
        self.act = hip.Q8Act(torch.zeros((M, Kmax), dtype=torch.int8, device="cuda"),
                             torch.zeros((M, Kmax // 32), dtype=torch.float32, device="cuda"),
                             torch.zeros((M, Kmax // 32), dtype=torch.int32, device="cuda"))
        self.with_output = with_output
        # the batched chain with the quantizes in the producers' epilogues (layer_qchain):
        # Q8 rows of the residual, the attention-output stand-in, x and h
        self.qa = None
        if 3 <= M <= 32:
            q8 = lambda K: hip.Q8Act(torch.zeros((M, K), dtype=torch.int8, device="cuda"),
                                     torch.zeros((M, K // 32), dtype=torch.float32, device="cuda"),
                                     torch.zeros((M, K // 32), dtype=torch.int32, device="cuda"))
            self.qa = {"res": q8(E), "xo": q8(E), "x": q8(E), "h": q8(F)}
        # algorithmic bytes
        b_gemv = {"qkv": gemv_bytes(QKV, E, M), "o": gemv_bytes(E, E, M), "gateup": gemv_bytes(F, E, M, 1, 2),
                  "down": gemv_bytes(E, F, M, 2), "output": gemv_bytes(V, E, 1)}
        self.kind_bytes = b_gemv
        b_b3 = {"qkv": b3_bytes(QKV, E, M), "o": b3_bytes(E, E, M), "gateup": b3_bytes(F, E, M, 1, 2),
                "down": b3_bytes(E, F, M, 2), "output": b3_bytes(V, E, 1)}
        self.kind_bytes_b3 = b_b3
        self.b3_total_bytes = layers * (b_b3["qkv"] + b_b3["o"] + b_b3["gateup"] + b_b3["down"]) + \
            (b_b3["output"] + prep_bytes(E, 1) if with_output else 0) + \
            layers * (3 * prep_bytes(E, M) + prep_bytes(F, M))
        self.gemv_bytes = layers * (b_gemv["qkv"] + b_gemv["o"] + b_gemv["gateup"] + b_gemv["down"])
        self.prep_bytes = layers * (3 * prep_bytes(E, M) + prep_bytes(F, M))
        if with_output:
            self.gemv_bytes += b_gemv["output"]
            self.prep_bytes += prep_bytes(E, 1)
        self.total_bytes = self.gemv_bytes + self.prep_bytes
        self.weight_bytes = layers * sum((QKV * E, E * E, 2 * F * E, E * F)) * 17 // 64
        if with_output:
            self.weight_bytes += V * E * 17 // 64
        self.flops = 2 * M * layers * (QKV * E + E * E + 2 * F * E + E * F) + (2 * V * E if with_output else 0)

    def prep(self, x, K, M, st):
        self.S.hip.launch_prep(x, K, M, K, None, 0.0, None, None, 0, self.act, st)

    def gemv(self, segs, K, M, mode, st):
        self.S.hip.launch_gemv(segs, K, M, self.act, mode, st)

    def layer(self, l, st):
        S, M, G = self.S, self.M, self.S.hip.GemvMode
        self.prep(self.res, E, M, st)
        self.gemv([S.seg("qkv", l, self.qkv, QKV)], E, M, G.kStore, st)
        self.prep(self.xo, E, M, st)
        self.gemv([S.seg("o", l, self.x, E)], E, M, G.kStore, st)
        self.prep(self.x, E, M, st)
        self.gemv([S.seg("gate", l, self.h, F), S.seg("up", l, None, 0)], E, M, G.kSwiglu, st)
        self.prep(self.h, F, M, st)
        self.gemv([S.seg("down", l, self.res, E)], F, M, G.kAdd, st)

    def layer_chain(self, l, st):
        """The same layer with most quantizes inside the GEMV launches
        (btf_hip_launch_gemv_ex): QKV, o and gate/up quantize their fp32
        inputs themselves; down's 17408-wide input keeps its own quantize
        launch (re-reading it in every GEMV workgroup costs more)."""
        S, M, G, hip = self.S, self.M, self.S.hip.GemvMode, self.S.hip
        hip.launch_gemv_ex([S.seg("qkv", l, self.qkv, QKV)], E, M, x=self.res, ldx=E, mode=G.kStore, stream=st)
        hip.launch_gemv_ex([S.seg("o", l, self.x, E)], E, M, x=self.xo, ldx=E, mode=G.kStore, stream=st)
        hip.launch_gemv_ex([S.seg("gate", l, self.h, F), S.seg("up", l, None, 0)], E, M, x=self.x, ldx=E,
                           mode=G.kSwiglu, stream=st)
        self.prep(self.h, F, M, st)
        self.gemv([S.seg("down", l, self.res, E)], F, M, G.kAdd, st)

    def layer_qchain(self, l, st):
        """The layer of `layer` for a batch (3..32 rows) with the quantizes in
        the producers' epilogues (btf_hip_launch_gemv_ex with a Q8 output,
        one int8-MFMA launch each): o, gate+up and down write the Q8 rows of
        x, h and the residual for the GEMM after them; the attention-output
        stand-in keeps its own quantize launch. 5 launches instead of 8."""
        S, M, G, hip, qa = self.S, self.M, self.S.hip.GemvMode, self.S.hip, self.qa
        hip.launch_prep(self.xo, E, M, E, None, 0.0, None, None, 0, qa["xo"], st)
        hip.launch_gemv([S.seg("qkv", l, self.qkv, QKV)], E, M, qa["res"], G.kStore, st)
        hip.launch_gemv_ex([S.seg("o", l, self.x, E)], E, M, a=qa["xo"], mode=G.kStore, out=qa["x"], stream=st)
        hip.launch_gemv_ex([S.seg("gate", l, self.h, F), S.seg("up", l, None, 0)], E, M, a=qa["x"],
                           mode=G.kSwiglu, out=qa["h"], stream=st)
        hip.launch_gemv_ex([S.seg("down", l, self.res, E)], F, M, a=qa["h"], mode=G.kAdd, out=qa["res"], stream=st)

    def run_qchain(self, st):
        self.S.hip.launch_prep(self.res, E, self.M, E, None, 0.0, None, None, 0, self.qa["res"], st)
        for l in range(self.layers):
            self.layer_qchain(l, st)

    def run_chain(self, st):
        for l in range(self.layers):
            self.layer_chain(l, st)
        if self.with_output:
            self.prep(self.res, E, 1, st)
            self.gemv([self.S.seg("output", self.layers, self.logits, V)], E, 1, self.S.hip.GemvMode.kStore, st)

    def run(self, st):
        for l in range(self.layers):
            self.layer(l, st)
        if self.with_output:
            self.prep(self.res, E, 1, st)
            self.gemv([self.S.seg("output", self.layers, self.logits, V)], E, 1, self.S.hip.GemvMode.kStore, st)

    def layer_b3(self, l, st):
        """The layer of `layer` on the PTQ1_0 rows, read directly."""
        S, M, G, hip = self.S, self.M, self.S.hip.GemvMode, self.S.hip
        self.prep(self.res, E, M, st)
        hip.launch_gemv_ptq1_0([S.src_seg("qkv", l, self.qkv, QKV)], E, M, self.act, G.kStore, st)
        self.prep(self.xo, E, M, st)
        hip.launch_gemv_ptq1_0([S.src_seg("o", l, self.x, E)], E, M, self.act, G.kStore, st)
        self.prep(self.x, E, M, st)
        hip.launch_gemv_ptq1_0([S.src_seg("gate", l, self.h, F), S.src_seg("up", l, None, 0)], E, M, self.act,
                               G.kSwiglu, st)
        self.prep(self.h, F, M, st)
        hip.launch_gemv_ptq1_0([S.src_seg("down", l, self.res, E)], F, M, self.act, G.kAdd, st)

    def run_b3(self, st):
        for l in range(self.layers):
            self.layer_b3(l, st)
        if self.with_output:
            self.prep(self.res, E, 1, st)
            self.S.hip.launch_gemv_ptq1_0([self.S.src_seg("output", self.layers, self.logits, V)], E, 1, self.act,
                                          self.S.hip.GemvMode.kStore, st)

    def kind_launch_b3(self, kind, l, st):
        S, M, G, hip = self.S, self.M, self.S.hip.GemvMode, self.S.hip
        segs, K, mode = {
            "qkv": ([S.src_seg("qkv", l, self.qkv, QKV)], E, G.kStore),
            "o": ([S.src_seg("o", l, self.x, E)], E, G.kStore),
            "gateup": ([S.src_seg("gate", l, self.h, F), S.src_seg("up", l, None, 0)], E, G.kSwiglu),
            "down": ([S.src_seg("down", l, self.res, E)], F, G.kAdd),
            "output": ([S.src_seg("output", self.layers, self.logits, V)], E, G.kStore)}[kind]
        hip.launch_gemv_ptq1_0(segs, K, 1 if kind == "output" else M, self.act, mode, st)

    def reset(self):
        self.res.copy_(self.S.torch.from_numpy(self.res0).cuda())

    def program(self):
        """The same chain as one step program (batch 1). Vector slots:
        0 residual, 1 qkv, 2 attention-output stand-in, 3 x, 4 h, 5 logits."""
        hip, S, G = self.S.hip, self.S, self.S.hip.GemvMode
        assert self.M == 1
        vecs = [hip.StepVec(E, self.res), hip.StepVec(QKV, self.qkv), hip.StepVec(E, self.xo),
                hip.StepVec(E, self.x), hip.StepVec(F, self.h)]
        if self.with_output:
            vecs.append(hip.StepVec(V, self.logits))
        return hip.StepProgram(vecs, sweep_ops(hip, S.weights, self.layers, self.with_output))

    def kind_launch(self, kind, l, st, fused=False):
        """One GEMV launch of a given kind (for per-kernel timing); fused: the
        launch of the chain engine (quantizes fused in)."""
        S, M, G = self.S, self.M, self.S.hip.GemvMode
        if fused and M > 1:  # as in run_qchain
            qa, hip = self.qa, S.hip
            if kind == "qkv":
                hip.launch_gemv([S.seg("qkv", l, self.qkv, QKV)], E, M, qa["res"], G.kStore, st)
            elif kind == "o":
                hip.launch_gemv_ex([S.seg("o", l, self.x, E)], E, M, a=qa["xo"], mode=G.kStore, out=qa["x"], stream=st)
            elif kind == "gateup":
                hip.launch_gemv_ex([S.seg("gate", l, self.h, F), S.seg("up", l, None, 0)], E, M, a=qa["x"],
                                   mode=G.kSwiglu, out=qa["h"], stream=st)
            else:
                hip.launch_gemv_ex([S.seg("down", l, self.res, E)], F, M, a=qa["h"], mode=G.kAdd, out=qa["res"],
                                   stream=st)
            return
        if fused and kind in ("qkv", "o", "gateup"):  # as in run_chain
            x, segs, mode = {
                "qkv": (self.res, [S.seg("qkv", l, self.qkv, QKV)], G.kStore),
                "o": (self.xo, [S.seg("o", l, self.x, E)], G.kStore),
                "gateup": (self.x, [S.seg("gate", l, self.h, F), S.seg("up", l, None, 0)], G.kSwiglu)}[kind]
            S.hip.launch_gemv_ex(segs, E, M, x=x, ldx=E, mode=mode, stream=st)
            return
        if kind == "qkv":
            self.gemv([S.seg("qkv", l, self.qkv, QKV)], E, M, G.kStore, st)
        elif kind == "o":
            self.gemv([S.seg("o", l, self.x, E)], E, M, G.kStore, st)
        elif kind == "gateup":
            self.gemv([S.seg("gate", l, self.h, F), S.seg("up", l, None, 0)], E, M, G.kSwiglu, st)
        elif kind == "down":
            self.gemv([S.seg("down", l, self.res, E)], F, M, G.kAdd, st)
        else:
            self.gemv([S.seg("output", self.layers, self.logits, V)], E, 1, G.kStore, st)


class Token:
    """One whole decode step of the 27B shapes at batch 1, as the reference
    decoder runs it (src/cuda/gpu_decoder.cu:401-421, 452-486) minus the
    attention itself: the embedding lookup of the current token (inverse
    FWHT 1024 + signs), 64 x (QKV through the attention RMSNorm + FWHT 1024 +
    signs; o += W_o * (attention-output stand-in through FWHT 1024 + signs);
    gate/up swiglu through the FFN RMSNorm + FWHT 1024 + signs; down += through
    FWHT 1024 + signs), the output projection through the output RMSNorm +
    FWHT 1024 + signs, the greedy pick into the token and the position
    counter. Each step decodes the token the previous one picked. Seeded norm
    weights N(1, 0.1) and random signs; the weights are the sweep's."""

    BLOCK = 1024

    def __init__(self, S: Setup, layers, seed=1, prep="full"):
        """prep: "full" (the decoder's RMSNorms and transforms), or for
        measurement "hx" (transforms only), "norm" (norms only), "none"."""
        import numpy as np
        hip, torch = S.hip, S.torch
        self.S, self.layers = S, layers
        self.use_norm = prep in ("full", "norm")
        self.use_hx = prep in ("full", "hx")
        rng = np.random.default_rng(seed)
        dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
        sg = lambda n: dev(np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float32))
        nw = lambda n: dev((1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32))
        self.norm = [(nw(E), nw(E)) for _ in range(layers)]              # attention, FFN
        self.signs = [(sg(E), sg(E), sg(E), sg(F)) for _ in range(layers)]  # qkv, o, gate/up, down inputs
        self.out_norm, self.out_signs, self.emb_signs = nw(E), sg(E), sg(E)
        z = lambda n: torch.zeros(n, dtype=torch.float32, device="cuda")
        self.res, self.qkv, self.h, self.logits = z(E), z(QKV), z(F), z(V)
        self.att = dev((rng.standard_normal(E) * 2).astype(np.float32))
        self.tok0 = 7
        self.tok = dev(np.array([self.tok0], np.int32))
        self.pos = torch.zeros(1, dtype=torch.int32, device="cuda")
        self.act = hip.Q8Act(torch.zeros(F, dtype=torch.int8, device="cuda"),
                             torch.zeros(F // 32, dtype=torch.float32, device="cuda"),
                             torch.zeros(F // 32, dtype=torch.int32, device="cuda"))
        self.part = torch.zeros(hip.argmax_part_bytes(V) // 4, dtype=torch.int32, device="cuda")
        # algorithmic bytes: the embedding row and its output; per GEMV the
        # weights, the prep (fp32 input, norm weights, signs, the Q8 written
        # and read) and the outputs; the logits read by the pick
        prep_b = lambda K, norm: 4 * K + 2 * (K + K // 4) + 4 * K + (4 * K if norm else 0)
        per_layer = (gemv_bytes(QKV, E, 1) - (E + E // 4) + prep_b(E, True) +
                     gemv_bytes(E, E, 1, 2) - (E + E // 4) + prep_b(E, False) +
                     gemv_bytes(F, E, 1, 1, 2) - (E + E // 4) + prep_b(E, True) +
                     gemv_bytes(E, F, 1, 2) - (F + F // 4) + prep_b(F, False))
        self.total_bytes = (E // 4 + E // 64 + 4 * E + layers * per_layer +
                            gemv_bytes(V, E, 1) - (E + E // 4) + prep_b(E, True) + 4 * V)

    def reset(self):
        self.tok.fill_(self.tok0)
        self.pos.zero_()

    def hx(self, signs):
        return self.S.hip.Hx(block=self.BLOCK, signs=signs) if self.use_hx else None

    def nw(self, w):
        return w if self.use_norm else None

    def ops(self):
        """The step program's ops. Vector slots: 0 residual, 1 qkv, 2
        attention-output stand-in, 3 h, 4 logits."""
        return token_ops(self.S.hip, self.S.weights, self.layers, self.tok, self.pos, self.hx,
                         [tuple(self.nw(w) for w in ln) for ln in self.norm], self.signs,
                         self.nw(self.out_norm), self.out_signs, self.emb_signs)

    def vecs(self):
        hip = self.S.hip
        return [hip.StepVec(E, self.res), hip.StepVec(QKV, self.qkv), hip.StepVec(E, self.att),
                hip.StepVec(F, self.h), hip.StepVec(V, self.logits)]

    def run(self, st):
        """The same step as the reference decoder's launches: launch_embed,
        launch_prep + launch_gemv per GEMV, launch_argmax, launch_pos_add."""
        hip, S, G = self.S.hip, self.S, self.S.hip.GemvMode
        N_, K_, _, co, so = S.mats[("embed", self.layers)]
        base = S.arena.data_ptr()
        hip.launch_embed(base + co, base + so, self.tok, 1, E, self.hx(self.emb_signs), self.res, st)
        prep = lambda x, K, normw, signs: hip.launch_prep(x, K, 1, K, normw, 1e-6 if normw is not None else 0.0,
                                                          self.hx(signs), None, 0, self.act, st)
        for l in range(self.layers):
            na, nf = self.norm[l]
            sq, so_, sgu, sd = self.signs[l]
            prep(self.res, E, self.nw(na), sq)
            hip.launch_gemv([S.seg("qkv", l, self.qkv, QKV)], E, 1, self.act, G.kStore, st)
            prep(self.att, E, None, so_)
            hip.launch_gemv([S.seg("o", l, self.res, E)], E, 1, self.act, G.kAdd, st)
            prep(self.res, E, self.nw(nf), sgu)
            hip.launch_gemv([S.seg("gate", l, self.h, F), S.seg("up", l, None, 0)], E, 1, self.act, G.kSwiglu, st)
            prep(self.h, F, None, sd)
            hip.launch_gemv([S.seg("down", l, self.res, E)], F, 1, self.act, G.kAdd, st)
        prep(self.res, E, self.nw(self.out_norm), self.out_signs)
        hip.launch_gemv([S.seg("output", self.layers, self.logits, V)], E, 1, self.act, G.kStore, st)
        hip.launch_argmax(self.logits, V, self.part, self.tok, st)
        hip.launch_pos_add(self.pos, 1, st)


def run_token(S: Setup, hip, torch, layers, steps, warmup, prep="full", traffic_tab=None):
    """The whole decode step: one step-program launch per token, checked
    bit-exact against the op-by-op launches (vectors, token, position), then
    both timed over `steps` tokens (each decoding the previous pick)."""
    import numpy as np
    T = Token(S, layers, prep=prep)
    t0 = time.time()
    prog = hip.StepProgram(T.vecs(), T.ops())
    log(f"whole-token program built in {time.time() - t0:.2f} s")
    try:
        outs = []
        for run in (T.run, lambda st: prog.launch(st)):
            T.reset()
            torch.cuda.synchronize()
            run(torch.cuda.current_stream().cuda_stream)
            torch.cuda.synchronize()
            outs.append([t.cpu().numpy().copy() for t in (T.res, T.qkv, T.h, T.logits, T.tok, T.pos)])
        if prog.error():
            raise SystemExit("whole-token program reported a timeout")
        if prep != "full" and not all(np.isfinite(a).all() for a in outs[0][:4]):
            # without the RMSNorms the residual grows layer by layer until it
            # overflows; the quantize of non-finite values is not a defined
            # result to compare (a measurement mode only)
            log(f"whole-token program (prep {prep}): the residual overflows without norms; not compared")
        else:
            for name, a, b in zip(("res", "qkv", "h", "logits", "token", "pos"), *outs):
                if not np.array_equal(a.view(np.uint32), b.view(np.uint32)):
                    raise SystemExit(f"whole-token program != op-by-op launches ({name})")
            if not np.isfinite(outs[0][3]).all():
                raise SystemExit("whole-token logits are not finite")
            log(f"whole-token program vs op-by-op launches: bit-exact (token {int(outs[0][4][0])})")
        T.reset()
        ms = time_program(hip, torch, prog, steps, warmup)
    finally:
        prog.close()
    T.reset()
    gms = time_graph(hip, torch, T.run, steps, warmup)
    gbs = T.total_bytes / (ms * 1e-3) / 1e9
    tr = (traffic_tab or {}).get("token/step_kernel") if prep == "full" and layers == LAYERS else None
    log(f"whole token: step program {ms:.4f} ms ({1e3 / ms:.1f} tok/s, {gbs:.1f} GB/s), "
        f"op-by-op graph {gms:.4f} ms ({1e3 / gms:.1f} tok/s)")
    return {
        "workload": f"whole decode step of the 27B shapes at batch 1: embedding lookup (inverse FWHT 1024 + signs), "
                    f"{layers} x (QKV, o, gate+up swiglu, down) each with launch_prep's RMSNorm / FWHT 1024 / signs, "
                    "output 5120->248320 with RMSNorm + FWHT, greedy pick, position counter; each token decodes "
                    "the previous pick",
        "ms_per_token": round(ms, 4), "tok_s": round(1e3 / ms, 2), "bytes_per_token": T.total_bytes,
        "graph_ms_per_token": round(gms, 4), "graph_tok_s": round(1e3 / gms, 2),
        "kernels_per_token": {"step": 1, "graph": 2 + 2 * (4 * layers + 1) + 2},
        "verified": "step program bit-exact vs the op-by-op launches (vectors, token, position)",
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": tr["hbm_bytes"] if tr else None,
                     "traffic_source": tr["source"] if tr else None,
                     "kernel": "step_kernel<true> (the whole token, one launch)", "bytes_per_launch": T.total_bytes,
                     "avg_launch_us": round(ms * 1e3, 3)},
    }


def kind_timings(step, layers, steps, fused=False, b3=False):
    """Per-kind GEMV launch times: a graph of one launch per layer (distinct
    weights, far beyond the 256 MB MALL) -> the average per launch."""
    hip, torch = step.S.hip, step.S.torch
    kinds = ["qkv", "o", "gateup", "down"] + (["output"] if step.with_output else [])
    per = {}
    launch = step.kind_launch_b3 if b3 else (lambda kind, l, st: step.kind_launch(kind, l, st, fused))
    table = step.kind_bytes_b3 if b3 else step.kind_bytes
    for kind in kinds:
        reps = 1 if kind == "output" else layers
        fn = (lambda st, kind=kind: launch(kind, 0, st)) if kind == "output" else \
             (lambda st, kind=kind: [launch(kind, l, st) for l in range(layers)])
        kms = time_graph(hip, torch, fn, max(3, steps // 2), 1)
        avg_us = kms * 1e3 / reps
        b = table[kind]
        per[kind] = {"avg_us": round(avg_us, 3), "bytes": b, "GBs": round(b / (avg_us * 1e-6) / 1e9, 1),
                     "launches_per_step": 1 if kind == "output" else layers}
    return per


def gemm_roofline(step, per, traffic_tab=None, fused=False):
    """The dominant GEMV/GEMM kind of a batched step and its roofline (HBM
    below 33 rows, int8 MFMA above); the traffic of the engine's own
    instance (the Q8-output kernels for the fused engine) when profiled."""
    dom = max(per, key=lambda k: per[k]["avg_us"] * per[k]["launches_per_step"])
    d = per[dom]
    if step.M <= 32:
        tr = (traffic_tab or {}).get(f"batched{step.M}{'_fused' if fused else ''}/{dom}")
        kern = "gemv_dot4_kernel" if step.M < 3 else "gemm_kp_kernel" if step.M <= 16 else "gemm_ks_kernel"
        return dom, {"bound": "hbm", "achieved": d["GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(d["GBs"] / HBM_PEAK_GBS, 4), "traffic": tr["hbm_bytes"] if tr else None,
                     "traffic_source": tr["source"] if tr else None, "kernel": f"{dom} GEMM ({kern})",
                     "bytes_per_launch": d["bytes"], "avg_launch_us": d["avg_us"]}
    K_ = F if dom == "down" else E
    N_ = {"qkv": QKV, "o": E, "gateup": 2 * F, "down": E}[dom]
    tops = 2 * step.M * N_ * K_ / (d["avg_us"] * 1e-6) / 1e12
    return dom, {"bound": "mfma", "achieved": round(tops, 2), "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s",
                 "frac": round(tops / INT8_PEAK_TOPS, 4), "traffic": None,
                 "kernel": f"{dom} GEMM (gemm_pf2_kernel, int8 ops)", "ops_per_launch": 2 * step.M * N_ * K_,
                 "avg_launch_us": d["avg_us"]}


def run_batched_sub(S: Setup, M, layers, steps, warmup, traffic_tab):
    """Batched decode (M <= 32) or prefill (M = 512) on the first `layers`
    layers of the sweep's weights: the graph of quantize + GEMM launches and,
    for 3 <= M <= 32, the graph with the quantizes in the producers'
    epilogues (checked bit-exact against it); the faster one's dominant kind
    and its roofline."""
    step = Step(S, M, layers, with_output=False)
    hip, torch = S.hip, S.torch
    runs = {"graph": step.run}
    verified = None
    if step.qa is not None:
        ok, why = verify_vs_graph(torch, step, step.run_qchain)
        if not ok:
            raise SystemExit(f"M={M}: fused-quantize launches do not match the op-by-op launches: {why}")
        verified = why
        runs["fused"] = step.run_qchain
    ems = {}
    for name, fn in runs.items():
        step.reset()
        ems[name] = time_graph(hip, torch, fn, steps, warmup)
    best = min(ems, key=ems.get)
    ms = ems[best]
    per = kind_timings(step, layers, steps, fused=best == "fused")
    dom, roof = gemm_roofline(step, per, traffic_tab, fused=best == "fused")
    log(f"M={M}: {ms:.4f} ms per {layers}-layer step ({best}; " +
        ", ".join(f"{k} {v:.4f}" for k, v in ems.items()) + f"); dominant {dom} {per[dom]['avg_us']} us, "
        f"{roof['achieved']} {roof['unit']} ({100 * roof['frac']:.1f} %)")
    how = {"graph": "graph of quantize + GEMM launches",
           "fused": "graph of GEMM launches quantizing their outputs in the epilogue (+ the attention-output "
                    "stand-in's quantize)"}[best]
    out = {"workload": (f"batched decode, M={M}, " if M <= 32 else f"prefill, M={M}, ") +
                       f"{layers} layers of the 27B shapes, {how}",
           "batch": M, "ms_per_step": round(ms, 4), "bytes_per_step": step.total_bytes,
           "GBs": round(step.total_bytes / (ms * 1e-3) / 1e9, 1), "engines_ms": {k: round(v, 4) for k, v in ems.items()},
           "kinds": per, "roofline": roof}
    if verified:
        out["verified"] = f"fused vs graph: {verified}"
    return out


def stream_ceiling(S: Setup, reps=5):
    """The practical HBM read ceiling: btf_hip_stream_read (non-temporal
    16-byte loads, as the GEMV kernels read their weights) over the weight
    arena (6 GB, beyond the 256 MB memory-side cache), HIP events on its
    stream."""
    hip, torch = S.hip, S.torch
    nbytes = S.arena_bytes // 16 * 16
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    s = torch.cuda.Stream()
    hip.stream_read(S.arena, nbytes, sink, s.cuda_stream)
    e0, e1 = hip.Event(), hip.Event()
    try:
        e0.record(s)
        for _ in range(reps):
            hip.stream_read(S.arena, nbytes, sink, s.cuda_stream)
        e1.record(s)
        s.synchronize()
        ms = e0.elapsed_ms(e1) / reps
    finally:
        e0.close()
        e1.close()
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"what": "btf_hip_stream_read: non-temporal 16-byte loads over the weight arena (the practical HBM "
                    "read ceiling)", "bytes": nbytes, "ms": round(ms, 4), "GBs": round(gbs, 1),
            "frac_of_8TBs": round(gbs / HBM_PEAK_GBS, 4)}


def time_graph(hip, torch, fn, reps, warmup):
    """Capture fn(stream) in one graph, replay warmup + reps times; returns ms
    per replay. The graph and the events are released before returning."""
    s = torch.cuda.Stream()
    g, e0, e1 = None, None, None
    try:
        with torch.cuda.stream(s):
            fn(s.cuda_stream)  # eager pass (first-launch costs outside the graph)
            s.synchronize()
            g = hip.Graph(s)
            with g:
                fn(s.cuda_stream)
            for _ in range(warmup):
                g.launch()
            s.synchronize()
            e0, e1 = hip.Event(), hip.Event()
            torch.cuda.synchronize()
            e0.record(s)
            for _ in range(reps):
                g.launch()
            e1.record(s)
            s.synchronize()
            return e0.elapsed_ms(e1) / reps
    finally:
        s.synchronize()
        for o in (e0, e1, g):
            if o is not None:
                o.close()


def time_program(hip, torch, prog, reps, warmup):
    """warmup + reps launches of a step program on one stream; ms per launch
    from HIP events recorded on that stream."""
    s = torch.cuda.Stream()
    for _ in range(warmup):
        prog.launch(s.cuda_stream)
    s.synchronize()
    e0, e1 = hip.Event(), hip.Event()
    try:
        e0.record(s)
        for _ in range(reps):
            prog.launch(s.cuda_stream)
        e1.record(s)
        s.synchronize()
        if prog.error():
            raise RuntimeError("step program reported a timeout")
        return e0.elapsed_ms(e1) / reps
    finally:
        s.synchronize()
        e0.close()
        e1.close()


def verify_vs_graph(torch, step: Step, runner):
    """Bit-exact comparison of one run of another engine (a step-program
    launch, or the fused launches) with the op-by-op launches of the same
    chain from the same residual."""
    import numpy as np
    outs = []
    for run in (lambda st: step.run(st), runner):
        step.reset()
        torch.cuda.synchronize()
        run(torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        outs.append([t.cpu().numpy().copy() for t in (step.res, step.qkv, step.x, step.h, step.logits) if t is not None])
    for a, b in zip(*outs):
        if not np.array_equal(a.view(np.uint32), b.view(np.uint32)):
            return False, f"max |diff| {float(np.max(np.abs(a - b))):.3e}"
    if not all(np.isfinite(a).all() for a in outs[0]):
        return False, "non-finite outputs"
    return True, "bit-exact"


def cpu_info():
    """(model string, logical CPUs this process may run on, logical CPUs of the host)."""
    model = ""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        allowed = len(os.sched_getaffinity(0))
    except AttributeError:
        allowed = os.cpu_count() or 1
    return model, allowed, os.cpu_count() or allowed


def cpu_baseline(S: Setup, step: Step, budget_s=12.0):
    """The reference CPU emulator's GEMV (or the oracle port) on a bounded
    sample of the same workload: the projections of the first layers, M rows,
    each with its Q8 quantize, and the output projection. Threads as the
    reference's bd::ThreadPool(0) (ref/bonsai-decoder/src/cpu_ops.cpp:19-21):
    every CPU the process may run on, no cap; then the layer sets on one
    thread. budget_s is split 2:1 between the two runs (plus a sixth for the
    output projection). `value` is config 5's bytes over the composed token
    time: 64 x the mean measured layer set + the measured output projection."""
    import numpy as np
    sys.path.insert(0, ORACLE)
    from btf_oracle import Oracle, Ref, have_ref
    O = Oracle()
    kind = "reference" if have_ref() else "port"
    R = Ref() if kind == "reference" else None
    model, allowed, logical = cpu_info()
    M = step.M
    rng = np.random.default_rng(0)
    xe = rng.standard_normal((M, E)).astype(np.float32)
    qe, de, se = O.quantize_rows(xe)
    xf = rng.standard_normal((M, F)).astype(np.float32)
    qf, df, sf = O.quantize_rows(xf)
    # Host copies of up to 8 layers (about 750 MB, well beyond the host's
    # caches), cycled until the time budget is spent.
    nl = min(step.layers, 8)
    names = (("qkv", E), ("o", E), ("gate", E), ("up", E), ("down", F))
    host = {(name, l): S.host_mat(name, l) for l in range(nl) for name, _ in names}

    def run(threads, budget):
        total_t, total_b, sets, l = 0.0, 0, 0, 0
        while total_t < budget:
            for name, K in names:
                codes, scales = host[(name, l % nl)]
                q, d, s_ = (qe, de, se) if K == E else (qf, df, sf)
                t0 = time.perf_counter()
                O.quantize_rows(xe if K == E else xf)  # the Q8 quantize of the input
                tq = time.perf_counter() - t0
                if R is not None:
                    t, _ = R.emu_gemv_timed(codes, scales, K, q, d, s_, reps=1, threads=threads)
                else:
                    t0 = time.perf_counter()
                    O.gemv(codes, scales, K, q, d, s_, nthreads=threads)
                    t = time.perf_counter() - t0
                total_t += t + tq
                total_b += gemv_bytes(codes.shape[0], K, M) + prep_bytes(K, M)
            sets += 1
            l += 1
        return total_b / total_t / 1e9, sets, total_t

    gbs, sets, tt = run(allowed, budget_s * 2 / 3)
    gbs1, sets1, tt1 = run(1, budget_s / 3)
    # config 5 = 64 layer sets + the output projection 5120 -> 248320 (5.7 %
    # of its bytes): the projection timed too, on every allowed thread, and
    # the token composed as 64 x the mean measured layer set + it
    out_t = None
    if step.with_output and M == 1:
        codes, scales = S.host_mat("output", step.layers)
        reps, t_out = 0, 0.0
        while t_out < max(1.0, budget_s / 6) or reps < 2:
            t0 = time.perf_counter()
            O.quantize_rows(xe)
            tq = time.perf_counter() - t0
            if R is not None:
                t, _ = R.emu_gemv_timed(codes, scales, E, qe, de, se, reps=1, threads=allowed)
            else:
                t0 = time.perf_counter()
                O.gemv(codes, scales, E, qe, de, se, nthreads=allowed)
                t = time.perf_counter() - t0
            t_out += t + tq
            reps += 1
        out_t = t_out / reps
        del codes, scales
    layer_b = sum(gemv_bytes(N, K, M) + prep_bytes(K, M) for N, K in ((QKV, E), (E, E), (F, E), (F, E), (E, F)))
    t_layer = layer_b / (gbs * 1e9)  # mean measured time of one layer set
    token = None
    if out_t is not None:
        t_tok = LAYERS * t_layer + out_t
        token = {"per_token_s": round(t_tok, 4), "tok_s": round(1.0 / t_tok, 4),
                 "GBs_over_config5_bytes": round(step.total_bytes / t_tok / 1e9, 3),
                 "output_projection_s": round(out_t, 4), "layer_set_s": round(t_layer, 5),
                 "composition": "64 x the mean measured layer set (5 GEMVs with their quantizes) + the measured "
                                "output projection with its quantize, all on every allowed thread (config 5 on "
                                "the CPU: the sum of its 321 GEMVs and quantizes, BASELINE section 3)"}
    what = ("reference EmuDecoder::gemv (src/emu_decoder.cpp:143-165) built from the reference sources"
            if kind == "reference" else "oracle port of EmuDecoder::gemv")
    return {"value": round(token["GBs_over_config5_bytes"] if token else gbs, 3), "unit": "GB/s", "cores": allowed,
            "kind": kind, "config5_token": token,
            "layer_sets_GBs": round(gbs, 3),
            "tok_s_equiv": token["tok_s"] if token else (round(gbs * 1e9 / step.total_bytes, 4) if M == 1 else None),
            "value_1_thread": round(gbs1, 3),
            "tok_s_equiv_1_thread": round(gbs1 * 1e9 / step.total_bytes, 4) if M == 1 else None,
            "cpu_model": model, "logical_cpus_allowed": allowed, "logical_cpus_host": logical,
            "sample": f"{sets} layer GEMV set(s) on {allowed} threads ({tt:.2f} s) and {sets1} on 1 thread "
                      f"({tt1:.2f} s), cycling over {nl} distinct layers x (QKV 5120->7168, o 5120->5120, "
                      f"gate/up 5120->17408, down 17408->5120), M={M}, each GEMV with its Q8 quantize; {what}; "
                      f"host CPU: {model}, {allowed} of {logical} logical CPUs allowed"}


def write_synth_gguf(path, layers, seed=0, chunk=1 << 26):
    """A GGUF v3 file of the 27B shapes' PTQ1_0 matrices (per layer QKV, o,
    gate, up, down; the output projection), seeded random bytes (the PTQ1_0
    codec decodes every byte value), plus one F32 norm per layer; streamed to
    disk. Returns the PTQ1_0 bytes written."""
    import struct
    import numpy as np
    rng = np.random.default_rng(seed)
    mats = []
    for l in range(layers):
        mats += [(f"blk.{l}.attn_qkv.weight", E, QKV), (f"blk.{l}.attn_output.weight", E, E),
                 (f"blk.{l}.ffn_gate.weight", E, F), (f"blk.{l}.ffn_up.weight", E, F),
                 (f"blk.{l}.ffn_down.weight", F, E)]
    mats.append(("output.weight", E, V))
    tens = []  # (name, ne, type, bytes)
    for l in range(layers):
        tens.append((f"blk.{l}.attn_norm.weight", (E,), 0, 4 * E))
    for name, K, N in mats:
        tens.append((name, (K, N), 143, N * K // 128 * 28))
    align = 32

    def st(x):
        b = x.encode()
        return struct.pack("<Q", len(b)) + b
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tens), 2)
    head += st("general.architecture") + struct.pack("<I", 8) + st("qwen35")
    head += st("general.alignment") + struct.pack("<II", 4, align)
    off, offs = 0, []
    for name, ne, ty, nb in tens:
        offs.append(off)
        head += st(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", x) for x in ne)
        head += struct.pack("<IQ", ty, off)
        off = (off + nb + align - 1) // align * align
    head += b"\0" * ((-len(head)) % align)
    src = 0
    with open(path, "wb") as f:
        f.write(head)
        pos = 0
        for (name, ne, ty, nb), o in zip(tens, offs):
            if o > pos:
                f.write(b"\0" * (o - pos))
            left = nb
            while left:
                n = min(chunk, left)
                f.write(rng.integers(0, 256, size=n, dtype=np.uint8).tobytes())
                left -= n
            pos = o + nb
            src += nb if ty == 143 else 0
        f.write(b"\0" * (off - pos))
    return src


def run_load(args, hip, torch):
    """--workload load: the load sub-result as its own line."""
    layers = args.layers if args.layers != LAYERS else 8
    r = load_result(hip, torch, layers, args.steps, args.warmup, args.cpu_budget, args.no_cpu)
    out = {
        "metric": "PTQ1_0 GGUF load GB/s (file in page cache -> resident T2 layout)", "value": r["GBs"],
        "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": r["ms"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8",
        "data": "synthetic GGUF (seeded PTQ1_0 bytes) of the 27B shapes",
        "config": {"workload": r["workload"], "parallelism": "single GPU"},
        "load": r, "cpu_baseline": r["cpu_baseline"],
    }
    print(json.dumps(out), flush=True)


def load_result(hip, torch, layers, steps, warmup, cpu_budget, no_cpu):
    """GGUF file -> staged upload -> resident T2 layout of every PTQ1_0
    matrix (btf_hip_gguf_* + btf_hip_loader_*), from the page cache: PTQ1_0
    bytes read from the file / wall time of the whole upload (open, plan,
    every upload, finish), median of the timed loads; beside it the
    reference's host repack (btf::repack_rows, src/repack.cpp:16-27, as
    tools/btf_plan.cpp:72-110 times it) on the same matrices, on every
    allowed thread."""
    import tempfile
    import numpy as np
    staging = 64 << 20
    tmp = tempfile.mkdtemp(prefix="btf_load_")
    path = os.path.join(tmp, "synth.gguf")
    t0 = time.time()
    src_bytes = write_synth_gguf(path, layers)
    log(f"synthetic GGUF: {layers} layers + output, {os.path.getsize(path) / 1e9:.3f} GB file "
        f"({src_bytes / 1e9:.3f} GB of PTQ1_0) written in {time.time() - t0:.1f} s")
    with open(path, "rb") as f:  # into the page cache
        while f.read(1 << 26):
            pass
    arena, times, plan, phases = None, [], None, []
    for rep in range(warmup + steps):
        t0 = time.perf_counter()
        g = hip.Gguf(path)
        plan = g.plan(staging)
        if arena is None:
            arena = torch.empty(plan["arena_bytes"], dtype=torch.uint8, device="cuda")
        t1 = time.perf_counter()
        L = hip.Loader(staging)
        t2 = time.perf_counter()
        st = torch.cuda.current_stream().cuda_stream
        off, base = 0, arena.data_ptr()
        for t in g.tensors:
            if t.type != 143 or t.n_dims != 2:
                continue
            K, N = t.ne
            co = off
            so = co + (N * K // 4 + 255) // 256 * 256
            off = so + (N * K // 64 + 255) // 256 * 256
            L.upload_ptq1_0(t.data, N, K, base + co, base + so, st)
        n = L.finish()
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        L.close()
        g.close()
        assert n == plan["source_bytes"] == src_bytes
        if rep >= warmup:
            times.append(dt)
            phases.append((t1 - t0, t2 - t1, dt - (t2 - t0)))
    t = float(np.median(times))
    ph = np.median(np.array(phases), axis=0)
    log(f"load phases (median): open + plan {ph[0] * 1e3:.2f} ms, loader (pinned + device staging) "
        f"{ph[1] * 1e3:.2f} ms, uploads + finish {ph[2] * 1e3:.2f} ms")
    value = src_bytes / t / 1e9
    log(f"load: {t * 1e3:.1f} ms for {src_bytes / 1e9:.3f} GB of PTQ1_0 -> {plan['arena_bytes'] / 1e9:.3f} GB "
        f"resident: {value:.2f} GB/s")
    # stage rates on one 64 MiB slice: host copy from the mapping, DMA copy, repack kernel
    g = hip.Gguf(path)
    tm = g.tensor("blk.0.ffn_gate.weight")
    rows = staging // (tm.ne[0] // 128 * 28)
    nbytes = rows * (tm.ne[0] // 128 * 28)
    import ctypes as C
    pinned = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    t0 = time.perf_counter()
    for _ in range(5):
        C.memmove(pinned.data_ptr(), tm.data, nbytes)
    host_gbs = 5 * nbytes / (time.perf_counter() - t0) / 1e9
    dstage = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    e0, e1 = hip.Event(), hip.Event()
    st = torch.cuda.current_stream().cuda_stream
    e0.record(st)
    for _ in range(5):
        dstage.copy_(pinned, non_blocking=True)
    e1.record(st)
    torch.cuda.synchronize()
    dma_gbs = 5 * nbytes / (e0.elapsed_ms(e1) * 1e-3) / 1e9
    codes = torch.empty(rows * tm.ne[0] // 4, dtype=torch.uint8, device="cuda")
    scales = torch.empty(rows * tm.ne[0] // 128, dtype=torch.int16, device="cuda")
    e0.record(st)
    for _ in range(5):
        hip.launch_repack(dstage, rows * tm.ne[0] // 128, codes, scales, st)
    e1.record(st)
    torch.cuda.synchronize()
    rep_gbs = 5 * nbytes / (e0.elapsed_ms(e1) * 1e-3) / 1e9
    log(f"stages on a {nbytes / 2**20:.0f} MiB slice: host copy from the mapping {host_gbs:.2f} GB/s, "
        f"copy engine {dma_gbs:.2f} GB/s, repack kernel {rep_gbs:.1f} GB/s (of PTQ1_0 read)")
    e0.close()
    e1.close()
    g.close()
    cpu = None
    if not no_cpu:
        sys.path.insert(0, ORACLE)
        from concurrent.futures import ThreadPoolExecutor
        from btf_oracle import Oracle, Ref, have_ref
        kind = "reference" if have_ref() else "port"
        R = Ref() if kind == "reference" else Oracle()
        model, allowed, logical = cpu_info()
        g = hip.Gguf(path)
        # every PTQ1_0 matrix of layer 0 and the output projection (the
        # reference repacks matrix by matrix over a thread pool: row ranges
        # here, one per thread, the GIL released inside the library)
        srcs = []
        for ti in g.tensors:
            if ti.type == 143 and ti.n_dims == 2 and (ti.name.startswith("blk.0.") or ti.name == "output.weight"):
                K, N = ti.ne
                srcs.append((np.frombuffer(C.string_at(ti.data, ti.bytes), dtype=np.uint8).reshape(N, K // 128 * 28),
                             N, K))
        g.close()
        jobs = []
        for m, N, K in srcs:
            step_rows = (N + allowed - 1) // allowed
            for r0 in range(0, N, step_rows):
                jobs.append((np.ascontiguousarray(m[r0:r0 + step_rows]), min(step_rows, N - r0), K))
        nbytes = sum(j[0].size for j in jobs)
        done, tt, passes = 0, 0.0, 0
        with ThreadPoolExecutor(max_workers=allowed) as ex:
            while tt < cpu_budget:
                t0 = time.perf_counter()
                list(ex.map(lambda j: R.repack_rows(*j), jobs))
                tt += time.perf_counter() - t0
                done += nbytes
                passes += 1
        cpu = {"value": round(done / tt / 1e9, 3), "unit": "GB/s", "cores": allowed, "kind": kind,
               "sample": f"host repack of layer 0's five matrices and the output projection "
                         f"({nbytes / 1e6:.0f} MB of PTQ1_0), {passes} passes, {tt:.2f} s, row ranges over "
                         f"{allowed} threads; "
                         f"{'reference btf::repack_rows (src/repack.cpp:16-27) built from the reference sources' if kind == 'reference' else 'oracle port of repack_rows'}"
                         f"; the reference's published rate: 2.65 GB/s on 8 vCPUs (README.md:36)",
               "cpu_model": model}
    os.remove(path)
    os.rmdir(tmp)
    return {"workload": f"load {layers} layers x (QKV, o, gate, up, down) + output projection, "
                        f"{src_bytes} B of PTQ1_0 -> {plan['arena_bytes']} B resident, 2 x 64 MiB staging",
            "GBs": round(value, 2), "ms": round(t * 1e3, 2), "seconds": round(t, 4), "bytes": src_bytes,
            "stages_gbs": {"host_copy": round(host_gbs, 2), "copy_engine": round(dma_gbs, 2),
                           "repack_kernel": round(rep_gbs, 1)},
            "phases_ms": {"open_plan": round(ph[0] * 1e3, 2), "loader_create": round(ph[1] * 1e3, 2),
                          "uploads": round(ph[2] * 1e3, 2)},
            "cpu_baseline": cpu}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="sweep", choices=["sweep", "layer", "batched", "prefill", "load", "token"])
    ap.add_argument("--token-prep", default="full", choices=["full", "hx", "norm", "none"],
                    help="--workload token: the GEMV input preps (the decoder's norms and transforms, or a part)")
    ap.add_argument("--no-subs", action="store_true",
                    help="sweep: skip the sub-results (whole token, config 1, batched M=8, prefill M=512)")
    ap.add_argument("--batch", type=int, default=0, help="M for --workload batched (default 4,8,16,32 sweep)")
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--engine", default="auto", choices=["auto", "step", "chain", "graph"],
                    help="auto: at batch 1 every engine is timed and the fastest one is the value; "
                         "the graph otherwise")
    ap.add_argument("--no-kinds", action="store_true", help="skip the per-GEMV-kind graph timings")
    ap.add_argument("--b3", dest="b3", action="store_true", default=None,
                    help="also time the chain on the PTQ1_0 rows read directly (default: with --engine auto)")
    ap.add_argument("--no-b3", dest="b3", action="store_false")
    ap.add_argument("--mfma-min-m", type=int, default=0,
                    help="batch rows from which GEMVs run on the int8 MFMA kernels (0: the library default)")
    ap.add_argument("--allow-profiler", action="store_true",
                    help="launch step programs under rocprofv3 (see under_profiler)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="first run 3 device copies of 1 GiB (the scale reference for HBM counters)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(json.dumps({"error": "this build runs on one GPU only: the ternary matmul path has no "
                                   "multi-GPU code (a GPU would take a row share of every matrix; the design "
                                   "is written up beside the code)",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    launches_step = args.workload == "token" or (args.workload == "sweep" and args.engine in ("auto", "step"))
    if launches_step and under_profiler() and not args.allow_profiler:
        raise SystemExit("bench: this run would launch step programs (a cooperative launch) under rocprofv3, "
                         "whose teardown has ended every such run with a segmentation fault in the exit "
                         "handlers after the results were complete; step timings come from HIP events on the "
                         "kernel's stream. Pass --allow-profiler to run it anyway, or profile the other "
                         "workloads (--workload layer|batched|prefill, --engine chain|graph).")

    import torch
    sys.path.insert(0, PKG)
    import btf_hip as hip

    torch.cuda.set_device(0)
    hip.kernels_init(0)
    if args.mfma_min_m:
        hip.gemv_set_policy(args.mfma_min_m)
    info = hip.device_info(0)
    log(f"device {info['name']} {info['gcn_arch']} CUs={info['cu_count']}")

    if args.calib_copy:
        a = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        log("calibration: 3 device copies of 1 GiB (reads 1 GiB, writes 1 GiB each)")
        del a, b

    if args.workload == "load":
        run_load(args, hip, torch)
        return

    layers = args.layers if args.workload in ("sweep", "token") else (1 if args.workload == "layer" else 8)
    t0 = time.time()
    with_b3 = (args.engine == "auto" if args.b3 is None else args.b3) and args.workload in ("sweep", "layer")
    subs_on = args.workload == "sweep" and not args.no_subs
    S = Setup(hip, torch, layers, keep_src=with_b3, with_embed=subs_on or args.workload == "token")
    log(f"weights generated + repacked: {S.arena_bytes / 1e9:.3f} GB arena in {time.time() - t0:.2f} s")
    try:
        with open(os.path.join(ROOT, "profiles", "hbm_traffic.json")) as f:
            traffic_tab = json.load(f)
    except (OSError, ValueError):
        traffic_tab = {}

    if args.workload == "token":
        tok = run_token(S, hip, torch, layers, args.steps, args.warmup, args.token_prep, traffic_tab)
        out = {"metric": "whole-token decode step at batch 1 (tok/s)", "value": tok["tok_s"], "unit": "tok/s",
               "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": tok["ms_per_token"],
               "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
               "data": "synthetic (seeded ternary weights, norm weights N(1,0.1), random signs)",
               "config": {"workload": tok["workload"], "batch": 1, "parallelism": "single GPU"},
               "roofline": tok["roofline"], "whole_token": tok, "cpu_baseline": None}
        print(json.dumps(out))
        return

    if args.workload == "sweep":
        step = Step(S, 1, layers)
    elif args.workload == "layer":
        step = Step(S, 1, 1, with_output=False)
    elif args.workload == "batched":
        step = Step(S, args.batch or 8, layers, with_output=False)
    else:
        step = Step(S, 512, layers, with_output=False)

    engines = [args.engine] if args.engine != "auto" else (
        ["step", "chain", "graph"] if step.M == 1 else ["chain", "graph"] if step.qa is not None else ["graph"])
    if "step" in engines and step.M != 1:
        raise SystemExit("the step engine runs batch-1 chains only")
    if "chain" in engines and step.M != 1 and step.qa is None:
        raise SystemExit("the chain engine runs batch 1 or 3..32 rows")
    chain_fn = step.run_chain if step.M == 1 else step.run_qchain

    verified = {}
    engine_ms = {}
    if "step" in engines:
        t0 = time.time()
        prog = step.program()
        log(f"step program built in {time.time() - t0:.2f} s")
        ok, why = verify_vs_graph(torch, step, lambda st: prog.launch(st))
        if prog.error():
            ok, why = False, "step program reported a timeout"
        verified["step"] = why
        log(f"step program vs op-by-op launches: {why}")
        if not ok:
            raise SystemExit(f"step program does not match the op-by-op launches: {why}")
        step.reset()
        try:
            engine_ms["step"] = time_program(hip, torch, prog, args.steps, args.warmup)
        finally:
            prog.close()
        log(f"step engine: {engine_ms['step']:.4f} ms per step")
    if "chain" in engines:
        ok, why = verify_vs_graph(torch, step, chain_fn)
        verified["chain"] = why
        log(f"chain launches vs op-by-op launches: {why}")
        if not ok:
            raise SystemExit(f"chain launches do not match the op-by-op launches: {why}")
        step.reset()
        engine_ms["chain"] = time_graph(hip, torch, chain_fn, args.steps, args.warmup)
        log(f"chain engine: {engine_ms['chain']:.4f} ms per step")
    if "graph" in engines:
        step.reset()
        engine_ms["graph"] = time_graph(hip, torch, step.run, args.steps, args.warmup)
        log(f"graph engine: {engine_ms['graph']:.4f} ms per step")
    # The same chain on the PTQ1_0 rows read directly (btf_hip_launch_gemv_ptq1_0
    # in a graph of quantize + GEMV launches): checked bit-exact against the
    # graph engine, rated on its own algorithmic bytes (28 B per 128 weights).
    b3 = None
    if with_b3:
        ok, why = verify_vs_graph(torch, step, lambda st: step.run_b3(st))
        log(f"PTQ1_0-direct launches vs op-by-op launches: {why}")
        if not ok:
            raise SystemExit(f"PTQ1_0-direct launches do not match the op-by-op launches: {why}")
        step.reset()
        b3_ms = time_graph(hip, torch, step.run_b3, args.steps, args.warmup)
        b3 = {"ms_per_step": round(b3_ms, 4), "bytes_per_step": step.b3_total_bytes,
              "GBs": round(step.b3_total_bytes / (b3_ms / 1e3) / 1e9, 1), "tok_s_equiv": round(1e3 / b3_ms, 2),
              "verified": why, "kinds": {}}
        log(f"PTQ1_0-direct graph: {b3_ms:.4f} ms per step, {b3['GBs']} GB/s of its own bytes")
        for kind in ["qkv", "o", "gateup", "down"] + (["output"] if step.with_output else []):
            reps = 1 if kind == "output" else layers
            fn = (lambda st, kind=kind: step.kind_launch_b3(kind, 0, st)) if kind == "output" else \
                 (lambda st, kind=kind: [step.kind_launch_b3(kind, l, st) for l in range(layers)])
            kms = time_graph(hip, torch, fn, max(3, args.steps // 2), 1)
            avg_us = kms * 1e3 / reps
            bb = step.kind_bytes_b3[kind]
            b3["kinds"][kind] = {"avg_us": round(avg_us, 3), "bytes": bb, "GBs": round(bb / (avg_us * 1e-6) / 1e9, 1)}
            log(f"  PTQ1_0-direct {kind}: {avg_us:.3f} us/launch, {b3['kinds'][kind]['GBs']} GB/s")
    engine = min(engine_ms, key=engine_ms.get)
    ms = engine_ms[engine]
    kernels_per_step = {"step": 1, "chain": layers * 5 + (2 if step.with_output else 1)}.get(
        engine, layers * 8 + (2 if step.with_output else 0))
    log(f"{engine} engine reported: {ms:.4f} ms per step ({step.total_bytes / 1e9:.4f} GB algorithmic)")
    value = step.total_bytes / (ms / 1e3) / 1e9

    # Per-kind GEMV timing of the op-by-op path: a graph of one launch per
    # layer (distinct weights) -> average per launch.
    per = {}
    fk = engine == "chain"
    if not args.no_kinds or engine != "step":
        per = kind_timings(step, layers, args.steps, fused=fk)
        for kind, d in per.items():
            log(f"  op-by-op {kind}: {d['avg_us']:.3f} us/launch, {d['GBs']} GB/s")
    # The kernels either side of the GEMV chain, as separate launches (the
    # whole-token sub-result runs them inside the step program): the
    # embedding lookup of one token from the packed V x 5120 table (inverse
    # transform at block 1024 + signs), the greedy pick over V logits (two
    # launches) and the position counter; graphs of 64 launches each.
    ends = None
    if step.with_output and args.workload == "sweep":
        N_, K_, _, co, so = S.mats[("output", layers)]
        base = S.arena.data_ptr()
        toks = torch.arange(64, dtype=torch.int32, device="cuda") * 3877 % V
        signs = torch.where(torch.rand(E, device="cuda") < 0.5, -1.0, 1.0).to(torch.float32)
        xe = torch.zeros((1, E), dtype=torch.float32, device="cuda")
        inv = hip.Hx(block=1024, signs=signs)
        part = torch.zeros(hip.argmax_part_bytes(V) // 4, dtype=torch.int32, device="cuda")
        tok_out = torch.zeros(1, dtype=torch.int32, device="cuda")
        pos = torch.zeros(1, dtype=torch.int32, device="cuda")
        tp = toks.data_ptr()
        fns = {
            "embed": lambda st: [hip.launch_embed(base + co, base + so, tp + 4 * i, 1, E, inv, xe, st) for i in range(64)],
            "argmax": lambda st: [hip.launch_argmax(step.logits, V, part, tok_out, st) for _ in range(64)],
            "argmax_noalloc": lambda st: [hip.launch_argmax_noalloc(step.logits, V, tok_out, st) for _ in range(64)],
            "pos_add": lambda st: [hip.launch_pos_add(pos, 1, st) for _ in range(64)],
        }
        ends = {}
        for name, fn in fns.items():
            kms = time_graph(hip, torch, fn, max(3, args.steps // 2), 1)
            ends[f"{name}_us"] = round(kms * 1e3 / 64, 3)
        ends["embed_bytes"] = E // 4 + E // 64 + 4 * E
        ends["argmax_bytes"] = 4 * V
        log(f"decode-step ends: embed {ends['embed_us']} us, argmax {ends['argmax_us']} us "
            f"({ends['argmax_bytes'] / (ends['argmax_us'] * 1e3):.1f} GB/s), pos_add {ends['pos_add_us']} us")

    # HBM bytes per launch of the dominant kernel, from the committed rocprofv3
    # FETCH_SIZE / WRITE_SIZE runs (profiles/hbm_traffic.json), when they
    # cover this engine's dominant kernel; counters cannot be read live.
    if engine == "step":
        tr = traffic_tab.get("step/step_kernel") if step.M == 1 and args.workload == "sweep" and \
            layers == LAYERS else None
        roof = {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(value / HBM_PEAK_GBS, 4), "traffic": tr["hbm_bytes"] if tr else None,
                "traffic_source": tr["source"] if tr else None,
                "kernel": "step_kernel<false> (the whole GEMV chain, one launch per step)",
                "bytes_per_launch": step.total_bytes, "avg_launch_us": round(ms * 1e3, 3)}
    elif step.M == 1:
        dom = max(per, key=lambda k: per[k]["avg_us"] * per[k]["launches_per_step"])
        d = per[dom]
        tr = traffic_tab.get(f"{engine}/{dom}") if args.workload == "sweep" else None
        roof = {"bound": "hbm", "achieved": d["GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(d["GBs"] / HBM_PEAK_GBS, 4), "traffic": tr["hbm_bytes"] if tr else None,
                "traffic_source": tr["source"] if tr else None,
                "kernel": f"{dom} GEMV (gemv_dot4_kernel{', quantizes fused in' if fk else ''})",
                "bytes_per_launch": d["bytes"], "avg_launch_us": d["avg_us"]}
    else:
        _, roof = gemm_roofline(step, per, traffic_tab if not args.mfma_min_m else {}, fused=engine == "chain")

    # Sub-results of the default run, each with its own roofline: the whole
    # decode step in one launch; config 1 (the 5120 -> 5120 GEMV, 64 distinct
    # matrices rotated past the MALL, from the per-kind timings); config 3
    # (batched decode M = 8) and config 4 (prefill M = 512) on 8 layers.
    subs = None
    if subs_on:
        subs = {"whole_token": run_token(S, hip, torch, layers, args.steps, args.warmup, traffic_tab=traffic_tab)}
        if "o" in per:
            d = per["o"]
            subs["config1_gemv_5120x5120"] = {
                "workload": "GEMV M=1, K=5120 -> N=5120 (the o projection of 64 distinct layers, 445 MB rotated "
                            "past the 256 MB MALL), Q8 input quantized by its own launch",
                "avg_us": d["avg_us"], "bytes_per_launch": d["bytes"], "GBs": d["GBs"],
                "roofline": {"bound": "hbm", "achieved": d["GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(d["GBs"] / HBM_PEAK_GBS, 4),
                             "traffic": traffic_tab.get("config1/o", {}).get("hbm_bytes"),
                             "traffic_source": traffic_tab.get("config1/o", {}).get("source"),
                             "kernel": "gemv_dot4_kernel (o projection)", "bytes_per_launch": d["bytes"],
                             "avg_launch_us": d["avg_us"]}}
        for M in (4, 8, 16, 32):
            subs[f"config3_batched_m{M}"] = run_batched_sub(S, M, 8, args.steps, args.warmup, traffic_tab)
        subs["config4_prefill_m512"] = run_batched_sub(S, 512, 8, max(5, args.steps // 2), 2, traffic_tab)
        subs["stream_read_ceiling"] = stream_ceiling(S)
        log(f"stream read ceiling: {subs['stream_read_ceiling']['GBs']} GB/s")
        subs["load"] = load_result(hip, torch, 8, 3, 1, min(args.cpu_budget, 6.0), args.no_cpu)

    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded ternary weights p=0.3/0.4/0.3, fp16 scales U[0.01,0.05], N(0,1) activations)",
        "config": {
            "workload": {"sweep": f"27B-scale decode-step weight sweep: {layers} x (QKV 5120->7168, o 5120->5120, "
                                  "gate+up 5120->17408 swiglu, down 17408->5120) + output 5120->248320, "
                                  "batch 1, every GEMV fed by the Q8 quantize of its input",
                         "layer": "one decoder layer's projections at batch 1, each with its Q8 quantize",
                         "batched": f"batched decode, M={step.M}, {layers} layers of the 27B shapes",
                         "prefill": f"prefill M=512, {layers} layers of the 27B shapes"}[args.workload],
            "batch": step.M,
            "bytes_per_step": step.total_bytes,
            "weight_bytes_per_step": step.weight_bytes,
            "engine": engine,
            "kernels_per_step": kernels_per_step,
            "parallelism": "single GPU",
        },
        "frac_of_8TBs": round(value / HBM_PEAK_GBS, 4),
        "frac_of_stream_read": round(value / subs["stream_read_ceiling"]["GBs"], 4) if subs else None,
        "tok_s_equiv": round(1e3 / ms, 2) if args.workload == "sweep" else None,
        "roofline": roof,
        "verified": {"vs_graph_engine_bit_exact": verified} if verified else None,
        "engines_ms": {k: round(v, 4) for k, v in engine_ms.items()},
        "gemv_kinds": per,
        "sub_results": subs,
        "decode_step_ends": ends,
        "ptq1_0_direct": b3,
        "device": {"name": info["name"], "arch": info["gcn_arch"], "cus": info["cu_count"]},
    }
    if not args.no_cpu:
        log("cpu baseline ...")
        out["cpu_baseline"] = cpu_baseline(S, step, args.cpu_budget)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out))


if __name__ == "__main__":
    main()
