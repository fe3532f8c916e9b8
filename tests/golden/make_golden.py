#!/usr/bin/env python3
"""Writes tests/golden/golden.npz from the reference's own CPU code.

Run in a container that has the reference checkout, after `make -C oracle ref`
has built oracle/_ref/libbtf_ref.so from the reference's sources (the build
reads them in place; nothing is copied). Every array in the fixture is
produced by a reference function:

  ptq_w / ptq_src       bd::quant_row(T_PTQ1_0)   ref/bonsai-decoder/src/types.cpp:289-320
  rp_src / rp_codes /   btf::repack_rows           src/repack.cpp:16-27
    rp_scales           (random bytes: every byte value occurs)
  q8_x / q8_q/d/s       EmuDecoder::prep, no norm / transform   src/emu_decoder.cpp:122-140
  q8_round              bd::round_q8_0             ref/bonsai-decoder/src/cpu_ops.cpp:189-197
  prep{i}_*             EmuDecoder::prep on the reference's test_prep cases
                        (tests/test_gpu_kernels.cpp:557-561, reduced M)
  gemv_* / gemv{M}_y    EmuDecoder::gemv           src/emu_decoder.cpp:143-165
  gemv{M}_I             sub_dot_host - s           include/btf/packed.hpp:108-113
  mv_y                  bd::matvec_raw(ggml_act)   ref/bonsai-decoder/src/cpu_ops.cpp:199-221
  f16_*                 bd::f32_to_fp16 / fp16_to_f32
  fwht_*                bd::fwht                   ref/bonsai-decoder/src/cpu_ops.cpp:76-88
  emb_* / emb{b}_x      the emulator's embedding lookup (src/emu_decoder.cpp:171-180:
                        packed_code, fp16_to_f32, bd::hadamard_inverse)
  am{i}_l / am{i}_best  bd::Sampler::argmax        ref/bonsai-decoder/src/sampler.cpp:20-25

Inputs are drawn from numpy's PCG64 with fixed seeds; the fixture stores both
inputs and outputs, so the tests never need the reference.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
from btf_oracle import Ref  # noqa: E402


def main():
    R = Ref()
    rng = np.random.default_rng(20261201)
    g = {}

    # fp16 conversions: boundary-heavy f32 sample + every half
    specials = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.996, 65520.0, 65536.0, 1e-8, 2.0 ** -24,
                         2.0 ** -25, 2.0 ** -25 * 1.0000001, 2.0 ** -14, 2.0 ** -14 * 0.99999994, 3.1415927,
                         np.inf, -np.inf], np.float32)
    bits = rng.integers(0, 2 ** 32, 40000, dtype=np.uint64).astype(np.uint32)
    f = np.concatenate([specials, bits.view(np.float32)])
    f = f[~np.isnan(f)]
    g["f16_in"] = f
    g["f16_out"] = np.array([R.lib.ref_f32_to_fp16(float(v)) for v in f], np.uint16)
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    g["f16_widen"] = np.array([R.lib.ref_fp16_to_f32(int(v)) for v in h], np.float32)

    # PTQ1_0 encoder, as the reference tests make weights (30 % zeros)
    N, K = 37, 1024
    w = rng.standard_normal((N, K)).astype(np.float32) * (rng.random((N, K)) >= 0.3)
    g["ptq_w"] = w
    g["ptq_src"] = R.quant_ptq1_0(w)

    # repack of arbitrary bytes (every byte value) and of encoder output
    src = rng.integers(0, 256, (41, 1024 // 128 * 28), dtype=np.uint8)
    g["rp_src"] = src
    g["rp_codes"], g["rp_scales"] = R.repack_rows(src, 41, 1024)
    g["rpe_codes"], g["rpe_scales"] = R.repack_rows(g["ptq_src"], N, K)

    # Q8 quantize (no norm, no transform) incl. edge rows
    x = (rng.standard_normal((8, 1024)) * 3).astype(np.float32)
    x[0, :32] = 0.0
    x[0, 32:64] = -0.0
    x[1, :32] = np.where(np.arange(32) % 2 == 0, 2.5, -3.5)
    x[1, 31] = 127.0
    x[2, :32] = 1e-7 * (np.arange(32) - 16)
    x[3] *= 1e4
    g["q8_x"] = x
    g["q8_q"], g["q8_d"], g["q8_s"], _ = R.emu_prep(x)
    g["q8_round"] = R.round_q8_0(x)

    # the reference's prep cases (n, block, norm, perm, signs, M) with M <= 2
    cases = [(1024, 64, 1, 0, 1, 1), (5120, 1024, 1, 0, 1, 2), (2048, 128, 0, 1, 1, 2), (256, 0, 1, 0, 0, 2),
             (17408, 1024, 0, 0, 1, 1)]
    for i, (n, blk, norm, perm, signs, M) in enumerate(cases):
        xx = (rng.standard_normal((M, n)) * 3).astype(np.float32)
        ww = rng.standard_normal(n).astype(np.float32)
        sg = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float32)
        hd, nk, rep = (32, n // 64, 2) if perm else (0, 0, 0)
        q, d, s, xn = R.emu_prep(xx, ww if norm else None, 1e-6, blk, hd, nk, rep, sg if signs else None)
        g[f"prep{i}_case"] = np.array([n, blk, norm, perm, signs, M, hd, nk, rep], np.int32)
        g[f"prep{i}_x"], g[f"prep{i}_w"], g[f"prep{i}_signs"] = xx, ww, sg
        g[f"prep{i}_q"], g[f"prep{i}_d"], g[f"prep{i}_s"], g[f"prep{i}_xn"] = q, d, s, xn

    # GEMV: the emulator on packed encoder weights, M in {1, 3, 8, 13}
    codes, scales = g["rpe_codes"], g["rpe_scales"]
    g["gemv_codes"], g["gemv_scales"] = codes, scales
    for M in (1, 3, 8, 13):
        xm = (rng.standard_normal((M, K)) * 3).astype(np.float32)
        q, d, s, _ = R.emu_prep(xm)
        g[f"gemv{M}_x"], g[f"gemv{M}_q"], g[f"gemv{M}_d"], g[f"gemv{M}_s"] = xm, q, d, s
        g[f"gemv{M}_y"] = R.emu_gemv(codes, scales, K, q, d, s)
        y0 = rng.standard_normal((M, N)).astype(np.float32)
        g[f"gemv{M}_y0"] = y0
        g[f"gemv{M}_yadd"] = R.emu_gemv(codes, scales, K, q, d, s, y=y0.copy(), add=True)
        I = np.zeros((M, N, K // 32), np.int32)
        aw = q.view(np.uint32)
        cw = codes.view(np.uint32)
        for m in range(M):
            for r in range(N):
                for sb in range(K // 32):
                    I[m, r, sb] = R.lib.ref_sub_dot(int(cw[r, 2 * sb]), int(cw[r, 2 * sb + 1]),
                                                    aw[m, 8 * sb:8 * sb + 8].ctypes.data_as(
                                                        __import__("ctypes").c_void_p)) - int(s[m, sb])
        g[f"gemv{M}_I"] = I
    # matvec_raw with ggml activation rounding (test_packed.cpp:63-74)
    xv = g["gemv1_x"][0]
    g["mv_y"] = R.matvec_ptq1_0(g["ptq_src"], N, K, xv, True)

    # normalised FWHT of a few sizes
    for n in (2, 64, 1024):
        v = rng.standard_normal(n).astype(np.float32)
        out = v.copy()
        R.lib.ref_fwht(out.ctypes.data_as(__import__("ctypes").c_void_p), n)
        g[f"fwht{n}_in"], g[f"fwht{n}_out"] = v, out

    # embedding lookup from a packed table (the table itself from the
    # reference's encoder and repack), with and without the inverse transform
    Ve, Ee = 40, 2048
    we = (rng.standard_normal((Ve, Ee)) * (rng.random((Ve, Ee)) >= 0.3)).astype(np.float32)
    ecodes, escales = R.repack_rows(R.quant_ptq1_0(we), Ve, Ee)
    etoks = rng.integers(0, Ve, 5).astype(np.int32)
    esigns = np.where(rng.random(Ee) < 0.5, -1.0, 1.0).astype(np.float32)
    g["emb_codes"], g["emb_scales"], g["emb_toks"], g["emb_signs"] = ecodes, escales, etoks, esigns
    for blk in (0, 128, 1024):
        g[f"emb{blk}_x"] = R.emu_embed(ecodes, escales, etoks, Ee, Ve, blk, esigns if blk else None)
    # greedy pick: distinct values, a tie (first index wins), -inf and all-equal rows
    am = [rng.standard_normal(5000).astype(np.float32) for _ in range(4)]
    am[1][[17, 4000]] = np.float32(7.5)
    am[2][:] = -np.inf
    am[2][[300, 301]] = np.float32(-3.0)
    am[3][:] = np.float32(1.25)
    for i, l in enumerate(am):
        g[f"am{i}_l"], g[f"am{i}_best"] = l, np.int32(R.argmax(l))

    path = os.path.join(HERE, "golden.npz")
    np.savez_compressed(path, **g)
    print(f"wrote {path}: {len(g)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
