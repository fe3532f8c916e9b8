"""Input synthesis and comparison helpers shared by the tests.

Weights follow the reference tests' recipe (tests/test_gpu_kernels.cpp:65-71:
normal floats with 30 % zeros, quantized to PTQ1_0 by the encoder), or the
seeded benchmark generator. Activations are quantized by the oracle so GEMV
tests do not depend on the GPU quantizer.
"""
import numpy as np


def random_ptq(oracle, rng, N, K, scale=1.0):
    """PTQ1_0 bytes [N][K/128*28] like the reference's random_ptq (times
    `scale`, which sets the magnitude of the fp16 block scales)."""
    w = rng.standard_normal((N, K)).astype(np.float32) * np.float32(scale)
    w *= (rng.random((N, K)) >= 0.3).astype(np.float32)
    return oracle.quant_ptq1_0(w)


def random_mat(oracle, rng, N, K, scale=1.0):
    """(codes [N][K/4], scales [N][K/128]) of a random PTQ1_0 matrix."""
    src = random_ptq(oracle, rng, N, K, scale)
    return oracle.repack_rows(src, N, K)


def gen_mat(oracle, seed, mat, N, K):
    """(codes, scales) of the seeded synthetic generator's matrix."""
    src = oracle.gen_ptq1_0(seed, mat, N * K // 128)
    return oracle.repack_rows(src, N, K)


def random_act(oracle, rng, M, K, scale=1.0):
    x = (rng.standard_normal((M, K)) * scale).astype(np.float32)
    q, d, s = oracle.quantize_rows(x)
    return x, q, d, s


def rel_rms(a, ref):
    """The reference's rel-RMS error (tests/test_common.hpp:61-69)."""
    a = np.asarray(a, np.float64)
    ref = np.asarray(ref, np.float64)
    num = np.sum((a - ref) ** 2)
    den = np.sum(ref ** 2)
    return float(np.sqrt(num / den) if den > 0 else np.sqrt(num))


def assert_close_1e3(y, ref, what=""):
    """The path's float bar: rel-RMS <= 1e-3 and max |err| <= 1e-3 * max |ref|."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    rr = rel_rms(y, ref)
    mx = float(np.max(np.abs(y - ref))) if y.size else 0.0
    scale = float(np.max(np.abs(ref))) if ref.size else 0.0
    assert rr <= 1e-3, f"{what}: rel-rms {rr:.3e} > 1e-3"
    assert mx <= 1e-3 * max(scale, 1e-30), f"{what}: max err {mx:.3e} > 1e-3 * {scale:.3e}"
    return rr, mx
