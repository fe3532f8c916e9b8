"""CPU tests that pin the oracle (oracle/btf_oracle.c).

Each oracle function is checked three ways where possible:
  * against golden vectors written by the reference's own CPU code
    (tests/golden/golden.npz, see make_golden.py) -- runs everywhere;
  * against the reference build itself (oracle/_ref) on fresh random inputs
    -- runs where the reference checkout was available to build it;
  * against what the mathematics fixes, computed independently here in numpy
    (IEEE binary16 via numpy's float16, brute-force integer dots, the
    closed-form T2 addressing, the Sylvester Hadamard matrix, exhaustive
    base-3 round trips), chosen so a dropped term, wrong index or transposed
    operand fails.
"""
import os

import numpy as np
import pytest

from helpers import rel_rms

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


# ---------------------------------------------------------------- fp16
def test_fp16_widen_exhaustive(oracle, golden):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = np.array([oracle.fp16_to_f32(int(v)) for v in h], np.float32)
    ref_np = h.view(np.float16).astype(np.float32)
    finite = ~np.isnan(ref_np)
    assert np.array_equal(got[finite].view(np.uint32), ref_np[finite].view(np.uint32))
    assert np.all(np.isnan(got[~finite]))
    assert np.array_equal(got.view(np.uint32), golden["f16_widen"].view(np.uint32))


def test_fp16_round_matches_ieee_and_reference(oracle, golden):
    f = golden["f16_in"]
    got = np.array([oracle.f32_to_fp16(float(v)) for v in f], np.uint16)
    assert np.array_equal(got, golden["f16_out"])  # the reference's bd::f32_to_fp16
    with np.errstate(over="ignore"):
        ieee = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ieee)  # IEEE RNE (numpy)
    # every rounding boundary of the binary16 range: midpoints between
    # consecutive halves must go to the even neighbour
    h = np.arange(0x0000, 0x7bff, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)
    exact = mid.astype(np.float64) == (lo + hi) / 2
    got = np.array([oracle.f32_to_fp16(float(v)) for v in mid[exact]], np.uint16)
    even = np.where(h[exact] % 2 == 0, h[exact], h[exact] + 1).astype(np.uint16)
    assert np.array_equal(got, even)
    assert oracle.f32_to_fp16(float("nan")) & 0x7e00 == 0x7e00


def test_fp16_vs_reference_random(oracle, ref):
    rng = np.random.default_rng(11)
    f = rng.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    a = np.array([oracle.f32_to_fp16(float(v)) for v in f], np.uint16)
    b = np.array([ref.lib.ref_f32_to_fp16(float(v)) for v in f], np.uint16)
    assert np.array_equal(a, b)


# ---------------------------------------------------------------- PTQ1_0
def test_ptq_digit_decode_exhaustive(oracle):
    """Every 5-digit base-3 value encodes to a byte whose decode gives the
    digits back (qs bytes), and every 4-digit value for qh bytes."""
    codes = np.array(np.unravel_index(np.arange(243), (3,) * 5)).T  # digit 0 most significant
    for c in codes:
        trits = np.zeros(128, np.int8)
        for n in range(5):  # qs byte 0 holds elements 0, 16, 32, 48, 64
            trits[16 * n] = c[n] - 1
        for n in range(5):  # qs byte 16 holds elements 80, 88, 96, 104, 112
            trits[80 + 8 * n] = c[n] - 1
        for n in range(4):  # qh byte 24 holds elements 120, 122, 124, 126
            trits[120 + 2 * n] = c[n] - 1
        blk = oracle.encode_trits(trits, 0x3c00)
        assert [oracle.trit(blk, e) for e in range(128)] == list(trits)
        assert blk[26] == 0x00 and blk[27] == 0x3c


def test_ptq_encoder_matches_reference(oracle, golden):
    assert np.array_equal(oracle.quant_ptq1_0(golden["ptq_w"]), golden["ptq_src"])


def test_ptq_encoder_vs_reference_random(oracle, ref):
    rng = np.random.default_rng(3)
    w = rng.standard_normal((20, 2048)).astype(np.float32) * (rng.random((20, 2048)) >= 0.3)
    w[0] = 0.0  # all-zero blocks: scale 0, trits 0
    assert np.array_equal(oracle.quant_ptq1_0(w), ref.quant_ptq1_0(w))


def test_ptq_encoder_semantics(oracle, golden):
    """Decoded trits are lround(w / amax) of each 128-block; scale = fp16(amax)."""
    w = golden["ptq_w"]
    src = golden["ptq_src"]
    N, K = w.shape
    blocks = w.reshape(N, K // 128, 128)
    amax = np.abs(blocks).max(axis=2)
    inv = np.where(amax != 0, np.float32(1) / amax, 0).astype(np.float32)
    v = blocks * inv[:, :, None]
    want = np.where(np.abs(v) >= 0.5, np.sign(v), 0).astype(np.int8)  # lround: half away from zero
    blk = src.reshape(N, K // 128, 28).astype(np.int64)
    for r in range(0, N, 9):
        for b in range(K // 128):
            got = [oracle.trit(blk[r, b].astype(np.uint8), e) for e in range(128)]
            assert got == list(want[r, b])
            assert blk[r, b, 26] | (blk[r, b, 27] << 8) == amax[r, b].astype(np.float16).view(np.uint16)


# ---------------------------------------------------------------- T2 repack
def _numpy_repack(src, N, K):
    """Independent restatement: decode trits with the byte formula, place code
    (trit + 1) of column e at byte (e/32)*8 + ((e/16)%2)*4 + e%4, bit
    ((e/4)%4)*2 of its 128-block (docs/packed-layout.md:31-36)."""
    blk = src.reshape(N, K // 128, 28).astype(np.uint32)
    e = np.arange(128)
    byte_idx = np.where(e < 80, e % 16, np.where(e < 120, 16 + (e - 80) % 8, 24 + (e - 120) % 2))
    digit = np.where(e < 80, e // 16, np.where(e < 120, (e - 80) // 8, (e - 120) // 2))
    p3 = np.array([1, 3, 9, 27, 81], np.int64)[digit]
    b = blk[:, :, byte_idx].astype(np.int64)
    code = (((b * p3) & 0xFF) * 3) >> 8  # trit + 1
    out_byte = (e // 32) * 8 + ((e // 16) % 2) * 4 + e % 4
    shift = ((e // 4) % 4) * 2
    codes = np.zeros((N, K // 128, 32), np.int64)
    for j in range(128):
        codes[:, :, out_byte[j]] |= code[:, :, j] << shift[j]
    scales = (blk[:, :, 26] | (blk[:, :, 27] << 8)).astype(np.uint16)
    return codes.astype(np.uint8).reshape(N, K // 4), scales.reshape(N, K // 128)


def test_repack_matches_reference_fixture(oracle, golden):
    c, s = oracle.repack_rows(golden["rp_src"], 41, 1024)
    assert np.array_equal(c, golden["rp_codes"]) and np.array_equal(s, golden["rp_scales"])
    c, s = oracle.repack_rows(golden["ptq_src"], 37, 1024)
    assert np.array_equal(c, golden["rpe_codes"]) and np.array_equal(s, golden["rpe_scales"])


def test_repack_matches_closed_form(oracle):
    rng = np.random.default_rng(17)
    src = rng.integers(0, 256, (29, 2048 // 128 * 28), dtype=np.uint8)
    c, s = oracle.repack_rows(src, 29, 2048)
    cn, sn = _numpy_repack(src, 29, 2048)
    assert np.array_equal(c, cn) and np.array_equal(s, sn)


def test_repack_codes_equal_trits(oracle, golden):
    """test_packed.cpp:29-41: every packed code is the source trit + 1."""
    src, (N, K) = golden["ptq_src"], golden["ptq_w"].shape
    codes, scales = oracle.repack_rows(src, N, K)
    blk = src.reshape(N, K // 128, 28)
    hist = np.zeros(3, int)
    for r in range(N):
        for e in range(0, K, 7):
            c = oracle.packed_code(codes[r], e)
            assert c == oracle.trit(blk[r, e // 128], e % 128) + 1
            hist[c] += 1
    assert (hist > 0).all()


def test_repack_vs_reference_random(oracle, ref):
    rng = np.random.default_rng(23)
    src = rng.integers(0, 256, (64, 5120 // 128 * 28), dtype=np.uint8)
    a = oracle.repack_rows(src, 64, 5120)
    b = ref.repack_rows(src, 64, 5120)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


# ---------------------------------------------------------------- Q8
def _numpy_q8(x):
    """IEEE float32 restatement of quantize_row_q8_0 (round half to even)."""
    xb = x.reshape(x.shape[0], -1, 32).astype(np.float32)
    amax = np.abs(xb).max(axis=2)
    d = (amax / np.float32(127)).astype(np.float16).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(amax != 0, np.float32(127) / amax, np.float32(0)).astype(np.float32)
    q = np.rint(xb * idv[:, :, None]).astype(np.int32)
    return q.reshape(x.shape).astype(np.int8), d, q.sum(axis=2).astype(np.int32)


def test_q8_matches_reference_fixture(oracle, golden):
    q, d, s = oracle.quantize_rows(golden["q8_x"])
    assert np.array_equal(q, golden["q8_q"])
    assert np.array_equal(d.view(np.uint32), golden["q8_d"].view(np.uint32))
    assert np.array_equal(s, golden["q8_s"])


def test_q8_matches_ieee_restatement(oracle):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((16, 2048)) * 3).astype(np.float32)
    x[3] *= 1e-6
    x[4, :64] = 0.0
    q, d, s = oracle.quantize_rows(x)
    qn, dn, sn = _numpy_q8(x)
    assert np.array_equal(q, qn) and np.array_equal(s, sn)
    assert np.array_equal(np.abs(d), dn)  # zero blocks may carry -0 (see below)


def test_q8_invariants(oracle, golden):
    """test_packed.cpp:44-59: q * d == round_q8_0(x) exactly, sum q == s;
    zero block -> d = q = s = 0; +-amax -> +-127; .5 ties go to even."""
    x = golden["q8_x"]
    q, d, s = oracle.quantize_rows(x)
    deq = q.reshape(x.shape[0], -1, 32).astype(np.float32) * d[:, :, None]
    assert np.array_equal(deq.reshape(x.shape), oracle.round_q8_0(x))
    assert np.array_equal(oracle.round_q8_0(x), golden["q8_round"])
    assert np.array_equal(q.reshape(x.shape[0], -1, 32).astype(np.int32).sum(axis=2), s)
    assert d[0, 0] == 0 and not q[0, :32].any() and s[0, 0] == 0
    assert np.signbit(d[0, 1])  # all -0 block: the CPU loop keeps the last zero's sign
    assert q[1, 31] == 127
    assert list(q[1, :4]) == [2, -4, 2, -4]  # id = 1: rint(2.5) = 2, rint(-3.5) = -4


def test_q8_vs_reference_random(oracle, ref):
    rng = np.random.default_rng(29)
    x = (rng.standard_normal((9, 4096)) * 5).astype(np.float32)
    a = oracle.quantize_rows(x)
    b = ref.emu_prep(x)
    for u, v in zip(a, b[:3]):
        assert np.array_equal(u.view(np.uint8), v.view(np.uint8))


# ---------------------------------------------------------------- prep
def test_prep_matches_reference_fixture(oracle, golden):
    for i in range(5):
        n, blk, norm, perm, signs, M, hd, nk, rep = golden[f"prep{i}_case"]
        q, d, s, xn = oracle.prep(golden[f"prep{i}_x"], golden[f"prep{i}_w"] if norm else None, 1e-6, int(blk),
                                  int(hd), int(nk), int(rep), golden[f"prep{i}_signs"] if signs else None)
        assert np.array_equal(q, golden[f"prep{i}_q"]), i
        assert np.array_equal(d.view(np.uint32), golden[f"prep{i}_d"].view(np.uint32)), i
        assert np.array_equal(s, golden[f"prep{i}_s"]), i
        assert np.array_equal(xn.view(np.uint32), golden[f"prep{i}_xn"].view(np.uint32)), i


def test_fwht_matches_reference_and_hadamard(oracle, golden):
    for n in (2, 64, 1024):
        v = golden[f"fwht{n}_in"]
        out = oracle.fwht(v)
        assert np.array_equal(out.view(np.uint32), golden[f"fwht{n}_out"].view(np.uint32))
        # Sylvester matrix H[r][c] = (-1)^popcount(r & c), normalised
        r = np.arange(n)
        H = (-1.0) ** np.array([[bin(a & b).count("1") for b in r] for a in r])
        assert np.allclose(out, H @ v.astype(np.float64) / np.sqrt(n), rtol=1e-5, atol=1e-5)


def test_hadamard_perm_is_tiled_to_grouped(oracle):
    """out[d + hd*(r + rep*k)] = x[d + hd*(k + nk*r)] before signs and WHT:
    with block 1 the WHT is the identity (one element, scale 1/sqrt(1))."""
    hd, nk, rep = 4, 3, 2
    n = hd * nk * rep
    x = np.arange(n, dtype=np.float32)
    out = np.zeros(n, np.float32)
    import ctypes as C
    oracle.lib.btf_or_hadamard_input(1, hd, nk, rep, None, x.ctypes.data_as(C.c_void_p), n,
                                     out.ctypes.data_as(C.c_void_p))
    want = np.zeros(n, np.float32)
    for k in range(nk):
        for r in range(rep):
            for d in range(hd):
                want[d + hd * (r + rep * k)] = x[d + hd * (k + nk * r)]
    assert np.array_equal(out, want)


def test_prep_vs_reference_random(oracle, ref):
    rng = np.random.default_rng(31)
    for n, blk, norm, perm, signs in [(1024, 256, 1, 1, 1), (3072, 1024, 1, 0, 0), (512, 0, 0, 0, 0)]:
        x = (rng.standard_normal((3, n)) * 2).astype(np.float32)
        w = rng.standard_normal(n).astype(np.float32)
        sg = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float32)
        hd, nk, rep = (32, n // 64, 2) if perm else (0, 0, 0)
        args = (x, w if norm else None, 1e-5, blk, hd, nk, rep, sg if signs else None)
        for u, v in zip(oracle.prep(*args), ref.emu_prep(*args)):
            assert np.array_equal(u.view(np.uint8), v.view(np.uint8))


# ---------------------------------------------------------------- GEMV
def _trits_from_codes(codes, K):
    """Decode T2 codes with the closed-form addressing (docs/packed-layout.md)."""
    N = codes.shape[0]
    e = np.arange(K)
    byte = (e // 128) * 32 + ((e % 128) // 32) * 8 + ((e % 128 // 16) % 2) * 4 + e % 4
    shift = ((e % 128 // 4) % 4) * 2
    return ((codes[:, byte] >> shift) & 3).astype(np.int64) - 1


@pytest.mark.parametrize("M", [1, 3, 8, 13])
def test_gemv_int_matches_fixture_and_brute_force(oracle, golden, M):
    codes, K = golden["gemv_codes"], 1024
    q, s = golden[f"gemv{M}_q"], golden[f"gemv{M}_s"]
    I = oracle.gemv_i32(codes, K, q, s)
    assert np.array_equal(I, golden[f"gemv{M}_I"])
    t = _trits_from_codes(codes, K)  # [N][K]
    brute = np.einsum("nsk,msk->mns", t.reshape(t.shape[0], K // 32, 32),
                      q.astype(np.int64).reshape(M, K // 32, 32))
    assert np.array_equal(I, brute)


@pytest.mark.parametrize("M", [1, 3, 8, 13])
def test_gemv_float_matches_emulator_fixture(oracle, golden, M):
    codes, scales, K = golden["gemv_codes"], golden["gemv_scales"], 1024
    q, d, s = golden[f"gemv{M}_q"], golden[f"gemv{M}_d"], golden[f"gemv{M}_s"]
    y = oracle.gemv(codes, scales, K, q, d, s, nthreads=1)
    assert np.array_equal(y.view(np.uint32), golden[f"gemv{M}_y"].view(np.uint32))
    y3 = oracle.gemv(codes, scales, K, q, d, s, nthreads=3)  # threads split rows only
    assert np.array_equal(y3.view(np.uint32), y.view(np.uint32))
    ya = oracle.gemv(codes, scales, K, q, d, s, y=golden[f"gemv{M}_y0"].copy(), add=True)
    assert np.array_equal(ya.view(np.uint32), golden[f"gemv{M}_yadd"].view(np.uint32))
    # double-precision restatement (the reference's ref_gemv, test_gpu_kernels.cpp:177-193)
    I = golden[f"gemv{M}_I"].astype(np.float64)
    f = scales.astype(np.uint16).view(np.float16).astype(np.float64)
    fs = np.repeat(f, 4, axis=1)  # scale of sub-block s = scale[s/4]
    yd = np.einsum("mns,ns,ms->mn", I, fs, d.astype(np.float64))
    assert rel_rms(y, yd) <= 1e-5


def test_gemv_matches_matvec_raw(oracle, golden):
    """test_packed.cpp:63-85: packed dot == matvec_raw with ggml activation rounding."""
    codes, scales, K = golden["gemv_codes"], golden["gemv_scales"], 1024
    q, d, s = oracle.quantize_rows(golden["gemv1_x"])
    y = oracle.gemv(codes, scales, K, q, d, s)[0]
    assert rel_rms(y, golden["mv_y"]) < 1e-5


def test_gemv_vs_reference_random(oracle, ref):
    rng = np.random.default_rng(37)
    w = rng.standard_normal((50, 3072)).astype(np.float32) * (rng.random((50, 3072)) >= 0.3)
    codes, scales = oracle.repack_rows(oracle.quant_ptq1_0(w), 50, 3072)
    for M in (1, 5):
        x = (rng.standard_normal((M, 3072)) * 2).astype(np.float32)
        q, d, s = oracle.quantize_rows(x)
        a = oracle.gemv(codes, scales, 3072, q, d, s)
        b = ref.emu_gemv(codes, scales, 3072, q, d, s)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_swiglu_is_silu_times_up(oracle):
    g = np.linspace(-30, 30, 1001).astype(np.float32)
    u = np.linspace(2, -2, 1001).astype(np.float32)
    got = oracle.swiglu(g, u)
    want = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.allclose(got, want, rtol=1e-6, atol=1e-30)


# ---------------------------------------------------------------- generator
def test_generator_distribution_and_determinism(oracle):
    nb = 20000
    src = oracle.gen_ptq1_0(0, 3, nb)
    codes, scales = oracle.repack_blocks(src, nb)
    t = _trits_from_codes(codes.reshape(1, -1), nb * 128)[0]
    frac = np.bincount(t + 1, minlength=3) / t.size
    assert np.allclose(frac, [0.3, 0.4, 0.3], atol=0.003)
    f = scales.view(np.float16).astype(np.float64)
    assert f.min() >= 0.00999 and f.max() <= 0.05001
    assert abs(f.mean() - 0.03) < 0.001
    assert np.array_equal(oracle.gen_ptq1_0(0, 3, 500, first_block=777), src[777:1277])
    assert not np.array_equal(oracle.gen_ptq1_0(0, 4, 10), src[:10])
    assert not np.array_equal(oracle.gen_ptq1_0(1, 3, 10), src[:10])


# ---------------------------------------------------------------- either side of the chain
@pytest.mark.parametrize("block", [0, 128, 1024])
def test_embed_matches_fixture(oracle, golden, block):
    E, V = 2048, 40
    x = oracle.embed(golden["emb_codes"], golden["emb_scales"], golden["emb_toks"], E, V, block,
                     golden["emb_signs"] if block else None)
    assert np.array_equal(x.view(np.uint32), golden[f"emb{block}_x"].view(np.uint32))


def test_embed_inverse_transform_round_trip(oracle, golden):
    """The forward input transform (signs, then the normalised FWHT per block,
    ref/bonsai-decoder/src/cpu_ops.cpp:90-111) undoes the embedding's inverse
    one (FWHT, then signs): both factors are involutions, so the order and
    the 1/sqrt(block) scaling are pinned."""
    E, V = 2048, 40
    x0 = oracle.embed(golden["emb_codes"], golden["emb_scales"], golden["emb_toks"], E, V, 0)
    sg = golden["emb_signs"]
    for block in (128, 1024):
        xi = oracle.embed(golden["emb_codes"], golden["emb_scales"], golden["emb_toks"], E, V, block, sg)
        back = np.stack([np.concatenate([oracle.fwht((r * sg)[b:b + block]) for b in range(0, E, block)]) for r in xi])
        assert np.max(np.abs(back - x0)) <= 1e-5 * max(1.0, float(np.max(np.abs(x0))))
        assert not np.allclose(xi, x0)


def test_embed_rejects_token_out_of_range(oracle, golden):
    with pytest.raises(ValueError):
        oracle.embed(golden["emb_codes"], golden["emb_scales"], np.array([0, 40], np.int32), 2048, 40)


def test_argmax_matches_fixture_and_numpy(oracle, golden):
    for i in range(4):
        l = golden[f"am{i}_l"]
        assert oracle.argmax(l) == int(golden[f"am{i}_best"]) == int(np.argmax(l))


def test_embed_and_argmax_vs_reference_random(oracle, ref):
    from helpers import random_mat
    rng = np.random.default_rng(77)
    for E, block in [(1024, 0), (5120, 1024), (3072, 256)]:
        V = 50
        codes, scales = random_mat(oracle, rng, V, E)
        toks = rng.integers(0, V, 6).astype(np.int32)
        sg = np.where(rng.random(E) < 0.5, -1.0, 1.0).astype(np.float32) if block else None
        a = oracle.embed(codes, scales, toks, E, V, block, sg)
        b = ref.emu_embed(codes, scales, toks, E, V, block, sg)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    for n in (1, 7, 1000, 248320):
        l = rng.standard_normal(n).astype(np.float32)
        if n > 10:
            l[[3, n - 2]] = l.max() + 1
        assert oracle.argmax(l) == ref.argmax(l)


def test_base3_digit_identity_of_the_direct_gemv():
    """The PTQ1_0-direct GEMV (csrc/gemv_b3.hip) forms digit n of a block byte
    b as H(n+1) - 3 H(n), H(n) = floor(b 3^n / 256), instead of the
    reference's ((u8)(b 3^n) * 3) >> 8 (src/types.hpp:70-78): equal for every
    byte and digit, with the operand bounds the kernel relies on (b 3^5 fits
    16-bit lanes, H(n) <= 80 for n <= 4 is a signed dot4 operand, 3 H(4)
    fits a byte)."""
    for b in range(256):
        H = [(b * 3 ** n) >> 8 for n in range(6)]
        assert b * 3 ** 5 < 1 << 16 and max(H[:5]) <= 80 and 3 * H[4] <= 240
        for n in range(5):
            ref = (((b * 3 ** n) & 0xFF) * 3) >> 8
            assert ref == H[n + 1] - 3 * H[n], (b, n)
