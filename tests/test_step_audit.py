"""CPU tests of the step program's host planning (btf_hip_step_audit: no
device is touched).

* Store audit: every global store a launch of the benchmark's programs makes
  -- the 27B-shape sweep (64 layers + the 248,320-row output projection) and
  the whole-token program (embedding, 257 prepped GEMVs, greedy pick) -- is
  replayed over all workgroups with the kernel's own placement and address
  functions and must lie inside a buffer the program owns or was given. The
  reference's build runs a resource check over its kernels
  (cmake/check_kernel_resources.cmake:15-61); this is the same kind of gate
  for the step kernel's stores.
* Store count: on small programs the replay visits exactly the stores the
  publish code makes (counted here from the op shapes), for several grid
  sizes, so the audit covers every unit of every workgroup.
* Write-after-read guards: an op that reads only a prefix of its input
  vector observes only the writers of that prefix; a guard the full read
  would make redundant must stay when only the prefix is read.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "bonsai-ternary-fast_amd", "libbtf_hip.so")
pytestmark = pytest.mark.skipif(not os.path.exists(LIB), reason="libbtf_hip.so not built")


@pytest.fixture(scope="module")
def lib():
    import btf_hip
    return btf_hip


@pytest.fixture(scope="module")
def bench():
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    import bench as b
    return b


class FakeWeights:
    """Distinct 256-byte-aligned addresses for every matrix (never read)."""

    def __init__(self):
        self.next = 0x7A0000000000
        self.tab = {}

    def __call__(self, name, l):
        if (name, l) not in self.tab:
            self.tab[(name, l)] = (self.next, self.next + (1 << 32))
            self.next += 1 << 33
        return self.tab[(name, l)]


def host_vecs(lib, lengths):
    """Vectors with host buffers (only their addresses are used)."""
    bufs = [np.zeros(n, np.float32) for n in lengths]
    return [lib.StepVec(n, b.ctypes.data) for n, b in zip(lengths, bufs)], bufs


def check(res):
    assert res["outside"] == 0, res["first_outside"]
    assert res["stores"] > 0


@pytest.mark.parametrize("G", [256, 240])
def test_audit_sweep_27b(lib, bench, G):
    """The benchmark's default program: 257 GEMVs, one plain prologue."""
    vecs, keep = host_vecs(lib, bench.SWEEP_VECS)
    ops = bench.sweep_ops(lib, FakeWeights(), bench.LAYERS)
    res = lib.step_audit(vecs, ops, G)
    check(res)
    assert not res["full"] and res["ops"] == 4 * bench.LAYERS + 1 + 2  # + prologue quantizes of slots 0 and 2
    del keep


def test_audit_whole_token_27b(lib, bench):
    """The whole-token program: embedding, prepped GEMVs, pick and counter."""
    vecs, keep = host_vecs(lib, bench.TOKEN_VECS)
    tok, pos = np.zeros(1, np.int32), np.zeros(1, np.int32)
    sg = lambda n: np.ones(n, np.float32)
    nw = lambda n: np.ones(n, np.float32)
    arrays = []

    def a(x):
        arrays.append(x)
        return x.ctypes.data

    norms = [(a(nw(bench.E)), a(nw(bench.E))) for _ in range(bench.LAYERS)]
    signs = [(a(sg(bench.E)), a(sg(bench.E)), a(sg(bench.E)), a(sg(bench.F))) for _ in range(bench.LAYERS)]
    hx = lambda s: lib.Hx(block=1024, signs=s)
    ops = bench.token_ops(lib, FakeWeights(), bench.LAYERS, tok.ctypes.data, pos.ctypes.data, hx, norms, signs,
                          a(nw(bench.E)), a(sg(bench.E)), a(sg(bench.E)))
    res = lib.step_audit(vecs, ops, 256)
    check(res)
    assert res["full"]
    # no GEMV of the whole token keeps a write-after-read wait (the data flow orders every read)
    assert res["guards"] == 0
    del keep, arrays


def expected_stores(units_wg, N, q8, f32, plain, sq):
    """Stores of publish_unit over the given units (32 values each)."""
    n = 0
    for u in units_wg:
        valid = max(0, min(32, N - 32 * u))
        n += valid * ((1 if f32 else 0) + (1 if plain else 0))
        n += 10 if q8 else 0
        n += 2 if sq else 0
    return n


@pytest.mark.parametrize("G", [1, 7, 64, 256])
def test_audit_counts_every_store(lib, G):
    """Two chained GEMVs, the second with a partial last unit: the replay
    visits each published value, Q8 word and control word exactly once."""
    Gm = lib.GemvMode
    N2 = 2044
    vecs, keep = host_vecs(lib, (1024, 1024, N2))
    w = FakeWeights()
    ops = [lib.StepGemv(Gm.kStore, 1024, 1024, *w("a", 0), 0, 1),
           lib.StepGemv(Gm.kStore, 1024, N2, *w("b", 0), 1, 2)]
    res = lib.step_audit(vecs, ops, G)
    check(res)
    units = lambda n: range((n + 31) // 32)
    # the prologue quantize of slot 0 (its Q8 words only), op 0 (Q8 words for op 1, fp32 LL words,
    # the plain output: it is slot 1's final writer), op 1 (fp32 LL words, plain output); 3 control
    # words per workgroup
    want = (expected_stores(units(1024), 1024, True, False, False, False) +
            expected_stores(units(1024), 1024, True, True, True, False) +
            expected_stores(units(N2), N2, False, True, True, False) + 3 * G)
    assert res["stores"] == want
    del keep


def guard_program(lib, K_read):
    """Vector 1 (D, 1024 values, user data) is read, rewritten twice, read,
    and written a fourth time by op 6, whose Q8 buffer is then the one its
    version 0 used: op 6 must wait until every workgroup has read version 0
    (op 0), unless the data flow already orders it. Op 6 reads the first
    K_read values of vector 0 (8192 values), which op 5 writes on every
    workgroup (256 units); reading all of it tells op 6's workgroups that
    every workgroup had finished op 4 (and so op 0), reading a prefix tells
    them that only of the prefix's writers."""
    Gm = lib.GemvMode
    w = FakeWeights()
    g = lambda mode, K, N, name, i, o: lib.StepGemv(mode, K, N, *w(name, 0), i, o)
    return [g(Gm.kStore, 1024, 1024, "z", 1, 2),       # 0: reads D v0
            g(Gm.kStore, 1024, 1024, "d1", 4, 1),      # 1: D v1
            g(Gm.kStore, 1024, 1024, "r1", 1, 2),      # 2: reads D v1
            g(Gm.kStore, 1024, 1024, "d2", 4, 1),      # 3: D v2
            g(Gm.kStore, 1024, 1024, "r2", 1, 2),      # 4: reads D v2
            g(Gm.kStore, 1024, 8192, "x", 4, 0),       # 5: A, all workgroups write
            g(Gm.kStore, K_read, 1024, "r", 0, 1),     # 6: D v3 (reuses v0's Q8 buffer)
            g(Gm.kStore, 1024, 1024, "r3", 1, 3)]      # 7: reads D v3


def test_guard_kept_when_only_a_prefix_is_read(lib):
    lengths = (8192, 1024, 1024, 1024, 1024)
    vecs, keep = host_vecs(lib, lengths)
    full = lib.step_audit(vecs, guard_program(lib, 8192), 256)
    prefix = lib.step_audit(vecs, guard_program(lib, 1024), 256)
    check(full)
    check(prefix)
    # reading all of vector 0 implies op 6's wait; reading 1024 of its 8192
    # values observes 32 of the 256 writers, so the wait stays
    assert prefix["guards"] == full["guards"] + 1
    del keep
