"""GPU test of the no-allocation greedy pick (btf_hip_launch_argmax_noalloc):
its scratch is the library's static per-GPU array, so it takes no workspace.
Checked against btf_hip_launch_argmax (with its `part` workspace) through the
C ABI on two calls in a row, the second with a smaller input (the static
scratch keeps the first call's keys; the second must not read them), and
on the edge inputs of the greedy pick (ties, all -inf, NaN, all NaN)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def dev(a):
    return _torch().from_numpy(np.ascontiguousarray(a).copy()).cuda()


def host(t):
    _torch().cuda.synchronize()
    return t.cpu().numpy()


def stream():
    return _torch().cuda.current_stream().cuda_stream


def pick_both(hip, logits):
    torch = _torch()
    V = logits.size
    x = dev(logits)
    part = torch.zeros(hip.argmax_part_bytes(V) // 4, dtype=torch.int32, device="cuda")
    a = torch.full((1,), -5, dtype=torch.int32, device="cuda")
    b = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    hip.launch_argmax(x, V, part, a, stream())
    hip.launch_argmax_noalloc(x, V, b, stream())
    return int(host(a)[0]), int(host(b)[0])


def test_noalloc_pick_matches_the_workspace_pick(hip, oracle):
    rng = np.random.default_rng(41)
    # 600000 logits (256 parts: the whole static scratch), then 1000 (one
    # part): the second call leaves 255 stale keys in the scratch
    big = rng.standard_normal(600000).astype(np.float32)
    big[123456] = 50.0
    small = rng.standard_normal(1000).astype(np.float32)
    for l in (big, small):
        a, b = pick_both(hip, l)
        assert a == b == oracle.argmax(l)
    # a smaller input whose maximum is below the first call's: stale keys would win
    tiny = (rng.standard_normal(3000) - 10).astype(np.float32)
    a, b = pick_both(hip, tiny)
    assert a == b == oracle.argmax(tiny)
    V = 248320
    cases = []
    t = rng.standard_normal(V).astype(np.float32)
    t[[V // 3, V - 2]] = t.max() + 2
    cases.append(t)
    t = np.full(V, -np.inf, np.float32)
    t[[5, V - 1]] = -7.0
    cases.append(t)
    t = rng.standard_normal(V).astype(np.float32)
    t[V // 2] = np.nan
    cases.append(t)
    cases.append(np.full(V, np.nan, np.float32))
    for l in cases:
        a, b = pick_both(hip, l)
        assert a == b == oracle.argmax(l)


def test_noalloc_pick_rejects_bad_arguments(hip):
    torch = _torch()
    x = torch.zeros(16, dtype=torch.float32, device="cuda")
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    assert hip.launch_argmax_noalloc_raw(x, 0, out) == hip.BTF_ERR_ARGS
    assert hip.launch_argmax_noalloc_raw(None, 16, out) == hip.BTF_ERR_ARGS
    assert hip.launch_argmax_noalloc_raw(x, 16, None) == hip.BTF_ERR_ARGS
