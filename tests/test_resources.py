"""Static resource gate of the HIP kernels (CPU; no GPU needed).

Every .hip source of the library is compiled for gfx950 with the compiler's
kernel-resource remarks (-Rpass-analysis=kernel-resource-usage), with the
library's own flags. The test fails if any kernel uses scratch memory
(ScratchSize > 0: a private stack frame or spilled registers, whose accesses
count in the same memory counter as the weight stream and would stall it) or
spills VGPRs or SGPRs. This is the AMD counterpart of the reference's build
check on its NVIDIA kernels (cmake/check_kernel_resources.cmake:15-61, which
fails on spill stores/loads, local memory or a stack frame).
"""
import os
import re
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "bonsai-ternary-fast_amd")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def _flags():
    """HIPFLAGS of the library's Makefile (one source of truth)."""
    text = open(os.path.join(PKG, "Makefile")).read().replace("\\\n", " ")
    m = re.search(r"^HIPFLAGS\s*:=\s*(.*)$", text, re.M)
    flags = m.group(1).replace("$(ARCH)", "gfx950").split()
    per_file = {}
    for f, extra in re.findall(r"^_build/(\w+)\.o:\s*HIPFLAGS\s*\+=\s*(.*)$", text, re.M):
        per_file[f] = extra.split()
    return flags, per_file


def _sources():
    text = open(os.path.join(PKG, "Makefile")).read().replace("\\\n", " ")
    m = re.search(r"^SRCS\s*:=\s*(.*)$", text, re.M)
    return m.group(1).split()


def _remarks(src):
    flags, per_file = _flags()
    stem = os.path.splitext(os.path.basename(src))[0]
    cmd = [HIPCC] + flags + per_file.get(stem, []) + ["--cuda-device-only", "-c", os.path.join(PKG, src),
                                                      "-o", os.devnull, "-Rpass-analysis=kernel-resource-usage"]
    p = subprocess.run(cmd, capture_output=True, text=True, cwd=PKG)
    assert p.returncode == 0, f"{src} does not compile:\n{p.stderr[-2000:]}"
    kernels, cur = [], None
    for line in p.stderr.splitlines():
        m = re.search(r"remark:\s+(Function Name|ScratchSize \[bytes/lane\]|VGPRs Spill|SGPRs Spill|VGPRs|"
                      r"TotalSGPRs|Occupancy \[waves/SIMD\]|LDS Size \[bytes/block\]):\s*(\S+)", line)
        if not m:
            continue
        key, val = m.group(1), m.group(2)
        if key == "Function Name":
            cur = {"name": val}
            kernels.append(cur)
        elif cur is not None:
            cur[key] = int(val)
    return kernels


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_no_kernel_uses_scratch_or_spills():
    srcs = _sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        results = dict(zip(srcs, ex.map(_remarks, srcs)))
    bad, n = [], 0
    for src, kernels in results.items():
        for k in kernels:
            n += 1
            if k.get("ScratchSize [bytes/lane]", 0) or k.get("VGPRs Spill", 0) or k.get("SGPRs Spill", 0):
                bad.append(f"{src}: {k['name']}: scratch {k.get('ScratchSize [bytes/lane]')} B/lane, "
                           f"VGPR spill {k.get('VGPRs Spill')}, SGPR spill {k.get('SGPRs Spill')}, "
                           f"VGPRs {k.get('VGPRs')}")
    assert n > 0, "no kernel resource remarks were parsed"
    assert not bad, "kernels with scratch or spills:\n" + "\n".join(bad)


def _assembly(src):
    flags, per_file = _flags()
    stem = os.path.splitext(os.path.basename(src))[0]
    cmd = [HIPCC] + flags + per_file.get(stem, []) + ["--cuda-device-only", "-S", os.path.join(PKG, src), "-o", "-"]
    p = subprocess.run(cmd, capture_output=True, text=True, cwd=PKG)
    assert p.returncode == 0, f"{src} does not compile:\n{p.stderr[-2000:]}"
    return p.stdout


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_no_kernel_issues_flat_memory_instructions():
    """No kernel reaches memory through a flat (generic) instruction. A flat
    access counts in both the vector-memory and the LDS/scalar counters, so a
    wait for its result (or any LDS wait after it) also waits for every
    global load issued before it -- in the step kernel, the weight stream in
    flight. Pointers that come back generic from LDS are cast to the global
    or constant address space where they are used."""
    srcs = _sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        asm = dict(zip(srcs, ex.map(_assembly, srcs)))
    bad = []
    for src, text in asm.items():
        for line in text.splitlines():
            s = line.strip()
            if s.startswith(("flat_load", "flat_store", "flat_atomic")):
                bad.append(f"{src}: {s}")
    assert not bad, "flat memory instructions:\n" + "\n".join(bad[:20])
