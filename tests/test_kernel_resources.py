"""Register budget of every kernel, checked at compile time (no GPU): each HIP source is
compiled for gfx950 with the library's own flags and the compiler's kernel-resource remarks,
and no kernel may use scratch memory (spilled registers or arrays moved to private memory).
A spill in a row mover costs HBM traffic and occupancy (a refactor that took the address of
the mover's kernel argument once spilled 16 VGPRs and slowed the four-donor scatter 2.4x)."""

from __future__ import annotations

import re
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

from semblend_amd import _build


def _remarks(src):
    cmd = [_build._hipcc(), *_build.COMMON_FLAGS, *_build.FILE_FLAGS.get(src.name, []),
           "-Rpass-analysis=kernel-resource-usage", "--cuda-device-only", "-c", str(src),
           "-o", "/dev/null"]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    out, cur = {}, None
    for line in r.stderr.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            cur = m.group(1)
            out[cur] = {}
            continue
        m = re.search(r"remark:\s+(VGPRs|ScratchSize \[bytes/lane\]|VGPRs Spill|Occupancy "
                      r"\[waves/SIMD\]): (\d+)", line)
        if m and cur:
            out[cur][m.group(1)] = int(m.group(2))
    return src.name, out


@pytest.fixture(scope="module")
def resources():
    try:
        _build._hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    srcs = sorted(_build.CSRC.glob("*.hip"))
    with ThreadPoolExecutor(len(srcs)) as ex:
        return dict(ex.map(_remarks, srcs))


def test_no_kernel_uses_scratch(resources):
    bad = {f"{f}: {k}": v for f, ks in resources.items() for k, v in ks.items()
           if v.get("ScratchSize [bytes/lane]", 0) or v.get("VGPRs Spill", 0)}
    assert not bad, bad


def test_hot_kernels_keep_their_occupancy(resources):
    """Plain and delta-rotating row movers run 8 waves per SIMD (the other rotation forms at
    least 5), the attention kernel 2."""
    ks = {k: v for f in resources.values() for k, v in f.items()}
    movers = {k: v for k, v in ks.items() if "move_rows_kernel" in k}
    # mangled template arguments: <DT, VB, ROT, SRCM, DSTM, INLINE>; ROT 0 plain, 1 delta
    fast = {k: v for k, v in movers.items()
            if re.search(r"move_rows_kernelILi\d+ELi\d+ELi[01]E", k)}
    assert fast and all(v["Occupancy [waves/SIMD]"] == 8 for v in fast.values()), fast
    assert all(v["Occupancy [waves/SIMD]"] >= 5 for v in movers.values())
    attn = [v for k, v in ks.items() if "attn_mfma_kernel" in k]
    assert attn and all(v["Occupancy [waves/SIMD]"] >= 2 for v in attn)
