"""The kernels' double-precision sin/cos (``sb::sincos_cw`` in semblend_amd/csrc/sb_sincos.h,
rounded to fp32 by ``sincos_rn``) against the C library's double sin and cos, both rounded to
float, on the CPU: every RoPE angle fp32(delta) * inv_freq for |delta| <= 65536 and the 64
inverse frequencies of head_dim 128 at bases 1e4, 5e5 and 1e6, plus 2^20 pseudo-random fp32
angles up to 2^32. The header is compiled for the host by g++ from tests/sincos_check.cpp.
Any float that differs from the library's rounding outside a near-midpoint band fails."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path_factory.mktemp("sincos") / "sincos_check"
    subprocess.run([gxx, "-O2", "-std=c++17", "-o", str(exe), str(HERE / "sincos_check.cpp"),
                    "-lm"], check=True, capture_output=True, text=True)
    return exe


@pytest.mark.parametrize("mode", ["grid", "wide"])
def test_sincos_cw_matches_libm_rounding(checker, mode):
    r = subprocess.run([str(checker), mode], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert " 0 outside the tie band" in r.stdout, r.stdout


def test_sincos_cw_catches_a_wrong_constant(tmp_path):
    """The check is sharp: the same header with 2/pi replaced by 4/pi (a plausible slip in
    the reduction constant) fails it."""
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    src = (HERE.parent / "semblend_amd" / "csrc" / "sb_sincos.h").read_text()
    bad = src.replace("kTwoOverPi = 0x1.45f306dc9c883p-1", "kTwoOverPi = 0x1.45f306dc9c883p+0")
    assert bad != src
    hdr_dir = tmp_path / "semblend_amd" / "csrc"
    hdr_dir.mkdir(parents=True)
    (hdr_dir / "sb_sincos.h").write_text(bad)
    tests_dir = tmp_path / "tests"
    tests_dir.mkdir()
    shutil.copy(HERE / "sincos_check.cpp", tests_dir / "sincos_check.cpp")
    exe = tmp_path / "bad_check"
    subprocess.run([gxx, "-O2", "-std=c++17", "-o", str(exe), str(tests_dir / "sincos_check.cpp"),
                    "-lm"], check=True, capture_output=True, text=True)
    r = subprocess.run([str(exe), "wide"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 1
