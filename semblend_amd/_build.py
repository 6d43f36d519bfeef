"""Build recipe for libsemblend_hip.so (gfx950).

Compiles every ``csrc/*.hip`` translation unit with hipcc for gfx950 only and links them into
``semblend_amd/libsemblend_hip.so``, next to the Python package that loads it. Object files
go to ``_build/`` at the repository root (git-ignored).

Usage: ``python -m semblend_amd._build`` or ``semblend_amd._build.build()``.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
REPO = PKG_DIR.parent
BUILD_DIR = REPO / "_build"
LIB_NAME = "libsemblend_hip.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"

# Flags shared by every translation unit. Packed-FP32 instructions are disabled for device
# code; the host pass warns that it does not know the feature, which is harmless.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]

# Per-file extras. The row movers implement RoPE with torch's CPU rounding order (no fused
# multiply-add), so contraction is off there.
FILE_FLAGS = {
    "sb_move.hip": ["-ffp-contract=off"],
    "sb_qkv.hip": ["-ffp-contract=off"],
}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the semblend_amd HIP library cannot be built")


def _compile(src: Path, hipcc: str, verbose: bool) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc, *COMMON_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(ln for ln in res.stderr.splitlines() if noise not in ln)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = False) -> Path:
    """Compile all HIP sources and link the shared library. Always rebuilds."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources in {CSRC}")
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(lambda s: _compile(s, hipcc, verbose), sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
