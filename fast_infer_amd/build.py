"""Build the gfx950 HIP library ``libfastinfer_hip.so`` in-tree with hipcc.

Usage: ``python -m fast_infer_amd.build`` (or ``build_library()`` from Python).
Each ``csrc/*.hip`` is compiled to an object in ``csrc/_build/`` in parallel, then
linked into ``fast_infer_amd/libfastinfer_hip.so``.  The library exports only the
``extern "C"`` entry points declared in ``include/fast_infer_amd.h``.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = CSRC / "_build"
LIB_NAME = "libfastinfer_hip.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"

# -packed-fp32-ops: keep hipcc from emitting packed fp32 VALU instructions.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

# Per-source additions.  The prefill kernel's inputs are finite and its masked scores are
# -inf (not NaN), so its max operations need no NaN quieting (saves a v_max per input).
FILE_FLAGS = {
    "flash_prefill.hip": ["-fno-honor-nans"],
}


# Extra libraries linked into the extension (none: every kernel is built here).
LINK_LIBS: list = []


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def _compile(hipcc: str, src: Path, extra: list[str]) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, *FILE_FLAGS.get(src.name, []), *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{res.stdout}{res.stderr}")
    return obj


def build_library(verbose: bool = False, extra_flags: list[str] | None = None) -> Path:
    """Compile every csrc/*.hip for gfx950 and link the shared library; returns its path."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    extra = list(extra_flags or [])
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(lambda s: _compile(hipcc, s, extra), sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), *LINK_LIBS,
           "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build_library(verbose=True, extra_flags=sys.argv[1:])
