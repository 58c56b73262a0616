"""Checks on the gfx950 code the kernels compile to (CPU only: hipcc cross-compiles).

The direct-to-LDS copies of the decode and INT4 kernels are issued through inline asm
(``lds_copy16`` in csrc/common.h) that sets M0 without telling the compiler.  That is
sound only while nothing else in those kernels uses M0, so every M0 write in their device
code must be a copy helper's, immediately followed by its ``buffer_load_dwordx4 ... lds``,
and no other instruction may name M0.
"""

import re
import subprocess

import pytest

from fast_infer_amd import build

SOURCES = ["paged_decode.hip", "int4_gemm.hip"]


def _device_asm(src: str, tmp_path) -> str:
    try:
        hipcc = build._hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    out = tmp_path / (src + ".s")
    cmd = [hipcc, *build.HIPCC_FLAGS, *build.FILE_FLAGS.get(src, []), "--cuda-device-only",
           "-S", "-w", str(build.CSRC / src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    return out.read_text()


@pytest.mark.parametrize("src", SOURCES)
def test_m0_is_only_set_by_the_copy_helper(src, tmp_path):
    lines = [ln.split(";")[0].strip() for ln in _device_asm(src, tmp_path).splitlines()]
    lines = [ln for ln in lines if ln and not ln.startswith((".", "#"))]
    copies = 0
    for i, ln in enumerate(lines):
        if not re.search(r"\bm0\b", ln):
            continue
        assert re.fullmatch(r"s_mov_b32 m0, s\d+", ln), f"{src}: M0 used by `{ln}`"
        nxt = lines[i + 1]
        assert nxt.startswith("buffer_load_dwordx4") and nxt.endswith(" lds"), \
            f"{src}: M0 write not followed by a copy: `{ln}` / `{nxt}`"
        copies += 1
    assert copies > 0, f"{src}: no direct-to-LDS copies found"
