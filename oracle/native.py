"""Build and bind ``oracle/ref_algo.c`` (TEST INFRASTRUCTURE — see ``oracle/__init__.py``).

``build()`` compiles the C restatement with gcc (-O2 -fopenmp, no fast-math so fp32
operations are IEEE) into ``oracle/_build/libfi_oracle.so``.  ``flash_forward`` /
``paged_forward`` run it on numpy fp16 arrays.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SRC = HERE / "ref_algo.c"
OUT_DIR = HERE / "_build"
LIB = OUT_DIR / "libfi_oracle.so"

CFLAGS = ["-O2", "-fPIC", "-shared", "-fopenmp", "-std=c11", "-Wall", "-fno-fast-math",
          "-ffp-contract=off"]

_lib = None


def build(force: bool = True) -> Path:
    if LIB.exists() and not force:
        return LIB
    OUT_DIR.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = ["gcc", *CFLAGS, str(SRC), "-o", str(tmp), "-lm"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{' '.join(cmd)}\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


def load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = ctypes.CDLL(str(LIB))
        i64, ptr, f32, i32 = ctypes.c_int64, ctypes.c_void_p, ctypes.c_float, ctypes.c_int
        lib.oracle_flash_fwd.restype = i32
        lib.oracle_flash_fwd.argtypes = [ptr, ptr, ptr, ptr, i32, i32, i32, i32, i32,
                                         *([i64] * 12), f32, ptr, i32, i32]
        lib.oracle_paged_fwd.restype = i32
        lib.oracle_paged_fwd.argtypes = [ptr, i64, i64, ptr, ptr, i32, i32, i32, ptr, i64,
                                         ptr, i32, ptr, i64, i64, i32, i32, i32, f32, i32]
        lib.oracle_f32_to_f16.argtypes = [ptr, ptr, i64]
        lib.oracle_f16_to_f32.argtypes = [ptr, ptr, i64]
        _lib = lib
    return _lib


def _u16(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float16)).view(np.uint16)


def flash_forward(q, k, v, sm_scale=None, programs=None, threads: int = 0) -> np.ndarray:
    """q [B, H, S, D], k/v [B, H_kv, S, D] fp16 -> fp16 [B, H, S, D] (see ref_algo.c).
    `programs`: optional list of (b, h) to evaluate; others are left 0."""
    q, k, v = _u16(q), _u16(k), _u16(v)
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    if sm_scale is None:
        sm_scale = D ** -0.5
    o = np.zeros_like(q)
    prog = None
    nprog = 0
    if programs is not None:
        prog = np.ascontiguousarray(np.asarray(programs, dtype=np.int32).reshape(-1, 2))
        nprog = prog.shape[0]
    rc = load().oracle_flash_fwd(
        q.ctypes.data, k.ctypes.data, v.ctypes.data, o.ctypes.data, B, H, Hkv, S, D,
        H * S * D, S * D, D, Hkv * S * D, S * D, D, Hkv * S * D, S * D, D,
        H * S * D, S * D, D, float(sm_scale),
        None if prog is None else prog.ctypes.data, nprog, threads)
    if rc:
        raise RuntimeError(f"oracle_flash_fwd failed ({rc})")
    return o.view(np.float16)


def paged_forward(q, k_cache, v_cache, block_table, block_size, context_lens,
                  sm_scale=None, threads: int = 0) -> np.ndarray:
    """q [B, H, D]; pools [N, bs, H_kv, D]; table int32 [B, M]; context_lens: int (one
    length for all rows, as the reference) or per-row sequence -> fp16 [B, H, D]."""
    q = _u16(q)
    kc, vc = _u16(k_cache), _u16(v_cache)
    bt = np.ascontiguousarray(np.asarray(block_table, dtype=np.int32))
    B, H, D = q.shape
    N, bs, Hkv, _ = kc.shape
    if sm_scale is None:
        sm_scale = D ** -0.5
    if isinstance(context_lens, (int, np.integer)):
        lens, ntok = None, int(context_lens)
    else:
        lens = np.ascontiguousarray(np.asarray(context_lens, dtype=np.int32))
        ntok = 0
    o = np.zeros_like(q)
    rc = load().oracle_paged_fwd(
        q.ctypes.data, H * D, D, kc.ctypes.data, vc.ctypes.data, N, bs, Hkv,
        bt.ctypes.data, bt.shape[1], None if lens is None else lens.ctypes.data, ntok,
        o.ctypes.data, H * D, D, B, H, D, float(sm_scale), threads)
    if rc:
        raise RuntimeError(f"oracle_paged_fwd failed ({rc})")
    return o.view(np.float16)


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    load().oracle_f32_to_f16(x.ctypes.data, y.ctypes.data, x.size)
    return y.view(np.float16)


def f16_to_f32(x: np.ndarray) -> np.ndarray:
    x = _u16(x)
    y = np.empty(x.shape, dtype=np.float32)
    load().oracle_f16_to_f32(x.ctypes.data, y.ctypes.data, x.size)
    return y
