"""numpy restatement of the reference's rotary position embedding
(TEST INFRASTRUCTURE — see ``oracle/__init__.py``).

* ``precompute_freqs`` — kernels/rope.py:9-16: angle(p, i) = p * theta^(-2j/D) with
  j = i mod D/2 (the half-width frequency vector concatenated twice), cos/sin in fp32.
* ``rotate_half`` — kernels/rope.py:19-23: [x1, x2] -> [-x2, x1] on the last axis.
* ``apply_rope`` — kernels/rope.py:26-44 as the reference's fp16 tensor arithmetic,
  op by op: ``q * cos`` (fp16 result), ``rotate_half(q) * sin`` (fp16), their sum (fp16);
  each product/sum formed in fp32 and rounded to fp16 (numpy ``astype`` rounds to
  nearest even).  Positions broadcast over the head axis (``cos.unsqueeze(1)``).
* ``rope_store_kv`` — apply_rope at table rows ``start + t`` followed by the pool
  placement of ``kv.scatter`` for rotated k and v (model.py:101 then :117 / :120).

Pinned (tests/test_rope_oracle.py) by closed forms, not by restating the formula:
position 0 (cos = 1, sin = 0) is the identity bit for bit; every output is within one
fp16 rounding of the float64 rotation x·cos + rotate_half(x)·sin; rotations compose
(angle a then b equals a+b within rounding) and preserve each pair's norm; a quarter
turn maps the pair (x_i, x_{i+64}) to (-x_{i+64}, x_i) exactly; planted pairing and sign
mistakes fail those checks.
"""

from __future__ import annotations

import numpy as np

from . import kv as OK


def precompute_freqs(head_dim: int, max_seq_len: int, theta: float = 500000.0):
    """kernels/rope.py:9-16 in float32 -> (cos, sin) [max_seq_len, head_dim]."""
    freq = (1.0 / (np.float32(theta) ** (np.arange(0, head_dim, 2, dtype=np.float32)
                                          / np.float32(head_dim)))).astype(np.float32)
    pos = np.arange(max_seq_len, dtype=np.float32)
    ang = np.outer(pos, freq).astype(np.float32)
    ang = np.concatenate([ang, ang], axis=-1)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def rotate_half(x: np.ndarray) -> np.ndarray:
    """kernels/rope.py:19-23."""
    d = x.shape[-1]
    return np.concatenate([-x[..., d // 2:], x[..., :d // 2]], axis=-1)


def _mul16(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    return (a.astype(np.float32) * b.astype(np.float32)).astype(np.float16)


def _add16(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    return (a.astype(np.float32) + b.astype(np.float32)).astype(np.float16)


def rope_rows(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """x [..., T, H, D] fp16; cos/sin [T, D] fp16 -> fp16, the arithmetic of rope.py:37-42."""
    c = cos.astype(np.float16)[:, None, :]
    s = sin.astype(np.float16)[:, None, :]
    return _add16(_mul16(x, c), _mul16(rotate_half(x), s))


def apply_rope(q: np.ndarray, k: np.ndarray, cos: np.ndarray, sin: np.ndarray):
    """kernels/rope.py:26-44: q [B, S, Hq, D], k [B, S, Hkv, D] fp16; cos/sin [S, D] fp16."""
    return rope_rows(q, cos, sin), rope_rows(k, cos, sin)


def rope_store_kv(q, k, v, cos_table, sin_table, starts, k_pool=None, v_pool=None,
                  table=None, block_size=None):
    """Rotate q, k at table rows start_b + t (starts: int or per-row list) and, with pools,
    scatter rotated k and v like ``kv.scatter``.  A token whose row is outside the table
    is skipped entirely: its q/k rows are returned unrotated (the kernel leaves them
    unwritten) and nothing of it reaches the pool.  Returns (q_rot, k_rot); pools are
    updated in place."""
    B, T = q.shape[:2]
    st = [int(starts)] * B if np.isscalar(starts) else [int(s) for s in starts]
    q_rot = q.copy()
    k_rot = k.copy()
    rows = cos_table.shape[0]
    for b in range(B):
        lo = min(max(0, -st[b]), T)           # valid tokens: 0 <= start + t < rows
        hi = max(lo, min(T, rows - st[b]))
        if hi <= lo:
            continue
        pos = np.arange(lo, hi) + st[b]
        c = cos_table[pos]
        s = sin_table[pos]
        q_rot[b, lo:hi] = rope_rows(q[b, lo:hi], c, s)
        k_rot[b, lo:hi] = rope_rows(k[b, lo:hi], c, s)
        if k_pool is not None:
            OK.scatter(k_pool, v_pool, [table[b]], k_rot[b:b + 1, lo:hi], v[b:b + 1, lo:hi],
                       st[b] + lo, block_size)
    return q_rot, k_rot
