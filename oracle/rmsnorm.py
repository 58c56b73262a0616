"""numpy restatement of the reference's RMSNorm (TEST INFRASTRUCTURE — see
``oracle/__init__.py``).

* ``rms_norm_exact`` — kernels/rms_norm.py:8-24 in float64: y = x / sqrt(mean(x^2) + eps)
  * weight (the reference computes it in fp32 and rounds y to fp16).
* ``rms_norm`` — the same rounded to fp16.
* ``norm_bound`` — how far an fp32 evaluation rounded to fp16 may land from the float64
  value: one fp16 rounding (2^-11 relative, 2^-25 absolute below the normal range) plus the
  fp32 errors of the sum of squares, the reciprocal square root and the two products,
  well under another 2^-11 — so one fp16 ulp, 2^-10 relative, with 2^-24 absolute.

Pinned (tests/test_rmsnorm_oracle.py): against torch.nn.functional.rms_norm on the CPU (the
reference's own check, README.md:140-143); a constant row c gives c / sqrt(c^2 + eps) *
weight; scaling x leaves y unchanged while eps is negligible; planted mistakes (sum in
place of the mean, eps left out, weight squared) fail.
"""

from __future__ import annotations

import numpy as np


def rms_norm_exact(x: np.ndarray, weight: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    x64 = x.astype(np.float64)
    r = 1.0 / np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True) + eps)
    return x64 * r * weight.astype(np.float64)


def rms_norm(x: np.ndarray, weight: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    return rms_norm_exact(x, weight, eps).astype(np.float16)


def norm_bound(exact: np.ndarray) -> np.ndarray:
    return np.abs(exact) * 2.0 ** -10 + 2.0 ** -24
