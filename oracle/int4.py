"""numpy restatement of the reference's INT4 weight format and linear layer
(TEST INFRASTRUCTURE — see ``oracle/__init__.py``).

* ``quantize_int4_groupwise`` — loader.py:9-41 with the reference's fp16 tensor
  arithmetic as torch runs it on a CUDA device: ``amax = |w|.amax`` over each 128-wide
  group (fp16, exact); ``clamp(min=1e-6)`` against the fp16 value of 1e-6;
  ``w_max / 7.0`` — a CUDA tensor divided by a Python scalar is multiplied by the fp32
  reciprocal of the scalar (ATen's BinaryDivTrueKernel.cu), then rounded to fp16;
  ``round(w / scale)`` — an fp32 quotient rounded to fp16, then rounded half to even;
  clamp to [-8, 7]; packing (:31-36) puts k = 2j in the low nibble of byte j.
* ``unpack`` / ``dequantize`` — matmul.py:309-326 (``_dequant_storage``): nibble >= 8 means
  nibble - 16; weight = fp16(fp32(q) * fp32(scale)).
* ``matmul_exact`` — sum_k x[m, k] * w[n, k] in float64, the value an fp32-accumulating
  kernel approximates (matmul.py:14-132 fused; :135-186 on dequantized weights).

Pinned (tests/test_int4_oracle.py): hand-packed bytes; quantize then dequantize within half
a scale step of the input (plus fp16 rounding); each group's largest |w| maps to +-7;
scale within one fp16 rounding of amax/7; ``dequantize`` bit-exact against torch's own
CPU ops running the reference's ``_dequant_storage`` expression; planted nibble-order and
sign-extension mistakes fail.  The scale's reciprocal multiply and a true division give
the same fp16 scale for every possible fp16 ``w_max`` (checked exhaustively), and the GPU
tests compare the quantizer bit for bit with the reference's expression run by torch on
the device itself.
"""

from __future__ import annotations

import numpy as np

GROUP = 128
_INV7 = np.float32(1.0) / np.float32(7.0)      # fp32 reciprocal, as ATen computes it
_LO = np.float32(np.float16(1e-6))              # clamp bound after conversion to fp16


def quantize_int4_groupwise(w: np.ndarray, groupsize: int = GROUP, true_division=False):
    """fp16 w [N, K] -> (packed int8 [N, K/2], scales fp16 [N, K/groupsize]).
    ``true_division`` computes the scale as fp32(amax) / 7 (torch's CPU kernel) instead
    of the CUDA reciprocal multiply."""
    N, K = w.shape
    g = w.reshape(N, K // groupsize, groupsize).astype(np.float32)
    amax = np.abs(g).max(axis=-1, keepdims=True)                     # :24
    amax = np.maximum(amax, _LO)                                      # :25
    if true_division:
        scale = (amax / np.float32(7.0)).astype(np.float16)
    else:
        scale = (amax * _INV7).astype(np.float32).astype(np.float16)  # :26
    q16 = (g / scale.astype(np.float32)).astype(np.float32).astype(np.float16)  # :29
    q = np.clip(np.rint(q16.astype(np.float32)), -8, 7).astype(np.int8)          # :29-30
    q = q.reshape(N, K // 2, 2)
    packed = ((q[..., 0] & 0xF) | ((q[..., 1] & 0xF) << 4)).astype(np.uint8)   # :34-36
    return packed.view(np.int8), scale.reshape(N, K // groupsize)


def unpack(packed: np.ndarray) -> np.ndarray:
    """int8 [N, K/2] -> int8 [N, K] in [-8, 7] (matmul.py:316-321)."""
    b = packed.view(np.uint8).astype(np.int16)
    low = b & 0xF
    high = (b >> 4) & 0xF
    low = np.where(low >= 8, low - 16, low)
    high = np.where(high >= 8, high - 16, high)
    return np.stack([low, high], axis=-1).reshape(packed.shape[0], -1).astype(np.int8)


def dequantize(packed: np.ndarray, scales: np.ndarray, groupsize: int = GROUP) -> np.ndarray:
    """matmul.py:309-326 -> fp16 [N, K]."""
    q = unpack(packed).astype(np.float32)
    N, K = q.shape
    s = np.repeat(scales.astype(np.float32), groupsize, axis=1)
    return (q * s).astype(np.float16)


def matmul_exact(x: np.ndarray, w16: np.ndarray) -> np.ndarray:
    """x fp16 [M, K], w16 fp16 [N, K] -> float64 [M, N]."""
    return x.astype(np.float64) @ w16.astype(np.float64).T


def matmul_bound(x: np.ndarray, w16: np.ndarray) -> np.ndarray:
    """Error allowed for an fp16 output of an fp32-accumulated dot product: half an fp16
    ulp of the result (2^-11 relative, 2^-24 absolute below the normal range) plus one
    fp32 rounding of sum_k |x w| per sequential accumulation step (K/32 MFMA steps, a
    split reduction and slack: (K/32 + 16) * 2^-24).  A single misplaced weight moves
    the result by about sum_k |x w| / K, far above this."""
    K = x.shape[1]
    exact = matmul_exact(x, w16)
    mag = np.abs(x.astype(np.float64)) @ np.abs(w16.astype(np.float64)).T
    return np.abs(exact) * 2.0 ** -11 + mag * (K / 32 + 16) * 2.0 ** -24 + 2.0 ** -24
