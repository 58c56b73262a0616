"""Pins for oracle/rmsnorm.py (CPU only)."""

import numpy as np
import torch

from oracle import rmsnorm as ON


def _rows(seed, M=16, H=3072, scale=1.0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((M, H)) * scale).astype(np.float16)


def test_matches_torch_rms_norm():
    """torch.nn.functional.rms_norm in fp32 on the CPU (the reference's own check of its
    kernel, README.md:140-143) agrees with the float64 form to fp32 accuracy."""
    x = _rows(0)
    w = (np.random.default_rng(1).standard_normal(3072) * 0.5 + 1).astype(np.float16)
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x).float(), (3072,),
                                       torch.from_numpy(w).float(), eps=1e-5).double().numpy()
    exact = ON.rms_norm_exact(x, w)
    assert np.max(np.abs(ref - exact) / (np.abs(exact) + 1e-6)) < 1e-5
    assert np.all(np.abs(ref.astype(np.float16).astype(np.float64) - exact) <= ON.norm_bound(exact))


def test_constant_row_closed_form_and_scale_invariance():
    w = (np.linspace(0.5, 2.0, 256)).astype(np.float16)
    for c in (0.25, 3.0, -7.5):
        x = np.full((1, 256), c, np.float16)
        y = ON.rms_norm_exact(x, w)
        assert np.allclose(y, c / np.sqrt(c * c + 1e-5) * w.astype(np.float64), rtol=1e-12)
    x = _rows(2, 4, 256)
    y1 = ON.rms_norm_exact(x, w)
    y2 = ON.rms_norm_exact((x.astype(np.float32) * 4).astype(np.float16), w)  # exact scaling
    assert np.allclose(y1, y2, rtol=1e-5)


def test_planted_mistakes_fail():
    x = _rows(3, 4, 512)
    w = (np.random.default_rng(4).standard_normal(512) * 0.3 + 1).astype(np.float16)
    exact = ON.rms_norm_exact(x, w)
    x64, w64 = x.astype(np.float64), w.astype(np.float64)
    summed = x64 / np.sqrt(np.sum(x64 * x64, -1, keepdims=True) + 1e-5) * w64
    no_eps = x64 / np.sqrt(np.mean(x64 * x64, -1, keepdims=True)) * w64
    squared = x64 / np.sqrt(np.mean(x64 * x64, -1, keepdims=True) + 1e-5) * w64 * w64
    for wrong in (summed, squared):
        assert np.mean(np.abs(wrong - exact) > ON.norm_bound(exact)) > 0.5
    tiny = (x * np.float16(1e-3)).astype(np.float16)   # eps matters when x is small
    assert np.any(np.abs(ON.rms_norm_exact(tiny, w) - tiny.astype(np.float64)
                         / np.sqrt(np.mean(tiny.astype(np.float64) ** 2, -1, keepdims=True)) * w64)
                  > ON.norm_bound(ON.rms_norm_exact(tiny, w)))
    assert no_eps.shape == exact.shape
