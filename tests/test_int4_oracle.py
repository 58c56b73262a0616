"""Pins for oracle/int4.py (CPU only).

The reference ships no INT4 vectors; the oracle is pinned by hand-packed bytes, by the
closed-form properties of symmetric rounding quantization, and by torch's own CPU
arithmetic running the reference's expressions (loader.py:20-38, matmul.py:309-326) —
torch as an independent fp16/fp32 arithmetic engine, not the reference's code.
"""

import numpy as np
import pytest
import torch

from oracle import int4 as OI

U16 = 2.0 ** -11


def _weights(rng, N, K, scale=0.05):
    w = rng.standard_normal((N, K)).astype(np.float32) * scale
    w[0, :128] = 0.0                       # an all-zero group (clamped amax)
    w[1, 128:256] *= 1e-4                  # tiny groups: subnormal scales
    w[2, :128] = 3.0e4 * np.sign(w[2, :128])  # near the top of fp16
    return w.astype(np.float16)


def test_hand_packed_bytes_and_nibble_order():
    w = np.zeros((1, 128), np.float16)
    w[0, :8] = [1, -1, 7, -7, 0, 3, -2, 5]      # amax 7 -> scale fp16(7 * fp32(1/7)) = 1
    packed, scales = OI.quantize_int4_groupwise(w)
    assert scales[0, 0] == np.float16(1.0)
    assert packed.view(np.uint8)[0, :4].tolist() == [0xF1, 0x97, 0x30, 0x5E]
    assert np.array_equal(OI.unpack(packed)[0, :8], [1, -1, 7, -7, 0, 3, -2, 5])
    # planted mistakes: high nibble first, or n >= 8 read as n - 8
    b = packed.view(np.uint8)[0, :4].astype(int)
    swapped = np.stack([b >> 4, b & 0xF], -1).reshape(-1)
    assert not np.array_equal(np.where(swapped >= 8, swapped - 16, swapped), [1, -1, 7, -7, 0, 3, -2, 5])
    wrong_sign = np.stack([b & 0xF, b >> 4], -1).reshape(-1)
    assert not np.array_equal(np.where(wrong_sign >= 8, wrong_sign - 8, wrong_sign), [1, -1, 7, -7, 0, 3, -2, 5])


def test_unpack_full_byte_range():
    packed = np.arange(256, dtype=np.uint8).view(np.int8).reshape(1, 256)
    q = OI.unpack(packed)[0].reshape(256, 2)
    for byte in range(256):
        lo, hi = byte & 0xF, byte >> 4
        assert q[byte, 0] == (lo - 16 if lo >= 8 else lo)
        assert q[byte, 1] == (hi - 16 if hi >= 8 else hi)


def test_quantize_round_trip_bounds():
    rng = np.random.default_rng(0)
    w = _weights(rng, 64, 512)
    packed, scales = OI.quantize_int4_groupwise(w)
    deq = OI.dequantize(packed, scales).astype(np.float64)
    s = np.repeat(scales.astype(np.float64), 128, axis=1)
    w64 = w.astype(np.float64)
    # |q - w/s| <= 1/2 + the fp16 rounding of the quotient; then one fp16 rounding of q*s
    bound = s * (0.5 + 8 * U16) + np.abs(deq) * U16 + 2.0 ** -24
    assert np.all(np.abs(deq - w64) <= bound)
    # each group's largest |w| maps to +-7 (unless the group is below the clamp)
    q = OI.unpack(packed).astype(int).reshape(64, 4, 128)
    g = np.abs(w64).reshape(64, 4, 128)
    idx = g.argmax(-1)
    top = np.take_along_axis(np.abs(q), idx[..., None], -1)[..., 0]
    amax = g.max(-1)
    assert np.all(top[amax > 1e-5] == 7)
    # the scale is amax / 7 within one fp16 rounding (two roundings through fp32)
    sc = scales.astype(np.float64)
    ref = np.maximum(amax, float(np.float16(1e-6))) / 7
    assert np.all(np.abs(sc - ref) <= ref * (U16 + 2.0 ** -23) + 2.0 ** -24)


def test_dequantize_matches_torch_cpu_ops():
    """_dequant_storage's expression (matmul.py:203-214) run by torch on the CPU."""
    rng = np.random.default_rng(1)
    packed = rng.integers(-128, 128, (48, 384), dtype=np.int16).astype(np.int8)
    scales = (rng.standard_normal((48, 6)) * 0.01).astype(np.float16)
    scales[0, 0] = np.float16(1.2e-7)   # subnormal
    p = torch.from_numpy(packed).to(torch.uint8)
    low = (p & 0xF).to(torch.int8)
    high = ((p >> 4) & 0xF).to(torch.int8)
    low = torch.where(low >= 8, low - 16, low).to(torch.float16)
    high = torch.where(high >= 8, high - 16, high).to(torch.float16)
    wq = torch.stack([low, high], dim=-1).reshape(48, 768).reshape(48, 6, 128)
    ref = (wq.float() * torch.from_numpy(scales).unsqueeze(-1).float()).reshape(48, 768).half()
    got = OI.dequantize(packed, scales)
    assert np.array_equal(got.view(np.uint16), ref.numpy().view(np.uint16))


def test_quantize_matches_torch_cpu_ops():
    """loader.py:20-38's expressions run by torch on the CPU, where ``w_max / 7.0`` is a
    true fp32 division: bit-exact with the oracle's ``true_division`` form, and with the
    reciprocal form the device uses (the two agree on every fp16 input, below)."""
    rng = np.random.default_rng(2)
    w = _weights(rng, 256, 1024)
    wt = torch.from_numpy(w).reshape(256, -1, 128)
    w_max = torch.clamp(wt.abs().amax(dim=-1, keepdim=True), min=1e-6)
    scale = w_max / 7.0
    wq = torch.clamp(torch.round(wt / scale.to(wt.dtype)), -8, 7).to(torch.int8)
    wq = wq.reshape(256, -1, 64, 2)
    packed_t = ((wq[..., 0] & 0xF) | ((wq[..., 1] & 0xF) << 4)).reshape(256, 512).to(torch.int8)
    p_div, s_div = OI.quantize_int4_groupwise(w, true_division=True)
    assert np.array_equal(p_div, packed_t.numpy())
    assert np.array_equal(s_div.view(np.uint16), scale.reshape(256, 8).numpy().view(np.uint16))
    p_rec, s_rec = OI.quantize_int4_groupwise(w)
    assert np.array_equal(p_rec, p_div) and np.array_equal(s_rec.view(np.uint16), s_div.view(np.uint16))


def test_scale_reciprocal_and_division_agree_on_every_fp16():
    """``w_max / 7.0`` on a device tensor multiplies by the fp32 reciprocal of 7; on the CPU
    it divides.  Over every positive finite fp16 ``w_max`` (and the clamp value fp16(1e-6))
    both give the same fp16 scale, so the scale step is pinned whichever form runs."""
    h = np.arange(1, 0x7C00, dtype=np.uint16).view(np.float16)
    a = np.maximum(h.astype(np.float32), np.float32(np.float16(1e-6)))
    rec = (a * (np.float32(1.0) / np.float32(7.0))).astype(np.float16)
    div = (a / np.float32(7.0)).astype(np.float16)
    assert np.array_equal(rec.view(np.uint16), div.view(np.uint16))
    # the oracle's two forms agree on the same inputs
    w = np.zeros((h.size // 128, 128), np.float16)
    w[:, 0] = h[: w.shape[0] * 128].reshape(-1, 128)[:, -1]
    _, s_rec = OI.quantize_int4_groupwise(w)
    _, s_div = OI.quantize_int4_groupwise(w, true_division=True)
    assert np.array_equal(s_rec.view(np.uint16), s_div.view(np.uint16))


@pytest.mark.parametrize("seed", [3, 4])
def test_matmul_bound_catches_a_misplaced_weight(seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((8, 3072))).astype(np.float16)
    w = (rng.standard_normal((64, 3072)) * 0.02).astype(np.float16)
    exact = OI.matmul_exact(x, w)
    bound = OI.matmul_bound(x, w)
    assert np.all(np.abs(exact.astype(np.float16).astype(np.float64) - exact) <= bound)
    w2 = w.copy()
    w2[:, [10, 11]] = w2[:, [11, 10]]           # two neighbouring k swapped (nibble swap)
    moved = np.abs(OI.matmul_exact(x, w2) - exact)
    assert np.mean(moved > bound) > 0.9


def test_matmul_exact_small_integers():
    x = np.array([[1, 2, 3, 4]], np.float16)
    w = np.array([[1, 0, -1, 2], [0.5, 0.5, 0.5, 0.5]], np.float16)
    assert OI.matmul_exact(x, w).tolist() == [[6.0, 5.0]]
