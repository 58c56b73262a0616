"""Pins for oracle/rope.py (CPU only).

The reference holds no RoPE vectors; its own checks are "Triton RoPE vs x*cos +
rotate_half(x)*sin" (README.md:140-143).  The oracle is pinned by what the mathematics
fixes instead: the float64 closed form of the table, the identity at position 0, the
exact quarter turn, the error bound of a two-rounding rotation, norm preservation and
composition; each test also shows that a plausible mistake (rotation partner off by one,
sign flipped, half-width vector not repeated, a fused single rounding) fails it.
"""

import numpy as np
import pytest
import torch

from oracle import kv as OK
from oracle import rope as OR

U16 = 2.0 ** -11        # fp16 unit roundoff
TINY16 = 2.0 ** -25     # half the smallest fp16 subnormal: absolute error of one rounding


def _rows(rng, *shape, scale=4.0):
    return (rng.standard_normal(shape) * scale).astype(np.float16)


def _exact(x, c, s, partner):
    """float64 rotation x*c + partner(x)*s with c/s broadcast over the head axis."""
    x64 = x.astype(np.float64)
    return x64 * c[:, None, :] + partner(x64) * s[:, None, :]


def _half_partner(x):
    d = x.shape[-1]
    return np.concatenate([-x[..., d // 2:], x[..., :d // 2]], axis=-1)


def _bound(x, c, s):
    """|fl(fl(xc) + fl(ys)) - (xc + ys)| <= u(|xc| + |ys|) + u|xc + ys| (1 + u) + 3 tiny."""
    x64 = x.astype(np.float64)
    a = np.abs(x64 * c[:, None, :])
    b = np.abs(_half_partner(x64) * s[:, None, :])
    return U16 * (a + b) * (2 + U16) + 3 * TINY16


# --- the table ---------------------------------------------------------------------------

def test_freqs_match_float64_closed_form():
    cos, sin = OR.precompute_freqs(128, 4096, 500000.0)
    assert cos.shape == (4096, 128) and cos.dtype == np.float32
    p = np.arange(4096, dtype=np.float64)[:, None]
    j = np.arange(128) % 64
    ang = p * 500000.0 ** (-2.0 * j / 128)
    # angles are formed in fp32: error <= |angle| * 2^-23 (+ cos/sin rounding)
    tol = np.abs(ang) * 2.0 ** -22 + 2.0 ** -23
    assert np.all(np.abs(cos - np.cos(ang)) <= tol)
    assert np.all(np.abs(sin - np.sin(ang)) <= tol)
    # half-width frequency vector repeated twice: columns i and i+64 share an angle
    assert np.array_equal(cos[:, :64], cos[:, 64:]) and np.array_equal(sin[:, :64], sin[:, 64:])
    # a planted interleaved layout (j = i // 2, the other common RoPE convention) fails
    bad = p * 500000.0 ** (-2.0 * (np.arange(128) // 2) / 128)
    assert not np.all(np.abs(cos - np.cos(bad)) <= tol)


def test_freqs_match_torch_restatement_of_the_model():
    """fast_infer_amd.precompute_freqs (torch, the model's table builder) and the numpy
    oracle agree to the fp32 rounding of the angle: the two libraries' pow differ in the
    last bit of some frequencies, which position p scales by p.  (About 1% of the fp16
    entries then round differently, so parity tests hand both sides the same table: the
    kernels take the table as an input.)"""
    from fast_infer_amd.rope import precompute_freqs as torch_freqs

    c_t, s_t = torch_freqs(128, 4096, 500000.0)
    c_n, s_n = OR.precompute_freqs(128, 4096, 500000.0)
    p = np.arange(4096, dtype=np.float64)[:, None]
    ang = p * 500000.0 ** (-2.0 * (np.arange(128) % 64) / 128)
    tol = np.abs(ang) * 2.0 ** -21 + 2.0 ** -22
    assert np.all(np.abs(c_t.numpy() - c_n) <= tol)
    assert np.all(np.abs(s_t.numpy() - s_n) <= tol)


# --- application --------------------------------------------------------------------------

def test_position_zero_is_identity():
    rng = np.random.default_rng(0)
    x = _rows(rng, 5, 3, 128)
    c = np.ones((5, 128), np.float16)
    s = np.zeros((5, 128), np.float16)
    out = OR.rope_rows(x, c, s)
    assert np.array_equal(out, x)  # values (-0 == +0)


def test_quarter_turn_is_exact_rotate_half():
    rng = np.random.default_rng(1)
    x = _rows(rng, 4, 2, 128)
    c = np.zeros((4, 128), np.float16)
    s = np.ones((4, 128), np.float16)
    out = OR.rope_rows(x, c, s)
    assert np.array_equal(out[..., :64], -x[..., 64:])
    assert np.array_equal(out[..., 64:], x[..., :64])
    # a planted partner mistake (neighbour instead of i + 64) fails
    wrong = np.concatenate([-x[..., 1::2], x[..., 0::2]], axis=-1)
    assert not np.array_equal(out, wrong)


@pytest.mark.parametrize("scale", [4.0, 1e-3, 3e3])
def test_within_two_roundings_of_float64_rotation(scale):
    rng = np.random.default_rng(2)
    cos, sin = OR.precompute_freqs(128, 4096)
    pos = rng.integers(0, 4096, 64)
    c = cos[pos].astype(np.float16)
    s = sin[pos].astype(np.float16)
    x = _rows(rng, 64, 8, 128, scale=scale)
    out = OR.rope_rows(x, c, s).astype(np.float64)
    c64, s64 = c.astype(np.float64), s.astype(np.float64)
    err = np.abs(out - _exact(x, c64, s64, _half_partner))
    assert np.all(err <= _bound(x, c64, s64))

    # planted mistakes fail: sign of the partner flipped, or partner off by one
    flipped = _exact(x, c64, s64, lambda y: -_half_partner(y))
    assert np.any(np.abs(out - flipped) > _bound(x, c64, s64))
    shifted = _exact(x, c64, s64, lambda y: np.roll(_half_partner(y), 1, axis=-1))
    assert np.any(np.abs(out - shifted) > _bound(x, c64, s64))


def test_two_roundings_not_one():
    """The reference rounds the products to fp16 before adding (three fp16 tensor ops);
    a fused x*c + y*s with one rounding differs on some inputs — the oracle follows the
    reference's form."""
    rng = np.random.default_rng(3)
    cos, sin = OR.precompute_freqs(128, 4096)
    pos = rng.integers(1, 4096, 256)
    c = cos[pos].astype(np.float16)
    s = sin[pos].astype(np.float16)
    x = _rows(rng, 256, 4, 128)
    out = OR.rope_rows(x, c, s)
    fused = _exact(x, c.astype(np.float64), s.astype(np.float64), _half_partner).astype(np.float16)
    assert np.any(out != fused)


def test_matches_torch_fp16_tensor_ops_on_cpu():
    """The reference's fp16 arithmetic (kernels/rope.py:37-42) executed by torch on the CPU:
    each fp16 product and sum is one fp32 op rounded to fp16, which is how the oracle
    models it.  Bit-exact."""
    rng = np.random.default_rng(4)
    cos, sin = OR.precompute_freqs(128, 4096)
    pos = rng.integers(0, 4096, 32)
    c = torch.from_numpy(cos[pos]).half().unsqueeze(1)
    s = torch.from_numpy(sin[pos]).half().unsqueeze(1)
    x = _rows(rng, 2, 32, 8, 128)
    xt = torch.from_numpy(x)
    rh = torch.cat([-xt[..., 64:], xt[..., :64]], dim=-1)
    ref = (xt * c + rh * s).numpy()
    out = OR.rope_rows(x, cos[pos], sin[pos])
    assert np.array_equal(out.view(np.uint16), ref.view(np.uint16))


def test_norm_preserved_and_rotations_compose():
    rng = np.random.default_rng(5)
    cos, sin = OR.precompute_freqs(128, 4096)
    x = _rows(rng, 1, 16, 128, scale=1.0)
    a, b = 700, 1300
    one = lambda y, p: OR.rope_rows(y, cos[[p]], sin[[p]])
    ab = one(one(x, a), b).astype(np.float64)
    direct = one(x, a + b).astype(np.float64)
    x64 = x.astype(np.float64)
    pair_norm = lambda y: np.hypot(y[..., :64], y[..., 64:])
    # each pair (x_i, x_{i+64}) keeps its norm within a few fp16 roundings
    assert np.all(np.abs(pair_norm(direct) - pair_norm(x64)) <= 4 * U16 * pair_norm(x64) + 1e-6)
    # composition: angle a then b equals a + b up to rounding (table angles add exactly
    # because the frequency vector is shared; the fp32 table rounding is below fp16's)
    assert np.max(np.abs(ab - direct)) <= 8 * U16 * np.max(np.abs(x64))


# --- the fused store ----------------------------------------------------------------------

def test_rope_store_kv_places_rotated_rows_and_skips_out_of_table():
    rng = np.random.default_rng(6)
    cos, sin = OR.precompute_freqs(128, 200)
    c16, s16 = cos.astype(np.float16), sin.astype(np.float16)
    B, T, Hq, Hkv, bs = 3, 40, 4, 2, 16
    q = _rows(rng, B, T, Hq, 128)
    k = _rows(rng, B, T, Hkv, 128)
    v = _rows(rng, B, T, Hkv, 128)
    starts = [0, 170, -5]       # row 1 runs past the 200-row table; row 2 starts before it
    table = np.full((B, 16), -1, np.int32)
    table[:, :13] = rng.permutation(64)[:39].reshape(B, 13)
    kp = _rows(rng, 64, bs, Hkv, 128)
    vp = _rows(rng, 64, bs, Hkv, 128)
    kp0, vp0 = kp.copy(), vp.copy()
    q_rot, k_rot = OR.rope_store_kv(q, k, v, c16, s16, starts, kp, vp, table, bs)

    written = np.zeros(kp.shape[:2], bool)
    for b, st in enumerate(starts):
        for t in range(T):
            p = st + t
            if not 0 <= p < 200:
                assert np.array_equal(q_rot[b, t], q[b, t]) and np.array_equal(k_rot[b, t], k[b, t])
                continue
            assert np.array_equal(q_rot[b, t], OR.rope_rows(q[b, t][None, None], c16[[p]], s16[[p]])[0, 0])
            phys, slot = table[b, p // bs], p % bs
            assert phys >= 0
            assert np.array_equal(kp[phys, slot], k_rot[b, t])
            assert np.array_equal(vp[phys, slot], v[b, t])
            written[phys, slot] = True
    # every other slot keeps its bytes
    assert np.array_equal(kp[~written], kp0[~written]) and np.array_equal(vp[~written], vp0[~written])
    assert written.sum() == 40 + 30 + 35


def test_rope_store_kv_equals_apply_then_scatter():
    """With every position inside the table the fused oracle is apply_rope followed by
    the pinned kv.scatter."""
    rng = np.random.default_rng(7)
    cos, sin = OR.precompute_freqs(128, 512)
    c16, s16 = cos.astype(np.float16), sin.astype(np.float16)
    B, T, bs = 2, 100, 64
    q, k, v = _rows(rng, B, T, 6, 128), _rows(rng, B, T, 2, 128), _rows(rng, B, T, 2, 128)
    table = np.arange(2 * 8, dtype=np.int32).reshape(2, 8)[:, ::-1].copy()
    kp = np.zeros((16, bs, 2, 128), np.float16)
    vp = np.zeros_like(kp)
    q_rot, k_rot = OR.rope_store_kv(q, k, v, c16, s16, 37, kp, vp, table, bs)
    qa, ka = OR.apply_rope(q, k, c16[37:37 + T], s16[37:37 + T])
    assert np.array_equal(q_rot, qa) and np.array_equal(k_rot, ka)
    kp2, vp2 = np.zeros_like(kp), np.zeros_like(vp)
    OK.scatter(kp2, vp2, table, ka, v, 37, bs)
    assert np.array_equal(kp, kp2) and np.array_equal(vp, vp2)
