"""GPU parity tests of RMSNorm (``fi_rmsnorm``) and RMSNorm fused with the INT4 projection
(``fi_rmsnorm_int4_matmul``), marked ``gpu``.

* rms_norm within one fp16 ulp of the float64 form (oracle/rmsnorm.py) — the reference
  computes in fp32 with its own sum order and rsqrt, so the last bit is not pinned — and
  the fraction of elements off the correctly rounded value reported and bounded;
* the fused call against the float64 product of the normalized rows and the dequantized
  weights, for the in-GEMM norm (few rows) and the separate-pass form (more rows).
"""

import numpy as np
import pytest
import torch

from conftest import banner
from oracle import int4 as OI
from oracle import rmsnorm as ON

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _inputs(seed, M, H, scale=1.0):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((M, H)) * scale).astype(np.float16)
    w = (rng.standard_normal(H) * 0.3 + 1.0).astype(np.float16)
    return x, w


@pytest.mark.parametrize("M,H,scale", [(1, 3072, 1.0), (64, 3072, 4.0), (1000, 3072, 0.01),
                                       (7, 256, 1.0), (3, 8192, 30.0)])
def test_rms_norm_vs_oracle(hip, M, H, scale):
    banner(f"rms_norm M={M} H={H}")
    from fast_infer_amd import rms_norm

    x, w = _inputs(M + H, M, H, scale)
    y = rms_norm(torch.from_numpy(x).to(DEV), torch.from_numpy(w).to(DEV))
    torch.cuda.synchronize()
    got = y.float().cpu().numpy().astype(np.float64)
    exact = ON.rms_norm_exact(x, w)
    assert np.all(np.abs(got - exact) <= ON.norm_bound(exact))
    off = np.mean(y.cpu().numpy() != exact.astype(np.float16))
    print(f"[rms_norm] fraction not correctly rounded: {off:.2e}")
    assert off < 0.01


def test_rms_norm_strided_rows_and_batch_dims(hip):
    banner("rms_norm strided")
    from fast_infer_amd import rms_norm

    rng = np.random.default_rng(5)
    big = rng.standard_normal((2, 5, 3072 + 64)).astype(np.float16)
    w = (rng.standard_normal(3072) * 0.3 + 1.0).astype(np.float16)
    xt = torch.from_numpy(big).to(DEV)[..., 32:32 + 3072]
    y = rms_norm(xt, torch.from_numpy(w).to(DEV))
    assert y.shape == (2, 5, 3072)
    exact = ON.rms_norm_exact(big[..., 32:32 + 3072].reshape(10, 3072), w)
    got = y.reshape(10, 3072).float().cpu().numpy()
    assert np.all(np.abs(got - exact) <= ON.norm_bound(exact))


@pytest.mark.parametrize("M", [1, 3, 4, 5, 16, 17, 64, 300])
@pytest.mark.parametrize("packed_weights", [True, False])
def test_rms_norm_int4_matmul_vs_oracle(hip, M, packed_weights):
    banner(f"rms_norm_int4_matmul M={M} packed={packed_weights}")
    from fast_infer_amd import (dequantize_int4, int4_matmul, quantize_int4_groupwise, rms_norm,
                                rms_norm_int4_matmul)

    N, K = 5120, 3072
    x, nw = _inputs(M, M, K, 2.0)
    rng = np.random.default_rng(99)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float16)
    packed, scales = quantize_int4_groupwise(torch.from_numpy(w).to(DEV))
    w16 = dequantize_int4(packed, scales)
    weight = (packed, scales) if packed_weights else w16
    xd, nwd = torch.from_numpy(x).to(DEV), torch.from_numpy(nw).to(DEV)
    out = rms_norm_int4_matmul(xd, nwd, weight)
    two_step = int4_matmul(rms_norm(xd, nwd), weight)
    torch.cuda.synchronize()
    xn = ON.rms_norm(x, nw)
    w16n = w16.cpu().numpy()
    exact = OI.matmul_exact(xn, w16n)
    mag = np.abs(xn.astype(np.float64)) @ np.abs(w16n.astype(np.float64)).T
    # the normalized rows may differ from the oracle's by one fp16 ulp here and there
    bound = OI.matmul_bound(xn, w16n) + mag * 2.0 ** -10
    for got in (out, two_step):
        g = got.float().cpu().numpy().astype(np.float64)
        assert np.all(np.abs(g - exact) <= bound), float(np.max(np.abs(g - exact) - bound))
