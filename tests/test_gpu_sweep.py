"""Seeded sweeps of random valid configurations against the oracle (marked ``gpu``).

* paged decode: block sizes 16..128 (seeds 0..11) and 1..100 off the 16-token tile grid
  (seeds 12..19), GQA groups 1..8 (and 32 query heads per kv head),
  1..12 ragged rows including empty ones, shuffled tables wider than needed with -1
  padding, sm_scale of either sign;
* causal prefill: GQA groups 1..8 (every heads-per-workgroup instantiation), lengths
  around the 64-row tiles, the model's strided [B, S, H, D] views or contiguous
  [B, H, S, D] tensors, sm_scale of either sign, with and without the fused pool write
  (pool rows bit-exact against the brute-force copy);
* the INT4 linear layer: odd M, N (down to 1) and K, packed and fp16 weights.

Each case derives every size from its seed, prints it before the GPU step, and is
checked with the same tolerances as the fixed-shape tests (max-abs 2e-3 for attention,
the fp32-accumulation bound for the linear layer).
"""

import math

import numpy as np
import pytest
import torch

from conftest import ATOL, banner
from oracle import attention as OA
from oracle import int4 as OI

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
D = 128


def _maxabs(a, b):
    return float((torch.as_tensor(a).float().cpu() - torch.as_tensor(b).float().cpu()).abs().max())


DECODE_HEADS = [(24, 8), (8, 8), (16, 8), (32, 8), (12, 4), (6, 2), (64, 8), (10, 5), (7, 7),
                (64, 2), (40, 8), (3, 1)]


@pytest.mark.parametrize("seed", range(20))
def test_paged_decode_random(hip, seed):
    from fast_infer_amd import paged_attention

    rng = np.random.default_rng(1000 + seed)
    Hq, Hkv = DECODE_HEADS[seed % len(DECODE_HEADS)]
    sizes = [16, 32, 64, 128] if seed < 12 else [1, 2, 4, 8, 12, 24, 40, 100]
    bs = int(rng.choice(sizes))
    B = int(rng.integers(1, 13))
    lens = [int(x) for x in rng.integers(0, 900, B)]
    if B > 2:
        lens[int(rng.integers(0, B))] = 0
    lens[int(rng.integers(0, B))] = max(1, lens[0])
    nblk = [math.ceil(n / bs) for n in lens]
    width = max(nblk) + int(rng.integers(0, 3))
    N = sum(nblk) + int(rng.integers(1, 8))
    perm = rng.permutation(N)
    table = np.full((B, width), -1, dtype=np.int32)
    pos = 0
    for b in range(B):
        table[b, :nblk[b]] = perm[pos:pos + nblk[b]]
        pos += nblk[b]
    scale = D ** -0.5 * float(rng.choice([1.0, 0.6, -1.0]))
    banner(f"decode sweep seed={seed} Hq={Hq} Hkv={Hkv} bs={bs} B={B} lens={lens} N={N} "
           f"width={width} scale={scale:.4f}")
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, D, generator=g).half()
    kc = torch.randn(N, bs, Hkv, D, generator=g).half()
    vc = torch.randn(N, bs, Hkv, D, generator=g).half()
    tt = torch.from_numpy(table)
    cl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    out = paged_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), tt.to(DEV), bs, max(lens), scale,
                          context_lens=cl)
    torch.cuda.synchronize()
    ref = OA.paged_attention(q, kc, vc, tt, bs, lens, sm_scale=scale)
    assert _maxabs(out, ref) <= ATOL
    for b, n in enumerate(lens):
        if n == 0:
            assert float(out[b].abs().max()) == 0.0


PREFILL_HEADS = [(24, 8), (8, 8), (16, 8), (20, 4), (12, 2), (6, 6), (15, 3), (40, 8), (32, 4),
                 (5, 1)]


@pytest.mark.parametrize("seed", range(10))
def test_flash_prefill_random(hip, seed):
    from fast_infer_amd import flash_attention

    rng = np.random.default_rng(2000 + seed)
    H, Hkv = PREFILL_HEADS[seed]
    B = int(rng.integers(1, 4))
    S = int(rng.choice([1, 2, 63, 64, 65, 127, 128, 129, 200, 333]))
    strided = bool(rng.integers(0, 2))
    pool = bool(rng.integers(0, 2))
    scale = D ** -0.5 * float(rng.choice([1.0, 0.7, -1.0]))
    banner(f"prefill sweep seed={seed} H={H} Hkv={Hkv} B={B} S={S} strided={strided} "
           f"pool={pool} scale={scale:.4f}")
    g = torch.Generator().manual_seed(seed)
    if strided:  # the model's layout: [B, S, heads, D] viewed as [B, heads, S, D]
        q = torch.randn(B, S, H, D, generator=g).half().transpose(1, 2)
        k = torch.randn(B, S, Hkv, D, generator=g).half().transpose(1, 2)
        v = torch.randn(B, S, Hkv, D, generator=g).half().transpose(1, 2)
    else:
        q = torch.randn(B, H, S, D, generator=g).half()
        k = torch.randn(B, Hkv, S, D, generator=g).half()
        v = torch.randn(B, Hkv, S, D, generator=g).half()
    qd, kd, vd = (t.to(DEV) for t in (q, k, v))
    kw = {}
    if pool:
        nb = math.ceil(S / 64)
        N = B * nb + 3
        table = torch.from_numpy(rng.permutation(N)[:B * nb].astype(np.int32)).view(B, nb)
        kc = torch.zeros(N, 64, Hkv, D, dtype=torch.float16, device=DEV)
        vc = torch.zeros_like(kc)
        kw = dict(k_cache=kc, v_cache=vc, block_table=table.to(DEV))
    out = flash_attention(qd, kd, vd, scale, **kw)
    torch.cuda.synchronize()
    ref = OA.causal_attention(q, k, v, scale)
    assert _maxabs(out, ref) <= ATOL
    if pool:
        t = torch.arange(S)
        kcc, vcc = kc.cpu(), vc.cpu()
        for b in range(B):
            phys = table[b, t // 64].long()
            assert torch.equal(kcc[phys, t % 64], k[b].transpose(0, 1))
            assert torch.equal(vcc[phys, t % 64], v[b].transpose(0, 1))
        used = set(table.flatten().tolist())
        for blk in range(N):
            if blk not in used:
                assert float(kcc[blk].abs().max()) == 0.0


INT4_SHAPES = [(1, 1, 128), (3, 7, 256), (17, 33, 384), (64, 100, 1024), (130, 257, 512),
               (5, 640, 3072)]


@pytest.mark.parametrize("M,N,K", INT4_SHAPES)
def test_int4_matmul_random(hip, M, N, K):
    from fast_infer_amd import dequantize_int4, int4_matmul, quantize_int4_groupwise

    banner(f"int4 sweep M={M} N={N} K={K}")
    rng = np.random.default_rng(M * 1000 + N + K)
    w = (rng.standard_normal((N, K)) * 0.03).astype(np.float16)
    x = torch.from_numpy((rng.standard_normal((M, K))).astype(np.float16))
    packed, scales = quantize_int4_groupwise(torch.from_numpy(w).to(DEV))
    ep, es = OI.quantize_int4_groupwise(w)
    out = int4_matmul(x.to(DEV), (packed, scales))
    w16 = dequantize_int4(packed, scales)
    out16 = int4_matmul(x.to(DEV), w16)
    torch.cuda.synchronize()
    assert np.array_equal(packed.cpu().numpy(), ep)
    assert np.array_equal(scales.cpu().numpy().view(np.uint16), es.view(np.uint16))
    wd = OI.dequantize(ep, es)
    exact = OI.matmul_exact(x.numpy(), wd)
    bound = OI.matmul_bound(x.numpy(), wd)
    for got in (out, out16):
        g = got.float().cpu().numpy().astype(np.float64)
        assert np.all(np.abs(g - exact) <= bound), float(np.max(np.abs(g - exact) - bound))
