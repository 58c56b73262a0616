"""head_dim below 128 (multiples of 8; of 16 for RoPE), marked ``gpu``.

The reference's kernels take any head_dim up to their power-of-two block (masking the rest,
kernels/attention.py:91, :141-142, :215); Llama-3.2-1B-shaped models use 64.  The attention
kernels here keep their 128-column layout and load the columns past head_dim as zeros, so
each case below is checked like the 128-column ones: paged decode and causal prefill
against the fp32 oracle within max-abs 2e-3 (one and several partitions, ragged rows), the
fused prefill pool write, the KV scatter and RoPE + pool write bit for bit, and bytes past
each row's head_dim untouched.
"""

import math

import numpy as np
import pytest
import torch

from conftest import ATOL, banner
from golden import specs
from oracle import attention as OA
from oracle import kv as OK
from oracle import rope as OR

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _maxabs(a, b):
    return float((torch.as_tensor(a).float().cpu() - torch.as_tensor(b).float().cpu()).abs().max())


@pytest.mark.parametrize("D", [64, 96, 80, 8])
@pytest.mark.parametrize("lens", [[1, 190, 70], [600, 3000, 513, 64, 65]])
def test_paged_decode_head_dim(hip, D, lens):
    # three short rows (one partition, direct output) and rows past 512 tokens (partitions
    # and the merge); GQA group 3 as in the model
    banner(f"paged decode head_dim {D} lens {lens}")
    from fast_infer_amd import paged_attention

    sp = dict(B=len(lens), Hq=12, Hkv=4, D=D, bs=64, N=128, lens=lens, seed=70 + D)
    q, kc, vc, table, lens = specs.decode_inputs(sp)
    cl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    out = paged_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), 64, max(lens),
                          context_lens=cl)
    torch.cuda.synchronize()
    assert out.shape == q.shape
    assert _maxabs(out, OA.paged_attention(q, kc, vc, table, 64, lens)) <= ATOL


def test_paged_decode_head_dim_64_strided_output_untouched(hip):
    # q and o as views of wider rows: the columns past head_dim keep their bytes
    banner("paged decode head_dim 64, strided q/o")
    from fast_infer_amd import paged_attention

    sp = dict(B=2, Hq=8, Hkv=2, D=64, bs=64, N=32, lens=[700, 90], seed=5)
    q, kc, vc, table, lens = specs.decode_inputs(sp)
    qw = torch.zeros(2, 8, 128, dtype=torch.float16)
    qw[..., :64] = q
    qd = qw.to(DEV)[..., :64]
    out = paged_attention(qd, kc.to(DEV), vc.to(DEV), table.to(DEV), 64, 700,
                          context_lens=torch.tensor(lens, dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    assert _maxabs(out, OA.paged_attention(q, kc, vc, table, 64, lens)) <= ATOL


@pytest.mark.parametrize("D", [64, 96])
@pytest.mark.parametrize("S", [1, 200, 700])
def test_flash_prefill_head_dim(hip, D, S):
    banner(f"flash prefill head_dim {D} S={S}")
    from fast_infer_amd import flash_attention

    B, H, Hkv = 2, 6, 2
    g = torch.Generator().manual_seed(D * 1000 + S)
    q = torch.randn(B, S, H, D, generator=g).half().transpose(1, 2)
    k = torch.randn(B, S, Hkv, D, generator=g).half().transpose(1, 2)
    v = torch.randn(B, S, Hkv, D, generator=g).half().transpose(1, 2)
    out = flash_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    torch.cuda.synchronize()
    assert out.shape == q.shape
    assert _maxabs(out, OA.causal_attention(q, k, v)) <= ATOL


@pytest.mark.parametrize("D", [64, 96])
def test_flash_prefill_head_dim_pool_write(hip, D):
    # the fused pool write with [blocks, 64, Hkv, D] pools: the written blocks equal the
    # scatter of K/V bit for bit, every other block keeps its bytes, the output is the plain one
    banner(f"flash prefill head_dim {D} fused pool write")
    from fast_infer_amd import flash_attention

    B, S, H, Hkv, N = 2, 300, 6, 2, 16
    g = torch.Generator().manual_seed(D)
    q = torch.randn(B, S, H, D, generator=g).half().to(DEV).transpose(1, 2)
    k = torch.randn(B, S, Hkv, D, generator=g).half().to(DEV)
    v = torch.randn(B, S, Hkv, D, generator=g).half().to(DEV)
    perm = torch.randperm(N, generator=torch.Generator().manual_seed(D + 1)).int()
    nb = math.ceil(S / 64)
    table = perm[:B * nb].view(B, nb)
    kc0 = torch.randn(N, 64, Hkv, D, generator=g).half()
    vc0 = torch.randn(N, 64, Hkv, D, generator=g).half()
    kc, vc = kc0.to(DEV), vc0.to(DEV)
    out = flash_attention(q, k.transpose(1, 2), v.transpose(1, 2), k_cache=kc, v_cache=vc,
                          block_table=table.to(DEV))
    plain = flash_attention(q, k.transpose(1, 2), v.transpose(1, 2))
    torch.cuda.synchronize()
    assert torch.equal(out, plain)
    ek, ev = kc0.numpy().copy(), vc0.numpy().copy()
    OK.scatter(ek, ev, table.tolist(), k.cpu().numpy(), v.cpu().numpy(), 0, 64)
    assert np.array_equal(kc.cpu().numpy().view(np.uint16), ek.view(np.uint16))
    assert np.array_equal(vc.cpu().numpy().view(np.uint16), ev.view(np.uint16))


@pytest.mark.parametrize("D", [64, 8, 200])
def test_store_kv_head_dim(hip, D):
    banner(f"store_kv head_dim {D}")
    from fast_infer_amd import store_kv

    B, T, Hkv, N = 2, 70, 3, 8
    g = torch.Generator().manual_seed(D)
    k = torch.randn(B, T, Hkv, D, generator=g).half()
    v = torch.randn(B, T, Hkv, D, generator=g).half()
    table = torch.tensor([[3, 6], [1, 5]], dtype=torch.int32)
    kc0 = torch.randn(N, 64, Hkv, D, generator=g).half()
    vc0 = torch.randn(N, 64, Hkv, D, generator=g).half()
    kc, vc = kc0.to(DEV), vc0.to(DEV)
    store_kv(k.to(DEV), v.to(DEV), kc, vc, table.to(DEV), 0)
    torch.cuda.synchronize()
    ek, ev = kc0.numpy().copy(), vc0.numpy().copy()
    OK.scatter(ek, ev, table.tolist(), k.numpy(), v.numpy(), 0, 64)
    assert np.array_equal(kc.cpu().numpy().view(np.uint16), ek.view(np.uint16))
    assert np.array_equal(vc.cpu().numpy().view(np.uint16), ev.view(np.uint16))


@pytest.mark.parametrize("D", [64, 32])
def test_rope_store_kv_head_dim(hip, D):
    # rotate-half pairs i with i + D/2; rotated q/k and the pool rows bit-exact
    banner(f"rope_store_kv head_dim {D}")
    from fast_infer_amd import rope_store_kv

    B, T, Hq, Hkv, N = 2, 90, 6, 2, 8
    g = torch.Generator().manual_seed(D)
    q = (torch.randn(B, T, Hq, D, generator=g) * 3).half()
    k = (torch.randn(B, T, Hkv, D, generator=g) * 3).half()
    v = torch.randn(B, T, Hkv, D, generator=g).half()
    c, s = OR.precompute_freqs(D, 200)
    cos, sin = torch.from_numpy(c).half(), torch.from_numpy(s).half()
    table = torch.tensor([[2, 7], [4, 0]], dtype=torch.int32)
    kc0 = torch.randn(N, 64, Hkv, D, generator=g).half()
    vc0 = torch.randn(N, 64, Hkv, D, generator=g).half()
    kc, vc = kc0.to(DEV), vc0.to(DEV)
    qr, kr = rope_store_kv(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV), 10,
                           kc, vc, table.to(DEV))
    torch.cuda.synchronize()
    ek, ev = kc0.numpy().copy(), vc0.numpy().copy()
    eq, ekr = OR.rope_store_kv(q.numpy(), k.numpy(), v.numpy(), cos.numpy(), sin.numpy(), 10,
                               ek, ev, table.tolist(), 64)
    assert np.array_equal(qr.cpu().numpy().view(np.uint16), eq.view(np.uint16))
    assert np.array_equal(kr.cpu().numpy().view(np.uint16), ekr.view(np.uint16))
    assert np.array_equal(kc.cpu().numpy().view(np.uint16), ek.view(np.uint16))
    assert np.array_equal(vc.cpu().numpy().view(np.uint16), ev.view(np.uint16))
