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


_SENTINEL = 0x7C01  # an fp16 NaN bit pattern no kernel produces


@pytest.mark.parametrize("lens", [[300, 90], [700, 90]])
def test_paged_decode_head_dim_64_leaves_bytes_past_head_dim(hip, lens):
    # fi_paged_attention_fwd through the C ABI with q and o as views of 128-wide rows: the
    # single-pass kernel (rows within one partition) and the partition + merge launches
    # write the 64 columns of each head and nothing past them
    banner(f"paged decode head_dim 64, C ABI, o columns 64..127 untouched, lens {lens}")
    from fast_infer_amd import _lib

    sp = dict(B=2, Hq=8, Hkv=2, D=64, bs=64, N=32, lens=lens, seed=5)
    q, kc, vc, table, lens = specs.decode_inputs(sp)
    qw = torch.zeros(2, 8, 128, dtype=torch.float16, device=DEV)
    qw[..., :64] = q.to(DEV)
    ow = torch.full((2, 8, 128), 0, dtype=torch.int16, device=DEV).fill_(_SENTINEL)
    ow = ow.view(torch.float16)
    kcd, vcd, td = kc.to(DEV), vc.to(DEV), table.to(DEV)
    cl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    lib = _lib.load()
    nbytes = lib.fi_paged_attention_workspace_size(2, 8, 2, max(lens), 64)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=DEV)
    rc = lib.fi_paged_attention_fwd(
        qw.data_ptr(), qw.stride(0), qw.stride(1), kcd.data_ptr(), vcd.data_ptr(), 32, 64, 2,
        td.data_ptr(), td.stride(0), td.shape[1], cl.data_ptr(), max(lens),
        ow.data_ptr(), ow.stride(0), ow.stride(1), 2, 8, 64, 64 ** -0.5,
        ws.data_ptr() if nbytes else None, nbytes, _lib.stream_handle(torch.device(DEV)))
    _lib.check(rc, "paged_attention")
    torch.cuda.synchronize()
    assert torch.all(ow.view(torch.int16)[..., 64:] == _SENTINEL)
    assert _maxabs(ow[..., :64], OA.paged_attention(q, kc, vc, table, 64, lens)) <= ATOL


@pytest.mark.parametrize("S", [70, 300])
def test_flash_prefill_head_dim_64_leaves_bytes_past_head_dim(hip, S):
    # fi_flash_attention_fwd through the C ABI with o a view of 128-wide rows
    banner(f"flash prefill head_dim 64, C ABI, o columns 64..127 untouched, S={S}")
    from fast_infer_amd import _lib

    B, H, Hkv, D = 2, 6, 2, 64
    g = torch.Generator().manual_seed(S)
    q = torch.randn(B, S, H, D, generator=g).half()
    k = torch.randn(B, S, Hkv, D, generator=g).half()
    v = torch.randn(B, S, Hkv, D, generator=g).half()
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    ow = torch.empty(B, S, H, 128, dtype=torch.int16, device=DEV).fill_(_SENTINEL)
    ow = ow.view(torch.float16)
    lib = _lib.load()
    rc = lib.fi_flash_attention_fwd(
        qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), ow.data_ptr(), B, H, Hkv, S, D,
        qd.stride(0), qd.stride(2), qd.stride(1), kd.stride(0), kd.stride(2), kd.stride(1),
        vd.stride(0), vd.stride(2), vd.stride(1), ow.stride(0), ow.stride(2), ow.stride(1),
        D ** -0.5, None, None, 0, 64, None, 0, 0, _lib.stream_handle(torch.device(DEV)))
    _lib.check(rc, "flash_attention")
    torch.cuda.synchronize()
    assert torch.all(ow.view(torch.int16)[..., 64:] == _SENTINEL)
    ref = OA.causal_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2))
    assert _maxabs(ow[..., :64].transpose(1, 2), ref) <= ATOL


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
