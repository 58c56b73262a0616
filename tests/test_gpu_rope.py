"""GPU parity tests of the fused RoPE + KV write (``fi_rope_store_kv``), marked ``gpu``.

Every output is compared bit for bit: rotated q / k against the oracle's fp16
arithmetic (oracle/rope.py) and against the reference's formula run as eager torch
fp16 ops on the same GPU; pool bytes against the oracle's scatter, including the bytes
that must stay untouched.  Both sides are handed the same fp16 cos/sin tables.
"""

import numpy as np
import pytest
import torch

from conftest import banner
from oracle import kv as OK
from oracle import rope as OR

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _tables(rows, device=DEV):
    c, s = OR.precompute_freqs(128, rows)
    return (torch.from_numpy(c).half().to(device), torch.from_numpy(s).half().to(device))


def _bits(t):
    return (t.detach().cpu().numpy() if isinstance(t, torch.Tensor) else t).view(np.uint16)


def _torch_rope(x, cos, sin):
    """kernels/rope.py:37-42 as eager fp16 torch ops (cos/sin [T, 128])."""
    c, s = cos.unsqueeze(1), sin.unsqueeze(1)
    rh = torch.cat([-x[..., 64:], x[..., :64]], dim=-1)
    return x * c + rh * s


def _qkv(B, T, Hq, Hkv, seed, device=DEV):
    """q, k, v as strided views of one projection output, like model.py:88-98."""
    g = torch.Generator(device=device).manual_seed(seed)
    qkv = torch.randn(B, T, (Hq + 2 * Hkv) * 128, device=device, generator=g).half() * 3
    q, k, v = qkv.split([Hq * 128, Hkv * 128, Hkv * 128], dim=-1)
    return (q.view(B, T, Hq, 128), k.view(B, T, Hkv, 128), v.view(B, T, Hkv, 128))


@pytest.mark.parametrize("B,T,Hq,Hkv", [(1, 1, 24, 8), (2, 300, 24, 8), (3, 77, 4, 1)])
def test_apply_rope_bitexact(hip, B, T, Hq, Hkv):
    banner(f"apply_rope B={B} T={T} Hq={Hq} Hkv={Hkv}")
    from fast_infer_amd import apply_rope

    q, k, _ = _qkv(B, T, Hq, Hkv, seed=B * 1000 + T)
    cos, sin = _tables(T + 5)
    cos, sin = cos[5:], sin[5:]  # rows of positions 5.., as the model's cos[positions]
    qr, kr = apply_rope(q, k, cos, sin)
    torch.cuda.synchronize()
    eq, ek = OR.apply_rope(q.cpu().numpy(), k.cpu().numpy(), cos.cpu().numpy(), sin.cpu().numpy())
    assert np.array_equal(_bits(qr), _bits(eq))
    assert np.array_equal(_bits(kr), _bits(ek))
    assert torch.equal(qr, _torch_rope(q, cos, sin))
    assert torch.equal(kr, _torch_rope(k, cos, sin))


def test_rope_store_kv_pool_per_row_starts(hip):
    banner("rope_store_kv pool, per-row starts, out-of-table tokens")
    from fast_infer_amd import rope_store_kv

    B, T, Hq, Hkv, bs, N, rows = 4, 90, 8, 2, 16, 48, 200
    q, k, v = _qkv(B, T, Hq, Hkv, seed=11)
    cos, sin = _tables(rows)
    starts = [0, 150, -7, 33]           # row 1 runs past the table, row 2 starts before it
    g = torch.Generator().manual_seed(12)
    table = torch.full((B, 16), -1, dtype=torch.int32)
    table[:, :12] = torch.randperm(N, generator=g)[:48].view(B, 12).int()
    table[3, 4] = -1                    # a hole: those 16 tokens go nowhere
    table[0, 5] = N + 3                 # outside the pool: skipped
    kp = (torch.randn(N, bs, Hkv, 128, generator=g) * 5).half()
    vp = (torch.randn(N, bs, Hkv, 128, generator=g) * 5).half()
    kp_d, vp_d = kp.to(DEV), vp.to(DEV)
    q_out = torch.full(q.shape, 7.0, dtype=torch.float16, device=DEV)
    qr, kr = rope_store_kv(q, k, v, cos, sin, 0, kp_d, vp_d, table.to(DEV),
                           start_positions=torch.tensor(starts, dtype=torch.int32),
                           q_out=q_out)
    torch.cuda.synchronize()

    ekp, evp = kp.numpy().copy(), vp.numpy().copy()
    eq, ek = OR.rope_store_kv(q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(),
                              cos.cpu().numpy(), sin.cpu().numpy(), starts, ekp, evp,
                              table.numpy(), bs)
    assert np.array_equal(_bits(kp_d), _bits(ekp))
    assert np.array_equal(_bits(vp_d), _bits(evp))
    for b, st in enumerate(starts):
        lo, hi = max(0, -st), min(T, rows - st)
        assert np.array_equal(_bits(qr[b, lo:hi]), _bits(eq[b, lo:hi]))
        assert np.array_equal(_bits(kr[b, lo:hi]), _bits(ek[b, lo:hi]))
        # skipped tokens leave the caller's q_out untouched
        assert bool((qr[b, :lo] == 7.0).all()) and bool((qr[b, hi:] == 7.0).all())


def test_rope_store_kv_no_k_out_and_contiguous_inputs(hip):
    banner("rope_store_kv return_k=False, contiguous inputs")
    from fast_infer_amd import rope_store_kv

    B, T, Hq, Hkv, bs, N = 2, 130, 24, 8, 64, 8
    q, k, v = (t.contiguous() for t in _qkv(B, T, Hq, Hkv, seed=13))
    cos, sin = _tables(4096)
    table = torch.tensor([[5, 2, 7, -1], [0, 1, 3, 4]], dtype=torch.int32, device=DEV)
    kp = torch.zeros(N, bs, Hkv, 128, dtype=torch.float16, device=DEV)
    vp = torch.zeros_like(kp)
    qr, kr = rope_store_kv(q, k, v, cos, sin, 60, kp, vp, table, return_k=False)
    torch.cuda.synchronize()
    assert kr is None
    ekp, evp = np.zeros(kp.shape, np.float16), np.zeros(vp.shape, np.float16)
    eq, _ = OR.rope_store_kv(q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(),
                             cos.cpu().numpy(), sin.cpu().numpy(), 60, ekp, evp,
                             table.cpu().numpy(), bs)
    assert np.array_equal(_bits(qr), _bits(eq))
    assert np.array_equal(_bits(kp), _bits(ekp)) and np.array_equal(_bits(vp), _bits(evp))


def test_rope_store_kv_rejects_positions_outside_table(hip):
    from fast_infer_amd import rope_store_kv

    q, k, v = _qkv(1, 10, 8, 8, seed=14)
    cos, sin = _tables(64)
    with pytest.raises(IndexError):
        rope_store_kv(q, k, v, cos, sin, 60)
    with pytest.raises(IndexError):
        rope_store_kv(q, k, v, cos, sin, -1)


def test_kvcache_rope_prefill_then_decode(hip):
    """rope_store_kv_prefill / _decode on a KVCache against the oracle's flow:
    apply_rope, then the pinned store_prefill / store_decode (model.py:101, :117, :120)."""
    banner("KVCache rope prefill + decode")
    from fast_infer_amd import KVCache, rope_store_kv_decode, rope_store_kv_prefill

    L, Hq, Hkv, S, B, rows = 2, 16, 4, 150, 2, 512
    fi = KVCache(L, Hkv, 128, max_seq_len=rows, block_size=64, device=DEV, num_blocks=20)
    ok = OK.OracleKVCache(L, Hkv, 128, max_seq_len=rows, block_size=64, num_blocks=20)
    cos, sin = _tables(rows)
    c_np, s_np = cos.cpu().numpy(), sin.cpu().numpy()
    for layer in range(L):
        q, k, v = _qkv(B, S, Hq, Hkv, seed=20 + layer)
        qr, kr = rope_store_kv_prefill(fi, layer, q, k, v, cos, sin)
        eq, ek = OR.apply_rope(q.cpu().numpy(), k.cpu().numpy(), c_np[:S], s_np[:S])
        OK.store_prefill(ok, layer, ek, v.cpu().numpy())
        torch.cuda.synchronize()
        assert np.array_equal(_bits(qr), _bits(eq)) and np.array_equal(_bits(kr), _bits(ek))
    for pos in (150, 191, 192):
        for layer in range(L):
            q, k, v = (t.squeeze(1) for t in _qkv(B, 1, Hq, Hkv, seed=pos * 7 + layer))
            qr = rope_store_kv_decode(fi, layer, q, k, v, cos, sin, pos)
            eq, ek = OR.apply_rope(q.cpu().numpy()[:, None], k.cpu().numpy()[:, None],
                                   c_np[pos:pos + 1], s_np[pos:pos + 1])
            OK.store_decode(ok, layer, ek[:, 0], v.cpu().numpy(), pos)
            torch.cuda.synchronize()
            assert np.array_equal(_bits(qr), _bits(eq[:, 0]))
    assert fi.block_table.cpu().tolist() == ok.block_table
    assert fi.num_tokens == ok.num_tokens
    assert np.array_equal(_bits(fi.k), _bits(ok.k))
    assert np.array_equal(_bits(fi.v), _bits(ok.v))


def test_rope_store_kv_batch4_seq4096_full_size(hip):
    """Batch 4 x 4096 tokens, 24 q / 8 kv heads, block_size 64, shuffled 256-block table:
    q and k equal the reference formula as eager fp16 torch ops on the same GPU, bit for
    bit; gathering every token back through the table returns rotated k and raw v; two
    sampled rows are checked against the oracle."""
    banner("rope_store_kv 4x4096 full size")
    from fast_infer_amd import rope_store_kv

    B, S, Hq, Hkv, bs, N = 4, 4096, 24, 8, 64, 256
    q, k, v = _qkv(B, S, Hq, Hkv, seed=30)
    cos, sin = _tables(S)
    g = torch.Generator(device=DEV).manual_seed(31)
    table = torch.randperm(N, device=DEV, generator=g).int().view(B, N // B)
    kp = torch.zeros(N, bs, Hkv, 128, dtype=torch.float16, device=DEV)
    vp = torch.zeros_like(kp)
    qr, kr = rope_store_kv(q, k, v, cos, sin, 0, kp, vp, table)
    assert torch.equal(qr, _torch_rope(q, cos, sin))
    assert torch.equal(kr, _torch_rope(k, cos, sin))
    t = torch.arange(S, device=DEV)
    for b in range(B):
        phys = table[b, t // bs].long()
        assert torch.equal(kp[phys, t % bs], kr[b])
        assert torch.equal(vp[phys, t % bs], v[b])
    for b, t0 in ((1, 4000), (3, 17)):
        eq, ek = OR.apply_rope(q[b:b + 1, t0:t0 + 64].cpu().numpy(),
                               k[b:b + 1, t0:t0 + 64].cpu().numpy(),
                               cos[t0:t0 + 64].cpu().numpy(), sin[t0:t0 + 64].cpu().numpy())
        assert np.array_equal(_bits(qr[b:b + 1, t0:t0 + 64]), _bits(eq))
        assert np.array_equal(_bits(kr[b:b + 1, t0:t0 + 64]), _bits(ek))
