"""Paged decode with block sizes that are not multiples of 16, marked ``gpu``.

The reference's decode kernel takes the block size as a compile-time range
(kernels/attention.py:128, :153), so any power of two runs there; the engine's default is 64
(config.py:23).  Here a multiple of 16 keeps whole 16-token tiles inside one pool block; any
other size takes a kernel instance that addresses each tile row through its own block: by
per-lane offsets into one descriptor over the pool when the pool is under 4 GiB, else by one
descriptor per row.  Checked: the fp32 oracle within max-abs 2e-3 for sizes 1..100 (one partition with the
direct output, several partitions with the merge, ragged rows, head_dim 64), table entries
that are -1 or outside the pool dropping out of the softmax, and, at the full decode size
(batch 32, contexts 512..4096), bit-identical outputs for one logical context stored with
block sizes 64, 48, 8 and 1 (the partitions and tiles are laid over token positions, so
the block size may only change where a row's bytes come from), and bit-identical outputs of
the per-row path on 4.3 GB pools and the per-lane path on a small one.  The fused prefill
pool write at block sizes other than 64 is checked bit for bit against the oracle scatter.
"""

import math

import pytest
import torch

from conftest import ATOL, banner
from golden import specs
from oracle import attention as OA

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _maxabs(a, b):
    return float((torch.as_tensor(a).float().cpu() - torch.as_tensor(b).float().cpu()).abs().max())


def _inputs(bs, lens, Hq=12, Hkv=4, D=128, seed=0):
    need = sum(math.ceil(n / bs) for n in lens)
    sp = dict(B=len(lens), Hq=Hq, Hkv=Hkv, D=D, bs=bs, N=need + 5, lens=lens, seed=seed)
    return specs.decode_inputs(sp)


@pytest.mark.parametrize("bs", [1, 2, 4, 8, 24, 40, 100])
@pytest.mark.parametrize("lens", [[1, 16, 37, 300], [600, 2500, 1025]])
def test_paged_decode_block_size_vs_oracle(hip, bs, lens):
    banner(f"paged decode block_size {bs} lens {lens}")
    from fast_infer_amd import paged_attention

    q, kc, vc, table, lens = _inputs(bs, lens, seed=bs)
    cl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    out = paged_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), bs, max(lens),
                          context_lens=cl)
    torch.cuda.synchronize()
    assert out.shape == q.shape
    assert _maxabs(out, OA.paged_attention(q, kc, vc, table, bs, lens)) <= ATOL


@pytest.mark.parametrize("bs", [1, 8])
def test_paged_decode_block_size_head_dim_64(hip, bs):
    banner(f"paged decode block_size {bs} head_dim 64")
    from fast_infer_amd import paged_attention

    q, kc, vc, table, lens = _inputs(bs, [700, 90, 33], Hq=8, Hkv=2, D=64, seed=3 + bs)
    cl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    out = paged_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), bs, 700,
                          context_lens=cl)
    torch.cuda.synchronize()
    assert _maxabs(out, OA.paged_attention(q, kc, vc, table, bs, lens)) <= ATOL


@pytest.mark.parametrize("bs", [8, 1])
def test_paged_decode_block_size_invalid_entries(hip, bs):
    # a -1 and an out-of-pool entry inside the contexts: their tokens drop out of the
    # softmax, the rest of each row is attended as usual
    banner(f"paged decode block_size {bs} invalid table entries")
    from fast_infer_amd import paged_attention

    lens = [200, 700]
    q, kc, vc, table, lens = _inputs(bs, lens, seed=11)
    t = table.clone()
    drops = {0: {3, 4}, 1: {math.ceil(600 / bs) - 1}}
    for b, blks in drops.items():
        for i, blk in enumerate(sorted(blks)):
            t[b, blk] = -1 if i == 0 else 10 ** 6
    out = paged_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), t.to(DEV), bs, 700,
                          context_lens=torch.tensor(lens, dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    for b, n in enumerate(lens):
        toks = [x for x in range(n) if x // bs not in drops[b]]
        K = torch.stack([kc[int(table[b, x // bs]), x % bs] for x in toks]).float()
        V = torch.stack([vc[int(table[b, x // bs]), x % bs] for x in toks]).float()
        K, V = K.repeat_interleave(3, 1).transpose(0, 1), V.repeat_interleave(3, 1).transpose(0, 1)
        s = torch.matmul(K, q[b].float().unsqueeze(-1)).squeeze(-1) * 128 ** -0.5
        ref = torch.matmul(torch.softmax(s, -1).unsqueeze(1), V).squeeze(1)
        assert _maxabs(out[b], ref) <= ATOL


def _pool(K, V, lens, bs, seed):
    """Store the logical rows K/V [B, L, Hkv, D] in pools of block size bs under a
    shuffled table."""
    B, L, Hkv, D = K.shape
    need = [math.ceil(n / bs) for n in lens]
    N = sum(need) + 3
    perm = torch.randperm(N, generator=torch.Generator().manual_seed(seed)).int()
    table = specs.make_table(perm, B, N, bs, lens, "deal")
    kc = torch.zeros(N * bs, Hkv, D, dtype=torch.float16, device=DEV)
    vc = torch.zeros_like(kc)
    for b, n in enumerate(lens):
        t = torch.arange(n)
        slot = (table[b, t // bs].long() * bs + t % bs).to(DEV)
        kc[slot] = K[b, :n]
        vc[slot] = V[b, :n]
    return kc.view(N, bs, Hkv, D), vc.view(N, bs, Hkv, D), table


def test_paged_decode_block_sizes_bit_identical_full_size(hip):
    banner("paged decode batch32 ragged 512..4096, block sizes 64/48/8/1")
    from fast_infer_amd import paged_attention

    B, Hq, Hkv, D, L = 32, 24, 8, 128, 4096
    lens = torch.randint(512, L + 1, (B,), generator=torch.Generator().manual_seed(4)).tolist()
    g = torch.Generator(device=DEV).manual_seed(4)
    q = torch.randn(B, Hq, D, device=DEV, generator=g).half()
    K = torch.randn(B, L, Hkv, D, device=DEV, generator=g).half()
    V = torch.randn(B, L, Hkv, D, device=DEV, generator=g).half()
    cl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    outs = {}
    for bs in (64, 48, 8, 1):
        kc, vc, table = _pool(K, V, lens, bs, seed=bs)
        outs[bs] = paged_attention(q, kc, vc, table.to(DEV), bs, L, context_lens=cl)
        torch.cuda.synchronize()
        if bs == 8:
            rows = torch.tensor([0, 31])
            ref = OA.paged_attention(q.cpu()[rows], kc.cpu(), vc.cpu(), table[rows], bs,
                                     [lens[r] for r in rows.tolist()])
            assert _maxabs(outs[bs].cpu()[rows], ref) <= ATOL
        del kc, vc
    for bs in (48, 8, 1):
        assert torch.equal(outs[bs], outs[64]), bs


def test_paged_decode_block_size_pool_over_4gib(hip):
    # Pools above 4 GiB with block_size 8 take the per-row descriptors instead of per-lane
    # offsets into one descriptor: the same contexts, moved to blocks spread over such a
    # pool, give outputs bit-identical to the small pool's, and the oracle agrees.
    banner("paged decode block_size 8, 4.3 GB pools")
    from fast_infer_amd import paged_attention

    B, Hq, Hkv, D, bs = 4, 24, 8, 128, 8
    lens = [3000, 1, 700, 2048]
    g = torch.Generator(device=DEV).manual_seed(9)
    q = torch.randn(B, Hq, D, device=DEV, generator=g).half()
    K = torch.randn(B, max(lens), Hkv, D, device=DEV, generator=g).half()
    V = torch.randn(B, max(lens), Hkv, D, device=DEV, generator=g).half()
    cl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    kc, vc, table = _pool(K, V, lens, bs, seed=9)
    small = paged_attention(q, kc, vc, table.to(DEV), bs, max(lens), context_lens=cl)

    big_n = (1 << 32) // (bs * Hkv * D * 2) + 64
    ids = torch.randperm(big_n - 1, generator=torch.Generator().manual_seed(10))[:kc.shape[0]]
    ids[int(table[0, 0])] = big_n - 1  # the pool's last block holds row 0's first tokens
    kb = torch.empty(big_n, bs, Hkv, D, dtype=torch.float16, device=DEV)
    vb = torch.empty_like(kb)
    kb[ids.to(DEV)] = kc
    vb[ids.to(DEV)] = vc
    tb = torch.where(table >= 0, ids[table.clamp(min=0).long()].int(), table)
    big = paged_attention(q, kb, vb, tb.to(DEV), bs, max(lens), context_lens=cl)
    torch.cuda.synchronize()
    assert int(tb.max()) == big_n - 1
    assert torch.equal(big, small)
    ref = OA.paged_attention(q.cpu(), kc.cpu(), vc.cpu(), table, bs, lens)
    assert _maxabs(small, ref) <= ATOL


@pytest.mark.parametrize("bs", [8, 1])
def test_paged_decode_block_size_graph_replay(hip, bs):
    # captured once, replayed with other decode calls and synchronisation between replays;
    # each replay equals the eager call bit for bit (the kernels record no memset)
    banner(f"paged decode block_size {bs}, HIP graph replay")
    from fast_infer_amd import paged_attention, paged_attention_workspace

    lens = [900, 3000, 17, 2048]
    q, kc, vc, table, lens = _inputs(bs, lens, Hq=24, Hkv=8, seed=20 + bs)
    q, kc, vc, table = q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV)
    cl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    ws = paged_attention_workspace(len(lens), 24, 8, 3000, 128, DEV)
    ref = paged_attention(q, kc, vc, table, bs, 3000, context_lens=cl, workspace=ws).clone()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        paged_attention(q, kc, vc, table, bs, 3000, context_lens=cl, workspace=ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = paged_attention(q, kc, vc, table, bs, 3000, context_lens=cl, workspace=ws)
    torch.cuda.synchronize()
    for rep in range(3):
        paged_attention(torch.randn_like(q), kc, vc, table, bs, 3000, context_lens=cl,
                        workspace=ws)
        torch.cuda.synchronize()
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), rep


@pytest.mark.parametrize("bs", [1, 8, 24, 100, 128])
@pytest.mark.parametrize("S,D", [(1, 128), (300, 128), (700, 64)])
def test_flash_prefill_pool_write_block_size(hip, bs, S, D):
    # the fused prefill pool write at block sizes other than 64: the written slots equal the
    # scatter of K/V bit for bit, every other slot keeps its bytes, the output is the plain
    # call's (a row's table is one block short, so its last tokens are not written)
    banner(f"flash prefill fused pool write, block_size {bs}, S={S}, head_dim {D}")
    import numpy as np

    from fast_infer_amd import flash_attention
    from oracle import kv as OK

    B, H, Hkv = 2, 6, 2
    g = torch.Generator().manual_seed(bs * 7 + S)
    q = torch.randn(B, S, H, D, generator=g).half().to(DEV).transpose(1, 2)
    k = torch.randn(B, S, Hkv, D, generator=g).half().to(DEV)
    v = torch.randn(B, S, Hkv, D, generator=g).half().to(DEV)
    nb = math.ceil(S / bs)
    N = 2 * nb + 3
    perm = torch.randperm(N, generator=torch.Generator().manual_seed(bs)).int()
    table = perm[:2 * nb].view(2, nb).clone()
    if nb > 1:
        table[1, nb - 1] = -1  # row 1's last block missing
    kc0 = torch.randn(N, bs, Hkv, D, generator=g).half()
    vc0 = torch.randn(N, bs, Hkv, D, generator=g).half()
    kc, vc = kc0.to(DEV), vc0.to(DEV)
    out = flash_attention(q, k.transpose(1, 2), v.transpose(1, 2), k_cache=kc, v_cache=vc,
                          block_table=table.to(DEV), block_size=bs)
    plain = flash_attention(q, k.transpose(1, 2), v.transpose(1, 2))
    torch.cuda.synchronize()
    assert torch.equal(out, plain)
    ek, ev = kc0.numpy().copy(), vc0.numpy().copy()
    OK.scatter(ek, ev, table.tolist(), k.cpu().numpy(), v.cpu().numpy(), 0, bs)
    assert np.array_equal(kc.cpu().numpy().view(np.uint16), ek.view(np.uint16))
    assert np.array_equal(vc.cpu().numpy().view(np.uint16), ev.view(np.uint16))


@pytest.mark.parametrize("bs", [8, 64])
def test_flash_prefill_pool_write_narrow_table(hip, bs):
    # a table one block narrower than the sequence needs, and an entry outside the pool:
    # tokens past the table or in that block are not written, everything else is
    banner(f"flash prefill fused pool write, block_size {bs}, narrow table")
    import numpy as np

    from fast_infer_amd import flash_attention
    from oracle import kv as OK

    B, S, H, Hkv, D = 2, 200, 6, 2, 128
    g = torch.Generator().manual_seed(bs + 99)
    q = torch.randn(B, S, H, D, generator=g).half().to(DEV).transpose(1, 2)
    k = torch.randn(B, S, Hkv, D, generator=g).half().to(DEV)
    v = torch.randn(B, S, Hkv, D, generator=g).half().to(DEV)
    nb = math.ceil(S / bs)
    N = 2 * nb + 1
    perm = torch.randperm(N, generator=torch.Generator().manual_seed(bs)).int()
    table = perm[:2 * nb].view(2, nb)[:, :nb - 1].clone()  # one block short
    table[0, 1] = 10 ** 6                                  # outside the pool
    kc0 = torch.randn(N, bs, Hkv, D, generator=g).half()
    vc0 = torch.randn(N, bs, Hkv, D, generator=g).half()
    kc, vc = kc0.to(DEV), vc0.to(DEV)
    out = flash_attention(q, k.transpose(1, 2), v.transpose(1, 2), k_cache=kc, v_cache=vc,
                          block_table=table.to(DEV), block_size=bs)
    plain = flash_attention(q, k.transpose(1, 2), v.transpose(1, 2))
    torch.cuda.synchronize()
    assert torch.equal(out, plain)
    ek, ev = kc0.numpy().copy(), vc0.numpy().copy()
    OK.scatter(ek, ev, table.tolist(), k.cpu().numpy(), v.cpu().numpy(), 0, bs)
    assert np.array_equal(kc.cpu().numpy().view(np.uint16), ek.view(np.uint16))
    assert np.array_equal(vc.cpu().numpy().view(np.uint16), ev.view(np.uint16))
