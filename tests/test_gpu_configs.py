"""Parity at the benchmarked workload sizes (marked ``gpu``).

* Batch 64, 28-layer decode step over per-layer 4096-block pools, lognormal contexts
  (median 1024, sigma 0.5, clipped to [64, 4096]), built with the seeds the benchmark
  uses: every row of four layers and sampled rows of the others against the fp32 oracle
  (max-abs 2e-3).
* The same workload as a serving loop runs it: ``PagedKVCache.append`` of one token per
  row, then per layer the fused RoPE + pool write at the rows' positions and paged
  attention over the rows' lengths (4 layers, 4096-block pools).  The written pool slots
  are compared bit for bit with the oracle's RoPE, and the attention with the oracle chain.
* Causal prefill with the fused pool write at batch 4 x 4096 (256-block shuffled pool)
  and batch 1 x 512 (64-block shuffled pool): the pool gathered back through the table
  equals K/V bit for bit, blocks outside the table stay zero, and the output equals the
  call without a pool bit for bit (batch 1 x 512 also against the reference-kernel
  goldens and the fp32 oracle).

Reference: model.py:77 (layer loop), :123-130 (decode call), :162-183 (prefill store).
"""

import math

import numpy as np
import pytest
import torch

from conftest import ATOL, banner
from golden import specs
from oracle import attention as OA
from oracle import rope as OR

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
HQ, HKV, D, BS = 24, 8, 128, 64


def _maxabs(a, b):
    return float((torch.as_tensor(a).float().cpu() - torch.as_tensor(b).float().cpu()).abs().max())


def _lognormal_lens(B=64, seed=4):
    gen = torch.Generator().manual_seed(seed)
    lens = torch.exp(torch.randn(B, generator=gen) * 0.5 + math.log(1024)).round()
    return lens.clamp(64, 4096).int()


def _dealt_table(lens, pool_blocks, seed, width=64):
    """One seeded permutation of the pool dealt row-major to the rows' blocks; -1 after."""
    perm = torch.randperm(pool_blocks, generator=torch.Generator().manual_seed(seed)).int()
    table = torch.full((len(lens), width), -1, dtype=torch.int32)
    pos = 0
    for b, n in enumerate(lens):
        nb = math.ceil(int(n) / BS)
        table[b, :nb] = perm[pos:pos + nb]
        pos += nb
    assert pos <= pool_blocks
    return table


def _row_oracle(q_row, kpool, vpool, table_row, n):
    """fp32 oracle for one row: gather the row's blocks (in table order) on the host and
    attend over its first n tokens."""
    nb = math.ceil(n / BS)
    ids = table_row[:nb].to(torch.int64)
    kb = kpool.index_select(0, ids.to(kpool.device)).cpu()
    vb = vpool.index_select(0, ids.to(vpool.device)).cpu()
    local = torch.arange(nb, dtype=torch.int32).view(1, nb)
    return OA.paged_attention(q_row.cpu().view(1, HQ, D), kb, vb, local, BS, [n])[0]


def test_decode_28layer_b64_lognormal_vs_oracle(hip):
    """28 layers x batch 64, per-layer 4096-block pools and shuffled tables."""
    from fast_infer_amd import paged_attention, paged_attention_workspace

    L, B, N = 28, 64, 4096
    lens = _lognormal_lens(B, 4)
    banner(f"decode 28 layers batch {B}, lognormal contexts {int(lens.min())}..{int(lens.max())}, "
           f"sum {int(lens.sum())}")
    g = torch.Generator(device=DEV).manual_seed(4)
    kpool = torch.empty(L, N, BS, HKV, D, device=DEV, dtype=torch.float16)
    vpool = torch.empty_like(kpool)
    for layer in range(L):
        kpool[layer].normal_(generator=g)
        vpool[layer].normal_(generator=g)
    tables = [_dealt_table(lens.tolist(), N, 100 + layer) for layer in range(L)]
    qs = torch.randn(L, B, HQ, D, device=DEV, generator=g, dtype=torch.float16)
    cl = lens.to(DEV)
    ws = paged_attention_workspace(B, HQ, HKV, 4096, D, DEV)
    outs = []
    for layer in range(L):
        outs.append(paged_attention(qs[layer], kpool[layer], vpool[layer], tables[layer].to(DEV),
                                    BS, 4096, context_lens=cl, workspace=ws))
    torch.cuda.synchronize()
    outs = torch.stack(outs).cpu()
    assert bool(torch.isfinite(outs.float()).all())

    rng = np.random.default_rng(4)
    order = np.argsort(lens.numpy())
    checked = 0
    worst = 0.0
    for layer in range(L):
        if layer in (0, 9, 18, 27):
            rows = range(B)
        else:  # the shortest and longest rows plus two random ones
            rows = sorted({int(order[0]), int(order[-1]), *rng.integers(0, B, 2).tolist()})
        for b in rows:
            ref = _row_oracle(qs[layer, b], kpool[layer], vpool[layer], tables[layer][b],
                              int(lens[b]))
            err = _maxabs(outs[layer, b], ref)
            worst = max(worst, err)
            assert err <= ATOL, (layer, b, int(lens[b]), err)
            checked += 1
    print(f"[case] checked {checked} (layer, row) pairs, worst max-abs {worst:.2e}", flush=True)


def test_decode_step_paged_b64_lognormal_vs_oracle_chain(hip):
    """The serving-loop step: append one token per row, then per layer RoPE + pool write at
    the rows' positions and attention over the rows' lengths (4 layers, 4096-block pools)."""
    from fast_infer_amd import (PagedKVCache, paged_attention, paged_attention_workspace,
                                precompute_freqs, rope_store_kv)

    L, B, N = 4, 64, 4096
    lens = _lognormal_lens(B, 4)
    max_len = 4096 + 8
    banner(f"decode step with block manager, {L} layers, batch {B}, pools {N} blocks")
    cache = PagedKVCache(L, HKV, D, max_len, BS, DEV, max_batch=B, num_blocks=N)
    g = torch.Generator(device=DEV).manual_seed(4)
    cache.k.normal_(generator=g)
    cache.v.normal_(generator=g)
    cache.append(lens.to(DEV))
    cache.check()
    cos, sin = precompute_freqs(D, max_len, device=DEV)
    cos, sin = cos.half(), sin.half()
    qkv = torch.randn(L, B, 1, (HQ + 2 * HKV) * D, device=DEV, generator=g, dtype=torch.float16)
    q = qkv[..., :HQ * D].view(L, B, 1, HQ, D)
    k = qkv[..., HQ * D:(HQ + HKV) * D].view(L, B, 1, HKV, D)
    v = qkv[..., (HQ + HKV) * D:].view(L, B, 1, HKV, D)
    q_rot = torch.empty(L, B, 1, HQ, D, device=DEV, dtype=torch.float16)
    ws = paged_attention_workspace(B, HQ, HKV, max_len, D, DEV)

    starts, ctx = cache.append(1)
    outs = []
    for layer in range(L):
        rope_store_kv(q[layer], k[layer], v[layer], cos, sin, 0, cache.k[layer], cache.v[layer],
                      cache.block_table, start_positions=starts, return_k=False,
                      q_out=q_rot[layer])
        outs.append(paged_attention(q_rot[layer][:, 0], cache.k[layer], cache.v[layer],
                                    cache.block_table, BS, max_len, context_lens=ctx,
                                    workspace=ws))
    torch.cuda.synchronize()
    cache.check()
    starts_h, ctx_h = starts.cpu(), ctx.cpu()
    assert torch.equal(starts_h, lens) and torch.equal(ctx_h, lens + 1)
    table = cache.block_table.cpu()
    cos_h, sin_h = cos.cpu().numpy(), sin.cpu().numpy()

    worst = 0.0
    for layer in range(L):
        q_exp, k_exp = OR.rope_store_kv(q[layer].cpu().numpy(), k[layer].cpu().numpy(),
                                        v[layer].cpu().numpy(), cos_h, sin_h,
                                        starts_h.tolist())
        # the rotated q the attention used
        assert np.array_equal(q_rot[layer].cpu().numpy().view(np.uint16), q_exp.view(np.uint16))
        for b in range(B):
            pos = int(starts_h[b])
            phys = int(table[b, pos // BS])
            slot = pos % BS
            got_k = cache.k[layer, phys, slot].cpu().numpy()
            got_v = cache.v[layer, phys, slot].cpu().numpy()
            assert np.array_equal(got_k.view(np.uint16), k_exp[b, 0].view(np.uint16)), (layer, b)
            assert np.array_equal(got_v.view(np.uint16),
                                  v[layer, b, 0].cpu().numpy().view(np.uint16)), (layer, b)
            ref = _row_oracle(torch.from_numpy(q_exp[b, 0]), cache.k[layer], cache.v[layer],
                              table[b], pos + 1)
            err = _maxabs(outs[layer][b], ref)
            worst = max(worst, err)
            assert err <= ATOL, (layer, b, pos + 1, err)
    print(f"[case] {L} layers x {B} rows, worst max-abs {worst:.2e}", flush=True)


def _pool_prefill_case(B, S, pool_blocks, seed, table_blocks=None):
    from fast_infer_amd import flash_attention

    table_blocks = table_blocks or pool_blocks
    per_row = table_blocks // B
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(B, S, HQ, D, device=DEV, generator=g, dtype=torch.float16).transpose(1, 2)
    k = torch.randn(B, S, HKV, D, device=DEV, generator=g, dtype=torch.float16).transpose(1, 2)
    v = torch.randn(B, S, HKV, D, device=DEV, generator=g, dtype=torch.float16).transpose(1, 2)
    kc = torch.zeros(pool_blocks, BS, HKV, D, device=DEV, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    perm = torch.randperm(pool_blocks, generator=torch.Generator().manual_seed(seed)).int()
    table = perm[:per_row * B].view(B, per_row).to(DEV)
    out = flash_attention(q, k, v, k_cache=kc, v_cache=vc, block_table=table)
    plain = flash_attention(q, k, v)
    torch.cuda.synchronize()
    assert torch.equal(out, plain)
    nb = math.ceil(S / BS)
    used = table[:, :nb].to(torch.int64)
    # gather the pool back through the table: [B, nb * BS, HKV, D], first S tokens
    gk = kc.index_select(0, used.reshape(-1)).view(B, nb * BS, HKV, D)[:, :S]
    gv = vc.index_select(0, used.reshape(-1)).view(B, nb * BS, HKV, D)[:, :S]
    assert torch.equal(gk, k.transpose(1, 2))
    assert torch.equal(gv, v.transpose(1, 2))
    # slots past S in the last block and every block outside the table stay zero
    if S % BS:
        tail = kc.index_select(0, used[:, -1])[:, S % BS:]
        assert not bool(tail.any())
    mask = torch.ones(pool_blocks, dtype=torch.bool, device=DEV)
    mask[used.reshape(-1)] = False
    assert not bool(kc[mask].any()) and not bool(vc[mask].any())
    return q, k, v, out, int(mask.sum())


def test_prefill_pool_write_b4_s4096(hip):
    """Batch 4 x 4096 with the K/V write into a 256-block shuffled pool."""
    banner("prefill batch 4 x 4096 with pool write (256-block pool)")
    q, k, v, out, untouched = _pool_prefill_case(4, 4096, 256, 3)
    assert untouched == 0
    rows = [0, 63, 64, 2047, 4095]
    heads = [0, 5, 23]
    ref = OA.causal_attention_rows(q.cpu(), k.cpu(), v.cpu(), rows, heads)
    assert _maxabs(out.cpu()[:, heads][:, :, rows], ref) <= ATOL


def test_prefill_pool_write_b4_s4096_spare_blocks(hip):
    """The same call with a 288-block pool: the 32 blocks outside the table stay zero."""
    banner("prefill batch 4 x 4096 with pool write (288-block pool, 256 used)")
    _, _, _, _, untouched = _pool_prefill_case(4, 4096, 288, 3, table_blocks=256)
    assert untouched == 32


def test_prefill_pool_write_b1_s512(hip, golden):
    """Batch 1 x 512 with the K/V write into a 64-block shuffled pool (8 blocks used): the
    output also against the reference-kernel goldens and the fp32 oracle."""
    banner("prefill batch 1 x 512 with pool write (64-block pool)")
    from fast_infer_amd import KVCache, allocate_prefill, flash_attention

    q, k, v, out, untouched = _pool_prefill_case(1, 512, 64, 1, table_blocks=64)
    assert untouched == 56
    arrays, _ = golden
    sp = specs.PREFILL_CASES["prefill_b1_s512"]
    gq, gk, gv = specs.prefill_inputs(sp)
    cache = KVCache(1, HKV, D, max_seq_len=4096, block_size=BS, device=DEV, num_blocks=64)
    allocate_prefill(cache, 1, 512)
    # golden inputs through the fused call: output matches the goldens and the oracle
    o = flash_attention(gq.to(DEV), gk.to(DEV), gv.to(DEV), k_cache=cache.k[0],
                        v_cache=cache.v[0], block_table=cache.block_table)
    torch.cuda.synchronize()
    rows = arrays["prefill_b1_s512__rows"]
    assert _maxabs(o.cpu()[:, :, rows], arrays["prefill_b1_s512__out"]) <= ATOL
    assert _maxabs(o.cpu(), OA.causal_attention(gq, gk, gv)) <= ATOL
