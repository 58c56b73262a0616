"""GPU tests of the device block manager (``fi_kv_append`` / ``fi_kv_release`` /
``fi_kv_reset`` through ``PagedKVCache``), marked ``gpu``.

* Random append / release walks compared after every call with the oracle
  (oracle/block_manager.py): block table, lengths, free-queue order, status, and the
  returned start positions and lengths, exactly.
* A continuous-batching decode run end to end: ragged prompts, rows retired and new
  sequences admitted mid-run, every step's RoPE + pool write (``rope_store_kv`` with the
  manager's start positions) and paged attention (with its per-row lengths) against the
  oracle chain (block manager, RoPE, scatter, fp32 paged attention) at max-abs 2e-3, and
  the pool bytes bit-exact.
"""

import random

import numpy as np
import pytest
import torch

from conftest import ATOL, banner
from oracle import attention as OA
from oracle import block_manager as OB
from oracle import kv as OK
from oracle import rope as OR

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _compare(cache, m: OB.OracleBlockManager):
    torch.cuda.synchronize()
    table = cache.block_table.cpu().tolist()
    assert table == [row[:cache.max_blocks_per_seq] for row in m.block_table]
    assert cache.seq_lens.cpu().tolist() == m.seq_lens
    assert cache.num_alloc.cpu().tolist() == [m.cache.allocated(b) for b in range(m.max_batch)]
    assert cache.free_list() == m.free_blocks
    code, row, free = cache.status()
    assert (code, row) == m.status and free == len(m.free_blocks)


@pytest.mark.parametrize("B,N,bs,maxlen,seed", [(8, 64, 16, 192, 0), (3000, 20000, 64, 1024, 1)])
def test_random_walk_matches_oracle(hip, B, N, bs, maxlen, seed):
    banner(f"block manager walk B={B} N={N}")
    from fast_infer_amd import PagedKVCache

    cache = PagedKVCache(1, 1, 128, maxlen, bs, DEV, max_batch=B, num_blocks=N)
    m = OB.OracleBlockManager(N, cache.max_blocks_per_seq, B, bs)
    _compare(cache, m)
    rng = random.Random(seed)
    for step in range(60):
        r = rng.random()
        if r < 0.15:
            rows = rng.sample(range(B), rng.randint(1, max(1, B // 4)))
            cache.release(rows)
            m.release(rows)
        elif r < 0.2:
            cache.reset()
            m.reset()
        else:
            batch = rng.choice([B, max(1, B // 2), 1])
            if rng.random() < 0.3:
                n = rng.choice([0, 1, 64])
                starts, lens = cache.append(n, batch)
                es, el = m.append(n, batch)
            else:
                ns = [rng.choice([0, 1, 1, 2, 15, 63, 130]) for _ in range(batch)]
                starts, lens = cache.append(torch.tensor(ns, dtype=torch.int32), batch)
                es, el = m.append(ns, batch)
            torch.cuda.synchronize()
            assert starts.cpu().tolist() == es
            assert lens.cpu().tolist() == el
        _compare(cache, m)


def test_errors_recorded_and_check_raises(hip):
    banner("block manager errors")
    from fast_infer_amd import PagedKVCache
    from fast_infer_amd._lib import FastInferError

    cache = PagedKVCache(1, 1, 128, 32, 8, DEV, max_batch=4, num_blocks=6)
    m = OB.OracleBlockManager(6, 4, 4, 8)
    cache.append(torch.tensor([8, 40, 8, 8], dtype=torch.int32))
    m.append([8, 40, 8, 8])
    _compare(cache, m)
    with pytest.raises(FastInferError, match="block table full"):
        cache.check()
    cache.reset()
    m.reset()
    cache.append(16)
    m.append(16)
    _compare(cache, m)
    with pytest.raises(FastInferError, match="out of memory"):
        cache.check()
    cache.reset()
    cache.append(torch.tensor([1, -1, 1, 1], dtype=torch.int32))
    m.reset()
    m.append([1, -1, 1, 1])
    _compare(cache, m)
    cache.reset()
    cache.check()  # clear again


@pytest.mark.parametrize("bs", [16, 8, 5])
def test_continuous_batching_decode_end_to_end(hip, bs):
    # block sizes 8 and 5 run the decode kernel's per-row block addressing
    banner(f"continuous batching: rope + pool write + paged decode, block_size {bs}")
    from fast_infer_amd import PagedKVCache, paged_attention, rope_store_kv

    L, Hq, Hkv, D, B, maxlen = 2, 8, 2, 128, 6, 256
    N = 90 * 16 // bs
    cache = PagedKVCache(L, Hkv, D, maxlen, bs, DEV, max_batch=B, num_blocks=N)
    m = OB.OracleBlockManager(N, cache.max_blocks_per_seq, B, bs)
    cos, sin = OR.precompute_freqs(D, maxlen)
    c16, s16 = cos.astype(np.float16), sin.astype(np.float16)
    cos_d, sin_d = torch.from_numpy(c16).to(DEV), torch.from_numpy(s16).to(DEV)
    kpool = np.zeros((L, N, bs, Hkv, D), np.float16)   # oracle pools
    vpool = np.zeros_like(kpool)
    g = torch.Generator().manual_seed(40)

    def qkv(T):
        return (torch.randn(B, T, Hq, D, generator=g).half(),
                torch.randn(B, T, Hkv, D, generator=g).half(),
                torch.randn(B, T, Hkv, D, generator=g).half())

    def write(rows, T, counts):
        """One call that adds counts[b] tokens to each row (a prompt or a decode token)."""
        starts, lens = cache.append(torch.tensor(counts, dtype=torch.int32))
        es, el = m.append(counts)
        outs = []
        for layer in range(L):
            q, k, v = qkv(T)
            sel = torch.tensor(rows)
            st_rows = starts[sel.to(DEV)]
            q_rot, _ = rope_store_kv(q[sel].to(DEV), k[sel].to(DEV), v[sel].to(DEV), cos_d,
                                     sin_d, 0, cache.k[layer], cache.v[layer],
                                     cache.block_table[sel.to(DEV)],
                                     start_positions=st_rows, return_k=False)
            table = [m.block_table[r] for r in rows]
            eq, _ = OR.rope_store_kv(q[sel].numpy(), k[sel].numpy(), v[sel].numpy(), c16, s16,
                                     [es[r] for r in rows], kpool[layer], vpool[layer], table, bs)
            outs.append((q_rot, eq))
        return lens, el, outs

    # ragged prompts for rows 0..4; row 5 stays empty
    prompts = [5, 17, 1, 33, 16, 0]
    rows = [0, 1, 2, 3, 4]
    write(rows, max(prompts), prompts)
    active = [True] * 5 + [False]
    for step in range(40):
        if step == 12:                       # retire row 1, admit a 9-token prompt there
            cache.release([1])
            m.release([1])
            write([1], 9, [0, 9, 0, 0, 0, 0])
        if step == 20:                       # row 5 joins with a 24-token prompt
            write([5], 24, [0, 0, 0, 0, 0, 24])
            active[5] = True
        if step == 30:                       # row 2 finishes
            cache.release([2])
            m.release([2])
            active[2] = False
        live = [b for b in range(B) if active[b]]
        counts = [1 if active[b] else 0 for b in range(B)]
        lens, el, outs = write(live, 1, counts)
        for layer, (q_rot, eq) in enumerate(outs):
            qd = torch.zeros(B, Hq, D, dtype=torch.float16, device=DEV)
            qd[torch.tensor(live, device=DEV)] = q_rot[:, 0]
            o = paged_attention(qd, cache.k[layer], cache.v[layer], cache.block_table, bs, lens)
            qo = np.zeros((B, Hq, D), np.float16)
            qo[live] = eq[:, 0]
            table = np.array([row[:cache.max_blocks_per_seq] for row in m.block_table])
            ref = OA.paged_attention(torch.from_numpy(qo), torch.from_numpy(kpool[layer]),
                                     torch.from_numpy(vpool[layer]), table, bs, el)
            torch.cuda.synchronize()
            got = o.float().cpu()
            err = float((got[live] - ref[live]).abs().max())
            assert err <= ATOL, (step, layer, err)
    _compare(cache, m)
    # every live row's context in the pool equals the oracle's, bit for bit
    torch.cuda.synchronize()
    kc, vc = cache.k.cpu().numpy(), cache.v.cpu().numpy()
    for b in range(B):
        for p in range(m.seq_lens[b]):
            phys, slot = m.block_table[b][p // bs], p % bs
            assert np.array_equal(kc[:, phys, slot].view(np.uint16), kpool[:, phys, slot].view(np.uint16))
            assert np.array_equal(vc[:, phys, slot].view(np.uint16), vpool[:, phys, slot].view(np.uint16))
