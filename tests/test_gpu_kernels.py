"""GPU parity tests of the HIP kernels through the C ABI (marked ``gpu``).

* MFMA fragment layout self-test (the layout every attention kernel assumes).
* KV scatter: bit-exact against the brute-force oracle, untouched bytes preserved.
* Paged decode: reference-kernel goldens and the fp32 oracle within max-abs 2e-3.
* Causal prefill: reference-kernel goldens and the fp32 oracle within max-abs 2e-3;
  fused pool write bit-exact.
Full-size workloads are checked on sampled rows / heads against the oracle and
through size-independent properties.
"""

import math

import numpy as np
import pytest
import torch

from conftest import ATOL, banner
from golden import specs
from oracle import attention as OA
from oracle import kv as OK

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _maxabs(a, b):
    return float((torch.as_tensor(a).float().cpu() - torch.as_tensor(b).float().cpu()).abs().max())


# --------------------------------------------------------------------------- MFMA


def test_mfma_fragment_layout(hip):
    banner("mfma 16x16x32 f16 layout")
    from fast_infer_amd import _lib

    rs = np.random.RandomState(0)
    A = rs.randint(-4, 5, size=(16, 32)).astype(np.float16)
    B = rs.randint(-4, 5, size=(32, 16)).astype(np.float16)
    a = np.zeros((64, 8), np.float16)
    b = np.zeros((64, 8), np.float16)
    for lane in range(64):
        for s in range(8):
            a[lane, s] = A[lane % 16, 8 * (lane // 16) + s]
            b[lane, s] = B[8 * (lane // 16) + s, lane % 16]
    ta = torch.from_numpy(a).to(DEV)
    tb = torch.from_numpy(b).to(DEV)
    tc = torch.zeros(64, 4, dtype=torch.float32, device=DEV)
    rc = hip.fi_selftest_mfma_f16(ta.data_ptr(), tb.data_ptr(), tc.data_ptr(),
                                  _lib.stream_handle(torch.device(DEV)))
    _lib.check(rc, "selftest")
    c = tc.cpu().numpy()
    C = A.astype(np.float32) @ B.astype(np.float32)
    got = np.zeros((16, 16), np.float32)
    for lane in range(64):
        for i in range(4):
            got[4 * (lane // 16) + i, lane % 16] = c[lane, i]
    assert np.array_equal(got, C)


# --------------------------------------------------------------------------- KV scatter


def _rand_pool(N, bs, H, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(N, bs, H, 128, generator=g).half()


@pytest.mark.parametrize("per_row", [False, True])
def test_store_kv_bitexact_vs_bruteforce(hip, per_row):
    banner(f"store_kv per_row={per_row}")
    from fast_infer_amd import store_kv

    B, T, H, bs, N = 3, 100, 8, 16, 40
    g = torch.Generator().manual_seed(1)
    # k/v as strided views of a wider buffer (like the model's qkv split)
    big = torch.randn(B, T, H * 128 * 3, generator=g).half()
    k = big[:, :, :H * 128].view(B, T, H, 128)
    v = big[:, :, 2 * H * 128:].view(B, T, H, 128)
    table = torch.full((B, 10), -1, dtype=torch.int32)
    perm = torch.randperm(N, generator=g).int()
    table[:, :8] = perm[:24].view(3, 8)
    table[1, 3] = -1          # unallocated entry inside the range: skipped
    table[2, 5] = N + 7       # out-of-pool entry: skipped
    starts = [0, 20, 57] if per_row else 9
    pk, pv = _rand_pool(N, bs, H, 2), _rand_pool(N, bs, H, 3)
    ek, ev = pk.numpy().copy(), pv.numpy().copy()
    OK.scatter(ek, ev, table.tolist(), k.numpy(), v.numpy(), starts, bs)
    dk, dv = pk.to(DEV), pv.to(DEV)
    sp = torch.tensor(starts, dtype=torch.int32, device=DEV) if per_row else None
    store_kv(k.to(DEV), v.to(DEV), dk, dv, table.to(DEV), 0 if per_row else starts,
             start_positions=sp)
    torch.cuda.synchronize()
    assert np.array_equal(dk.cpu().numpy().view(np.uint16), ek.view(np.uint16))
    assert np.array_equal(dv.cpu().numpy().view(np.uint16), ev.view(np.uint16))


def test_kvcache_prefill_decode_stores_match_reference_semantics(hip):
    banner("KVCache prefill+decode stores")
    from fast_infer_amd import KVCache, store_kv_decode, store_kv_prefill

    L, H, S, B = 2, 8, 150, 2
    fi = KVCache(L, H, 128, max_seq_len=512, block_size=64, device=DEV, num_blocks=20)
    ok = OK.OracleKVCache(L, H, 128, max_seq_len=512, block_size=64, num_blocks=20)
    g = torch.Generator().manual_seed(4)
    for layer in range(L):
        k = torch.randn(B, S, H, 128, generator=g).half()
        v = torch.randn(B, S, H, 128, generator=g).half()
        store_kv_prefill(fi, layer, k.to(DEV), v.to(DEV))
        OK.store_prefill(ok, layer, k.numpy(), v.numpy())
    for pos in (150, 191, 192):
        for layer in range(L):
            k = torch.randn(B, H, 128, generator=g).half()
            v = torch.randn(B, H, 128, generator=g).half()
            store_kv_decode(fi, layer, k.to(DEV), v.to(DEV), pos)
            OK.store_decode(ok, layer, k.numpy(), v.numpy(), pos)
    torch.cuda.synchronize()
    assert fi.block_table.cpu().tolist() == ok.block_table
    assert fi.num_tokens == ok.num_tokens
    assert np.array_equal(fi.k.cpu().numpy().view(np.uint16), ok.k.view(np.uint16))
    assert np.array_equal(fi.v.cpu().numpy().view(np.uint16), ok.v.view(np.uint16))


def test_kvcache_store_and_store_batch(hip):
    banner("KVCache store/store_batch")
    from fast_infer_amd import KVCache

    fi = KVCache(1, 4, 128, max_seq_len=256, block_size=16, device=DEV)
    ok = OK.OracleKVCache(1, 4, 128, max_seq_len=256, block_size=16)
    for _ in range(6):
        fi.alloc_block(0)
        ok.alloc_block(0)
    g = torch.Generator().manual_seed(5)
    k = torch.randn(50, 4, 128, generator=g).half()
    fi.store_batch(0, 1, 3, k.to(DEV), (k * 2).to(DEV))
    OK.store_batch(ok, 0, 1, 3, k.numpy(), (k * 2).numpy())
    one = torch.randn(4, 128, generator=g).half()
    fi.store(0, 4, 9, one.to(DEV), one.to(DEV))
    OK.store(ok, 0, 4, 9, one.numpy(), one.numpy())
    torch.cuda.synchronize()
    assert np.array_equal(fi.k.cpu().numpy().view(np.uint16), ok.k.view(np.uint16))
    assert np.array_equal(fi.v.cpu().numpy().view(np.uint16), ok.v.view(np.uint16))


def test_store_kv_full_size_round_trip(hip):
    # batch 4 x 4096 tokens into a 256-block pool (block_size 64), shuffled table:
    # gathering every token back through the table returns the input bytes.
    banner("store_kv 4x4096 round trip")
    from fast_infer_amd import store_kv

    B, S, H, bs, N = 4, 4096, 8, 64, 256
    g = torch.Generator(device=DEV).manual_seed(6)
    k = torch.randn(B, S, H, 128, device=DEV, generator=g).half()
    v = torch.randn(B, S, H, 128, device=DEV, generator=g).half()
    table = torch.randperm(N, device=DEV, generator=g).int().view(B, N // B)
    pk = torch.zeros(N, bs, H, 128, dtype=torch.float16, device=DEV)
    pv = torch.zeros_like(pk)
    store_kv(k, v, pk, pv, table, 0)
    t = torch.arange(S, device=DEV)
    for b in range(B):
        phys = table[b, t // bs].long()
        assert torch.equal(pk[phys, t % bs], k[b])
        assert torch.equal(pv[phys, t % bs], v[b])


# --------------------------------------------------------------------------- decode


def _decode_case(name):
    sp = {**specs.DECODE_CASES, **specs.RAGGED_CASES}[name]
    return sp, specs.decode_inputs(sp)


@pytest.mark.parametrize("name", list(specs.DECODE_CASES))
def test_paged_decode_vs_reference_and_oracle(hip, golden, name):
    banner(f"paged decode {name}")
    from fast_infer_amd import paged_attention

    arrays, _ = golden
    sp, (q, kc, vc, table, lens) = _decode_case(name)
    out = paged_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), sp["bs"], sp["ctx"])
    torch.cuda.synchronize()
    assert out.shape == q.shape and out.dtype == torch.float16
    ref = arrays[f"{name}__out"]
    assert _maxabs(out, ref) <= ATOL
    assert _maxabs(out, OA.paged_attention(q, kc, vc, table, sp["bs"], lens)) <= ATOL


@pytest.mark.parametrize("name", list(specs.RAGGED_CASES))
@pytest.mark.parametrize("as_num_tokens", [False, True])
def test_paged_decode_ragged(hip, golden, name, as_num_tokens):
    banner(f"paged decode ragged {name} as_num_tokens={as_num_tokens}")
    from fast_infer_amd import paged_attention

    arrays, _ = golden
    sp, (q, kc, vc, table, lens) = _decode_case(name)
    cl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    args = (q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), sp["bs"])
    if as_num_tokens:
        out = paged_attention(*args, cl)
    else:
        out = paged_attention(*args, max(lens), context_lens=cl)
    torch.cuda.synchronize()
    assert _maxabs(out, arrays[f"{name}__out"]) <= ATOL
    for b, n in enumerate(lens):
        if n == 0:
            assert float(out[b].abs().max()) == 0.0


def test_paged_decode_zero_tokens_returns_zeros(hip):
    from fast_infer_amd import paged_attention

    sp, (q, kc, vc, table, _) = _decode_case("decode_ctx63")
    out = paged_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), sp["bs"], 0)
    assert float(out.abs().max()) == 0.0 and out.shape == q.shape


def test_paged_decode_skips_invalid_table_entries(hip):
    # a -1 / out-of-pool entry inside the context is never dereferenced; its tokens
    # drop out of the softmax (the reference would index block -1)
    banner("paged decode invalid table entries")
    from fast_infer_amd import paged_attention

    sp, (q, kc, vc, table, lens) = _decode_case("decode_ctx200")
    t = table.clone()
    t[0, 1] = -1
    t[1, 2] = 10 ** 6
    out = paged_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), t.to(DEV), sp["bs"], sp["ctx"])
    torch.cuda.synchronize()
    # oracle: attention over the remaining tokens only (move them to a clean table)
    for b, drop in ((0, 1), (1, 2)):
        keep = [blk for blk in range(math.ceil(lens[b] / 64)) if blk != drop]
        toks = [x for blk in keep for x in range(blk * 64, min(lens[b], blk * 64 + 64))]
        K = torch.stack([kc[int(table[b, x // 64]), x % 64] for x in toks]).float()
        V = torch.stack([vc[int(table[b, x // 64]), x % 64] for x in toks]).float()
        K, V = K.repeat_interleave(3, 1), V.repeat_interleave(3, 1)
        s = torch.einsum("hd,nhd->hn", q[b].float(), K) * 128 ** -0.5
        ref = torch.einsum("hn,nhd->hd", torch.softmax(s, -1), V)
        assert _maxabs(out[b], ref) <= ATOL


def test_paged_decode_strided_q(hip):
    banner("paged decode strided q")
    from fast_infer_amd import paged_attention

    sp, (q, kc, vc, table, lens) = _decode_case("decode_ctx65")
    wide = torch.zeros(q.shape[0], q.shape[1], 256, dtype=torch.float16)
    wide[..., 64:192] = q
    qd = wide.to(DEV)[..., 64:192]
    out = paged_attention(qd, kc.to(DEV), vc.to(DEV), table.to(DEV), sp["bs"], sp["ctx"])
    assert _maxabs(out, OA.paged_attention(q, kc, vc, table, sp["bs"], lens)) <= ATOL


@pytest.mark.parametrize("Hq,Hkv", [(15, 5), (64, 2), (12, 6), (6, 1), (40, 8), (24, 8),
                                     (16, 8), (32, 4), (8, 8)])
@pytest.mark.parametrize("batch", [3, 9])
def test_paged_decode_head_layouts(hip, Hq, Hkv, batch):
    # GQA groups of 1..8 query heads per kv head, odd kv-head counts (15/5, 6/1) and a
    # group wider than one workgroup's 16 MFMA columns (64/2: 32 query heads per kv head,
    # served by two workgroups), at 3 rows (one partition) and 9 rows with contexts past
    # 512 (split partitions and the merge).  Every layout against the oracle.
    banner(f"paged decode heads {Hq}/{Hkv} batch {batch}")
    from fast_infer_amd import paged_attention

    lens = [1, 190, 70, 600, 513, 64, 65, 300, 1000][:batch]
    sp = dict(B=batch, Hq=Hq, Hkv=Hkv, D=128, bs=64, N=64, lens=lens, seed=40 + Hq)
    q, kc, vc, table, lens = specs.decode_inputs(sp)
    cl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    out = paged_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), 64, max(lens),
                          context_lens=cl)
    torch.cuda.synchronize()
    assert _maxabs(out, OA.paged_attention(q, kc, vc, table, 64, lens)) <= ATOL


def _big_decode_inputs(B, lens, N, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(B, 24, 128, device=DEV, generator=g).half()
    kc = torch.randn(N, 64, 8, 128, device=DEV, generator=g).half()
    vc = torch.randn(N, 64, 8, 128, device=DEV, generator=g).half()
    perm = torch.randperm(N, generator=torch.Generator().manual_seed(seed)).int()
    table = specs.make_table(perm, B, N, 64, lens, "deal", width=64)
    return q, kc, vc, table


def test_paged_decode_batch32_ragged_full_size(hip):
    # batch 32, contexts uniform in [512, 4096], 2048-block pool, shuffled table
    banner("paged decode batch32 ragged 512..4096")
    from fast_infer_amd import paged_attention

    lens = torch.randint(512, 4097, (32,), generator=torch.Generator().manual_seed(2)).tolist()
    q, kc, vc, table = _big_decode_inputs(32, lens, 2048, 2)
    cl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    out = paged_attention(q, kc, vc, table.to(DEV), 64, 4096, context_lens=cl)
    torch.cuda.synchronize()
    rows = [0, 7, 13, 31]
    sub = torch.tensor(rows)
    ref = OA.paged_attention(q.cpu()[sub], kc.cpu(), vc.cpu(), table[sub], 64,
                             [lens[r] for r in rows])
    assert _maxabs(out.cpu()[sub], ref) <= ATOL
    # the same rows called one at a time agree (split boundaries differ per call)
    for r in rows[:2]:
        one = paged_attention(q[r:r + 1], kc, vc, table[r:r + 1].to(DEV), 64, lens[r])
        assert _maxabs(one[0], out[r]) <= ATOL


def test_paged_decode_workspace_reused_across_shapes(hip):
    # One workspace serves calls of different batch, lengths and split counts in a row
    # (partials of earlier calls left in it must not leak into later results).
    banner("paged decode: one workspace, several call shapes")
    from fast_infer_amd import paged_attention, paged_attention_workspace

    ws = paged_attention_workspace(32, 24, 8, 4096, 128, DEV)
    q, kc, vc, table = _big_decode_inputs(32, [4096] * 32, 2048, 5)
    calls = [(32, [4096] * 32), (4, [3000, 17, 4096, 1]), (32, [600 + 100 * i for i in range(32)]),
             (9, [0, 513, 4096, 2048, 1, 64, 65, 999, 4000]), (32, [4096] * 32)]
    for rep, (B, lens) in enumerate(calls):
        cl = torch.tensor(lens, dtype=torch.int32, device=DEV)
        out = paged_attention(q[:B], kc, vc, table[:B].to(DEV), 64, 4096, context_lens=cl,
                              workspace=ws)
        torch.cuda.synchronize()
        rows = sorted({0, B // 2, B - 1})
        sub = torch.tensor(rows)
        ref = OA.paged_attention(q.cpu()[sub], kc.cpu(), vc.cpu(), table[sub], 64,
                                 [lens[r] for r in rows])
        assert _maxabs(out.cpu()[sub], ref) <= ATOL, (rep, B)


# --------------------------------------------------------------------------- prefill


@pytest.mark.parametrize("name", list(specs.PREFILL_CASES))
@pytest.mark.parametrize("expanded", [False, True])
def test_flash_prefill_vs_reference_and_oracle(hip, golden, name, expanded):
    banner(f"flash prefill {name} expanded={expanded}")
    from fast_infer_amd import flash_attention

    arrays, _ = golden
    sp = specs.PREFILL_CASES[name]
    q, k, v = specs.prefill_inputs(sp)
    G = sp["H"] // sp["Hkv"]
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)   # [B, H, S, D] views of [B, S, H, D]
    if expanded:   # the reference call convention: K/V expanded (model.py:110-111)
        kd, vd = kd.repeat_interleave(G, 1), vd.repeat_interleave(G, 1)
    out = flash_attention(qd, kd, vd)
    torch.cuda.synchronize()
    assert out.shape == q.shape and out.stride() == qd.stride()
    rows = arrays[f"{name}__rows"]
    assert _maxabs(out.cpu()[:, :, rows], arrays[f"{name}__out"]) <= ATOL
    assert _maxabs(out.cpu(), OA.causal_attention(q, k, v)) <= ATOL


@pytest.mark.parametrize("S,width", [(300, 3), (130, 1), (64, 1)])
def test_flash_prefill_pool_write_partial_table(hip, S, width):
    """A table narrower than the sequence, with a -1 entry and an entry past the pool: only
    the blocks with valid entries are written (bit-exact), every other pool byte keeps its
    value, and the attention output is the plain one."""
    banner(f"flash prefill pool write, S={S}, table width {width}")
    from fast_infer_amd import flash_attention

    B, H, Hkv, N = 3, 24, 8, 12
    g = torch.Generator().manual_seed(S + width)
    q = torch.randn(B, S, H, 128, generator=g).half().transpose(1, 2)
    k = torch.randn(B, S, Hkv, 128, generator=g).half().transpose(1, 2)
    v = torch.randn(B, S, Hkv, 128, generator=g).half().transpose(1, 2)
    table = torch.tensor([[4, 7, 1][:width], [-1, 2, 9][:width], [N + 5, 0, 3][:width]],
                         dtype=torch.int32)
    kc0 = torch.randn(N, 64, Hkv, 128, generator=g).half()
    vc0 = torch.randn(N, 64, Hkv, 128, generator=g).half()
    kc, vc = kc0.to(DEV), vc0.to(DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    out = flash_attention(qd, kd, vd, k_cache=kc, v_cache=vc, block_table=table.to(DEV))
    plain = flash_attention(qd, kd, vd)
    torch.cuda.synchronize()
    assert torch.equal(out, plain)
    ek, ev = kc0.clone(), vc0.clone()
    for b in range(B):
        for lb in range(min(width, math.ceil(S / 64))):
            phys = int(table[b, lb])
            if not 0 <= phys < N:
                continue
            n = min(64, S - 64 * lb)
            ek[phys, :n] = k[b, :, 64 * lb:64 * lb + n].transpose(0, 1)
            ev[phys, :n] = v[b, :, 64 * lb:64 * lb + n].transpose(0, 1)
    assert torch.equal(kc.cpu(), ek) and torch.equal(vc.cpu(), ev)


@pytest.mark.parametrize("S", [64, 200, 1000])
def test_flash_prefill_fused_pool_write(hip, S):
    banner(f"flash prefill fused pool write S={S}")
    from fast_infer_amd import allocate_prefill, flash_attention, KVCache

    B, H, Hkv = 2, 24, 8
    g = torch.Generator().manual_seed(40 + S)
    q = torch.randn(B, S, H, 128, generator=g).half().to(DEV).transpose(1, 2)
    k = torch.randn(B, S, Hkv, 128, generator=g).half().to(DEV)
    v = torch.randn(B, S, Hkv, 128, generator=g).half().to(DEV)
    cache = KVCache(1, Hkv, 128, max_seq_len=1024, block_size=64, device=DEV, num_blocks=40)
    # scramble the allocation order so tables are not identity-like
    cache._grow_batch(B)
    cache.alloc_block(1)
    allocate_prefill(cache, B, S)
    out = flash_attention(q, k.transpose(1, 2), v.transpose(1, 2), k_cache=cache.k[0],
                          v_cache=cache.v[0], block_table=cache.block_table)
    torch.cuda.synchronize()
    ek = np.zeros(tuple(cache.k[0].shape), np.float16)
    ev = np.zeros_like(ek)
    OK.scatter(ek, ev, cache.block_table.cpu().tolist(), k.cpu().numpy(), v.cpu().numpy(), 0, 64)
    assert np.array_equal(cache.k[0].cpu().numpy().view(np.uint16), ek.view(np.uint16))
    assert np.array_equal(cache.v[0].cpu().numpy().view(np.uint16), ev.view(np.uint16))
    plain = flash_attention(q, k.transpose(1, 2), v.transpose(1, 2))
    assert torch.equal(out, plain)


def test_flash_prefill_batch4_seq4096_sampled(hip):
    # batch 4, seq 4096, 24/8 heads: sampled query rows of sampled heads vs the oracle
    banner("flash prefill batch4 seq4096")
    from fast_infer_amd import flash_attention

    B, S, H, Hkv = 4, 4096, 24, 8
    g = torch.Generator(device=DEV).manual_seed(3)
    q = torch.randn(B, S, H, 128, device=DEV, generator=g).half().transpose(1, 2)
    k = torch.randn(B, S, Hkv, 128, device=DEV, generator=g).half().transpose(1, 2)
    v = torch.randn(B, S, Hkv, 128, device=DEV, generator=g).half().transpose(1, 2)
    out = flash_attention(q, k, v)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all())
    rows = [0, 1, 63, 64, 65, 1000, 2047, 2048, 4031, 4032, 4095]
    heads = [0, 2, 3, 13, 23]
    ref = OA.causal_attention_rows(q.cpu(), k.cpu(), v.cpu(), rows, heads)
    got = out.cpu()[:, heads][:, :, rows]
    assert _maxabs(got, ref) <= ATOL


@pytest.mark.parametrize("S", [1, 70, 200])
def test_zero_scale_prefill_and_decode(hip, S):
    """sm_scale == 0: uniform weights over the causal prefix (prefill) or the context
    (decode); masked keys must not turn into NaN."""
    banner(f"zero sm_scale prefill and decode, S={S}")
    from fast_infer_amd import flash_attention, paged_attention

    B, H, Hkv = 2, 24, 8
    g = torch.Generator().manual_seed(60 + S)
    q = torch.randn(B, S, H, 128, generator=g).half().transpose(1, 2)
    k = torch.randn(B, S, Hkv, 128, generator=g).half().transpose(1, 2)
    v = torch.randn(B, S, Hkv, 128, generator=g).half().transpose(1, 2)
    out = flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), 0.0)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all())
    assert _maxabs(out, OA.causal_attention(q, k, v, 0.0)) <= ATOL
    nb = math.ceil(S / 64)
    kc = torch.randn(B * nb + 1, 64, Hkv, 128, generator=g).half()
    vc = torch.randn(B * nb + 1, 64, Hkv, 128, generator=g).half()
    table = torch.arange(B * nb, dtype=torch.int32).view(B, nb).flip(0).contiguous()
    qd = torch.randn(B, H, 128, generator=g).half()
    od = paged_attention(qd.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), 64, S, 0.0)
    torch.cuda.synchronize()
    assert _maxabs(od, OA.paged_attention(qd, kc, vc, table, 64, S, sm_scale=0.0)) <= ATOL


def test_kvcache_device_table_keeps_in_place_writes(hip):
    """block_table is a device tensor updated in place: alloc_block writes only the
    entries it fills, so a caller's own writes to other entries persist."""
    banner("KVCache device table in-place writes")
    from fast_infer_amd import KVCache

    cache = KVCache(1, 8, 128, max_seq_len=512, block_size=64, device=DEV, num_blocks=20)
    cache._grow_batch(2)
    cache.alloc_block(0)
    table = cache.block_table
    table[1, 5] = 17            # the caller's own entry
    cache.alloc_block(0)
    cache.alloc_block(1)
    cache._grow_batch(3)
    cache.alloc_block(2)
    got = cache.block_table.cpu()
    expect = torch.full((3, 8), -1, dtype=torch.int32)
    expect[0, 0], expect[0, 1], expect[1, 0], expect[2, 0] = 0, 1, 2, 3
    expect[1, 5] = 17
    assert torch.equal(got, expect)
    assert cache.host_block_table()[1, 5] == -1   # not seen by the allocator
    cache.reset()
    assert bool((cache.block_table == -1).all())
