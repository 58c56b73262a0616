"""HIP graph capture of a decode step (marked ``gpu``).

Two layers of a decode step are captured once with ``torch.cuda.graph`` and replayed
several times, with other GPU work and host synchronisation between the replays:
  - RMSNorm fused with the INT4 QKV projection (one-pass kernel at 8 rows; a norm pass,
    then split-K GEMM plus reduction at 64 rows);
  - the fused RoPE + pool write at per-row positions;
  - paged attention over per-row lengths;
  - the INT4 O projection.

Each replay must equal the eager step bit for bit: the same kernels on the same inputs,
rewriting the same pool slots. None of these entry points records a memset or allocates
inside the library. The caller's caches (INT4 workspace, decode workspace) are set up by
an eager call before capture.

A captured ``PagedKVCache.append`` advances the device allocator once per replay, exactly
as the same number of eager appends on a twin cache does.
"""

import numpy as np
import pytest
import torch

from conftest import banner

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
HQ, HKV, D, BS, L = 24, 8, 128, 64, 2


def _setup(B, seed):
    from fast_infer_amd import precompute_freqs, quantize_int4_groupwise

    g = torch.Generator(device=DEV).manual_seed(seed)
    rng = np.random.default_rng(seed)
    lens = torch.from_numpy(rng.integers(200, 1000, B).astype(np.int32)).to(DEV)
    width = 16
    N = B * width + 4
    table = torch.from_numpy(rng.permutation(N)[:B * width].astype(np.int32)).view(B, width).to(DEV)
    pools = [(torch.randn(N, BS, HKV, D, device=DEV, generator=g).half(),
              torch.randn(N, BS, HKV, D, device=DEV, generator=g).half()) for _ in range(L)]
    weights = []
    for _ in range(L):
        wqkv = (torch.randn(5120, 3072, device=DEV, generator=g) * 0.02).half()
        wo = (torch.randn(3072, 3072, device=DEV, generator=g) * 0.02).half()
        weights.append((quantize_int4_groupwise(wqkv), quantize_int4_groupwise(wo)))
    cos, sin = precompute_freqs(D, 4096)
    x = torch.randn(B, 3072, device=DEV, generator=g).half()
    norm_w = (1.0 + 0.1 * torch.randn(3072, device=DEV, generator=g)).half()
    return dict(lens=lens, pos=(lens - 1).contiguous(), table=table, pools=pools, weights=weights,
                cos=cos.half().to(DEV), sin=sin.half().to(DEV), x=x, norm_w=norm_w)


def _step(st, x, ws):
    from fast_infer_amd import int4_matmul, paged_attention, rms_norm_int4_matmul, rope_store_kv

    B = x.shape[0]
    for layer in range(L):
        wqkv, wo = st["weights"][layer]
        kc, vc = st["pools"][layer]
        qkv = rms_norm_int4_matmul(x, st["norm_w"], wqkv)
        q = qkv[:, :HQ * D].view(B, 1, HQ, D)
        k = qkv[:, HQ * D:(HQ + HKV) * D].view(B, 1, HKV, D)
        v = qkv[:, (HQ + HKV) * D:].view(B, 1, HKV, D)
        q_rot, _ = rope_store_kv(q, k, v, st["cos"], st["sin"], 0, kc, vc, st["table"],
                                 start_positions=st["pos"], return_k=False)
        attn = paged_attention(q_rot.view(B, HQ, D), kc, vc, st["table"], BS, 1024,
                               context_lens=st["lens"], workspace=ws)
        x = int4_matmul(attn.view(B, HQ * D), wo)
    return x


@pytest.mark.parametrize("B", [8, 64])
def test_decode_step_graph_replay(hip, B):
    banner(f"graph capture of a 2-layer decode step, batch {B}")
    from fast_infer_amd import paged_attention, paged_attention_workspace

    st = _setup(B, 50 + B)
    ws = paged_attention_workspace(B, HQ, HKV, 1024, D, DEV)
    # eager reference (also sets up the INT4 workspace cache); the step rewrites the same
    # pool slots each time, so running it again leaves the pools unchanged
    ref = _step(st, st["x"], ws).clone()
    ref_pools = [(k.clone(), v.clone()) for k, v in st["pools"]]
    torch.cuda.synchronize()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _step(st, st["x"], ws)  # warm-up on the capture stream's side, as torch advises
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    static_x = st["x"].clone()
    with torch.cuda.graph(graph):
        out = _step(st, static_x, ws)
    torch.cuda.synchronize()

    for rep in range(3):
        # unrelated eager work between replays, including a different decode call
        noise = torch.randn(1 << 20, device=DEV).sum()
        paged_attention(torch.randn(B, HQ, D, device=DEV).half(), st["pools"][0][0],
                        st["pools"][0][1], st["table"], BS, 1024, context_lens=st["lens"],
                        workspace=ws)
        torch.cuda.synchronize()
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), (rep, float((out.float() - ref.float()).abs().max()))
        for (k, v), (rk, rv) in zip(st["pools"], ref_pools):
            assert torch.equal(k, rk) and torch.equal(v, rv), rep
        assert torch.isfinite(noise)


def test_int4_workspace_two_captures_shared_pool(hip):
    """Two graphs captured back to back on a shared memory pool, the second needing a larger
    split-K workspace than the first: the first graph's workspace must stay allocated, so
    replaying both (in either order, repeatedly) equals the eager results bit for bit."""
    banner("int4 split-K workspace across two captures (17 then 64 rows)")
    from fast_infer_amd import int4_matmul, quantize_int4_groupwise

    g = torch.Generator(device=DEV).manual_seed(77)
    w = quantize_int4_groupwise((torch.randn(5120, 3072, device=DEV, generator=g) * 0.02).half())
    xs = {m: torch.randn(m, 3072, device=DEV, generator=g).half() for m in (17, 64)}
    refs = {m: int4_matmul(x, w).clone() for m, x in xs.items()}
    torch.cuda.synchronize()
    pool = torch.cuda.graph_pool_handle()
    graphs, outs = {}, {}
    for m in (17, 64):
        graphs[m] = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graphs[m], pool=pool):
            outs[m] = int4_matmul(xs[m], w)
        torch.cuda.synchronize()
    for rep in range(3):
        for m in ((17, 64) if rep % 2 == 0 else (64, 17)):
            outs[m].zero_()
            graphs[m].replay()
        torch.cuda.synchronize()
        for m in (17, 64):
            assert torch.equal(outs[m], refs[m]), (rep, m)


def test_block_manager_append_graph_replay(hip):
    banner("graph capture of PagedKVCache.append")
    from fast_infer_amd import PagedKVCache

    B = 16
    a = PagedKVCache(1, 8, 128, 2048, 64, DEV, max_batch=B, num_blocks=400)
    b = PagedKVCache(1, 8, 128, 2048, 64, DEV, max_batch=B, num_blocks=400)
    lens0 = torch.randint(0, 700, (B,), generator=torch.Generator().manual_seed(3)).int()
    a.append(lens0.to(DEV))
    b.append(lens0.to(DEV))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        starts_g, lens_g = a.append(1)  # recorded, not run
    torch.cuda.synchronize()
    assert torch.equal(a.seq_lens, b.seq_lens)
    for rep in range(5):
        graph.replay()
        sb, lb = b.append(1)
        torch.cuda.synchronize()
        assert torch.equal(starts_g, sb) and torch.equal(lens_g, lb), rep
        assert torch.equal(a.block_table, b.block_table), rep
        assert torch.equal(a.seq_lens, b.seq_lens) and torch.equal(a.num_alloc, b.num_alloc), rep
        assert torch.equal(a.free_queue, b.free_queue) and torch.equal(a.state, b.state), rep
    a.check()
