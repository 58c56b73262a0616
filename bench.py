#!/usr/bin/env python3
"""Benchmark of the MI355X attention hot path (paged decode + causal prefill).

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Prints ONE JSON line.  Headline: paged decode at batch 32 (contexts uniform in
[512, 4096], 24/8 heads, d 128, block 64, 2048-block pool, shuffled table) in GB/s of
algorithmic HBM traffic; a "step" is one paged_attention call over the batch, with
the K/V pools rotated over four copies (2 GiB) so the 256 MB last-level cache cannot
serve them.  The same line carries:

* ``prefill`` — causal prefill batch 4 x seq 4096 with the K/V pool write, TFLOP/s;
* ``decode_b1_ctx256`` / ``prefill_b1_s512`` — the small configurations (latency), per
  eager call and per call of a HIP graph replay (GPU time without host launch cost);
* ``decode_step_28layer_b64_paged`` — the same step with the device block manager (one
  append per step) and the fused RoPE + pool write per layer before attention;
* ``int4_linear`` — the INT4 QKV / O projections around attention (decode batch 64 and 1
  over 28 layers of weights, GB/s; prefill QKV at 16384 tokens, TFLOP/s), RMSNorm fused
  into the QKV projection against the two-step form, and RMSNorm alone at 16384 rows;
* ``rope_store_kv`` — the fused RoPE + K/V pool write (batch 4 x 4096 prefill, batch 64
  decode), GB/s of algorithmic traffic;
* ``decode_28layer_b64`` — a 28-layer decode step over per-layer pools, batch 64,
  lognormal contexts (median 1024, sigma 0.5, clipped to [64, 4096]): step latency
  and decode tokens/s;
* ``roofline`` objects (achieved vs MI355X peak; ``traffic`` = HBM bytes per call measured by
  rocprofv3 FETCH_SIZE/WRITE_SIZE, profiles/hbm_traffic.txt) and ``cpu_baseline`` objects: the C
  restatement of the reference's kernels (oracle/ref_algo.c, OpenMP) timed on this
  host's cores on a bounded sample, plus the eager torch fp32 oracle.

Timing uses HIP events on torch's current stream, which is the stream every
fast_infer_amd kernel is launched on.  Inputs are resident in HBM before timing, and
every section rotates the inputs it reads over copies that together exceed 320 MB
(decode pools, prefill q/k/v, RoPE projections, the 28 layers' INT4 weights), so the
256 MB last-level cache does not serve them from one call to the next.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "decode attn GB/s + prefill attn TFLOP/s (% of MI355X roofline), fp16"
HQ, HKV, D, BS = 24, 8, 128, 64
# MFMA-bound kernels (prefill attention, the prefill GEMM) run 10-20% slower over their
# first few tens of milliseconds of back-to-back calls (same tensors; a GEMM load
# beforehand does not remove it), and on a GPU that has just been idle a 0.1 s warm-up
# still left the first process's prefill about 4% slower than a second process's.  The
# batch-32 decode, the first section a process times, runs 3-7% slower over its first
# hundred calls too.  These sections keep calling, untimed, for this long before timing.
WARM_S = 0.5


def _args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", default="",
                    help="comma list: decode,prefill,small,e2e,rope,int4")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 1 GiB device copy (reference for PMC byte counters)")
    return ap.parse_args()


def _traffic(workload: str):
    """HBM bytes per call (read + write) measured by rocprofv3 for this workload, from
    profiles/hbm_traffic.txt; None when not measured."""
    path = ROOT / "profiles" / "hbm_traffic.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        parts = line.split()
        if len(parts) == 3 and parts[0] == workload and not line.startswith("#"):
            return int(parts[1]) + int(parts[2])
    return None


# Host threads the CPU baseline may use: a one-GPU box grants 16 host cores per GPU, which
# the affinity mask does not necessarily show, so the thread count is capped there.
CPU_THREAD_CAP = 16


def _cores() -> tuple[int, int]:
    """(threads used by the CPU baseline, cores in this process's affinity mask)."""
    visible = len(os.sched_getaffinity(0))
    return max(1, min(CPU_THREAD_CAP, visible)), visible


class Timer:
    """HIP events on the current stream around `steps` calls of fn, after `warmup`
    untimed calls and, with `warm_s`, untimed calls until that much time has passed."""

    def __init__(self, torch):
        self.torch = torch

    def run(self, fn, steps: int, warmup: int, warm_s: float = 0.0) -> float:
        torch = self.torch
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < warm_s:
            for _ in range(8):
                fn()
            torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / 1e3 / steps  # seconds per call

    def graph(self, fn, calls: int, steps: int, warmup: int) -> float:
        """Seconds per call of fn with `calls` calls captured once into a HIP graph and the
        graph replayed: the GPU time of the calls without the host's per-launch cost."""
        torch = self.torch
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(calls):
                fn()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(calls):
                fn()
        t = self.run(graph.replay, steps, warmup)
        del graph
        return t / calls


# Inputs that a section reads on every call are kept in enough copies to exceed this many
# bytes, and the calls rotate over them, so the 256 MB last-level cache cannot serve them.
ROTATE_BYTES = 320 << 20


def _copies(nbytes: int) -> int:
    return max(2, -(-ROTATE_BYTES // max(1, nbytes)))


def _table(torch, lens, pool_blocks, seed, width):
    perm = torch.randperm(pool_blocks, generator=torch.Generator().manual_seed(seed)).int()
    table = torch.full((len(lens), width), -1, dtype=torch.int32)
    pos = 0
    for b, n in enumerate(lens):
        nb = math.ceil(n / BS)
        table[b, :nb] = perm[pos:pos + nb]
        pos += nb
    assert pos <= pool_blocks
    return table


def bench_decode_b32(torch, fi, timer, steps, warmup, dev):
    from fast_infer_amd import roofline as R

    B, N = 32, 2048
    lens = torch.randint(512, 4097, (B,), generator=torch.Generator().manual_seed(2)).tolist()
    g = torch.Generator(device=dev).manual_seed(2)
    pools = [(torch.randn(N, BS, HKV, D, device=dev, generator=g, dtype=torch.float16),
              torch.randn(N, BS, HKV, D, device=dev, generator=g, dtype=torch.float16))
             for _ in range(4)]
    q = torch.randn(B, HQ, D, device=dev, generator=g, dtype=torch.float16)
    table = _table(torch, lens, N, 2, 64).to(dev)
    cl = torch.tensor(lens, dtype=torch.int32, device=dev)
    ws = fi.paged_attention_workspace(B, HQ, HKV, 4096, D, dev)
    it = [0]

    def step():
        kc, vc = pools[it[0] & 3]
        it[0] += 1
        fi.paged_attention(q, kc, vc, table, BS, 4096, context_lens=cl, workspace=ws)

    # the same calls timed cold first (the process's first decode calls, after `warmup` of
    # them), then after WARM_S of untimed calls, which is what the headline reports
    t_cold = timer.run(step, steps, warmup)
    t = timer.run(step, steps, 0, WARM_S)
    nbytes = R.decode_bytes(lens, HQ, HKV, D, BS)
    gbs = nbytes / t / 1e9
    return dict(t=t, t_cold=t_cold, bytes=nbytes, gbs=gbs, lens=lens, q=q, pools=pools[0],
                table=table)


def bench_prefill(torch, fi, timer, steps, warmup, dev, B, S, pool_blocks, seed, warm_s=0.0,
                  graph=False):
    from fast_infer_amd import roofline as R

    g = torch.Generator(device=dev).manual_seed(seed)
    copies = _copies(B * S * (HQ + 2 * HKV) * D * 2)
    qkv = []
    for _ in range(copies):
        qkv.append(tuple(
            torch.randn(B, S, H, D, device=dev, generator=g, dtype=torch.float16).transpose(1, 2)
            for H in (HQ, HKV, HKV)))
    kc = torch.zeros(pool_blocks, BS, HKV, D, device=dev, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    per_row = pool_blocks // B
    table = torch.randperm(pool_blocks, generator=torch.Generator().manual_seed(seed)).int()
    table = table.view(B, per_row).to(dev)
    it = [0]

    def step():
        q, k, v = qkv[it[0] % copies]
        it[0] += 1
        fi.flash_attention(q, k, v, k_cache=kc, v_cache=vc, block_table=table)

    t = timer.run(step, steps, warmup, warm_s)
    t_graph = timer.graph(step, copies, steps, warmup) if graph else None
    flops = R.prefill_flops(B, HQ, S, D)
    q, k, v = qkv[0]
    return dict(t=t, t_graph=t_graph, flops=flops, tflops=flops / t / 1e12, q=q, k=k, v=v,
                copies=copies, scatter_bytes=R.prefill_scatter_bytes(B, S, HKV, D))


def bench_decode_b1(torch, fi, timer, steps, warmup, dev):
    from fast_infer_amd import roofline as R

    g = torch.Generator(device=dev).manual_seed(0)
    copies = 64  # 64 x 8 MiB pools rotate past the last-level cache
    pools = [(torch.randn(64, BS, HKV, D, device=dev, generator=g, dtype=torch.float16),
              torch.randn(64, BS, HKV, D, device=dev, generator=g, dtype=torch.float16))
             for _ in range(copies)]
    q = torch.randn(1, HQ, D, device=dev, generator=g, dtype=torch.float16)
    table = torch.randperm(64, generator=torch.Generator().manual_seed(0)).int().view(1, 64).to(dev)
    it = [0]

    def step():
        kc, vc = pools[it[0] % copies]
        it[0] += 1
        fi.paged_attention(q, kc, vc, table, BS, 256)

    t = timer.run(step, steps, warmup)
    t_graph = timer.graph(step, copies, steps, warmup)
    nbytes = R.decode_bytes([256], HQ, HKV, D, BS)
    return dict(t=t, t_graph=t_graph, bytes=nbytes, gbs=nbytes / t / 1e9)


def bench_decode_28layer(torch, fi, timer, steps, warmup, dev):
    from fast_infer_amd import roofline as R

    L, B, N = 28, 64, 4096
    gen = torch.Generator().manual_seed(4)
    lens = torch.exp(torch.randn(B, generator=gen) * 0.5 + math.log(1024)).round()
    lens = lens.clamp(64, 4096).int().tolist()
    g = torch.Generator(device=dev).manual_seed(4)
    kpool = torch.empty(L, N, BS, HKV, D, device=dev, dtype=torch.float16)
    vpool = torch.empty_like(kpool)
    for layer in range(L):
        kpool[layer].normal_(generator=g)
        vpool[layer].normal_(generator=g)
    tables = [_table(torch, lens, N, 100 + layer, 64).to(dev) for layer in range(L)]
    qs = torch.randn(L, B, HQ, D, device=dev, generator=g, dtype=torch.float16)
    cl = torch.tensor(lens, dtype=torch.int32, device=dev)
    ws = fi.paged_attention_workspace(B, HQ, HKV, 4096, D, dev)

    def step():
        for layer in range(L):
            fi.paged_attention(qs[layer], kpool[layer], vpool[layer], tables[layer], BS, 4096,
                               context_lens=cl, workspace=ws)

    t = timer.run(step, max(1, steps // 10), max(1, warmup // 5))
    nbytes = L * R.decode_bytes(lens, HQ, HKV, D, BS)
    return dict(t=t, bytes=nbytes, gbs=nbytes / t / 1e9, tok_s=B / t, lens=lens)


def bench_rope(torch, fi, timer, steps, warmup, dev, B, T, start, pool_blocks, return_k):
    """Fused RoPE + pool write on q/k/v views of one projection output (model.py:88-101)."""
    from fast_infer_amd import roofline as R

    g = torch.Generator(device=dev).manual_seed(7)
    copies = _copies(B * T * (HQ + 2 * HKV) * D * 2)
    views = []
    for _ in range(copies):
        qkv = torch.randn(B, T, (HQ + 2 * HKV) * D, device=dev, generator=g, dtype=torch.float16)
        q, k, v = qkv.split([HQ * D, HKV * D, HKV * D], dim=-1)
        views.append((q.view(B, T, HQ, D), k.view(B, T, HKV, D), v.view(B, T, HKV, D)))
    cos, sin = fi.precompute_freqs(D, 4096, device=dev)
    cos, sin = cos.half(), sin.half()
    kc = torch.zeros(pool_blocks, BS, HKV, D, device=dev, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    per_row = pool_blocks // B
    table = torch.randperm(pool_blocks, generator=torch.Generator().manual_seed(7)).int()
    table = table.view(B, per_row).to(dev)
    q_out = torch.empty(B, T, HQ, D, device=dev, dtype=torch.float16)
    it = [0]

    def step():
        q, k, v = views[it[0] % copies]
        it[0] += 1
        fi.rope_store_kv(q, k, v, cos, sin, start, kc, vc, table, return_k=return_k,
                         q_out=q_out)

    t = timer.run(step, steps, warmup)
    nbytes = R.rope_store_bytes(B, T, HQ, HKV, D, T, True, return_k)
    return dict(t=t, bytes=nbytes, gbs=nbytes / t / 1e9)


def bench_decode_step_paged(torch, fi, timer, steps, warmup, dev):
    """A 28-layer decode step as a serving loop runs it with the device block manager:
    one append of a token to every row, then per layer the fused RoPE + pool write at the
    rows' own positions and paged attention over the rows' own lengths.  Batch 64,
    lognormal contexts (median 1024, sigma 0.5, clipped to [64, 4096])."""
    from fast_infer_amd import roofline as R

    L, B = 28, 64
    gen = torch.Generator().manual_seed(4)
    lens = torch.exp(torch.randn(B, generator=gen) * 0.5 + math.log(1024)).round()
    lens = lens.clamp(64, 4096).int()
    extra = steps + warmup + 1
    max_len = 4096 + extra
    N = int(sum(math.ceil((int(n) + extra) / BS) for n in lens)) + B
    cache = fi.PagedKVCache(L, HKV, D, max_len, BS, dev, max_batch=B, num_blocks=N)
    g = torch.Generator(device=dev).manual_seed(4)
    cache.k.normal_(generator=g)
    cache.v.normal_(generator=g)
    cache.append(lens.to(dev))
    cache.check()
    cos, sin = fi.precompute_freqs(D, max_len, device=dev)
    cos, sin = cos.half(), sin.half()
    qkv = torch.randn(L, B, 1, (HQ + 2 * HKV) * D, device=dev, generator=g, dtype=torch.float16)
    q = qkv[..., :HQ * D].view(L, B, 1, HQ, D)
    k = qkv[..., HQ * D:(HQ + HKV) * D].view(L, B, 1, HKV, D)
    v = qkv[..., (HQ + HKV) * D:].view(L, B, 1, HKV, D)
    q_rot = torch.empty(B, 1, HQ, D, device=dev, dtype=torch.float16)
    ws = fi.paged_attention_workspace(B, HQ, HKV, max_len, D, dev)

    def step():
        starts, ctx = cache.append(1)
        for layer in range(L):
            fi.rope_store_kv(q[layer], k[layer], v[layer], cos, sin, 0, cache.k[layer],
                             cache.v[layer], cache.block_table, start_positions=starts,
                             return_k=False, q_out=q_rot)
            fi.paged_attention(q_rot[:, 0], cache.k[layer], cache.v[layer], cache.block_table,
                               BS, max_len, context_lens=ctx, workspace=ws)

    n_steps, n_warm = max(1, steps // 10), max(1, warmup // 5)
    t = timer.run(step, n_steps, n_warm)
    cache.check()
    mid = [int(n) + n_warm + n_steps // 2 + 1 for n in lens]
    nbytes = L * (R.decode_bytes(mid, HQ, HKV, D, BS)
                  + R.rope_store_bytes(B, 1, HQ, HKV, D, B, True, False))
    return dict(t=t, bytes=nbytes, gbs=nbytes / t / 1e9, tok_s=B / t, tokens=sum(mid))


def bench_decode_step_b1_graph(torch, fi, timer, steps, warmup, dev):
    """A batch-1 decode step over 28 layers, as single-stream serving runs it: per layer the
    fused RMSNorm + INT4 QKV projection, the fused RoPE + pool write, paged attention over a
    1024-token context and the INT4 O projection (364 MB of packed weights).  Timed as eager
    calls and as one HIP graph replay of the whole step (captured once; the graph removes
    the host's per-launch cost, which dominates at batch 1)."""
    L, B, ctx = 28, 1, 1024
    NQKV, K_HID = (HQ + 2 * HKV) * D, HQ * D
    g = torch.Generator(device=dev).manual_seed(11)
    layers = []
    for _ in range(L):
        wqkv = (torch.randn(NQKV, K_HID, device=dev, generator=g) * 0.02).half()
        wo = (torch.randn(K_HID, K_HID, device=dev, generator=g) * 0.02).half()
        layers.append((fi.quantize_int4_groupwise(wqkv), fi.quantize_int4_groupwise(wo)))
        del wqkv, wo
    norm_w = (1.0 + 0.1 * torch.randn(K_HID, device=dev, generator=g)).half()
    nblk = ctx // BS + 1
    kpool = torch.randn(L, nblk, BS, HKV, D, device=dev, generator=g, dtype=torch.float16)
    vpool = torch.randn_like(kpool)
    table = torch.randperm(nblk, generator=torch.Generator().manual_seed(11)).int()
    table = table.view(1, nblk).to(dev)
    cl = torch.tensor([ctx], dtype=torch.int32, device=dev)
    pos = torch.tensor([ctx - 1], dtype=torch.int32, device=dev)
    cos, sin = fi.precompute_freqs(D, 4096, device=dev)
    cos, sin = cos.half(), sin.half()
    ws = fi.paged_attention_workspace(B, HQ, HKV, ctx, D, dev)
    q_buf = torch.empty(B, 1, HQ, D, device=dev, dtype=torch.float16)
    x = torch.randn(B, K_HID, device=dev, generator=g).half()

    def step():
        h = x
        for layer in range(L):
            wqkv, wo = layers[layer]
            qkv = fi.rms_norm_int4_matmul(h, norm_w, wqkv)
            q = qkv[:, :HQ * D].view(B, 1, HQ, D)
            k = qkv[:, HQ * D:(HQ + HKV) * D].view(B, 1, HKV, D)
            v = qkv[:, (HQ + HKV) * D:].view(B, 1, HKV, D)
            fi.rope_store_kv(q, k, v, cos, sin, 0, kpool[layer], vpool[layer], table,
                             start_positions=pos, return_k=False, q_out=q_buf)
            attn = fi.paged_attention(q_buf[:, 0], kpool[layer], vpool[layer], table, BS, ctx,
                                      context_lens=cl, workspace=ws)
            h = fi.int4_matmul(attn.view(B, HQ * D), wo)
        return h

    n_steps, n_warm = max(1, steps // 5), max(1, warmup // 2)
    t_eager = timer.run(step, n_steps, n_warm)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    t_graph = timer.run(graph.replay, n_steps, n_warm)
    return dict(t_eager=t_eager, t_graph=t_graph, layers=L, ctx=ctx)


def bench_int4(torch, fi, timer, steps, warmup, dev):
    """INT4 QKV (N 5120) and O (N 3072) projections, K 3072, over 28 layers' weights (364
    MB packed, past the 256 MB last-level cache): decode at batch 64 and batch 1, and
    prefill at 4 x 4096 tokens."""
    from fast_infer_amd import roofline as R

    L, K, NQKV, NO = 28, 3072, (HQ + 2 * HKV) * D, HQ * D
    g = torch.Generator(device=dev).manual_seed(5)
    layers = []
    for _ in range(L):
        wq = (torch.randn(NQKV, K, device=dev, generator=g) * 0.02).half()
        wo = (torch.randn(NO, K, device=dev, generator=g) * 0.02).half()
        layers.append((fi.quantize_int4_groupwise(wq), fi.quantize_int4_groupwise(wo)))
        del wq, wo
    res = {}
    for M in (64, 1):
        x = torch.randn(M, K, device=dev, generator=g).half()
        ws = torch.empty(max(fi._lib.load().fi_int4_matmul_workspace_size(M, n, K)
                             for n in (NQKV, NO)) or 1, dtype=torch.uint8, device=dev)

        def step():
            for wqkv, wo in layers:
                fi.int4_matmul(x, wqkv, workspace=ws)
                fi.int4_matmul(x, wo, workspace=ws)

        t = timer.run(step, max(1, steps // 10), max(1, warmup // 5))
        # the same 56 calls captured once and replayed as one HIP graph (no host launch
        # cost between kernels; the workspace is the explicit one above)
        step()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        t_graph = timer.run(graph.replay, max(1, steps // 10), max(1, warmup // 5))
        del graph
        nbytes = L * (R.int4_matmul_bytes(M, NQKV, K) + R.int4_matmul_bytes(M, NO, K))
        res[f"decode_b{M}"] = dict(t=t, bytes=nbytes, gbs=nbytes / t / 1e9, t_graph=t_graph,
                                   gbs_graph=nbytes / t_graph / 1e9)
    # RMSNorm (model.py:82) fused with the QKV projection against the two-step form
    nws = [(torch.randn(K, device=dev, generator=g) * 0.1 + 1).half() for _ in range(L)]
    for M in (1, 64):
        x = torch.randn(M, K, device=dev, generator=g).half()

        def fused():
            for (wqkv, _), nw in zip(layers, nws):
                fi.rms_norm_int4_matmul(x, nw, wqkv)

        def two_step():
            for (wqkv, _), nw in zip(layers, nws):
                fi.int4_matmul(fi.rms_norm(x, nw), wqkv)

        res[f"norm_qkv_b{M}"] = dict(
            fused=timer.run(fused, max(1, steps // 10), max(1, warmup // 5)) / L,
            two_step=timer.run(two_step, max(1, steps // 10), max(1, warmup // 5)) / L)
    M = 4 * 4096
    x = torch.randn(M, K, device=dev, generator=g).half()
    t = timer.run(lambda: fi.rms_norm(x, nws[0]), steps, warmup)
    nbytes = 2 * M * K * 2 + K * 2
    res["rms_norm_prefill"] = dict(t=t, bytes=nbytes, gbs=nbytes / t / 1e9)
    wqkv = layers[0][0]
    t = timer.run(lambda: fi.int4_matmul(x, wqkv), max(1, steps // 10), max(1, warmup // 5),
                  WARM_S)
    fl = R.matmul_flops(M, NQKV, K)
    res["prefill_qkv"] = dict(t=t, flops=fl, tflops=fl / t / 1e12)
    return res


# ----------------------------------------------------------------------------- CPU


def cpu_baseline_decode(torch, res, cores):
    """C restatement (port) and torch fp32 oracle on the full batch-32 decode."""
    import numpy as np

    from oracle import attention as OA
    from oracle import native

    kc, vc = (t.cpu().numpy() for t in res["pools"])
    q = res["q"].cpu().numpy()
    table = res["table"].cpu().numpy()
    lens = res["lens"]
    native.load()
    t0 = time.perf_counter()
    reps = 0
    while True:
        native.paged_forward(q, kc, vc, table, BS, lens, threads=cores)
        reps += 1
        if time.perf_counter() - t0 > 2.0:
            break
    t_port = (time.perf_counter() - t0) / reps
    torch.set_num_threads(cores)
    tq, tk, tv, tt = (torch.from_numpy(np.ascontiguousarray(a)) for a in (q, kc, vc, table))
    t0 = time.perf_counter()
    OA.paged_attention(tq, tk, tv, tt, BS, lens)
    t_torch = time.perf_counter() - t0
    return dict(port=res["bytes"] / t_port / 1e9, torch=res["bytes"] / t_torch / 1e9,
                t_port=t_port, t_torch=t_torch, reps=reps)


def cpu_baseline_prefill(torch, res, cores, B, S, nprog=16):
    """C restatement on `nprog` of the B*24 (batch, head) programs, extrapolated;
    torch fp32 oracle on 4 heads of batch row 0, extrapolated."""
    from oracle import attention as OA
    from oracle import native

    q = res["q"].cpu().contiguous().numpy()
    k = res["k"].cpu().contiguous().numpy()
    v = res["v"].cpu().contiguous().numpy()
    total = B * HQ
    progs = [(i % B, (i * 7) % HQ) for i in range(nprog)]
    native.load()
    t0 = time.perf_counter()
    native.flash_forward(q, k, v, programs=progs, threads=cores)
    t_port = (time.perf_counter() - t0) * total / nprog
    torch.set_num_threads(cores)
    qt, kt, vt = (torch.from_numpy(a) for a in (q, k, v))
    heads = [0, 5, 11, 23]
    t0 = time.perf_counter()
    for h in heads:
        OA.causal_attention(qt[:1, h:h + 1], kt[:1, h // 3:h // 3 + 1], vt[:1, h // 3:h // 3 + 1])
    t_torch = (time.perf_counter() - t0) * total / len(heads)
    return dict(port=res["flops"] / t_port / 1e12, torch=res["flops"] / t_torch / 1e12,
                t_port=t_port, t_torch=t_torch, nprog=nprog, total=total)


def main():
    a = _args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {a.gpus} is not supported: the attention "
              "path runs on a single MI355X (a multi-GPU run would shard rows and kv heads "
              "across GPUs, each running this same single-GPU path).", file=sys.stderr)
        sys.exit(2)
    import torch

    import fast_infer_amd as fi
    from fast_infer_amd import roofline as R

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    timer = Timer(torch)
    only = set(filter(None, a.only.split(","))) or {"decode", "prefill", "small", "e2e", "rope",
                                                    "int4"}
    cores, cores_visible = _cores()
    core_note = {"cores_in_affinity_mask": cores_visible, "thread_cap": CPU_THREAD_CAP}
    steps, warm = a.steps, a.warmup
    out = {"metric": METRIC}

    if a.copy_calibration:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()

    dec = None
    if "decode" in only:
        dec = bench_decode_b32(torch, fi, timer, steps, warm, dev)
        print(f"[bench] decode b32: {dec['t'] * 1e6:.1f} us/call, {dec['gbs']:.0f} GB/s "
              f"(cold, first in the process: {dec['t_cold'] * 1e6:.1f} us/call)",
              file=sys.stderr, flush=True)
    pre = None
    pre_steps, pre_warm = max(1, steps // 5), max(1, warm // 2)
    if "prefill" in only:
        pre = bench_prefill(torch, fi, timer, pre_steps, pre_warm, dev, 4, 4096, 256, 3,
                            warm_s=WARM_S)
        print(f"[bench] prefill b4 s4096: {pre['t'] * 1e6:.1f} us/call, "
              f"{pre['tflops']:.1f} TFLOP/s", file=sys.stderr, flush=True)

    if dec is not None:
        out.update({
            "value": round(dec["gbs"], 1), "unit": "GB/s", "n_gpus": 1, "steps": steps,
            "warmup": warm, "ms_per_step": round(dec["t"] * 1e3, 5),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
            "data": "synthetic: seeded N(0,1) fp16 q and K/V pools, seeded shuffled block tables",
            "config": {"workload": "paged decode, batch 32, contexts U[512,4096], 24 q / 8 kv "
                                   "heads, head_dim 128, block_size 64, 2048-block pool",
                       "batch": 32, "context_tokens": sum(dec["lens"]),
                       "num_q_heads": HQ, "num_kv_heads": HKV, "head_dim": D,
                       "block_size": BS, "pool_blocks": 2048},
            "roofline": {"bound": "hbm", "achieved": round(dec["gbs"], 1),
                         "peak": R.HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(dec["gbs"] / R.HBM_PEAK_GBS, 4),
                         "traffic": _traffic("decode_b32"),
                         "kernel": "paged decode call (partition + merge launches)",
                         "algorithmic_bytes": dec["bytes"]},
            "cold": {"ms_per_step": round(dec["t_cold"] * 1e3, 5),
                     "value": round(dec["bytes"] / dec["t_cold"] / 1e9, 1),
                     "note": "the same steps timed first in the process, before the 0.5 s "
                             "of untimed calls after which value is timed"},
        })
    if pre is not None:
        out["prefill"] = {
            "workload": "causal prefill, batch 4, seq 4096, 24 q / 8 kv heads, head_dim 128, "
                        "with the K/V write into a 256-block pool (block_size 64)",
            "value": round(pre["tflops"], 2), "unit": "TFLOP/s",
            "ms_per_step": round(pre["t"] * 1e3, 5), "steps": pre_steps, "warmup": pre_warm,
            "warm_s": WARM_S,
            "roofline": {"bound": "mfma", "achieved": round(pre["tflops"], 2),
                         "peak": R.FP16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(pre["tflops"] / R.FP16_MFMA_PEAK_TFLOPS, 4),
                         "traffic": _traffic("prefill_b4_s4096"), "kernel": "fwd_kernel<3, false>",
                         "algorithmic_flops": pre["flops"],
                         "pool_write_bytes": pre["scatter_bytes"]},
        }
    if "small" in only:
        d1 = bench_decode_b1(torch, fi, timer, steps, warm, dev)
        p1 = bench_prefill(torch, fi, timer, steps, warm, dev, 1, 512, 64, 1, warm_s=WARM_S,
                           graph=True)
        out["decode_b1_ctx256"] = {"us_per_call": round(d1["t"] * 1e6, 2),
                                   "graph_us_per_call": round(d1["t_graph"] * 1e6, 2),
                                   "GB/s": round(d1["gbs"], 1),
                                   "graph_GB/s": round(d1["bytes"] / d1["t_graph"] / 1e9, 1),
                                   "bytes": d1["bytes"]}
        out["prefill_b1_s512"] = {"us_per_call": round(p1["t"] * 1e6, 2),
                                  "graph_us_per_call": round(p1["t_graph"] * 1e6, 2),
                                  "TFLOP/s": round(p1["tflops"], 2),
                                  "graph_TFLOP/s": round(p1["flops"] / p1["t_graph"] / 1e12, 2)}
        print(f"[bench] small: decode b1 {d1['t'] * 1e6:.1f} us (graph "
              f"{d1['t_graph'] * 1e6:.1f}), prefill s512 {p1['t'] * 1e6:.1f} us (graph "
              f"{p1['t_graph'] * 1e6:.1f})", file=sys.stderr, flush=True)
    if "e2e" in only:
        e = bench_decode_28layer(torch, fi, timer, steps, warm, dev)
        out["decode_28layer_b64"] = {
            "step_ms": round(e["t"] * 1e3, 4), "tokens_per_s": round(e["tok_s"], 1),
            "GB/s": round(e["gbs"], 1), "frac_hbm": round(e["gbs"] / R.HBM_PEAK_GBS, 4),
            "context_tokens": sum(e["lens"]), "lognormal_sigma": 0.5}
        print(f"[bench] 28-layer b64 step: {e['t'] * 1e3:.3f} ms, {e['gbs']:.0f} GB/s",
              file=sys.stderr, flush=True)
        del e
        f = bench_decode_step_paged(torch, fi, timer, steps, warm, dev)
        out["decode_step_28layer_b64_paged"] = {
            "workload": "28-layer decode step with the device block manager: append one token "
                        "per row, then per layer fused RoPE + pool write and paged attention "
                        "over per-row lengths; batch 64, lognormal contexts as above",
            "step_ms": round(f["t"] * 1e3, 4), "tokens_per_s": round(f["tok_s"], 1),
            "GB/s": round(f["gbs"], 1), "frac_hbm": round(f["gbs"] / R.HBM_PEAK_GBS, 4),
            "context_tokens": f["tokens"]}
        print(f"[bench] 28-layer b64 paged step (append + rope + attention): "
              f"{f['t'] * 1e3:.3f} ms, {f['gbs']:.0f} GB/s", file=sys.stderr, flush=True)
        del f
        gb = bench_decode_step_b1_graph(torch, fi, timer, steps, warm, dev)
        out["decode_step_28layer_b1_graph"] = {
            "workload": "batch-1 decode step over 28 layers: fused RMSNorm + INT4 QKV, fused "
                        "RoPE + pool write, paged attention over 1024 tokens, INT4 O projection",
            "eager_ms": round(gb["t_eager"] * 1e3, 4),
            "graph_ms": round(gb["t_graph"] * 1e3, 4),
            "graph_tokens_per_s": round(1.0 / gb["t_graph"], 1)}
        print(f"[bench] 28-layer b1 decode step: eager {gb['t_eager'] * 1e3:.3f} ms, "
              f"HIP graph {gb['t_graph'] * 1e3:.3f} ms", file=sys.stderr, flush=True)

    if "rope" in only:
        rp = bench_rope(torch, fi, timer, steps, warm, dev, 4, 4096, 0, 256, True)
        rd = bench_rope(torch, fi, timer, steps, warm, dev, 64, 1, 1000, 1024, False)
        out["rope_store_kv"] = {
            "workload": "fused RoPE + K/V pool write on strided q/k/v views, batch 4 x 4096 "
                        "tokens (prefill, rotated k returned) and batch 64 x 1 token at "
                        "position 1000 (decode); 24 q / 8 kv heads, block_size 64",
            "prefill_b4_s4096": {"us_per_call": round(rp["t"] * 1e6, 2),
                                 "GB/s": round(rp["gbs"], 1),
                                 "frac_hbm": round(rp["gbs"] / R.HBM_PEAK_GBS, 4),
                                 "algorithmic_bytes": rp["bytes"],
                                 "traffic": _traffic("rope_b4_s4096")},
            "decode_b64": {"us_per_call": round(rd["t"] * 1e6, 2), "GB/s": round(rd["gbs"], 1),
                           "algorithmic_bytes": rd["bytes"]}}
        print(f"[bench] rope+store b4 s4096: {rp['t'] * 1e6:.1f} us, {rp['gbs']:.0f} GB/s; "
              f"decode b64 {rd['t'] * 1e6:.2f} us", file=sys.stderr, flush=True)

    if "int4" in only:
        q = bench_int4(torch, fi, timer, steps, warm, dev)
        d64, d1, pq = q["decode_b64"], q["decode_b1"], q["prefill_qkv"]
        out["int4_linear"] = {
            "workload": "INT4 QKV (N 5120) + O (N 3072) projections, K 3072, groupsize 128, "
                        "over 28 layers of weights (364 MB packed); prefill: QKV at 4 x 4096 "
                        "tokens",
            "decode_b64": {"us_per_layer": round(d64["t"] / 28 * 1e6, 2),
                           "GB/s": round(d64["gbs"], 1),
                           "frac_hbm": round(d64["gbs"] / R.HBM_PEAK_GBS, 4),
                           "graph_us_per_layer": round(d64["t_graph"] / 28 * 1e6, 2),
                           "graph_GB/s": round(d64["gbs_graph"], 1)},
            "decode_b1": {"us_per_layer": round(d1["t"] / 28 * 1e6, 2),
                          "GB/s": round(d1["gbs"], 1),
                          "frac_hbm": round(d1["gbs"] / R.HBM_PEAK_GBS, 4),
                          "graph_us_per_layer": round(d1["t_graph"] / 28 * 1e6, 2),
                          "graph_GB/s": round(d1["gbs_graph"], 1)},
            "prefill_qkv_m16384": {"us_per_call": round(pq["t"] * 1e6, 1),
                                   "TFLOP/s": round(pq["tflops"], 1),
                                   "frac_mfma": round(pq["tflops"] / R.FP16_MFMA_PEAK_TFLOPS, 4)},
            "rms_norm_qkv": {f"b{M}": {"fused_us": round(q[f"norm_qkv_b{M}"]["fused"] * 1e6, 2),
                                       "two_step_us": round(q[f"norm_qkv_b{M}"]["two_step"] * 1e6,
                                                            2)}
                             for M in (1, 64)},
            "rms_norm_m16384": {"us_per_call": round(q["rms_norm_prefill"]["t"] * 1e6, 2),
                                "GB/s": round(q["rms_norm_prefill"]["gbs"], 1),
                                "frac_hbm": round(q["rms_norm_prefill"]["gbs"] / R.HBM_PEAK_GBS,
                                                  4)}}
        print(f"[bench] int4 decode b64 {d64['t'] / 28 * 1e6:.2f} us/layer {d64['gbs']:.0f} GB/s "
              f"(graph {d64['t_graph'] / 28 * 1e6:.2f}); b1 {d1['t'] / 28 * 1e6:.2f} us/layer "
              f"{d1['gbs']:.0f} GB/s (graph {d1['t_graph'] / 28 * 1e6:.2f}); prefill qkv "
              f"{pq['t'] * 1e6:.0f} us {pq['tflops']:.0f} TFLOP/s", file=sys.stderr, flush=True)
        print("[bench] norm+qkv fused/two-step us: " + ", ".join(
            f"b{M} {q[f'norm_qkv_b{M}']['fused'] * 1e6:.2f}/{q[f'norm_qkv_b{M}']['two_step'] * 1e6:.2f}"
            for M in (1, 64)) + f"; rms_norm 16384x3072 {q['rms_norm_prefill']['t'] * 1e6:.1f} us "
            f"{q['rms_norm_prefill']['gbs']:.0f} GB/s", file=sys.stderr, flush=True)

    if not a.no_cpu_baseline:
        if dec is not None:
            c = cpu_baseline_decode(torch, dec, cores)
            out["cpu_baseline"] = {
                "value": round(c["port"], 3), "unit": "GB/s", "cores": cores, "kind": "port",
                "sample": f"the full batch-32 decode call, C restatement of the reference "
                          f"kernel (oracle/ref_algo.c, OpenMP), {c['reps']} reps, "
                          f"{c['t_port'] * 1e3:.1f} ms/call",
                "torch_fp32_oracle": {"value": round(c["torch"], 3), "unit": "GB/s",
                                      "s_per_call": round(c["t_torch"], 3)}, **core_note}
            print(f"[bench] cpu decode: port {c['port']:.2f} GB/s, torch {c['torch']:.2f} GB/s",
                  file=sys.stderr, flush=True)
        if pre is not None:
            c = cpu_baseline_prefill(torch, pre, cores, 4, 4096)
            out["prefill"]["cpu_baseline"] = {
                "value": round(c["port"], 4), "unit": "TFLOP/s", "cores": cores,
                "kind": "port",
                "sample": f"C restatement on {c['nprog']} of {c['total']} (batch, head) "
                          f"programs, extrapolated to the full call "
                          f"({c['t_port']:.1f} s/call)",
                "torch_fp32_oracle": {"value": round(c["torch"], 4), "unit": "TFLOP/s",
                                      "sample": "4 heads of batch row 0, extrapolated"},
                **core_note}
            print(f"[bench] cpu prefill: port {c['port']:.4f} TFLOP/s", file=sys.stderr,
                  flush=True)

    out["device"] = torch.cuda.get_device_name(0)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
