"""Seeded synthetic inputs shared by the golden-vector generator and the tests.

Inputs are regenerated from (shape, seed) with torch's CPU generator rather than
stored; the fixtures record the SHA-256 of the generated fp16 bytes so a change in
the generator is detected instead of silently comparing different inputs.
"""

from __future__ import annotations

import hashlib
import math

import numpy as np
import torch

# Decode cases: the reference's single shared num_tokens (``ctx``) for every row.
DECODE_CASES = {
    # Paged decode, batch 1, 24/8 heads, d 128, ctx 256 in a 64-block pool whose
    # table is a seeded permutation of all 64 ids.
    "decode_b1_ctx256": dict(B=1, Hq=24, Hkv=8, D=128, bs=64, N=64, ctx=256, seed=0,
                             table="full"),
    "decode_ctx1": dict(B=2, Hq=24, Hkv=8, D=128, bs=64, N=16, ctx=1, seed=10, table="deal"),
    "decode_ctx63": dict(B=2, Hq=24, Hkv=8, D=128, bs=64, N=16, ctx=63, seed=11, table="deal"),
    "decode_ctx64": dict(B=2, Hq=24, Hkv=8, D=128, bs=64, N=16, ctx=64, seed=12, table="deal"),
    "decode_ctx65": dict(B=2, Hq=24, Hkv=8, D=128, bs=64, N=16, ctx=65, seed=13, table="deal"),
    "decode_ctx200": dict(B=3, Hq=24, Hkv=8, D=128, bs=64, N=24, ctx=200, seed=14,
                          table="deal"),
    "decode_mha_ctx100": dict(B=2, Hq=8, Hkv=8, D=128, bs=64, N=8, ctx=100, seed=15,
                              table="deal"),
    "decode_g4_ctx130": dict(B=2, Hq=32, Hkv=8, D=128, bs=64, N=8, ctx=130, seed=16,
                             table="deal"),
    "decode_bs16_ctx90": dict(B=2, Hq=24, Hkv=8, D=128, bs=16, N=16, ctx=90, seed=17,
                              table="deal"),
}

# Ragged decode: per-row lengths; the reference has no per-row lengths, so its
# goldens are produced by one call per row (batch 1, num_tokens = ctx_b).
RAGGED_CASES = {
    "ragged_b4": dict(B=4, Hq=24, Hkv=8, D=128, bs=64, N=16, lens=[1, 64, 129, 300],
                      seed=20),
    "ragged_b3_zero": dict(B=3, Hq=24, Hkv=8, D=128, bs=64, N=8, lens=[70, 0, 5], seed=21),
}

# Causal prefill: q [B, S, H, D], k/v [B, S, H_kv, D] (the model's layout), passed to
# attention as [B, H, S, D] views.  `rows` = query rows kept in the fixture (None = all).
PREFILL_CASES = {
    "prefill_s1": dict(B=1, H=24, Hkv=8, S=1, D=128, seed=30),
    "prefill_s16": dict(B=1, H=24, Hkv=8, S=16, D=128, seed=31),
    "prefill_s33": dict(B=1, H=24, Hkv=8, S=33, D=128, seed=32),
    "prefill_s100": dict(B=1, H=24, Hkv=8, S=100, D=128, seed=33, rows="sparse"),
    "prefill_b2_s130": dict(B=2, H=24, Hkv=8, S=130, D=128, seed=34, rows="sparse"),
    "prefill_mha_s70": dict(B=1, H=8, Hkv=8, S=70, D=128, seed=35),
    "prefill_g4_s65": dict(B=1, H=32, Hkv=8, S=65, D=128, seed=36, rows="sparse"),
    # Causal prefill, batch 1, seq 512, 24/8 heads: every 16th query row and the last.
    "prefill_b1_s512": dict(B=1, H=24, Hkv=8, S=512, D=128, seed=1, rows="every16"),
}


def sha256(*tensors) -> str:
    h = hashlib.sha256()
    for t in tensors:
        a = t.detach().cpu().contiguous().numpy() if isinstance(t, torch.Tensor) else t
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def make_table(perm: torch.Tensor, B: int, N: int, bs: int, lens, mode: str,
               width: int | None = None) -> torch.Tensor:
    """Block table int32 [B, width]: "full" = perm reshaped row-major (every entry
    valid); "deal" = perm dealt row-major, ceil(len_b / bs) ids per row, rest -1."""
    if mode == "full":
        return perm.to(torch.int32).view(B, N // B).clone()
    need = [math.ceil(int(n) / bs) for n in lens]
    width = width or max(max(need), 1)
    table = torch.full((B, width), -1, dtype=torch.int32)
    pos = 0
    for b, n in enumerate(need):
        table[b, :n] = perm[pos:pos + n].to(torch.int32)
        pos += n
    if pos > N:
        raise ValueError("pool too small for the requested contexts")
    return table


def decode_inputs(spec: dict):
    """-> q [B, Hq, D], k_cache, v_cache [N, bs, Hkv, D] fp16, table int32, lens list."""
    g = torch.Generator().manual_seed(spec["seed"])
    B, Hq, Hkv, D, bs, N = (spec[k] for k in ("B", "Hq", "Hkv", "D", "bs", "N"))
    q = torch.randn(B, Hq, D, generator=g).half()
    k_cache = torch.randn(N, bs, Hkv, D, generator=g).half()
    v_cache = torch.randn(N, bs, Hkv, D, generator=g).half()
    perm = torch.randperm(N, generator=g)
    lens = spec["lens"] if "lens" in spec else [spec["ctx"]] * B
    table = make_table(perm, B, N, bs, lens, spec.get("table", "deal"))
    return q, k_cache, v_cache, table, list(lens)


def prefill_inputs(spec: dict):
    """-> q [B, H, S, D], k/v [B, Hkv, S, D] fp16 views of [B, S, *, D] tensors."""
    g = torch.Generator().manual_seed(spec["seed"])
    B, H, Hkv, S, D = (spec[k] for k in ("B", "H", "Hkv", "S", "D"))
    q = torch.randn(B, S, H, D, generator=g).half()
    k = torch.randn(B, S, Hkv, D, generator=g).half()
    v = torch.randn(B, S, Hkv, D, generator=g).half()
    return q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)


def prefill_rows(spec: dict) -> np.ndarray:
    """Query rows kept in a fixture: all, every 16th (+ last), or "sparse" = the first
    rows, every 7th, the rows either side of 16/32/64-row tile edges, and the last."""
    S = spec["S"]
    mode = spec.get("rows")
    if mode == "every16":
        rows = np.append(np.arange(0, S, 16), S - 1)
    elif mode == "sparse":
        edges = [e + d for e in (16, 32, 64, 96, 128) for d in (-1, 0, 1)]
        rows = np.concatenate([np.arange(4), np.arange(0, S, 7), edges, [S - 1]])
    else:
        rows = np.arange(S)
    return np.unique(rows[(rows >= 0) & (rows < S)])
