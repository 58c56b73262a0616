"""Attention oracles (TEST INFRASTRUCTURE — see ``oracle/__init__.py``).

Two families:

1. fp32 closed forms, computed with torch on the CPU:
   * ``causal_attention`` — softmax(Q K^T * s + causal mask) V, query head h reading
     kv head h // (H / H_kv).  Restates what ``_flash_attn_fwd``
     (kernels/attention.py:8-77) computes on the K/V that model.py:110-111 expands.
   * ``paged_attention`` — per row, gather the first ctx tokens through the block
     table and apply softmax(q k^T * s) v.  Restates ``_paged_attention_kernel``
     (kernels/attention.py:116-188) with per-row lengths (the reference's single
     ``num_tokens`` is the special case ctx_b == num_tokens).
   Pinned by: the reference kernels' own outputs (golden vectors generated with
   TRITON_INTERPRET=1, tests/golden/), and textbook special cases — seq_len 1 gives
   o = v[0]; identical keys give the mean of V; one-hot V rows read back the softmax
   weights; a shuffled block table / pool permutation leaves decode unchanged; GQA
   equals the explicit repeat_interleave expansion.

2. numpy restatements of the reference's Triton programs, step for step:
   * ``reference_flash_forward`` — kernels/attention.py:80-113 (tile sizes :91-96) and
     :8-77 (serial Q tiles :34, causal K tiles :47, dot :55, masks :57-59, online
     softmax :61-66, PV :68-70, fp16 store :74-77).
   * ``reference_paged_forward`` — kernels/attention.py:191-233 and :116-188 (GQA
     routing :137-139, block loop :155-156, token mask :158-160, scores :168,
     online softmax :171-176, PV :178-182, fp16 store :186-188).
   Under TRITON_INTERPRET=1 the reference evaluates ``tl.dot`` as an fp32
   ``np.matmul`` and the rest as numpy fp32 element-wise ops; these restatements make
   the same calls in the same order.  Pinned by: the golden vectors (bit-exact or
   within one fp16 ulp), and against family 1 within tolerance.
"""

from __future__ import annotations

import numpy as np
import torch


def _f32(x) -> torch.Tensor:
    if isinstance(x, np.ndarray):
        x = torch.from_numpy(x)
    return x.detach().to("cpu", torch.float32)


def causal_attention(q, k, v, sm_scale: float | None = None,
                     dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """q [B, H, S, D], k/v [B, H_kv, S, D] (H % H_kv == 0) -> o [B, H, S, D] in `dtype`.

    Row m attends to keys n <= m (kernels/attention.py:57-58); scale defaults to
    D ** -0.5 (:88-89).
    """
    q, k, v = (_f32(t).to(dtype) for t in (q, k, v))
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    if H % Hkv:
        raise ValueError("H must be a multiple of H_kv")
    if sm_scale is None:
        sm_scale = D ** -0.5
    G = H // Hkv
    if G > 1:
        k = k.repeat_interleave(G, dim=1)
        v = v.repeat_interleave(G, dim=1)
    s = torch.matmul(q, k.transpose(-1, -2)) * sm_scale
    mask = torch.ones(S, S, dtype=torch.bool).triu(1)
    s = s.masked_fill(mask, float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, v)


def gather_context(k_cache, v_cache, block_table, block_size: int, b: int, ctx: int):
    """Tokens 0..ctx-1 of row b: position t lives in block block_table[b, t // bs],
    slot t % bs (kernels/attention.py:155-165).  Returns (K, V) [ctx, H_kv, D]."""
    bt = np.asarray(block_table)
    t = np.arange(ctx)
    phys = bt[b, t // block_size].astype(np.int64)
    if ctx and (phys.min() < 0 or phys.max() >= k_cache.shape[0]):
        raise ValueError(f"row {b}: block table maps a needed token outside the pool")
    slot = t % block_size
    return k_cache[phys, slot], v_cache[phys, slot]


def paged_attention(q, k_cache, v_cache, block_table, block_size: int, context_lens,
                    sm_scale: float | None = None,
                    dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """q [B, H, D]; pools [N, bs, H_kv, D]; table [B, max_blocks]; context_lens: int or
    per-row sequence.  -> o [B, H, D] in `dtype`; rows of length 0 give zeros
    (kernels/attention.py:205-206)."""
    q = _f32(q).to(dtype)
    kc = _f32(k_cache).to(dtype)
    vc = _f32(v_cache).to(dtype)
    bt = np.asarray(block_table.cpu() if isinstance(block_table, torch.Tensor) else block_table)
    B, H, D = q.shape
    Hkv = kc.shape[2]
    G = H // Hkv
    if sm_scale is None:
        sm_scale = D ** -0.5
    if isinstance(context_lens, (int, np.integer)):
        lens = [int(context_lens)] * B
    else:
        lens = [int(x) for x in (context_lens.cpu().tolist()
                                 if isinstance(context_lens, torch.Tensor) else context_lens)]
    out = torch.zeros(B, H, D, dtype=dtype)
    for b in range(B):
        n = lens[b]
        if n <= 0:
            continue
        K, V = gather_context(kc, vc, bt, block_size, b, n)  # [n, Hkv, D]
        K = K.repeat_interleave(G, dim=1).transpose(0, 1)     # [H, n, D]
        V = V.repeat_interleave(G, dim=1).transpose(0, 1)
        s = torch.matmul(K, q[b].unsqueeze(-1)).squeeze(-1) * sm_scale  # [H, n]
        p = torch.softmax(s, dim=-1)
        out[b] = torch.matmul(p.unsqueeze(1), V).squeeze(1)
    return out


# ---------------------------------------------------------------------------------
# numpy restatements of the reference Triton programs


def _next_pow2(n: int) -> int:
    return 1 if n <= 1 else 1 << (n - 1).bit_length()


def reference_block_sizes(seq_len: int, head_dim: int):
    """(BLOCK_M, BLOCK_N, BLOCK_D) chosen by flash_attention (kernels/attention.py:91-96)."""
    bd = _next_pow2(head_dim)
    bm = max(16, min(32, _next_pow2(seq_len)))
    return bm, bm, bd


def reference_flash_forward(q, k, v, sm_scale: float | None = None,
                            programs=None) -> np.ndarray:
    """Restatement of flash_attention -> _flash_attn_fwd (kernels/attention.py:80-113,
    :8-77) on fp16 numpy arrays q [B, H, S, D] and k/v [B, H_kv, S, D] (the reference
    requires H_kv == H; here head h reads kv head h // (H / H_kv), which is the same
    as passing the repeat_interleave-expanded K/V).  Returns fp16 [B, H, S, D].
    `programs` optionally restricts the (b, h) programs evaluated (others stay 0)."""
    q = np.asarray(q, dtype=np.float16)
    k = np.asarray(k, dtype=np.float16)
    v = np.asarray(v, dtype=np.float16)
    B, H, S, D = q.shape
    G = H // k.shape[1]
    if sm_scale is None:
        sm_scale = D ** -0.5
    BM, BN, BD = reference_block_sizes(S, D)
    scale = np.float32(sm_scale)
    o = np.zeros((B, H, S, D), dtype=np.float16)
    offs_m = np.arange(BM)
    offs_n = np.arange(BN)
    todo = programs if programs is not None else [(b, h) for b in range(B) for h in range(H)]
    with np.errstate(invalid="ignore", over="ignore"):
        for b, h in todo:
            qh, kh, vh = q[b, h], k[b, h // G], v[b, h // G]
            for start_m in range(0, S, BM):                       # :34
                m_offs = start_m + offs_m
                m_mask = m_offs < S
                m_i = np.full(BM, -np.inf, dtype=np.float32)     # :38-40
                l_i = np.zeros(BM, dtype=np.float32)
                acc = np.zeros((BM, BD), dtype=np.float32)
                qt = np.zeros((BM, BD), dtype=np.float32)        # :43-45 (masked load, other=0)
                qt[m_mask, :D] = qh[m_offs[m_mask]].astype(np.float32)
                for start_n in range(0, start_m + BM, BN):       # :47
                    n_offs = start_n + offs_n
                    n_mask = n_offs < S
                    kt = np.zeros((BN, BD), dtype=np.float32)    # :51-53
                    kt[n_mask, :D] = kh[n_offs[n_mask]].astype(np.float32)
                    qk = np.matmul(qt, kt.T) * scale             # :55
                    qk = np.where(m_offs[:, None] >= n_offs[None, :], qk,
                                  np.float32(-np.inf))           # :58
                    qk = np.where(m_mask[:, None] & n_mask[None, :], qk,
                                  np.float32(-np.inf))           # :59
                    m_new = np.maximum(m_i, np.max(qk, axis=1))  # :61
                    alpha = np.exp(m_i - m_new)                  # :62
                    p = np.exp(qk - m_new[:, None])              # :63
                    l_i = l_i * alpha + np.sum(p, axis=1)        # :65
                    acc = acc * alpha[:, None]                   # :66
                    vt = np.zeros((BN, BD), dtype=np.float32)    # :68-69
                    vt[n_mask, :D] = vh[n_offs[n_mask]].astype(np.float32)
                    acc = acc + np.matmul(p, vt)                 # :70
                    m_i = m_new                                  # :72
                res = (acc / l_i[:, None]).astype(np.float16)    # :74
                o[b, h, m_offs[m_mask]] = res[m_mask, :D]        # :76-77
    return o


def reference_paged_forward(q, k_cache, v_cache, block_table, block_size: int,
                            num_tokens: int, sm_scale: float | None = None) -> np.ndarray:
    """Restatement of paged_attention -> _paged_attention_kernel
    (kernels/attention.py:191-233, :116-188) on fp16 numpy arrays.  One shared
    num_tokens for every row, as in the reference.  Returns fp16 [B, H, D]."""
    q = np.asarray(q, dtype=np.float16)
    kc = np.asarray(k_cache, dtype=np.float16)
    vc = np.asarray(v_cache, dtype=np.float16)
    bt = np.asarray(block_table)
    if num_tokens == 0:
        return np.zeros_like(q)                                   # :205-206
    B, H, D = q.shape
    Hkv = kc.shape[2]
    if sm_scale is None:
        sm_scale = D ** -0.5                                      # :208-209
    scale = np.float32(sm_scale)
    num_blocks = (num_tokens + block_size - 1) // block_size      # :213
    groups = H // Hkv
    out = np.zeros((B, H, D), dtype=np.float16)
    offs_s = np.arange(block_size)
    with np.errstate(invalid="ignore", over="ignore"):
        for b in range(B):
            for h in range(H):
                kvh = h // groups                                 # :137-139
                qv = q[b, h].astype(np.float32)                   # :145-146
                m_i = np.full(1, -np.inf, dtype=np.float32)       # :149-151
                l_i = np.zeros(1, dtype=np.float32)
                acc = np.zeros(D, dtype=np.float32)
                for blk in range(num_blocks):                     # :155
                    phys = int(bt[b, blk])                        # :156
                    tok = blk * block_size + offs_s               # :158-160
                    tmask = tok < num_tokens
                    kt = np.zeros((block_size, D), dtype=np.float32)
                    kt[tmask] = kc[phys, offs_s[tmask], kvh].astype(np.float32)  # :163-165
                    scores = np.sum(qv[None, :] * kt, axis=1) * scale           # :168
                    scores = np.where(tmask, scores, np.float32(-np.inf))       # :169
                    m_new = np.maximum(m_i, np.max(scores))       # :172
                    alpha = np.exp(m_i - m_new)                   # :173
                    p = np.exp(scores - m_new)                    # :174
                    l_i = l_i * alpha + np.sum(p)                 # :175
                    acc = acc * alpha                             # :176
                    vt = np.zeros((block_size, D), dtype=np.float32)
                    vt[tmask] = vc[phys, offs_s[tmask], kvh].astype(np.float32)  # :179-181
                    acc = acc + np.sum(p[:, None] * vt, axis=0)   # :182
                    m_i = m_new                                   # :183
                out[b, h] = (acc / l_i).astype(np.float16)        # :186-188
    return out



def causal_attention_rows(q, k, v, rows, heads=None, sm_scale: float | None = None,
                          dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """``causal_attention`` restricted to query rows `rows` (and optionally heads):
    row m of head h = softmax(q[m] . K[:m+1]^T * s) V[:m+1] on kv head h // G.
    For full-size checks where the S x S score matrix is too large for the CPU.
    Returns [B, len(heads), len(rows), D]."""
    q, k, v = (_f32(t).to(dtype) for t in (q, k, v))
    B, H, S, D = q.shape
    G = H // k.shape[1]
    if sm_scale is None:
        sm_scale = D ** -0.5
    heads = list(range(H)) if heads is None else list(heads)
    rows = torch.as_tensor(rows, dtype=torch.long)
    out = torch.empty(B, len(heads), len(rows), D, dtype=dtype)
    keys = torch.arange(S)
    mask = keys[None, :] > rows[:, None]                    # [R, S]
    for hi, h in enumerate(heads):
        qh = q[:, h, rows]                                  # [B, R, D]
        s = torch.matmul(qh, k[:, h // G].transpose(-1, -2)) * sm_scale  # [B, R, S]
        s = s.masked_fill(mask, float("-inf"))
        out[:, hi] = torch.matmul(torch.softmax(s, -1), v[:, h // G])
    return out
