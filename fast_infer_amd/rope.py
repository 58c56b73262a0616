"""Rotary position embedding (kernels/rope.py) on the gfx950 kernel, optionally fused
with the paged K/V write of model.py:117 / :120.

``precompute_freqs`` and ``apply_rope`` keep the reference's names and signatures
(kernels/rope.py:9-16, :26-44).  ``apply_rope`` is bit-exact with the reference's fp16
tensor arithmetic.  ``rope_store_kv`` is the fused form: it rotates q and k at table
rows ``start + t`` and, given a pool, writes rotated k and v into it in the same pass
(replacing ``apply_rope`` followed by ``store_kv``); ``rope_store_kv_prefill`` /
``rope_store_kv_decode`` apply it to a ``KVCache`` with the model's allocation steps.
"""

from __future__ import annotations

import torch

from . import _lib
from .kv_store import allocate_decode, allocate_prefill


def precompute_freqs(head_dim: int, max_seq_len: int, theta: float = 500000.0,
                     device: torch.device | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """cos and sin tables ``[max_seq_len, head_dim]`` (fp32) as kernels/rope.py:9-16
    builds them: angle(p, i) = p / theta^(2(i mod head_dim/2)/head_dim), the half-width
    frequency vector repeated twice.  Table setup, not the hot path."""
    freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device).float() / head_dim))
    positions = torch.arange(max_seq_len, device=device).float()
    angles = torch.outer(positions, freq)
    angles = torch.cat([angles, angles], dim=-1)
    return angles.cos(), angles.sin()


# rope_store_kv runs once per layer and decode step, where its host time is of the order of
# the kernel's: tensors' shapes, strides and pointers are read once each, dtypes compared by
# identity and devices by index.

def _check_rows(name: str, t: torch.Tensor, heads: int | None = None,
                head_dim: int | None = None) -> torch.Size:
    """Validates a [batch, tokens, heads, head_dim] fp16 HIP tensor; returns its shape."""
    if t.dtype is not torch.float16:
        raise TypeError(f"{name} must be float16, got {t.dtype}")
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be on a HIP device; fast_infer_amd has no CPU path")
    shape = t.shape
    if len(shape) != 4 or shape[3] % 16 or (head_dim is not None and shape[3] != head_dim):
        raise ValueError(f"{name} must be [batch, tokens, heads, head_dim] with head_dim a "
                         f"multiple of 16{'' if head_dim is None else f' ({head_dim})'}, "
                         f"got {tuple(shape)}")
    if heads is not None and shape[2] != heads:
        raise ValueError(f"{name} has {shape[2]} heads, expected {heads}")
    return shape


def _rows(t: torch.Tensor) -> tuple[torch.Tensor, tuple, int]:
    """(t or a contiguous copy, its strides, its pointer): unit inner stride, other strides
    multiples of 8 elements, 16-byte aligned base."""
    st, ptr = t.stride(), t.data_ptr()
    if st[3] != 1 or st[0] % 8 or st[1] % 8 or st[2] % 8 or ptr % 16:
        t = t.contiguous()
        st, ptr = t.stride(), t.data_ptr()
    return t, st, ptr


def _table(name: str, t: torch.Tensor, dev: int, head_dim: int) -> torch.Tensor:
    """A cos or sin table as fp16 [rows, head_dim] on device index `dev`, contiguous."""
    if t.dim() != 2 or t.shape[1] != head_dim:
        raise ValueError(f"{name} must be [rows, {head_dim}], got {tuple(t.shape)}")
    if t.dtype is not torch.float16 or t.get_device() != dev:
        t = t.to(device=torch.device("cuda", dev), dtype=torch.float16)
    return t if t.is_contiguous() and t.data_ptr() % 16 == 0 else t.contiguous()


def rope_store_kv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor | None,
                  cos_table: torch.Tensor, sin_table: torch.Tensor, start_pos: int = 0,
                  k_cache: torch.Tensor | None = None, v_cache: torch.Tensor | None = None,
                  block_table: torch.Tensor | None = None, *,
                  start_positions: torch.Tensor | None = None, return_k: bool = True,
                  q_out: torch.Tensor | None = None
                  ) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Rotate q ``[B, T, Hq, D]`` and k ``[B, T, Hkv, D]`` (D a multiple of 16, 128 in the
    model) at table rows ``start + t`` (``start`` = ``start_positions[b]`` if given, else
    ``start_pos``), with fp16 tables ``cos_table`` / ``sin_table`` ``[rows, D]`` (fp32 tables are converted
    on every call; pass fp16 ones on the hot path).  With a pool, rotated k and v also go
    to ``block_table[b, pos // bs]``, slot ``pos % bs`` (block-table entries past the
    table or outside the pool are skipped).  Positions outside the table are an error for
    a scalar ``start_pos`` (the reference's table indexing fails there); with
    ``start_positions`` such tokens are skipped on the device, their q/k rows left
    unwritten.  Returns (q_rot, k_rot or None)."""
    q_shape = _check_rows("q", q)
    batch, tokens, num_q_heads, head_dim = q_shape
    k_shape = _check_rows("k", k, head_dim=head_dim)
    num_kv_heads = k_shape[2]
    if k_shape[0] != batch or k_shape[1] != tokens:
        raise ValueError(f"k {tuple(k_shape)} does not match q {tuple(q_shape)}")
    dev = q.get_device()
    pool = k_cache is not None
    if pool:
        if v is None or v_cache is None or block_table is None:
            raise ValueError("the pool write needs v, v_cache and block_table")
        v_shape = _check_rows("v", v, num_kv_heads, head_dim)
        if v_shape[0] != batch or v_shape[1] != tokens:
            raise ValueError(f"v {tuple(v_shape)} does not match q {tuple(q_shape)}")
        for name, t in (("k_cache", k_cache), ("v_cache", v_cache)):
            if t.dtype is not torch.float16 or not t.is_cuda:
                raise TypeError(f"{name} must be a float16 HIP tensor")
        pool_shape = k_cache.shape
        if (len(pool_shape) != 4 or v_cache.shape != pool_shape
                or pool_shape[2] != num_kv_heads or pool_shape[3] != head_dim):
            raise ValueError(f"pool {tuple(pool_shape)} does not match k {tuple(k_shape)}")
        if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
            raise ValueError("pools must be contiguous")
        if block_table.dtype is not torch.int32 or block_table.dim() != 2:
            raise TypeError("block_table must be a 2-D int32 tensor")
        bt_rows, bt_cols = block_table.shape
        if bt_rows < batch:
            raise ValueError("block_table has fewer rows than the batch")
        if block_table.stride(-1) != 1:
            block_table = block_table.contiguous()
    cos_t = _table("cos_table", cos_table, dev, head_dim)
    sin_t = _table("sin_table", sin_table, dev, head_dim)
    table_rows = cos_t.shape[0]
    if sin_t.shape[0] != table_rows:
        raise ValueError("cos and sin tables differ in shape")
    if start_positions is not None:
        if (start_positions.dtype is not torch.int32 or start_positions.get_device() != dev
                or not start_positions.is_contiguous()):
            start_positions = start_positions.to(device=q.device, dtype=torch.int32).contiguous()
        if start_positions.numel() < batch:
            raise ValueError("start_positions has fewer entries than the batch")
    elif tokens > 0 and (start_pos < 0 or start_pos + tokens > table_rows):
        raise IndexError(f"positions {start_pos}..{start_pos + tokens - 1} outside the "
                         f"{table_rows}-row table")
    if q_out is None:
        q_out = torch.empty(q_shape, dtype=q.dtype, device=q.device)
    elif q_out.shape != q_shape:
        raise ValueError("q_out must have q's shape")
    k_out = torch.empty(k_shape, dtype=k.dtype, device=k.device) if return_k else None
    if batch == 0 or tokens == 0:
        return q_out, k_out
    q, qs, q_ptr = _rows(q)
    k, ks, k_ptr = _rows(k)
    if v is not None:
        v, vs, v_ptr = _rows(v)
    else:
        vs, v_ptr = (0, 0, 0), None
    qo = q_out.stride()
    if k_out is not None:
        ko, ko_ptr = k_out.stride(), k_out.data_ptr()
    else:
        ko, ko_ptr = (0, 0, 0), None
    if pool:
        kc_ptr, vc_ptr, n_blocks, bs = k_cache.data_ptr(), v_cache.data_ptr(), pool_shape[0], pool_shape[1]
        bt_ptr, bt_stride = block_table.data_ptr(), block_table.stride(0)
    else:
        kc_ptr = vc_ptr = bt_ptr = None
        n_blocks = bs = bt_stride = bt_cols = 0
    rc = _lib.load().fi_rope_store_kv(
        q_ptr, qs[0], qs[1], qs[2], k_ptr, ks[0], ks[1], ks[2], v_ptr, vs[0], vs[1], vs[2],
        cos_t.data_ptr(), sin_t.data_ptr(), table_rows,
        q_out.data_ptr(), qo[0], qo[1], qo[2], ko_ptr, ko[0], ko[1], ko[2],
        kc_ptr, vc_ptr, n_blocks, bs, bt_ptr, bt_stride, bt_cols,
        batch, tokens, num_q_heads, num_kv_heads, head_dim,
        int(start_pos), None if start_positions is None else start_positions.data_ptr(),
        _lib.tensor_stream(q))
    _lib.check(rc, "rope_store_kv")
    return q_out, k_out


def apply_rope(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor,
               sin: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """kernels/rope.py:26-44: q ``[B, S, Hq, D]``, k ``[B, S, Hkv, D]`` fp16 (strided
    views fine), cos/sin ``[S, D]`` fp16 (the table rows of the S positions).
    Returns rotated (q, k), bit-exact with the reference."""
    if cos.dim() != 2 or cos.shape[0] != q.shape[1]:
        raise ValueError(f"cos must be [seq_len, head_dim] for seq_len {q.shape[1]}")
    return rope_store_kv(q, k, None, cos, sin, 0)


def rope_store_kv_prefill(kv_cache, layer_idx: int, q: torch.Tensor, k: torch.Tensor,
                          v: torch.Tensor, cos_table: torch.Tensor, sin_table: torch.Tensor,
                          return_k: bool = True):
    """model.py:101 + :117 (:162-183) in one pass: positions 0..S-1; at layer 0 sets
    ``num_tokens = S``; allocates each row's blocks; returns (q_rot, k_rot)."""
    batch_size, seq_len = q.shape[0], q.shape[1]
    if layer_idx == 0:
        kv_cache.num_tokens = seq_len
    allocate_prefill(kv_cache, batch_size, seq_len)
    return rope_store_kv(q, k, v, cos_table, sin_table, 0, kv_cache.k[layer_idx],
                         kv_cache.v[layer_idx], kv_cache.block_table, return_k=return_k)


def rope_store_kv_decode(kv_cache, layer_idx: int, q: torch.Tensor, k: torch.Tensor,
                         v: torch.Tensor, cos_table: torch.Tensor, sin_table: torch.Tensor,
                         token_pos: int) -> torch.Tensor:
    """model.py:101 + :120 (:185-201) in one pass for one token per row at position
    ``token_pos``: q ``[B, Hq, D]``, k/v ``[B, Hkv, D]``.  At layer 0 increments
    ``num_tokens``; allocates lazily; returns q_rot ``[B, Hq, D]``."""
    batch_size = q.shape[0]
    if layer_idx == 0:
        kv_cache.num_tokens += 1
    allocate_decode(kv_cache, batch_size, token_pos)
    q_rot, _ = rope_store_kv(q.unsqueeze(1), k.unsqueeze(1), v.unsqueeze(1), cos_table,
                             sin_table, token_pos, kv_cache.k[layer_idx], kv_cache.v[layer_idx],
                             kv_cache.block_table, return_k=False)
    return q_rot.squeeze(1)
