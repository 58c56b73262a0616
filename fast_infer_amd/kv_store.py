"""K/V writes into the paged pool (the copies of model.py:162-201 as one HIP launch).

``store_kv`` is the raw scatter.  ``store_kv_prefill`` / ``store_kv_decode`` restate
``LlamaForCausalLM._store_kv_prefill`` (model.py:162-183) and ``_store_kv_decode``
(model.py:185-201) on a ``KVCache``: the same allocation loop and the same token ->
(block, slot) placement, with the per-block ``.item()`` syncs and slice copies
replaced by one kernel launch per layer.
"""

from __future__ import annotations

import torch

from . import _lib


def _rows(t: torch.Tensor) -> torch.Tensor:
    if t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:-1]) or t.data_ptr() % 16:
        return t.contiguous()
    return t


def store_kv(k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
             block_table: torch.Tensor, start_pos: int = 0, *,
             start_positions: torch.Tensor | None = None) -> None:
    """Copy k, v ``[batch, num_tokens, num_kv_heads, head_dim]`` into one layer's pool.

    Token t of row b goes to position ``p = start + t`` (``start`` =
    ``start_positions[b]`` if given, else ``start_pos``): block
    ``block_table[b, p // block_size]``, slot ``p % block_size``.  Positions past the
    table width or mapped to an entry outside the pool (e.g. -1) are skipped.
    Byte-exact; asynchronous on the current stream.
    """
    if k.dim() != 4 or v.shape != k.shape:
        raise ValueError(f"k/v must be [batch, tokens, kv_heads, dim], got "
                         f"{tuple(k.shape)} / {tuple(v.shape)}")
    batch, num_tokens, num_kv_heads, head_dim = k.shape
    for name, t in (("k", k), ("v", v), ("k_cache", k_cache), ("v_cache", v_cache)):
        if t.dtype != torch.float16:
            raise TypeError(f"{name} must be float16, got {t.dtype}")
        if t.device.type != "cuda":
            raise RuntimeError(f"{name} must be on a HIP device; fast_infer_amd has no CPU path")
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("pools must be [num_blocks, block_size, kv_heads, dim]")
    if k_cache.shape[2] != num_kv_heads or k_cache.shape[3] != head_dim:
        raise ValueError(f"pool {tuple(k_cache.shape)} does not match k {tuple(k.shape)}")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("pools must be contiguous")
    if block_table.dtype != torch.int32 or block_table.dim() != 2:
        raise TypeError("block_table must be a 2-D int32 tensor")
    if block_table.shape[0] < batch:
        raise ValueError("block_table has fewer rows than the batch")
    if block_table.stride(-1) != 1:
        block_table = block_table.contiguous()
    if start_positions is not None:
        start_positions = start_positions.to(device=k.device, dtype=torch.int32).contiguous()
        if start_positions.numel() < batch:
            raise ValueError("start_positions has fewer entries than the batch")
    if batch == 0 or num_tokens == 0:
        return
    k, v = _rows(k), _rows(v)
    lib = _lib.load()
    rc = lib.fi_kv_store(
        k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
        v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.shape[0], k_cache.shape[1],
        num_kv_heads, head_dim,
        block_table.data_ptr(), block_table.stride(0), block_table.shape[1],
        batch, num_tokens, int(start_pos),
        None if start_positions is None else start_positions.data_ptr(),
        _lib.stream_handle(k.device))
    _lib.check(rc, "store_kv")


def allocate_prefill(kv_cache, batch_size: int, seq_len: int) -> None:
    """Allocation loop of model.py:172-174: give every row ceil(seq_len / bs) blocks."""
    num_needed = (seq_len + kv_cache.block_size - 1) // kv_cache.block_size
    kv_cache._grow_batch(batch_size)
    for b in range(batch_size):
        while kv_cache.allocated_blocks(b) < num_needed:
            kv_cache.alloc_block(b)


def store_kv_prefill(kv_cache, layer_idx: int, k: torch.Tensor, v: torch.Tensor) -> None:
    """model.py:162-183: k, v ``[batch, seq_len, num_kv_heads, head_dim]`` (post-RoPE).

    At layer 0 sets ``num_tokens = seq_len``; allocates each row's blocks; copies
    token t of row b to block ``block_table[b, t // bs]``, slot ``t % bs``.
    """
    batch_size, seq_len = k.shape[0], k.shape[1]
    if layer_idx == 0:
        kv_cache.num_tokens = seq_len
    allocate_prefill(kv_cache, batch_size, seq_len)
    store_kv(k, v, kv_cache.k[layer_idx], kv_cache.v[layer_idx], kv_cache.block_table, 0)


def store_kv_decode(kv_cache, layer_idx: int, k: torch.Tensor, v: torch.Tensor,
                    token_pos: int) -> None:
    """model.py:185-201: k, v ``[batch, num_kv_heads, head_dim]`` for position token_pos
    (the model's ``_token_count - 1``).  At layer 0 increments ``num_tokens``;
    allocates lazily; copies row b to block ``block_table[b, pos // bs]``, slot
    ``pos % bs``."""
    batch_size = k.shape[0]
    if layer_idx == 0:
        kv_cache.num_tokens += 1
    allocate_decode(kv_cache, batch_size, token_pos)
    store_kv(k.unsqueeze(1), v.unsqueeze(1), kv_cache.k[layer_idx], kv_cache.v[layer_idx],
             kv_cache.block_table, token_pos)


def allocate_decode(kv_cache, batch_size: int, token_pos: int) -> None:
    """Allocation loop of model.py:196-198: every row gets blocks up to token_pos's."""
    block_idx = token_pos // kv_cache.block_size
    kv_cache._grow_batch(batch_size)
    for b in range(batch_size):
        while kv_cache.allocated_blocks(b) <= block_idx:
            kv_cache.alloc_block(b)
