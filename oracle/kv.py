"""Pure-Python restatement of the KV pool writes and the block allocator
(TEST INFRASTRUCTURE — see ``oracle/__init__.py``).

* ``OracleKVCache`` — kv_cache.py:12-113 with lists: ``free_blocks.pop(0)`` (:54), first
  -1 entry of the row (:56-61), the two error messages (:52-53, :58-59), ``_grow_batch``
  (:41-48), ``reset`` (:108-113).
* ``store_prefill`` — model.py:162-183: per row allocate until ceil(S/bs) entries are
  non-negative, then copy block by block, ``k_pool[layer, phys, :n] = k[b, start:end]``.
* ``store_decode`` — model.py:185-201: pos = token_pos, block pos//bs, slot pos%bs,
  lazy allocation, one row per batch entry.
* ``store`` / ``store_batch`` — kv_cache.py:69-103 (row 0 only).
* ``scatter`` — the element-wise brute force used to pin the three functions above:
  position p of row b lands at (table[b][p // bs], p % bs), nothing else changes.

All loops are plain Python over tokens (pools are numpy arrays), sized for tests.
Pinned by brute force: ``scatter`` is the definition of the placement; the block
copies of ``store_prefill``/``store_decode`` are checked against it, and untouched
slots are checked to keep their previous bytes.
"""

from __future__ import annotations

import numpy as np


class OracleKVCache:
    """kv_cache.py:12-113 allocator state with numpy pools [L, N, bs, H, D]."""

    def __init__(self, num_layers, num_heads, head_dim, max_seq_len, block_size,
                 num_blocks=None):
        self.block_size = block_size
        per_seq = (max_seq_len + block_size - 1) // block_size     # :21
        self.num_blocks = per_seq if num_blocks is None else num_blocks
        self.max_blocks_per_seq = self.num_blocks if num_blocks is None else per_seq  # :22
        self.k = np.zeros((num_layers, self.num_blocks, block_size, num_heads, head_dim),
                          dtype=np.float16)                         # :25-28
        self.v = np.zeros_like(self.k)
        self.block_table = [[-1] * self.max_blocks_per_seq]         # :33-34
        self.free_blocks = list(range(self.num_blocks))             # :37
        self._allocated = 0
        self.num_tokens = 0

    def _grow_batch(self, batch_size):                             # :41-48
        while len(self.block_table) < batch_size:
            self.block_table.append([-1] * self.max_blocks_per_seq)

    def alloc_block(self, batch_idx=0):                            # :50-63
        if not self.free_blocks:
            raise RuntimeError("KV cache out of memory")
        phys = self.free_blocks.pop(0)
        row = self.block_table[batch_idx]
        for logical, entry in enumerate(row):
            if entry == -1:
                row[logical] = phys
                self._allocated += 1
                return logical
        raise RuntimeError("Sequence block table full")

    def allocated(self, b):
        return sum(1 for e in self.block_table[b] if e >= 0)

    def reset(self):                                               # :108-113
        self.block_table = [[-1] * self.max_blocks_per_seq for _ in self.block_table]
        self.free_blocks = list(range(self.num_blocks))
        self._allocated = 0
        self.num_tokens = 0


def scatter(k_pool, v_pool, table, k, v, start, block_size):
    """Brute force placement: k, v [B, T, H, D]; start int or per-row list; pools
    [N, bs, H, D] (one layer, modified in place).  Skips positions whose logical
    block is past the table or whose entry is outside the pool."""
    B, T = k.shape[:2]
    for b in range(B):
        s = start[b] if isinstance(start, (list, tuple, np.ndarray)) else start
        for t in range(T):
            p = s + t
            lb = p // block_size
            if lb >= len(table[b]):
                continue
            phys = table[b][lb]
            if phys < 0 or phys >= k_pool.shape[0]:
                continue
            k_pool[phys, p % block_size] = k[b, t]
            v_pool[phys, p % block_size] = v[b, t]


def store_prefill(cache: OracleKVCache, layer_idx, k, v):
    """model.py:162-183 with k, v [B, S, H, D] numpy fp16."""
    B, S = k.shape[:2]
    bs = cache.block_size
    num_needed = (S + bs - 1) // bs                                 # :166
    if layer_idx == 0:
        cache.num_tokens = S                                        # :169-170
    cache._grow_batch(B)
    for b in range(B):
        while cache.allocated(b) < num_needed:                      # :173-174
            cache.alloc_block(b)
        for blk in range(num_needed):                               # :176-183
            start = blk * bs
            end = min(start + bs, S)
            phys = cache.block_table[b][blk]
            cache.k[layer_idx, phys, :end - start] = k[b, start:end]
            cache.v[layer_idx, phys, :end - start] = v[b, start:end]


def store_decode(cache: OracleKVCache, layer_idx, k, v, token_pos):
    """model.py:185-201 with k, v [B, H, D] numpy fp16 at position token_pos."""
    B = k.shape[0]
    bs = cache.block_size
    block_idx = token_pos // bs                                     # :190
    offset = token_pos % bs                                         # :191
    if layer_idx == 0:
        cache.num_tokens += 1                                       # :193-194
    cache._grow_batch(B)
    for b in range(B):
        while cache.allocated(b) <= block_idx:                      # :197-198
            cache.alloc_block(b)
        phys = cache.block_table[b][block_idx]                      # :199
        cache.k[layer_idx, phys, offset] = k[b]                     # :200-201
        cache.v[layer_idx, phys, offset] = v[b]


def store(cache: OracleKVCache, layer_idx, logical_block, token_offset, k, v):
    """kv_cache.py:69-77: one token of row 0."""
    phys = cache.block_table[0][logical_block]
    cache.k[layer_idx, phys, token_offset] = k
    cache.v[layer_idx, phys, token_offset] = v


def store_batch(cache: OracleKVCache, layer_idx, start_block, start_offset, k, v):
    """kv_cache.py:79-103: consecutive tokens of row 0 from (start_block, start_offset)."""
    remaining = k.shape[0]
    block_idx, offset, pos = start_block, start_offset, 0
    while remaining > 0:
        phys = cache.block_table[0][block_idx]
        to_store = min(remaining, cache.block_size - offset)
        cache.k[layer_idx, phys, offset:offset + to_store] = k[pos:pos + to_store]
        cache.v[layer_idx, phys, offset:offset + to_store] = v[pos:pos + to_store]
        pos += to_store
        remaining -= to_store
        offset = 0
        block_idx += 1
