"""Paged KV pool with the reference's layout and allocator (drop-in for ``kv_cache.py``).

Layout and semantics follow kv_cache.py:6-113 exactly:

* pools ``k``/``v``: fp16 ``[num_layers, num_blocks, block_size, num_heads, head_dim]``,
  zero-initialised (:25-28);
* ``block_table``: int32 ``[batch, max_blocks_per_seq]``, -1 = unallocated (:33-34),
  grown with -1 rows by ``_grow_batch`` (:41-48);
* ``alloc_block(b)`` pops the lowest free physical id (``free_blocks.pop(0)``) into the
  first -1 entry of row b and returns that logical index; it raises
  ``RuntimeError("KV cache out of memory")`` / ``RuntimeError("Sequence block table
  full")`` under the same conditions (:50-63);
* ``reset()`` frees everything (:108-113).

Differences, all keyword-only or internal:

* ``num_blocks=`` sizes the pool independently of ``max_seq_len`` (the reference
  always has ``ceil(max_seq_len / block_size)`` blocks, shared by every row); rows
  then hold ``ceil(max_seq_len / block_size)`` entries.  Without it the reference
  sizes are used (rows as wide as the pool, :21-22).
* The allocator decides on a host copy of the table, so allocation never waits for
  the device (the reference's ``.item()`` at :60).  ``block_table`` is a device tensor
  like the reference's; the entries ``alloc_block`` fills are written into it (batched,
  before the tensor is next handed out, through pinned memory and an asynchronous copy,
  so the host never waits), never the whole table, so a caller's in-place
  writes to other entries persist.  Such writes are not seen by the allocator, which
  still picks the first entry it has not filled itself; assigning ``block_table``
  replaces both copies.
* ``store``/``store_batch`` (:69-103) copy with the HIP scatter kernel.  A position
  whose table entry is -1 is skipped (the reference's ``k[layer, -1, ...]`` would wrap
  to the last pool block).
"""

from __future__ import annotations

import numpy as np
import torch

from .kv_store import store_kv


class KVCache:
    """Paged KV cache for a batch of sequences sharing one pool of physical blocks."""

    def __init__(self, num_layers: int, num_heads: int, head_dim: int,
                 max_seq_len: int, block_size: int, device: torch.device, *,
                 num_blocks: int | None = None):
        self.num_layers = num_layers
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.max_seq_len = max_seq_len
        self.block_size = block_size
        self.device = torch.device(device)

        per_seq = (max_seq_len + block_size - 1) // block_size
        if num_blocks is None:
            self.num_blocks = per_seq
            self.max_blocks_per_seq = self.num_blocks  # one sequence may use all blocks
        else:
            self.num_blocks = int(num_blocks)
            self.max_blocks_per_seq = per_seq

        self.k = torch.zeros(num_layers, self.num_blocks, block_size, num_heads, head_dim,
                             dtype=torch.float16, device=self.device)
        self.v = torch.zeros(num_layers, self.num_blocks, block_size, num_heads, head_dim,
                             dtype=torch.float16, device=self.device)

        self._table = np.full((1, self.max_blocks_per_seq), -1, dtype=np.int32)
        self._table_dev = torch.full((1, self.max_blocks_per_seq), -1, dtype=torch.int32,
                                     device=self.device)
        self._pending: list[tuple[int, int, int]] = []  # (row, entry, block) not yet on device
        self._staging: list[tuple[torch.Tensor, torch.cuda.Event]] = []  # pinned, in flight

        self.free_blocks = list(range(self.num_blocks))
        self._allocated = 0
        self.num_tokens = 0

    # -- block table ---------------------------------------------------------------
    def _flush(self) -> None:
        """Write the entries alloc_block filled since the last flush into the device table.

        The (row, entry, block) triples go through pinned host memory with one
        asynchronous copy on the current stream, then a device scatter: nothing here waits
        for the device.  Each staging buffer is kept with an event recorded after its copy
        until that event has completed."""
        if not self._pending:
            return
        host = torch.tensor(self._pending, dtype=torch.int32).t().contiguous()
        self._pending = []
        if self.device.type == "cuda":
            self._staging = [(buf, ev) for buf, ev in self._staging if not ev.query()]
            host = host.pin_memory()
            dev = host.to(self.device, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(torch.cuda.current_stream(self.device))
            self._staging.append((host, ev))
        else:  # a host table (allocator tests without a GPU)
            dev = host
        idx = dev[:2].long()
        self._table_dev.index_put_((idx[0], idx[1]), dev[2])

    @property
    def block_table(self) -> torch.Tensor:
        """Device block table [batch, max_blocks_per_seq] (int32, -1 = unallocated)."""
        self._flush()
        return self._table_dev

    @block_table.setter
    def block_table(self, table: torch.Tensor) -> None:
        table = torch.as_tensor(table)
        if table.dim() != 2:
            raise ValueError("block_table must be 2-D")
        self._table = table.detach().to("cpu", torch.int32).numpy().copy()
        self._table_dev = table.detach().to(self.device, torch.int32).contiguous()
        self._pending = []

    def host_block_table(self) -> np.ndarray:
        """Read-only view of the allocator's host copy of the table (no device traffic)."""
        v = self._table.view()
        v.flags.writeable = False
        return v

    def _grow_batch(self, batch_size: int):
        """Add rows of -1 entries until the table has batch_size rows (kv_cache.py:41-48)."""
        rows = self._table.shape[0]
        if batch_size <= rows:
            return
        new_table = np.full((batch_size, self.max_blocks_per_seq), -1, dtype=np.int32)
        new_table[:rows] = self._table
        self._table = new_table
        self._flush()
        new_dev = torch.full((batch_size, self.max_blocks_per_seq), -1, dtype=torch.int32,
                             device=self.device)
        new_dev[:rows] = self._table_dev
        self._table_dev = new_dev

    def alloc_block(self, batch_idx: int = 0) -> int:
        """Take the lowest free physical block id, put it in the first unallocated entry of
        row ``batch_idx`` and return that entry's index (kv_cache.py:50-63)."""
        if not self.free_blocks:
            raise RuntimeError("KV cache out of memory")
        phys_block = self.free_blocks.pop(0)
        row = self._table[batch_idx]
        empty_slots = np.flatnonzero(row == -1)
        if len(empty_slots) == 0:
            raise RuntimeError("Sequence block table full")
        logical_idx = int(empty_slots[0])
        row[logical_idx] = phys_block
        self._allocated += 1
        self._pending.append((int(batch_idx), logical_idx, int(phys_block)))
        return logical_idx

    def allocated_blocks(self, batch_idx: int = 0) -> int:
        """Number of non-negative table entries of a row ((block_table[b] >= 0).sum())."""
        return int(np.count_nonzero(self._table[batch_idx] >= 0))

    def get_physical_blocks(self, batch_idx: int = 0) -> torch.Tensor:
        """Row ``batch_idx`` of the device table (kv_cache.py:65-67)."""
        return self.block_table[batch_idx]

    # -- stores ----------------------------------------------------------------------
    def store(self, layer_idx: int, logical_block: int, token_offset: int,
              k: torch.Tensor, v: torch.Tensor):
        """Store one token's K, V ([num_heads, head_dim]) of row 0 (kv_cache.py:69-77)."""
        pos = logical_block * self.block_size + token_offset
        store_kv(k.reshape(1, 1, *k.shape[-2:]), v.reshape(1, 1, *v.shape[-2:]),
                 self.k[layer_idx], self.v[layer_idx], self.block_table[:1], pos)

    def store_batch(self, layer_idx: int, start_block: int, start_offset: int,
                    k: torch.Tensor, v: torch.Tensor):
        """Store consecutive tokens' K, V ([num_tokens, num_heads, head_dim]) of row 0
        starting at (start_block, start_offset) (kv_cache.py:79-103)."""
        pos = start_block * self.block_size + start_offset
        store_kv(k.unsqueeze(0), v.unsqueeze(0), self.k[layer_idx], self.v[layer_idx],
                 self.block_table[:1], pos)

    def allocated_tokens(self, batch_idx: int = 0) -> int:
        """Number of tokens currently stored for a sequence (upper bound, :104-106)."""
        return self._allocated * self.block_size

    def reset(self):
        """Every entry back to -1, every block back on the free list, token count 0
        (kv_cache.py:108-113)."""
        self._table.fill(-1)
        self._pending = []
        self._table_dev.fill_(-1)
        self.free_blocks = list(range(self.num_blocks))
        self._allocated = 0
        self.num_tokens = 0
