"""Paged K/V pool with a device-resident allocator and per-sequence lengths.

``KVCache`` (kv_cache.py:6-113) allocates on the host one block at a time and the model
keeps one token count for the whole batch (model.py:169-170, :193-194).  ``PagedKVCache``
keeps the same pool layout and attribute names but moves the allocator state to HBM:

* ``append(num_new)`` adds tokens to every row in one launch (``fi_kv_append``) and
  returns the rows' start positions and new lengths as device tensors, ready for
  ``rope_store_kv(start_positions=...)`` and ``paged_attention(context_lens=...)``;
* ``release(rows)`` retires finished rows and returns their blocks to the free queue
  (``fi_kv_release``), so new sequences can join a running batch;
* nothing syncs the host; errors (out of blocks, a full row) are recorded on the device
  and raised by ``check()`` when the caller chooses to look.

Allocation order is the reference's: rows in order, each row's new blocks taken from
the front of the free list (kv_cache.py:54, ``free_blocks.pop(0)``).
"""

from __future__ import annotations

import torch

from . import _lib

_STATUS_TEXT = {
    _lib.FI_KV_OUT_OF_BLOCKS: "KV cache out of memory",
    _lib.FI_KV_TABLE_FULL: "Sequence block table full",
    _lib.FI_KV_NEGATIVE_COUNT: "negative token count",
}


class PagedKVCache:
    """Pool ``k`` / ``v`` ``[num_layers, num_blocks, block_size, num_heads, head_dim]`` fp16
    with device state ``block_table`` ``[max_batch, max_blocks_per_seq]``, ``num_alloc`` and
    ``seq_lens`` ``[max_batch]``, ``free_queue`` ``[num_blocks]`` and ``state`` ``[4]``
    (queue head, free count, status, row of the status), all int32."""

    def __init__(self, num_layers: int, num_heads: int, head_dim: int, max_seq_len: int,
                 block_size: int, device, max_batch: int, num_blocks: int | None = None):
        self.num_layers = num_layers
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.max_seq_len = max_seq_len
        self.block_size = block_size
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise RuntimeError("PagedKVCache lives on a HIP device; fast_infer_amd has no CPU path")
        self.max_batch = int(max_batch)
        self.max_blocks_per_seq = (max_seq_len + block_size - 1) // block_size
        self.num_blocks = int(num_blocks) if num_blocks is not None else \
            self.max_blocks_per_seq * self.max_batch
        shape = (num_layers, self.num_blocks, block_size, num_heads, head_dim)
        self.k = torch.zeros(shape, dtype=torch.float16, device=self.device)
        self.v = torch.zeros(shape, dtype=torch.float16, device=self.device)
        i32 = dict(dtype=torch.int32, device=self.device)
        self.block_table = torch.full((self.max_batch, self.max_blocks_per_seq), -1, **i32)
        self.num_alloc = torch.zeros(self.max_batch, **i32)
        self.seq_lens = torch.zeros(self.max_batch, **i32)
        self.free_queue = torch.empty(self.num_blocks, **i32)
        self.state = torch.empty(4, **i32)
        self.reset()

    def _state_args(self):
        return (self.block_table.data_ptr(), self.block_table.stride(0),
                self.max_blocks_per_seq)

    def reset(self) -> None:
        """kv_cache.py:108-113: every row empty, free queue 0..num_blocks-1, status clear."""
        lib = _lib.load()
        rc = lib.fi_kv_reset(*self._state_args(), self.max_batch, self.num_alloc.data_ptr(),
                             self.seq_lens.data_ptr(), self.free_queue.data_ptr(),
                             self.state.data_ptr(), self.num_blocks,
                             _lib.stream_handle(self.device))
        _lib.check(rc, "PagedKVCache.reset")

    def append(self, num_new, batch: int | None = None):
        """Add ``num_new`` tokens (an int for every row, or an int32 tensor ``[batch]``) to
        rows ``0..batch-1`` (default all ``max_batch``), allocating blocks as needed.
        Returns ``(start_positions, context_lens)``: int32 device tensors ``[batch]`` with
        each row's length before and after the call."""
        batch = self.max_batch if batch is None else int(batch)
        if not 0 <= batch <= self.max_batch:
            raise ValueError(f"batch {batch} outside [0, {self.max_batch}]")
        if isinstance(num_new, torch.Tensor):
            per_row = num_new.to(device=self.device, dtype=torch.int32).contiguous()
            if per_row.dim() != 1 or per_row.numel() < batch:
                raise ValueError(f"num_new must be [batch >= {batch}], got {tuple(num_new.shape)}")
            n_all = 0
        else:
            per_row = None
            n_all = int(num_new)
            if n_all < 0:
                raise ValueError("num_new must be >= 0")
        starts = torch.empty(batch, dtype=torch.int32, device=self.device)
        lens = torch.empty(batch, dtype=torch.int32, device=self.device)
        if batch == 0:
            return starts, lens
        lib = _lib.load()
        rc = lib.fi_kv_append(*self._state_args(), self.num_alloc.data_ptr(),
                              self.seq_lens.data_ptr(), self.free_queue.data_ptr(),
                              self.state.data_ptr(), self.num_blocks, self.block_size, batch,
                              None if per_row is None else per_row.data_ptr(), n_all,
                              starts.data_ptr(), lens.data_ptr(),
                              _lib.stream_handle(self.device))
        _lib.check(rc, "PagedKVCache.append")
        return starts, lens

    def release(self, rows) -> None:
        """Retire rows: a bool / int mask tensor ``[max_batch]`` (nonzero = release) or a
        sequence of row indices.  Their blocks go to the back of the free queue."""
        if isinstance(rows, torch.Tensor) and rows.numel() == self.max_batch and \
                rows.dtype in (torch.bool, torch.int32, torch.int64, torch.uint8):
            mask = rows.to(device=self.device, dtype=torch.int32).contiguous()
        else:
            idx = [int(r) for r in (rows.tolist() if isinstance(rows, torch.Tensor) else rows)]
            if any(not 0 <= r < self.max_batch for r in idx):
                raise IndexError(f"row outside [0, {self.max_batch})")
            host = torch.zeros(self.max_batch, dtype=torch.int32)
            host[idx] = 1
            mask = host.to(self.device)
        lib = _lib.load()
        rc = lib.fi_kv_release(*self._state_args(), self.num_alloc.data_ptr(),
                               self.seq_lens.data_ptr(), self.free_queue.data_ptr(),
                               self.state.data_ptr(), self.num_blocks, self.max_batch,
                               mask.data_ptr(), _lib.stream_handle(self.device))
        _lib.check(rc, "PagedKVCache.release")

    # -- host-side inspection (each of these waits for the stream) -----------------------

    def status(self) -> tuple[int, int, int]:
        """(status code, row of the first error or -1, free blocks)."""
        head, count, code, row = self.state.tolist()
        return code, row, count

    def num_free_blocks(self) -> int:
        return self.status()[2]

    def check(self) -> None:
        """Raise if an append since the last reset could not be served."""
        code, row, _ = self.status()
        if code != _lib.FI_KV_OK:
            raise _lib.FastInferError(f"{_STATUS_TEXT.get(code, code)} (row {row})")

    def free_list(self) -> list[int]:
        """Free block ids in the order they will be handed out."""
        head, count, _, _ = self.state.tolist()
        q = self.free_queue.tolist()
        return [q[(head + i) % self.num_blocks] for i in range(count)]
