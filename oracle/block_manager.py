"""Pure-Python restatement of the device block manager
(TEST INFRASTRUCTURE — see ``oracle/__init__.py``).

``OracleBlockManager`` drives the reference allocator restated in ``kv.OracleKVCache``
(kv_cache.py:50-63: ``free_blocks.pop(0)``, first -1 entry of the row) with per-row
token counts:

* ``append`` — the allocation loops of model.py:172-174 (prefill: until the row has
  ceil(S / bs) blocks) and :196-198 (decode: until it covers the new position), run for
  rows in order with each row's own length.  Before allocating it finds the first row
  that cannot be served (negative count; more than ``max_blocks_per_seq`` blocks — the
  reference's "Sequence block table full"; or past the free list — "KV cache out of
  memory") and leaves that row and every later one untouched.  The reference raises
  instead, after a partial allocation; the difference only shows once it has failed.
* ``release`` — no counterpart in the reference (it only has ``reset``,
  kv_cache.py:108-113): a released row's blocks are appended to ``free_blocks`` in
  logical order, rows in order; its entries become -1 and its length 0.
* ``reset`` — kv_cache.py:108-113.

Pinned (tests/test_block_manager_oracle.py): ``append`` reproduces the tables that the
pinned ``kv.store_prefill`` / ``kv.store_decode`` build; conservation (every block is in
exactly one table entry or once in the free list) and ``allocated == ceil(len / bs)``
hold under random append / release sequences; failing rows leave the state unchanged.
"""

from __future__ import annotations

from .kv import OracleKVCache

OK = 0
OUT_OF_BLOCKS = 1
TABLE_FULL = 2
NEGATIVE_COUNT = 3


class OracleBlockManager:
    def __init__(self, num_blocks: int, max_blocks_per_seq: int, max_batch: int,
                 block_size: int):
        self.block_size = block_size
        self.max_blocks_per_seq = max_blocks_per_seq
        self.max_batch = max_batch
        self.cache = OracleKVCache(1, 1, 1, max_seq_len=max_blocks_per_seq * block_size,
                                   block_size=block_size, num_blocks=num_blocks)
        self.cache._grow_batch(max_batch)
        self.seq_lens = [0] * max_batch
        self.status = (OK, -1)

    @property
    def block_table(self):
        return self.cache.block_table

    @property
    def free_blocks(self):
        return self.cache.free_blocks

    def _need(self, b, n):
        return -(-(self.seq_lens[b] + n) // self.block_size)

    def append(self, num_new, batch=None):
        batch = self.max_batch if batch is None else batch
        ns = [int(num_new)] * batch if isinstance(num_new, int) else [int(x) for x in num_new]
        fail, kind = batch, OK
        free, cum = len(self.cache.free_blocks), 0
        for b in range(batch):
            if ns[b] < 0:
                fail, kind = b, NEGATIVE_COUNT
                break
            need = self._need(b, ns[b])
            if need > self.max_blocks_per_seq:
                fail, kind = b, TABLE_FULL
                break
            cum += max(0, need - self.cache.allocated(b))
            if cum > free:
                fail, kind = b, OUT_OF_BLOCKS
                break
        starts = self.seq_lens[:batch]
        for b in range(fail):
            need = self._need(b, ns[b])
            while self.cache.allocated(b) < need:            # model.py:173-174 / :197-198
                self.cache.alloc_block(b)
            self.seq_lens[b] += ns[b]
        if fail < batch and self.status[0] == OK:
            self.status = (kind, fail)
        return starts, self.seq_lens[:batch]

    def release(self, rows):
        for b in sorted(set(int(r) for r in rows)):
            row = self.cache.block_table[b]
            for j, e in enumerate(row):
                if e >= 0:
                    self.cache.free_blocks.append(e)
                    row[j] = -1
            self.seq_lens[b] = 0

    def reset(self):
        self.cache.reset()
        self.seq_lens = [0] * self.max_batch
        self.status = (OK, -1)
