"""Pins for oracle/block_manager.py (CPU only).

The block manager's append is the reference's allocation loop with per-row lengths; it
is pinned against the restated ``store_prefill`` / ``store_decode`` allocation (model.py
:172-174, :196-198, itself pinned in test_kv_oracle.py), and by the invariants any
allocator with release must keep: conservation of blocks, ``allocated == ceil(len/bs)``,
and failing rows leaving the state unchanged.
"""

import random

import numpy as np
import pytest

from oracle import block_manager as OB
from oracle import kv as OK


def _invariants(m: OB.OracleBlockManager, num_blocks: int):
    seen = [e for row in m.block_table for e in row if e >= 0] + list(m.free_blocks)
    assert sorted(seen) == list(range(num_blocks)), "a block is lost or held twice"
    for b, row in enumerate(m.block_table):
        held = [e for e in row if e >= 0]
        assert row[:len(held)] == held, "a row's blocks are not a dense prefix"
        assert len(held) == -(-m.seq_lens[b] // m.block_size)


@pytest.mark.parametrize("S", [1, 63, 64, 65, 200])
def test_append_matches_reference_prefill_then_decode_allocation(S):
    B, bs, N = 3, 64, 40
    ref = OK.OracleKVCache(1, 1, 1, max_seq_len=512, block_size=bs, num_blocks=N)
    one = np.zeros((B, S, 1, 1), np.float16)
    OK.store_prefill(ref, 0, one, one)
    m = OB.OracleBlockManager(N, 8, B, bs)
    starts, lens = m.append(S)
    assert starts == [0] * B and lens == [S] * B
    assert m.block_table == ref.block_table and m.free_blocks == ref.free_blocks
    for pos in range(S, S + 70):
        OK.store_decode(ref, 0, np.zeros((B, 1, 1), np.float16), np.zeros((B, 1, 1), np.float16),
                        pos)
        starts, lens = m.append(1)
        assert starts == [pos] * B and lens == [pos + 1] * B
        assert m.block_table == ref.block_table and m.free_blocks == ref.free_blocks
    _invariants(m, N)


def test_planted_row_order_mistake_is_caught():
    """Serving rows in reverse order (or taking blocks from the back) builds a different
    table than the reference loop: the comparison above would fail."""
    B, bs, N, S = 3, 16, 20, 40
    ref = OK.OracleKVCache(1, 1, 1, max_seq_len=256, block_size=bs, num_blocks=N)
    one = np.zeros((B, S, 1, 1), np.float16)
    OK.store_prefill(ref, 0, one, one)
    wrong = OK.OracleKVCache(1, 1, 1, max_seq_len=256, block_size=bs, num_blocks=N)
    wrong._grow_batch(B)
    for b in reversed(range(B)):
        while wrong.allocated(b) < 3:
            wrong.alloc_block(b)
    assert wrong.block_table != ref.block_table
    lifo = OB.OracleBlockManager(N, 16, B, bs)
    lifo.cache.free_blocks.reverse()
    lifo.append(S)
    assert lifo.block_table != ref.block_table


def test_random_append_release_keeps_invariants():
    rng = random.Random(0)
    N, maxb, B, bs = 64, 12, 8, 16
    m = OB.OracleBlockManager(N, maxb, B, bs)
    for step in range(400):
        if rng.random() < 0.2:
            rows = rng.sample(range(B), rng.randint(1, 3))
            m.release(rows)
            assert all(m.seq_lens[r] == 0 for r in rows)
        else:
            ns = [rng.choice([0, 0, 1, 1, 1, 5, 17]) for _ in range(B)]
            before = list(m.seq_lens)
            free_before = len(m.free_blocks)
            starts, lens = m.append(ns)
            assert starts == before
            if m.status[0] != OB.OK:
                kind, row = m.status
                assert lens[row:] == before[row:]         # failing rows untouched
                assert kind in (OB.OUT_OF_BLOCKS, OB.TABLE_FULL)
                m.status = (OB.OK, -1)                     # continue the walk
                m.release(range(B))
            else:
                assert lens == [a + n for a, n in zip(before, ns)]
                assert len(m.free_blocks) <= free_before
        _invariants(m, N)


def test_release_returns_blocks_to_the_back_in_order():
    m = OB.OracleBlockManager(10, 5, 3, 4)
    m.append([5, 9, 2])             # row0: 0,1  row1: 2,3,4  row2: 5
    assert m.block_table[:3] == [[0, 1, -1, -1, -1], [2, 3, 4, -1, -1], [5, -1, -1, -1, -1]]
    m.release([1, 0])
    assert m.free_blocks == [6, 7, 8, 9, 0, 1, 2, 3, 4]
    m.append([4, 0, 0])             # row0 reuses the front of the queue
    assert m.block_table[0][:1] == [6]


def test_failures_leave_later_rows_unchanged_and_are_sticky():
    m = OB.OracleBlockManager(6, 4, 4, 8)
    starts, lens = m.append([8, 40, 8, 8])          # row 1 needs 5 > 4 blocks
    assert m.status == (OB.TABLE_FULL, 1)
    assert lens == [8, 0, 0, 0] and starts == [0, 0, 0, 0]
    m.append([0, 0, 30, 30])                        # row 2 takes 4, row 3 runs out
    assert m.status == (OB.TABLE_FULL, 1)           # the first error stays
    assert m.seq_lens == [8, 0, 30, 0]
    m.reset()
    assert m.status == (OB.OK, -1) and m.free_blocks == list(range(6))
    m.append([1, -1, 1, 1])
    assert m.status == (OB.NEGATIVE_COUNT, 1) and m.seq_lens == [1, 0, 0, 0]
    m.reset()
    m.append([16, 16, 16, 16])                      # 2 blocks each, 6 free: row 3 fails
    assert m.status == (OB.OUT_OF_BLOCKS, 3) and m.seq_lens == [16, 16, 16, 0]
