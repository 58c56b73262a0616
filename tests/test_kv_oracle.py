"""Pin the KV-write / allocator oracle (oracle/kv.py) by brute force, and check the
host-side allocator of fast_infer_amd.KVCache against it (CPU only: the allocator
never touches the device table until it is read)."""

import numpy as np
import pytest
import torch

from oracle import kv as OK


def _rand(shape, seed):
    return np.random.RandomState(seed).standard_normal(shape).astype(np.float16)


def test_store_prefill_matches_brute_force_scatter():
    cache = OK.OracleKVCache(2, 8, 128, max_seq_len=512, block_size=64, num_blocks=40)
    cache._grow_batch(3)
    # pre-allocate a few blocks out of order to make the table non-trivial
    for b in (2, 0, 2, 1):
        cache.alloc_block(b)
    k = _rand((3, 150, 8, 128), 1)
    v = _rand((3, 150, 8, 128), 2)
    before_k = cache.k.copy()
    OK.store_prefill(cache, 1, k, v)
    assert cache.num_tokens == 0  # layer 1 does not set num_tokens (model.py:169-170)
    # brute force on a copy of the pre-store pool with the final table
    bk, bv = before_k[1].copy(), np.zeros_like(before_k[1])
    OK.scatter(bk, bv, cache.block_table, k, v, 0, 64)
    assert np.array_equal(cache.k[1], bk) and np.array_equal(cache.v[1], bv)
    assert np.array_equal(cache.k[0], before_k[0])  # other layer untouched
    # each row got exactly ceil(150/64) = 3 blocks
    assert [cache.allocated(b) for b in range(3)] == [3, 3, 3]


def test_store_prefill_layer0_sets_num_tokens_and_leaves_tail_slots():
    cache = OK.OracleKVCache(1, 2, 128, max_seq_len=256, block_size=64)
    k = _rand((1, 70, 2, 128), 3)
    OK.store_prefill(cache, 0, k, k)
    assert cache.num_tokens == 70
    phys1 = cache.block_table[0][1]
    assert np.all(cache.k[0, phys1, 6:] == 0)  # slots 6..63 of the last block stay zero
    assert np.array_equal(cache.k[0, phys1, :6], k[0, 64:70])


def test_store_decode_matches_brute_force_and_allocates_lazily():
    cache = OK.OracleKVCache(1, 8, 128, max_seq_len=256, block_size=64, num_blocks=16)
    cache._grow_batch(2)
    k = _rand((2, 8, 128), 4)
    v = _rand((2, 8, 128), 5)
    OK.store_decode(cache, 0, k, v, token_pos=64)  # needs logical block 1 -> allocates 2 per row
    assert cache.num_tokens == 1
    assert [cache.allocated(b) for b in range(2)] == [2, 2]
    assert cache.block_table[0][:2] == [0, 1] and cache.block_table[1][:2] == [2, 3]
    bk = np.zeros_like(cache.k[0])
    bv = np.zeros_like(cache.v[0])
    OK.scatter(bk, bv, cache.block_table, k[:, None], v[:, None], 64, 64)
    assert np.array_equal(cache.k[0], bk) and np.array_equal(cache.v[0], bv)


def test_store_and_store_batch_match_scatter():
    cache = OK.OracleKVCache(1, 4, 128, max_seq_len=256, block_size=16)
    for _ in range(5):
        cache.alloc_block(0)
    k = _rand((40, 4, 128), 6)
    OK.store_batch(cache, 0, 1, 5, k, k)
    bk = np.zeros_like(cache.k[0])
    OK.scatter(bk, bk.copy(), cache.block_table, k[None], k[None], 16 + 5, 16)
    assert np.array_equal(cache.k[0], bk)
    one = _rand((4, 128), 7)
    OK.store(cache, 0, 2, 3, one, one)
    assert np.array_equal(cache.k[0, cache.block_table[0][2], 3], one)


def test_allocator_closed_form_and_errors():
    cache = OK.OracleKVCache(1, 1, 128, max_seq_len=128, block_size=64)  # 2 blocks
    assert cache.alloc_block(0) == 0 and cache.block_table[0] == [0, -1]
    assert cache.alloc_block(0) == 1 and cache.block_table[0] == [0, 1]
    with pytest.raises(RuntimeError, match="KV cache out of memory"):
        cache.alloc_block(0)
    cache.reset()
    assert cache.block_table[0] == [-1, -1] and cache.free_blocks == [0, 1]
    cache2 = OK.OracleKVCache(1, 1, 128, max_seq_len=64, block_size=64, num_blocks=4)
    cache2.alloc_block(0)
    with pytest.raises(RuntimeError, match="Sequence block table full"):
        cache2.alloc_block(0)


# --- fast_infer_amd.KVCache allocator vs the oracle (no device work) -----------------


def _fi_cache(**kw):
    from fast_infer_amd.kv_cache import KVCache

    return KVCache(device="cpu", **kw)


@pytest.mark.parametrize("num_blocks", [None, 12])
def test_kvcache_allocator_matches_oracle(num_blocks):
    args = dict(num_layers=1, num_heads=2, head_dim=128, max_seq_len=256, block_size=64)
    fi = _fi_cache(**args, num_blocks=num_blocks)
    ok = OK.OracleKVCache(**args, num_blocks=num_blocks)
    assert fi.num_blocks == ok.num_blocks and fi.max_blocks_per_seq == ok.max_blocks_per_seq
    assert tuple(fi.k.shape) == (1, ok.num_blocks, 64, 2, 128)
    assert fi.k.dtype == torch.float16 and float(fi.k.abs().sum()) == 0.0
    fi._grow_batch(3)
    ok._grow_batch(3)
    seq = [0, 2, 2, 1, 0, 2, 1]
    for b in seq:
        try:
            r_ok = ok.alloc_block(b)
        except RuntimeError as e:
            with pytest.raises(RuntimeError, match=str(e)):
                fi.alloc_block(b)
            continue
        assert fi.alloc_block(b) == r_ok
    assert fi.block_table.tolist() == ok.block_table
    assert fi.free_blocks == ok.free_blocks
    fi.reset()
    ok.reset()
    assert fi.block_table.tolist() == ok.block_table and fi.num_tokens == 0


def test_kvcache_errors_match_reference_messages():
    fi = _fi_cache(num_layers=1, num_heads=1, head_dim=128, max_seq_len=128, block_size=64)
    fi.alloc_block(0)
    fi.alloc_block(0)
    with pytest.raises(RuntimeError, match="^KV cache out of memory$"):
        fi.alloc_block(0)
    fi2 = _fi_cache(num_layers=1, num_heads=1, head_dim=128, max_seq_len=64, block_size=64,
                    num_blocks=3)
    fi2.alloc_block(0)
    with pytest.raises(RuntimeError, match="^Sequence block table full$"):
        fi2.alloc_block(0)


def test_kvcache_block_table_assignment_and_grow():
    fi = _fi_cache(num_layers=1, num_heads=1, head_dim=128, max_seq_len=256, block_size=64)
    fi.block_table = torch.tensor([[3, -1, -1, -1]], dtype=torch.int32)
    assert fi.allocated_blocks(0) == 1
    fi._grow_batch(2)
    assert fi.block_table.tolist() == [[3, -1, -1, -1], [-1, -1, -1, -1]]
    assert fi.alloc_block(1) == 0 and fi.block_table[1, 0].item() == 0
