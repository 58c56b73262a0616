"""The KVCache drop-in never makes the host wait for the device.

The model's attention path (model.py:162-201 for the K/V writes, kernels/attention.py:191-233
for decode) runs ``store_kv_prefill``, ``store_kv_decode`` and ``paged_attention`` on a
``KVCache`` layer by layer.  Each allocation that fills new table entries is flushed to the
device table the next time ``block_table`` is read; that flush goes through pinned memory
and an asynchronous copy.  Here the whole flow -- prefill, then decode steps that cross block
boundaries, so that the allocator runs mid-stream -- executes under
``torch.cuda.set_sync_debug_mode("error")``, which raises on any synchronizing call, and the
device table must equal the allocator's host copy afterwards.
"""

import numpy as np
import pytest
import torch

from fast_infer_amd import KVCache, paged_attention, store_kv_decode, store_kv_prefill

pytestmark = pytest.mark.gpu


def test_kvcache_prefill_and_decode_never_sync():
    dev = torch.device("cuda")
    layers, hq, hkv, d, bs = 2, 24, 8, 128, 64
    batch, prompt, steps = 3, 100, 40  # positions 100..139 cross the block at 128
    cache = KVCache(layers, hkv, d, 512, bs, dev, num_blocks=32)
    g = torch.Generator(device=dev).manual_seed(7)
    k = torch.randn(batch, prompt, hkv, d, device=dev, generator=g, dtype=torch.float16)
    v = torch.randn(batch, prompt, hkv, d, device=dev, generator=g, dtype=torch.float16)
    kd = torch.randn(steps, batch, hkv, d, device=dev, generator=g, dtype=torch.float16)
    vd = torch.randn(steps, batch, hkv, d, device=dev, generator=g, dtype=torch.float16)
    q = torch.randn(steps, batch, hq, d, device=dev, generator=g, dtype=torch.float16)
    torch.cuda.synchronize()
    outs = []
    torch.cuda.set_sync_debug_mode("error")
    try:
        for layer in range(layers):
            store_kv_prefill(cache, layer, k, v)
        for t in range(steps):
            pos = prompt + t
            for layer in range(layers):
                store_kv_decode(cache, layer, kd[t], vd[t], pos)
                outs.append(paged_attention(q[t], cache.k[layer], cache.v[layer],
                                            cache.block_table, bs, cache.num_tokens))
    finally:
        torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()
    host = cache.host_block_table()
    assert np.array_equal(cache.block_table.cpu().numpy(), host)
    # three rows of ceil(140 / 64) = 3 blocks each, handed out in row order
    assert (host[:, :3] >= 0).all() and (host[:, 3:] == -1).all()
    assert all(torch.isfinite(o.float()).all() for o in outs)


def test_sync_detector_catches_a_blocking_table_write():
    """Positive control: the pattern the flush replaced (a pageable host tensor copied to the
    device with a blocking copy, then scattered) is reported by the same debug mode."""
    dev = torch.device("cuda")
    table = torch.full((2, 4), -1, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        with pytest.raises(RuntimeError):
            vals = torch.tensor([3, 5], dtype=torch.int32).to(dev)
            table.index_put_((torch.tensor([0, 1], device=dev), torch.tensor([0, 0], device=dev)),
                             vals)
    finally:
        torch.cuda.set_sync_debug_mode("default")
