"""Long contexts: paged decode up to the call's limit of 4096 × 1024 tokens, and a
32,000-position prefill with the fused pool write (marked ``gpu``).

Past 384 × 1024 tokens the partitions grow with the context (at most 1024 per row), up to
4096 tokens each; the merge then combines hundreds of partials per (row, head).  One kv head
with three query heads keeps the pools at 1 GiB or less.  Checked against the fp32 oracle
within max-abs 2e-3: two rows of 1,000,000 and 523,777 tokens at block sizes 64 and 1, and
one row at the 4,194,304-token limit at block size 16.
"""

import math

import pytest
import torch

from conftest import ATOL, banner
from oracle import attention as OA

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
HQ, HKV, D = 3, 1, 128


def _case(lens, bs, seed):
    need = [math.ceil(n / bs) for n in lens]
    N = sum(need) + 2
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(len(lens), HQ, D, device=DEV, generator=g).half()
    kc = torch.randn(N, bs, HKV, D, device=DEV, generator=g).half()
    vc = torch.randn(N, bs, HKV, D, device=DEV, generator=g).half()
    perm = torch.randperm(N, generator=torch.Generator().manual_seed(seed)).int()
    table = torch.full((len(lens), max(need)), -1, dtype=torch.int32)
    pos = 0
    for b, n in enumerate(need):
        table[b, :n] = perm[pos:pos + n]
        pos += n
    return q, kc, vc, table


@pytest.mark.parametrize("lens,bs", [([1_000_000, 523_777], 64), ([1_000_000, 523_777], 1),
                                     ([4096 * 1024], 16)])
def test_paged_decode_long_context(hip, lens, bs):
    banner(f"paged decode long context lens {lens} block_size {bs}")
    from fast_infer_amd import paged_attention

    q, kc, vc, table = _case(lens, bs, seed=len(lens) + bs)
    cl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    out = paged_attention(q, kc, vc, table.to(DEV), bs, max(lens), context_lens=cl)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    ref = OA.paged_attention(q.cpu(), kc.cpu(), vc.cpu(), table, bs, lens)
    assert float((out.float().cpu() - ref).abs().max()) <= ATOL


def test_flash_prefill_long_sequence_with_pool(hip):
    # batch 1 x 32,000 positions (500 query tiles, the last one partial), 24 / 8 heads:
    # sampled rows of every head against the oracle, and the fused pool write gathered back
    # through a shuffled table bit for bit
    S, H, Hkv, bs = 32_000, 24, 8, 64
    banner(f"flash prefill batch 1 x {S} with pool write")
    from fast_infer_amd import flash_attention

    g = torch.Generator(device=DEV).manual_seed(5)
    q = torch.randn(1, S, H, D, device=DEV, generator=g).half().transpose(1, 2)
    k = torch.randn(1, S, Hkv, D, device=DEV, generator=g).half()
    v = torch.randn(1, S, Hkv, D, device=DEV, generator=g).half()
    nb = math.ceil(S / bs)
    N = nb + 3
    table = torch.randperm(N, generator=torch.Generator().manual_seed(6)).int()[:nb].view(1, nb)
    kc = torch.zeros(N, bs, Hkv, D, device=DEV, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    out = flash_attention(q, k.transpose(1, 2), v.transpose(1, 2), k_cache=kc, v_cache=vc,
                          block_table=table.to(DEV))
    torch.cuda.synchronize()
    rows = [0, 1, 63, 64, 4095, 20_001, S - 1]
    ref = OA.causal_attention_rows(q.cpu(), k.transpose(1, 2).cpu(), v.transpose(1, 2).cpu(), rows)
    got = out[:, :, rows].float().cpu()
    assert float((got - ref).abs().max()) <= ATOL
    t = torch.arange(S)
    slot = (table[0, t // bs].long() * bs + t % bs).to(DEV)
    assert torch.equal(kc.view(-1, Hkv, D)[slot], k[0])
    assert torch.equal(vc.view(-1, Hkv, D)[slot], v[0])
    unused = sorted(set(range(N)) - set(table[0].tolist()))
    assert float(kc[unused].abs().max()) == 0.0 and float(vc[unused].abs().max()) == 0.0
