"""Large batches (marked ``gpu``): paged decode over 700 ragged rows and causal prefill over
96 short sequences, against the fp32 oracle within max-abs 2e-3 on sampled rows.

The decode grid's row axis then holds 700 rows, each split into 384-token partitions (the
call allows 1500 tokens) that the merge combines; the empty row gives zeros.  The prefill
grid's first axis holds batch × kv heads workgroups.
"""

import math

import pytest
import torch

from conftest import ATOL, banner
from oracle import attention as OA

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def test_paged_decode_batch_700_ragged(hip):
    banner("paged decode batch 700, contexts 0..1500")
    from fast_infer_amd import paged_attention

    B, Hq, Hkv, D, bs = 700, 24, 8, 128, 64
    gen = torch.Generator().manual_seed(12)
    lens = torch.randint(0, 1501, (B,), generator=gen).tolist()
    lens[3] = 0
    need = [math.ceil(n / bs) for n in lens]
    N = sum(need) + 5
    g = torch.Generator(device=DEV).manual_seed(12)
    q = torch.randn(B, Hq, D, device=DEV, generator=g).half()
    kc = torch.randn(N, bs, Hkv, D, device=DEV, generator=g).half()
    vc = torch.randn(N, bs, Hkv, D, device=DEV, generator=g).half()
    perm = torch.randperm(N, generator=gen).int()
    table = torch.full((B, max(need)), -1, dtype=torch.int32)
    pos = 0
    for b, n in enumerate(need):
        table[b, :n] = perm[pos:pos + n]
        pos += n
    cl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    out = paged_attention(q, kc, vc, table.to(DEV), bs, 1500, context_lens=cl)
    torch.cuda.synchronize()
    assert float(out[3].abs().max()) == 0.0
    rows = [0, 3, 1, 250, 499, 698, 699]
    sub = torch.tensor(rows)
    ref = OA.paged_attention(q.cpu()[sub], kc.cpu(), vc.cpu(), table[sub], bs,
                             [lens[r] for r in rows])
    assert float((out.cpu()[sub].float() - ref).abs().max()) <= ATOL


def test_flash_prefill_batch_96(hip):
    banner("flash prefill batch 96 x 130")
    from fast_infer_amd import flash_attention

    B, S, H, Hkv, D = 96, 130, 24, 8, 128
    g = torch.Generator(device=DEV).manual_seed(13)
    q = torch.randn(B, S, H, D, device=DEV, generator=g).half().transpose(1, 2)
    k = torch.randn(B, S, Hkv, D, device=DEV, generator=g).half().transpose(1, 2)
    v = torch.randn(B, S, Hkv, D, device=DEV, generator=g).half().transpose(1, 2)
    out = flash_attention(q, k, v)
    torch.cuda.synchronize()
    for b in (0, 47, 95):
        ref = OA.causal_attention(q[b:b + 1].cpu(), k[b:b + 1].cpu(), v[b:b + 1].cpu())
        assert float((out[b:b + 1].float().cpu() - ref).abs().max()) <= ATOL
