"""The allocation-free decode entry point ``fi_paged_attention_fwd_noalloc`` (marked ``gpu``).

Called through the C ABI, its output must equal ``fi_paged_attention_fwd``'s (with a
caller workspace) bit for bit: both run the same kernels, only the split-K scratch
differs.  Two calls in a row, the second smaller, so the second runs over scratch the
first left behind.  A request larger than the static scratch is refused before any launch.
"""

import ctypes

import numpy as np
import pytest
import torch

from conftest import ATOL, banner
from oracle import attention as OA

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
HQ, HKV, D, BS = 24, 8, 128, 64


def _case(B, lo, hi, seed, N):
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, B).astype(np.int32)
    g = torch.Generator(device=DEV).manual_seed(seed)
    kc = torch.randn(N, BS, HKV, D, device=DEV, generator=g, dtype=torch.float16)
    vc = torch.randn(N, BS, HKV, D, device=DEV, generator=g, dtype=torch.float16)
    q = torch.randn(B, HQ, D, device=DEV, generator=g, dtype=torch.float16)
    width = 64
    table = torch.full((B, width), -1, dtype=torch.int32)
    perm = rng.permutation(N)
    pos = 0
    for b, n in enumerate(lens):
        nb = -(-int(n) // BS)
        table[b, :nb] = torch.from_numpy(perm[pos:pos + nb].astype(np.int32))
        pos += nb
    return q, kc, vc, table.to(DEV), torch.from_numpy(lens).to(DEV), lens


def _args(q, kc, vc, table, cl, num_tokens, o):
    return (q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(), kc.shape[0],
            BS, HKV, table.data_ptr(), table.stride(0), table.shape[1], cl.data_ptr(),
            num_tokens, o.data_ptr(), o.stride(0), o.stride(1), q.shape[0], HQ, D,
            ctypes.c_float(D ** -0.5))


def _both(hip, q, kc, vc, table, cl, num_tokens):
    from fast_infer_amd import _lib

    stream = _lib.stream_handle(torch.device(DEV))
    need = hip.fi_paged_attention_workspace_size(q.shape[0], HQ, HKV, num_tokens, D)
    assert 0 < need <= 32 << 20
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    o_ws = torch.full_like(q, float("nan"))
    o_na = torch.full_like(q, float("nan"))
    _lib.check(hip.fi_paged_attention_fwd(*_args(q, kc, vc, table, cl, num_tokens, o_ws),
                                          ws.data_ptr(), need, stream), "with workspace")
    _lib.check(hip.fi_paged_attention_fwd_noalloc(*_args(q, kc, vc, table, cl, num_tokens, o_na),
                                                  stream), "noalloc")
    torch.cuda.synchronize()
    return o_ws, o_na


def test_noalloc_matches_workspace_entry_point_twice(hip):
    cases = [(32, 512, 4096, 2, 2048, 4096),   # batch 32, contexts U[512, 4096]
             (5, 600, 1500, 9, 200, 1536)]     # then a smaller call over the same scratch
    for B, lo, hi, seed, N, num_tokens in cases:
        banner(f"noalloc decode batch {B}, contexts [{lo}, {hi}], num_tokens {num_tokens}")
        q, kc, vc, table, cl, lens = _case(B, lo, hi, seed, N)
        o_ws, o_na = _both(hip, q, kc, vc, table, cl, num_tokens)
        assert torch.equal(o_na, o_ws)
        for b in (0, B - 1):  # and against the fp32 oracle on two rows
            n = int(lens[b])
            ref = OA.paged_attention(q[b:b + 1].cpu(), kc.cpu(), vc.cpu(), table[b:b + 1].cpu(),
                                     BS, [n])
            assert float((o_na[b:b + 1].float().cpu() - ref).abs().max()) <= ATOL


def test_noalloc_rejects_requests_beyond_its_scratch(hip):
    from fast_infer_amd import _lib

    banner("noalloc decode: oversize request refused before launch")
    B, num_tokens = 4096, 4096
    need = hip.fi_paged_attention_workspace_size(B, HQ, HKV, num_tokens, D)
    assert need > 32 << 20
    q = torch.zeros(B, HQ, D, device=DEV, dtype=torch.float16)
    kc = torch.zeros(1, BS, HKV, D, device=DEV, dtype=torch.float16)
    table = torch.zeros(B, 64, dtype=torch.int32, device=DEV)
    cl = torch.ones(B, dtype=torch.int32, device=DEV)
    o = torch.empty_like(q)
    rc = hip.fi_paged_attention_fwd_noalloc(*_args(q, kc, kc, table, cl, num_tokens, o),
                                            _lib.stream_handle(torch.device(DEV)))
    assert rc == _lib.FI_ERR_UNSUPPORTED
    assert b"scratch" in hip.fi_last_error()
