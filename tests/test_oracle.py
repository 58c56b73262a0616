"""Pin the CPU oracle (oracle/) before trusting it as the parity checker.

* The numpy restatements of the reference's Triton programs must reproduce the
  reference kernels' own outputs (golden vectors) bit for bit.
* The C restatement (CPU baseline) must agree with them within one fp16 ulp.
* The fp32 closed forms must agree with the goldens within the fp16 tolerance, and
  satisfy textbook special cases and invariants.
* Planted mistakes in the oracle (dropped causal mask, off-by-one, wrong GQA map,
  transposed operand, wrong block mapping) must fail those same checks.
"""

import numpy as np
import pytest
import torch

from conftest import ATOL
from golden import specs
from oracle import attention as OA
from oracle import native


@pytest.fixture(scope="module", autouse=True)
def _build_native():
    native.build(force=False)


def _maxabs(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float32) - np.asarray(b, np.float32))))


def _assert_ulp_close(out, ref):
    """Differences come only from fp32 summation order (C loops vs numpy): at most one
    fp16 ulp of the larger magnitude (two across a binade edge) plus 1e-6 for values
    that cancel to near zero, and rare."""
    out32, ref32 = out.astype(np.float32), ref.astype(np.float32)
    d = np.abs(out32 - ref32)
    big = np.maximum(np.abs(out32), np.abs(ref32)).astype(np.float16)
    assert np.all(d <= 2 * np.spacing(big).astype(np.float32) + 1e-6)
    assert d.max() <= 1e-3
    assert np.mean(out.view(np.uint16) != ref.view(np.uint16)) < 0.01


def test_golden_inputs_regenerate(golden):
    _, meta = golden
    for name, case in meta["cases"].items():
        sp = case["spec"]
        if case["kind"] == "prefill":
            got = specs.sha256(*specs.prefill_inputs(sp))
        else:
            q, kc, vc, table, _ = specs.decode_inputs(sp)
            got = specs.sha256(q, kc, vc, table)
        assert got == case["inputs_sha256"], f"{name}: generator drifted"


@pytest.mark.parametrize("name", list(specs.DECODE_CASES))
def test_paged_restatement_matches_reference_bitexact(golden, name):
    arrays, _ = golden
    sp = specs.DECODE_CASES[name]
    q, kc, vc, table, _ = specs.decode_inputs(sp)
    out = OA.reference_paged_forward(q.numpy(), kc.numpy(), vc.numpy(), table.numpy(),
                                     sp["bs"], sp["ctx"])
    ref = arrays[f"{name}__out"]
    assert np.array_equal(out.view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("name", [n for n in specs.PREFILL_CASES if specs.PREFILL_CASES[n]["S"] <= 130])
def test_flash_restatement_matches_reference_bitexact(golden, name):
    arrays, _ = golden
    sp = specs.PREFILL_CASES[name]
    q, k, v = specs.prefill_inputs(sp)
    out = OA.reference_flash_forward(q.numpy(), k.numpy(), v.numpy())
    rows = arrays[f"{name}__rows"]
    assert np.array_equal(out[:, :, rows].view(np.uint16), arrays[f"{name}__out"].view(np.uint16))


def test_flash_restatement_s512_sampled_programs(golden):
    arrays, _ = golden
    name = "prefill_b1_s512"
    sp = specs.PREFILL_CASES[name]
    q, k, v = specs.prefill_inputs(sp)
    progs = [(0, 0), (0, 13), (0, 23)]
    out = OA.reference_flash_forward(q.numpy(), k.numpy(), v.numpy(), programs=progs)
    rows = arrays[f"{name}__rows"]
    for b, h in progs:
        assert np.array_equal(out[b, h][rows].view(np.uint16),
                              arrays[f"{name}__out"][b, h].view(np.uint16))


@pytest.mark.parametrize("name", list(specs.DECODE_CASES) + list(specs.RAGGED_CASES))
def test_c_paged_within_one_ulp_of_reference(golden, name):
    arrays, _ = golden
    sp = {**specs.DECODE_CASES, **specs.RAGGED_CASES}[name]
    q, kc, vc, table, lens = specs.decode_inputs(sp)
    out = native.paged_forward(q.numpy(), kc.numpy(), vc.numpy(), table.numpy(), sp["bs"], lens)
    _assert_ulp_close(out, arrays[f"{name}__out"])


@pytest.mark.parametrize("name", list(specs.PREFILL_CASES))
def test_c_flash_within_one_ulp_of_reference(golden, name):
    arrays, _ = golden
    sp = specs.PREFILL_CASES[name]
    q, k, v = specs.prefill_inputs(sp)
    rows = arrays[f"{name}__rows"]
    out = native.flash_forward(q.numpy(), k.numpy(), v.numpy())[:, :, rows]
    _assert_ulp_close(out, arrays[f"{name}__out"])


@pytest.mark.parametrize("name", list(specs.DECODE_CASES) + list(specs.RAGGED_CASES))
def test_fp32_paged_oracle_vs_reference(golden, name):
    arrays, _ = golden
    sp = {**specs.DECODE_CASES, **specs.RAGGED_CASES}[name]
    q, kc, vc, table, lens = specs.decode_inputs(sp)
    out = OA.paged_attention(q, kc, vc, table, sp["bs"], lens)
    assert _maxabs(out, arrays[f"{name}__out"]) <= ATOL


@pytest.mark.parametrize("name", list(specs.PREFILL_CASES))
def test_fp32_causal_oracle_vs_reference(golden, name):
    arrays, _ = golden
    sp = specs.PREFILL_CASES[name]
    q, k, v = specs.prefill_inputs(sp)
    rows = arrays[f"{name}__rows"]
    out = OA.causal_attention(q, k, v)[:, :, rows]
    assert _maxabs(out, arrays[f"{name}__out"]) <= ATOL


# --- closed forms and invariants -------------------------------------------------


def test_causal_seq1_returns_v0():
    g = torch.Generator().manual_seed(5)
    q = torch.randn(2, 6, 1, 128, generator=g).half()
    k = torch.randn(2, 2, 1, 128, generator=g).half()
    v = torch.randn(2, 2, 1, 128, generator=g).half()
    o = OA.causal_attention(q, k, v)
    assert torch.equal(o, v.float().repeat_interleave(3, dim=1))


def test_causal_equal_keys_give_running_mean_of_v():
    # identical keys -> uniform weights over the causal prefix -> running mean of V
    g = torch.Generator().manual_seed(6)
    S = 40
    q = torch.randn(1, 2, S, 128, generator=g)
    k = torch.randn(1, 1, 1, 128, generator=g).expand(1, 1, S, 128)
    v = torch.randn(1, 1, S, 128, generator=g)
    o = OA.causal_attention(q, k, v, dtype=torch.float64)
    mean = torch.cumsum(v.double(), dim=2) / torch.arange(1, S + 1, dtype=torch.float64)[:, None]
    assert torch.allclose(o, mean.expand(1, 2, S, 128), atol=1e-12)


def test_zero_scale_gives_running_mean_of_v():
    # sm_scale == 0: every score is 0, so each row averages V over its causal prefix; the
    # decode oracle averages V over the context
    g = torch.Generator().manual_seed(16)
    S = 70
    q = torch.randn(1, 6, S, 128, generator=g)
    k = torch.randn(1, 2, S, 128, generator=g)
    v = torch.randn(1, 2, S, 128, generator=g)
    o = OA.causal_attention(q, k, v, 0.0, dtype=torch.float64)
    mean = torch.cumsum(v.double(), dim=2) / torch.arange(1, S + 1, dtype=torch.float64)[:, None]
    assert torch.allclose(o, mean.repeat_interleave(3, dim=1), atol=1e-12)
    sp = dict(specs.DECODE_CASES["decode_ctx200"])
    qd, kc, vc, table, lens = specs.decode_inputs(sp)
    od = OA.paged_attention(qd, kc, vc, table, sp["bs"], lens, sm_scale=0.0, dtype=torch.float64)
    _, V = OA.gather_context(kc.double(), vc.double(), table.numpy(), sp["bs"], 0, lens[0])
    assert torch.allclose(od[0], V.mean(0).repeat_interleave(3, dim=0), atol=1e-12)


def test_one_hot_v_reads_softmax_weights():
    g = torch.Generator().manual_seed(7)
    S = 20
    q = torch.randn(1, 1, S, 128, generator=g)
    k = torch.randn(1, 1, S, 128, generator=g)
    v = torch.zeros(1, 1, S, 128)
    v[0, 0, torch.arange(S), torch.arange(S)] = 1.0  # row j of V is e_j
    o = OA.causal_attention(q, k, v, dtype=torch.float64)
    s = (q.double()[0, 0] @ k.double()[0, 0].T) * 128 ** -0.5
    s = s.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(1), float("-inf"))
    w = torch.softmax(s, dim=-1)
    assert torch.allclose(o[0, 0, :, :S], w, atol=1e-12)
    # weights of a row sum to one and vanish above the diagonal
    assert torch.allclose(o[0, 0, :, :S].sum(-1), torch.ones(S, dtype=torch.float64))
    assert float(o[0, 0, :, :S].triu(1).abs().max()) == 0.0


def test_gqa_equals_explicit_expansion():
    g = torch.Generator().manual_seed(8)
    q = torch.randn(1, 6, 30, 128, generator=g)
    k = torch.randn(1, 2, 30, 128, generator=g)
    v = torch.randn(1, 2, 30, 128, generator=g)
    a = OA.causal_attention(q, k, v, dtype=torch.float64)
    b = OA.causal_attention(q, k.repeat_interleave(3, 1), v.repeat_interleave(3, 1),
                            dtype=torch.float64)
    assert torch.equal(a, b)


def test_paged_single_token_returns_v():
    sp = dict(specs.DECODE_CASES["decode_ctx1"])
    q, kc, vc, table, lens = specs.decode_inputs(sp)
    o = OA.paged_attention(q, kc, vc, table, sp["bs"], lens)
    for b in range(sp["B"]):
        phys = int(table[b, 0])
        assert torch.equal(o[b], vc[phys, 0].float().repeat_interleave(3, dim=0))


def test_paged_matches_dense_causal_last_row():
    # decode at position n-1 equals the last row of causal prefill over the same tokens
    sp = dict(specs.DECODE_CASES["decode_ctx200"])
    q, kc, vc, table, lens = specs.decode_inputs(sp)
    n = lens[0]
    K, V = OA.gather_context(kc, vc, table.numpy(), sp["bs"], 0, n)
    qq = torch.zeros(1, sp["Hq"], n, 128, dtype=torch.float16)
    qq[0, :, -1] = q[0]
    dense = OA.causal_attention(qq, K.permute(1, 0, 2)[None], V.permute(1, 0, 2)[None],
                                dtype=torch.float64)[0, :, -1]
    paged = OA.paged_attention(q, kc, vc, table, sp["bs"], lens, dtype=torch.float64)[0]
    assert torch.allclose(dense, paged, atol=1e-12)


def test_paged_invariant_under_pool_permutation():
    sp = dict(specs.DECODE_CASES["decode_ctx200"])
    q, kc, vc, table, lens = specs.decode_inputs(sp)
    perm = torch.randperm(sp["N"], generator=torch.Generator().manual_seed(3))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(sp["N"])
    kc2, vc2 = kc[perm], vc[perm]          # block p of the new pool = old block perm[p]
    t = table.clone()
    t[t >= 0] = inv[t[t >= 0].long()].int()
    a = OA.paged_attention(q, kc, vc, table, sp["bs"], lens, dtype=torch.float64)
    b = OA.paged_attention(q, kc2, vc2, t, sp["bs"], lens, dtype=torch.float64)
    assert torch.equal(a, b)


# --- planted mistakes must be caught ------------------------------------------------


def _mutated_causal(q, k, v, mistake):
    q, k, v = (t.float() for t in (q, k, v))
    B, H, S, D = q.shape
    G = H // k.shape[1]
    if mistake == "gqa_modulo":   # head h reads kv head h % H_kv instead of h // G
        idx = torch.arange(H) % k.shape[1]
        k, v = k[:, idx], v[:, idx]
    else:
        k, v = k.repeat_interleave(G, 1), v.repeat_interleave(G, 1)
    if mistake == "transpose_v":
        v = v.transpose(-1, -2)[..., :S, :D] if S >= D else v.flip(-1)
    s = torch.matmul(q, k.transpose(-1, -2)) * D ** -0.5
    diag = {"no_mask": None, "off_by_one": 0}.get(mistake, 1)
    if diag is not None:
        s = s.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(diag), float("-inf"))
    if mistake == "no_scale":
        s = s / (D ** -0.5)
    return torch.matmul(torch.softmax(s, -1), v)


@pytest.mark.parametrize("mistake", ["no_mask", "off_by_one", "gqa_modulo", "transpose_v", "no_scale"])
def test_planted_prefill_mistakes_fail_golden(golden, mistake):
    arrays, _ = golden
    name = "prefill_s33"
    sp = specs.PREFILL_CASES[name]
    q, k, v = specs.prefill_inputs(sp)
    out = _mutated_causal(q, k, v, mistake)
    if mistake == "off_by_one":
        # masking the diagonal leaves row 0 with no key: NaN, or a different answer
        out = torch.nan_to_num(out, nan=1e3)
    assert _maxabs(out, arrays[f"{name}__out"]) > 10 * ATOL


@pytest.mark.parametrize("mistake", ["slot_shift", "ignore_table", "one_short"])
def test_planted_decode_mistakes_fail_golden(golden, mistake):
    arrays, _ = golden
    name = "decode_ctx200"
    sp = specs.DECODE_CASES[name]
    q, kc, vc, table, lens = specs.decode_inputs(sp)
    t = table.clone()
    if mistake == "ignore_table":    # read logical block b as physical block b
        t = torch.arange(t.numel(), dtype=torch.int32).view(t.shape) % sp["N"]
        out = OA.paged_attention(q, kc, vc, t, sp["bs"], lens)
    elif mistake == "slot_shift":   # off-by-one slot within each block
        kc2 = torch.roll(kc, 1, dims=1)
        out = OA.paged_attention(q, kc2, vc, t, sp["bs"], lens)
    else:                            # drop the last context token
        out = OA.paged_attention(q, kc, vc, t, sp["bs"], [n - 1 for n in lens])
    assert _maxabs(out, arrays[f"{name}__out"]) > 10 * ATOL


def test_row_restricted_oracle_equals_full():
    g = torch.Generator().manual_seed(9)
    q = torch.randn(2, 6, 50, 128, generator=g)
    k = torch.randn(2, 2, 50, 128, generator=g)
    v = torch.randn(2, 2, 50, 128, generator=g)
    full = OA.causal_attention(q, k, v, dtype=torch.float64)
    rows, heads = [0, 7, 31, 49], [1, 4, 5]
    part = OA.causal_attention_rows(q, k, v, rows, heads, dtype=torch.float64)
    assert torch.allclose(part, full[:, heads][:, :, rows], atol=1e-12)
