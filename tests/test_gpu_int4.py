"""GPU parity tests of the INT4 linear layer (``fi_int4_quantize`` / ``fi_int4_dequantize`` /
``fi_int4_matmul``), marked ``gpu``.

* quantize and dequantize bit-exact against the oracle (oracle/int4.py), including
  all-zero groups, subnormal scales and values near the top of fp16;
* quantize bit-exact against the reference's own expression (loader.py:20-38) evaluated by
  torch on the same GPU, over groups whose maxima cover every positive fp16 value;
* group sizes 8..512 besides the reference's 128: quantize / dequantize bit-exact, and the
  matmul (on the dequantized weight) within the same bound;
* int4_matmul with packed weights within the fp32-accumulation bound of the float64
  product on the dequantized weights, for decode-sized M (1..64, split-K) and prefill
  sizes, odd N, strided X; the speed mode (dequantized fp16 weights) within the same
  bound;
* the split-K kernel that adds its K splits in the same launch (17..64 rows, packed
  weights): shapes whose tile and split counts change from call to call on one stream
  (each call leaves its arrival counters at zero for the next), calls on two streams in
  flight together (each stream has its own counters), and streams past the per-device
  counter sets, which take the two-launch path: all within the same bound, and the same
  bits on every stream that has counters.
"""

import numpy as np
import pytest
import torch

from conftest import banner
from oracle import int4 as OI

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _weights(seed, N, K, scale=0.05, big=False):
    """Random weights with an all-zero group and a tiny group (subnormal scales); with
    ``big`` also a group near the top of fp16 (products would overflow a matmul)."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * scale).astype(np.float32)
    w[0, :128] = 0.0
    w[1 % N, 128 % K:256 % K or K] *= 1e-4
    if big:
        w[2 % N, :128] = 3.0e4 * np.sign(w[2 % N, :128])
    return w.astype(np.float16)


@pytest.mark.parametrize("N,K", [(5120, 3072), (3, 256), (130, 8192)])
def test_quantize_dequantize_bitexact(hip, N, K):
    banner(f"int4 quantize/dequantize N={N} K={K}")
    from fast_infer_amd import dequantize_int4, quantize_int4_groupwise

    w = _weights(N + K, N, K, big=True)
    packed, scales = quantize_int4_groupwise(torch.from_numpy(w).to(DEV))
    ep, es = OI.quantize_int4_groupwise(w)
    torch.cuda.synchronize()
    assert np.array_equal(packed.cpu().numpy(), ep)
    assert np.array_equal(scales.cpu().numpy().view(np.uint16), es.view(np.uint16))
    deq = dequantize_int4(packed, scales)
    ed = OI.dequantize(ep, es)
    torch.cuda.synchronize()
    assert np.array_equal(deq.cpu().numpy().view(np.uint16), ed.view(np.uint16))


def _reference_quantize_on_device(w: torch.Tensor, groupsize: int = 128):
    """loader.py:20-38 run as torch tensor ops on the GPU: the reference's own arithmetic
    (``w_max / 7.0`` on a device tensor, ``torch.round(w / scale)``) on the same device."""
    out_features, in_features = w.shape
    w = w.reshape(out_features, -1, groupsize)
    w_max = torch.clamp(w.abs().amax(dim=-1, keepdim=True), min=1e-6)
    scale = w_max / 7.0
    w_q = torch.clamp(torch.round(w / scale.to(w.dtype)), -8, 7).to(torch.int8)
    w_q = w_q.reshape(out_features, -1, groupsize // 2, 2)
    packed = ((w_q[..., 0] & 0xF) | ((w_q[..., 1] & 0xF) << 4))
    packed = packed.reshape(out_features, in_features // 2).to(torch.int8)
    return packed, scale.reshape(out_features, in_features // groupsize).to(torch.float16)


@pytest.mark.parametrize("N,K", [(5120, 3072), (7, 1024)])
def test_quantize_matches_reference_expression_on_device(hip, N, K):
    """fi_int4_quantize against the reference's expression evaluated by torch on this GPU,
    bit for bit: random weights, an all-zero group (clamped to fp16(1e-6)), subnormal
    scales, values near the top of fp16, and one group per row whose maximum walks through
    every positive finite fp16 value in turn (so every possible scale is produced)."""
    banner(f"int4 quantize vs the reference expression on the GPU, N={N} K={K}")
    from fast_infer_amd import quantize_int4_groupwise

    w = _weights(N * 7 + K, N, K, big=True)
    every = np.arange(1, 0x7C00, dtype=np.uint16).view(np.float16)  # all positive finite fp16
    groups = N * (K // 128)
    maxima = np.resize(every, groups).reshape(N, K // 128)
    g = w.reshape(N, K // 128, 128).astype(np.float32)
    g = np.clip(g, -np.abs(maxima[..., None]).astype(np.float32), np.abs(maxima[..., None]))
    g[..., 5] = maxima  # each group's largest |w| is exactly this value
    g[..., 6] = -maxima * np.float16(0.5)
    w = g.reshape(N, K).astype(np.float16)
    wd = torch.from_numpy(w).to(DEV)
    packed, scales = quantize_int4_groupwise(wd)
    rp, rs = _reference_quantize_on_device(wd)
    torch.cuda.synchronize()
    assert torch.equal(scales.view(torch.int16), rs.view(torch.int16))
    assert torch.equal(packed, rp)
    ep, es = OI.quantize_int4_groupwise(w)
    assert np.array_equal(packed.cpu().numpy(), ep)
    assert np.array_equal(scales.cpu().numpy().view(np.uint16), es.view(np.uint16))


def _check(out, x, w16):
    got = out.float().cpu().numpy().astype(np.float64)
    exact = OI.matmul_exact(x, w16)
    bound = OI.matmul_bound(x, w16)
    assert np.all(np.abs(got - exact) <= bound), float(np.max(np.abs(got - exact) - bound))


@pytest.mark.parametrize("M", [1, 5, 16, 17, 33, 64, 100, 300])
@pytest.mark.parametrize("N,K", [(5120, 3072), (3072, 3072), (130, 1024)])
def test_int4_matmul_vs_oracle(hip, M, N, K):
    banner(f"int4_matmul M={M} N={N} K={K}")
    from fast_infer_amd import dequantize_int4, int4_matmul, quantize_int4_groupwise

    w = _weights(7, N, K, 0.02)
    packed, scales = quantize_int4_groupwise(torch.from_numpy(w).to(DEV))
    g = torch.Generator().manual_seed(M * 7 + N)
    x = torch.randn(M, K, generator=g).half()
    out = int4_matmul(x.to(DEV), (packed, scales))
    w16 = dequantize_int4(packed, scales)
    out16 = int4_matmul(x.to(DEV), w16)
    torch.cuda.synchronize()
    _check(out, x.numpy(), w16.cpu().numpy())      # memory mode (packed weights)
    _check(out16, x.numpy(), w16.cpu().numpy())    # speed mode (dequantized weights)


def test_int4_matmul_strided_x_and_batch_dims(hip):
    banner("int4_matmul strided x, [B, S, K] input")
    from fast_infer_amd import dequantize_int4, int4_matmul, quantize_int4_groupwise

    N, K = 640, 3072
    w = _weights(8, N, K, 0.02)
    packed, scales = quantize_int4_groupwise(torch.from_numpy(w).to(DEV))
    g = torch.Generator().manual_seed(9)
    big = torch.randn(2, 7, K + 256, generator=g).half()
    x = big[..., 128:128 + K]                 # [2, 7, K], row stride K + 256
    xd = big.to(DEV)[..., 128:128 + K]        # the same view on the device
    assert xd.stride(1) == K + 256
    out = int4_matmul(xd, (packed, scales))
    assert out.shape == (2, 7, N)
    torch.cuda.synchronize()
    _check(out.reshape(14, N), x.reshape(14, K).numpy(), dequantize_int4(packed, scales).cpu().numpy())


# 17..64 rows run the split-K kernel (gemm_sk_kernel): one K group, a two-way K split
# whose second part is shorter, an 8-way split of 64 groups, partial last column tiles,
# strided X rows, the QKV shape at 33 and 48 rows, an N that is not a multiple of 4 with
# and without a K split (scalar output stores), and a grid of 257 column tiles
@pytest.mark.parametrize("M,N,K,pad", [(17, 64, 128, 0), (20, 130, 640, 0), (40, 70, 8192, 264),
                                       (64, 200, 3072, 512), (33, 5120, 3072, 8),
                                       (48, 5120, 3072, 0), (36, 130, 3072, 0), (17, 66, 128, 0),
                                       (50, 16400, 256, 0)])
def test_int4_matmul_lds_staged_shapes(hip, M, N, K, pad):
    banner(f"int4_matmul staged M={M} N={N} K={K} row pad {pad}")
    from fast_infer_amd import dequantize_int4, int4_matmul, quantize_int4_groupwise

    w = _weights(M + N, N, K, 0.02)
    packed, scales = quantize_int4_groupwise(torch.from_numpy(w).to(DEV))
    g = torch.Generator().manual_seed(M * 31 + K)
    big = torch.randn(M, K + pad, generator=g).half()
    xd = big.to(DEV)[:, 8:8 + K] if pad else big.to(DEV)   # row stride K + pad on the device
    assert xd.stride(0) == K + pad
    out = int4_matmul(xd, (packed, scales))
    torch.cuda.synchronize()
    _check(out, xd.cpu().numpy(), dequantize_int4(packed, scales).cpu().numpy())


def test_int4_matmul_prefill_size_sampled(hip):
    """4 x 512 tokens through the fused QKV weight (N 5120, K 3072): sampled rows of the
    packed and the dequantized forms against float64."""
    banner("int4_matmul M=2048 N=5120 K=3072")
    from fast_infer_amd import dequantize_int4, int4_matmul, quantize_int4_groupwise

    M, N, K = 2048, 5120, 3072
    w = _weights(10, N, K, 0.02)
    packed, scales = quantize_int4_groupwise(torch.from_numpy(w).to(DEV))
    g = torch.Generator(device=DEV).manual_seed(11)
    x = torch.randn(M, K, device=DEV, generator=g).half()
    out = int4_matmul(x, (packed, scales))
    w16 = dequantize_int4(packed, scales)
    out16 = int4_matmul(x, w16)
    rows = torch.tensor([0, 1, 63, 64, 127, 128, 1000, 2047])
    _check(out[rows.to(DEV)], x[rows.to(DEV)].cpu().numpy(), w16.cpu().numpy())
    _check(out16[rows.to(DEV)], x[rows.to(DEV)].cpu().numpy(), w16.cpu().numpy())


# 129 rows and up: the weight dequantized once, then the 256 x 256-tile fp16 GEMM
# (wide_gemm_kernel).  Shapes: partial row and column tiles, two K steps (K 128) and
# 128 (K 8192), row tiles in multiples of 8 (the XCD-banded tile order, also with a partial
# last row tile) and not, N not a multiple of 8 (element stores), output rows with a stride
# and an output that is only 2-byte aligned (element stores), X rows with a stride; packed
# and fp16 weights, every row against float64.
@pytest.mark.parametrize("M,N,K,xpad,opad,ooff", [(129, 264, 128, 0, 0, 0),
                                                  (257, 130, 1024, 8, 6, 1),
                                                  (520, 640, 3072, 0, 0, 0),
                                                  (300, 1288, 3072, 264, 8, 0),
                                                  (2048, 256, 256, 0, 0, 0),
                                                  (4096, 520, 512, 0, 16, 0),
                                                  (2100, 72, 384, 0, 0, 3),
                                                  (1800, 264, 8192, 0, 0, 0)])
def test_int4_matmul_dense_path_shapes(hip, M, N, K, xpad, opad, ooff):
    banner(f"int4_matmul dense M={M} N={N} K={K} x pad {xpad} out pad {opad} out offset {ooff}")
    from fast_infer_amd import _lib, dequantize_int4, quantize_int4_groupwise

    lib = _lib.load()
    w = _weights(M + 3 * N, N, K, 0.02)
    packed, scales = quantize_int4_groupwise(torch.from_numpy(w).to(DEV))
    w16 = dequantize_int4(packed, scales)
    g = torch.Generator(device=DEV).manual_seed(M + K)
    xbig = torch.randn(M, K + xpad, device=DEV, generator=g).half()
    x = xbig[:, 8:8 + K] if xpad else xbig
    ld = N + opad
    ws = torch.empty(lib.fi_int4_matmul_workspace_size(M, N, K), dtype=torch.uint8, device=DEV)
    st = _lib.stream_handle(torch.device(DEV))
    for form in ("packed", "fp16"):
        buf = torch.full((M * ld + 8,), float("nan"), dtype=torch.float16, device=DEV)
        out_ptr = buf.data_ptr() + 2 * ooff
        if form == "packed":
            rc = lib.fi_int4_matmul(x.data_ptr(), x.stride(0), M, K, packed.data_ptr(), K // 2,
                                    scales.data_ptr(), K // 128, N, 128, out_ptr, ld,
                                    ws.data_ptr(), ws.numel(), st)
        else:
            rc = lib.fi_int4_matmul(x.data_ptr(), x.stride(0), M, K, w16.data_ptr(), K, None, 0,
                                    N, 128, out_ptr, ld, ws.data_ptr(), ws.numel(), st)
        _lib.check(rc, "fi_int4_matmul")
        torch.cuda.synchronize()
        rows = buf[ooff:ooff + M * ld].view(M, ld)
        _check(rows[:, :N], x.cpu().numpy(), w16.cpu().numpy())
        # nothing written between rows or past the last one
        assert torch.isnan(rows[:, N:]).all() and torch.isnan(buf[:ooff]).all()
        assert torch.isnan(buf[ooff + M * ld:]).all()


def test_int4_matmul_workspace(hip):
    """Split-K calls (dequantized weights, 17..64 rows) with a caller workspace: the same
    bits as with the cached one, one workspace reused across shapes, and too small a
    workspace rejected before launch."""
    banner("int4_matmul workspace")
    from fast_infer_amd import _lib, dequantize_int4, int4_matmul, quantize_int4_groupwise

    lib = _lib.load()
    N, K = 5120, 3072
    M = 40
    need = lib.fi_int4_matmul_workspace_size(M, N, K)
    assert need > 0
    # prefill sizes dequantize the packed weight once into the workspace
    assert lib.fi_int4_matmul_workspace_size(4096, N, K) == N * K * 2
    w = _weights(12, N, K, 0.02)
    packed, scales = quantize_int4_groupwise(torch.from_numpy(w).to(DEV))
    w16 = dequantize_int4(packed, scales)
    x = torch.randn(64, K, device=DEV).half()
    ws = torch.empty(max(lib.fi_int4_matmul_workspace_size(m, N, K) for m in (17, 40, 64)),
                     dtype=torch.uint8, device=DEV)
    for m in (40, 17, 64, 40):
        a = int4_matmul(x[:m], w16, workspace=ws)
        b = int4_matmul(x[:m], w16)
        assert torch.equal(a, b)
    # the size query covers both weight forms; the packed form needs all of it at 40 rows
    out = torch.empty(M, N, dtype=torch.float16, device=DEV)
    rc = lib.fi_int4_matmul(x.data_ptr(), K, M, K, packed.data_ptr(), K // 2, scales.data_ptr(),
                            K // 128, N, 128, out.data_ptr(), N, ws.data_ptr(), need - 16,
                            _lib.stream_handle(torch.device(DEV)))
    assert rc == _lib.FI_ERR_WORKSPACE


def test_int4_matmul_prefill_workspace_and_errors(hip):
    """The prefill path (dequantize once + fp16 GEMM): a caller workspace gives the same
    bits as the cached one, and one too small is rejected before launch."""
    banner("int4_matmul prefill workspace")
    from fast_infer_amd import _lib, int4_matmul, quantize_int4_groupwise

    lib = _lib.load()
    M, N, K = 512, 640, 1024
    w = _weights(13, N, K, 0.02)
    packed, scales = quantize_int4_groupwise(torch.from_numpy(w).to(DEV))
    x = torch.randn(M, K, device=DEV).half()
    need = lib.fi_int4_matmul_workspace_size(M, N, K)
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    assert torch.equal(int4_matmul(x, (packed, scales), workspace=ws), int4_matmul(x, (packed, scales)))
    out = torch.empty(M, N, dtype=torch.float16, device=DEV)
    rc = lib.fi_int4_matmul(x.data_ptr(), K, M, K, packed.data_ptr(), K // 2, scales.data_ptr(),
                            K // 128, N, 128, out.data_ptr(), N, ws.data_ptr(), need - 256,
                            _lib.stream_handle(torch.device(DEV)))
    assert rc == _lib.FI_ERR_WORKSPACE


@pytest.mark.filterwarnings("ignore:int4_matmul. packed weights with groupsize")
@pytest.mark.parametrize("gs", [8, 32, 64, 256, 512])
def test_other_group_sizes(hip, gs):
    # quantize / dequantize at group sizes other than the reference's 128, bit-exact against
    # the oracle; int4_matmul and the fused norm call on such weights (dequantized first)
    # within the fp32-accumulation bound
    banner(f"int4 group size {gs}")
    from fast_infer_amd import (dequantize_int4, int4_matmul, quantize_int4_groupwise, rms_norm,
                                rms_norm_int4_matmul)

    N, K = 130, 1024
    w = _weights(gs, N, K, big=True)
    packed, scales = quantize_int4_groupwise(torch.from_numpy(w).to(DEV), gs)
    ep, es = OI.quantize_int4_groupwise(w, gs)
    torch.cuda.synchronize()
    assert scales.shape == (N, K // gs)
    assert np.array_equal(packed.cpu().numpy(), ep)
    assert np.array_equal(scales.cpu().numpy().view(np.uint16), es.view(np.uint16))
    deq = dequantize_int4(packed, scales, gs)
    ed = OI.dequantize(ep, es, gs)
    torch.cuda.synchronize()
    assert np.array_equal(deq.cpu().numpy().view(np.uint16), ed.view(np.uint16))
    w = _weights(gs + 1, N, K, 0.02)
    packed, scales = quantize_int4_groupwise(torch.from_numpy(w).to(DEV), gs)
    w16 = dequantize_int4(packed, scales, gs).cpu().numpy()
    for M in (1, 40, 200):
        x = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).half()
        out = int4_matmul(x.to(DEV), (packed, scales), groupsize=gs)
        torch.cuda.synchronize()
        _check(out, x.numpy(), w16)
    nw = (1.0 + 0.1 * torch.randn(K, generator=torch.Generator().manual_seed(3))).half()
    x = torch.randn(4, K, generator=torch.Generator().manual_seed(4)).half()
    fused = rms_norm_int4_matmul(x.to(DEV), nw.to(DEV), (packed, scales), groupsize=gs)
    xn = rms_norm(x.to(DEV), nw.to(DEV))
    torch.cuda.synchronize()
    _check(fused, xn.cpu().numpy(), w16)


def _packed(seed, N, K):
    from fast_infer_amd import quantize_int4_groupwise
    w = _weights(seed, N, K, 0.02)
    return quantize_int4_groupwise(torch.from_numpy(w).to(DEV))


def test_int4_split_k_shapes_change_between_calls(hip):
    """One stream, shapes whose column-tile and K-split counts differ from call to call,
    three rounds: every call within the bound (a counter left non-zero by one call would
    make a later call finish a tile before all its splits are stored)."""
    banner("int4_matmul split-K: changing shapes on one stream")
    from fast_infer_amd import dequantize_int4, int4_matmul

    shapes = [(64, 5120, 3072), (17, 200, 640), (40, 1000, 1024), (64, 3072, 3072),
              (33, 130, 8192), (64, 64, 128)]
    ws = {shape: _packed(sum(shape), shape[1], shape[2]) for shape in shapes}
    g = torch.Generator().manual_seed(5)
    xs = {shape: torch.randn(shape[0], shape[2], generator=g).half() for shape in shapes}
    for _ in range(3):
        for shape in shapes:
            packed, scales = ws[shape]
            out = int4_matmul(xs[shape].to(DEV), (packed, scales))
            torch.cuda.synchronize()
            _check(out, xs[shape].numpy(), dequantize_int4(packed, scales).cpu().numpy())


def test_int4_split_k_two_streams_in_flight(hip):
    """Alternating calls on two streams with no synchronization between them: each stream
    has its own arrival counters, so the calls may overlap; every output has the same bits
    as a call on the default stream."""
    banner("int4_matmul split-K: two streams in flight")
    from fast_infer_amd import int4_matmul

    N, K = 5120, 3072
    packed, scales = _packed(21, N, K)
    g = torch.Generator(device=DEV).manual_seed(22)
    xs = [torch.randn(64, K, device=DEV, generator=g).half() for _ in range(8)]
    refs = [int4_matmul(x, (packed, scales)) for x in xs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(device=DEV), torch.cuda.Stream(device=DEV)]
    outs = [None] * len(xs)
    for rep in range(4):
        for i, x in enumerate(xs):
            with torch.cuda.stream(streams[i % 2]):
                outs[i] = int4_matmul(x, (packed, scales))
        torch.cuda.synchronize()
        for i in range(len(xs)):
            assert torch.equal(outs[i], refs[i]), (rep, i)


def test_int4_split_k_streams_past_the_counter_sets(hip):
    """More streams than the per-device counter sets (16): the streams without one take the
    two-launch path (partials, then a reduction launch); all within the bound."""
    banner("int4_matmul split-K: 20 streams")
    from fast_infer_amd import dequantize_int4, int4_matmul

    N, K = 3072, 3072
    packed, scales = _packed(31, N, K)
    w16 = dequantize_int4(packed, scales).cpu().numpy()
    g = torch.Generator().manual_seed(32)
    x = torch.randn(64, K, generator=g).half()
    xd = x.to(DEV)
    streams = [torch.cuda.Stream(device=DEV) for _ in range(20)]
    outs = []
    for st in streams:
        with torch.cuda.stream(st):
            outs.append(int4_matmul(xd, (packed, scales)))
        st.synchronize()
    for out in outs:
        _check(out, x.numpy(), w16)
