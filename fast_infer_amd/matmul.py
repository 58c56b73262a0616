"""INT4 group-quantized linear layers (kernels/matmul.py, loader.py:9-41) on gfx950.

``int4_matmul(x, w, scales=None, groupsize=128)`` keeps the reference's signature
(kernels/matmul.py:217-231): ``w`` is either a ``(packed_int8, scales)`` tuple — the
dequantization then runs inside the MFMA loop — or an fp16 ``[N, K]`` weight.
``quantize_int4_groupwise`` (loader.py:9-41) and ``dequantize_int4`` (the reference's
``_dequant_storage``, matmul.py:309-326) produce and expand the same wire format, bit for
bit.  ``rms_norm`` is kernels/rms_norm.py's; ``rms_norm_int4_matmul`` is the norm of
model.py:82 and the projection after it in one call.
"""

from __future__ import annotations

import warnings

import torch

from . import _lib

PACKED_GROUP = 128  # the group size the packed-weight kernels read (the reference's)


# These wrappers run once per projection and decode step, where their host time is of the
# order of the kernels': each tensor's shape, strides and pointer are read once, dtypes
# compared by identity, devices checked with is_cuda, and workspace sizes cached.

def _need_cuda(name: str, t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be on a HIP device; fast_infer_amd has no CPU path")


def _rows16(t: torch.Tensor, elem: int) -> tuple[torch.Tensor, int, int]:
    """(t with unit inner stride, 16-byte aligned rows and row stride a multiple of 16 B,
    its row stride, its pointer) for a 2-D t."""
    (s0, s1), ptr = t.stride(), t.data_ptr()
    if s1 != 1 or ptr % 16 or (s0 * elem) % 16 or s0 < t.shape[1]:
        t = t.contiguous()
        s0, ptr = t.stride(0), t.data_ptr()
        if ptr % 16 or (s0 * elem) % 16:
            raise ValueError("rows must be 16-byte aligned (K a multiple of 8 elements)")
    return t, s0, ptr


def _norm_weight(w: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """An RMSNorm weight as a contiguous fp16 tensor on x's device."""
    if w.dtype is not torch.float16 or w.get_device() != x.get_device():
        w = w.to(device=x.device, dtype=torch.float16)
    return w if w.is_contiguous() else w.contiguous()


# Split-K calls need a workspace for their fp32 partials; one per (device, stream), grown
# on demand, so back-to-back calls on a stream reuse it.  A buffer that is outgrown is
# kept alive, never returned to the allocator: a HIP graph captured earlier may hold its
# address (graphs captured on one stream share the key), and replaying that graph must
# not write into memory that was handed out again.
_workspaces: dict[tuple[int, int], torch.Tensor] = {}
_outgrown: list[torch.Tensor] = []


def _workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _outgrown.append(ws)
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


def int4_matmul(x: torch.Tensor, w, scales=None, groupsize: int = 128, *,
                workspace: torch.Tensor | None = None) -> torch.Tensor:
    """fp16 ``x [..., K]`` times a weight ``[N, K]`` -> fp16 ``[..., N]``
    (kernels/matmul.py:217-231).  ``w`` is ``(packed int8 [N, K/2], scales fp16 [N,
    K/groupsize])`` or an fp16 ``[N, K]`` tensor; ``scales`` is ignored as in the
    reference.  Accumulation is fp32, the output rounded to fp16 once.  ``workspace``
    (optional) must not be shared by calls that overlap in time; by default one cached
    workspace per device and stream is used.  The packed kernels read 128-wide groups (the
    reference's); packed weights with another group size are dequantized first (the same
    fp16 values) and take the fp16 form."""
    _need_cuda("x", x)
    w = _other_group_size(w, groupsize)
    N, K, w_ptr, w_stride, s_ptr, s_stride, _keep = _weight_args(w, groupsize)
    x_shape = x.shape
    if x_shape[-1] != K:
        raise ValueError(f"x has K = {x_shape[-1]}, the weight K = {K}")
    if K % groupsize:
        raise ValueError(f"K ({K}) must be multiple of groupsize ({groupsize})")
    if x.dtype is not torch.float16:
        x = x.to(torch.float16)
    x2, x_stride, x_ptr = _rows16(x if len(x_shape) == 2 else x.reshape(-1, K), 2)
    M = x2.shape[0]
    out = torch.empty(M, N, dtype=torch.float16, device=x.device)
    if M == 0 or N == 0:
        return out if len(x_shape) == 2 else out.reshape(*x_shape[:-1], N)
    stream = _lib.tensor_stream(x)
    need = _lib.workspace_size("fi_int4_matmul_workspace_size", M, N, K)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = _workspace(x.device, stream, need)
    ws_ptr = workspace.data_ptr() if need else None
    ws_bytes = workspace.numel() * workspace.element_size() if need else 0
    rc = _lib.load().fi_int4_matmul(x_ptr, x_stride, M, K, w_ptr, w_stride, s_ptr, s_stride, N,
                                    groupsize, out.data_ptr(), N, ws_ptr, ws_bytes, stream)
    _lib.check(rc, "int4_matmul")
    return out if len(x_shape) == 2 else out.reshape(*x_shape[:-1], N)


_warned_group_sizes: set[int] = set()


def _other_group_size(w, groupsize: int):
    """Packed weights whose group size is not 128 as the dequantized fp16 tensor.

    This costs every call a full dequantization: N x K fp16 written and read back, about
    4.5 times the packed weight's bytes.  Callers with such weights should dequantize once
    (``dequantize_int4``) and pass the fp16 weight; the first such call per group size
    warns."""
    if isinstance(w, tuple) and groupsize != PACKED_GROUP:
        if groupsize not in _warned_group_sizes:
            _warned_group_sizes.add(groupsize)
            warnings.warn(
                f"int4_matmul: packed weights with groupsize {groupsize} are dequantized on "
                f"every call (the packed kernels take groupsize {PACKED_GROUP}); dequantize "
                f"once with dequantize_int4 and pass the fp16 weight instead",
                RuntimeWarning, stacklevel=3)
        return dequantize_int4(w[0], w[1], groupsize)
    return w


def _weight_args(w, groupsize: int):
    """(N, K, weight pointer, its row stride, scales pointer, scales row stride, the
    tensors those pointers are into, kept alive for the call) for either weight form."""
    if isinstance(w, tuple):
        packed, sc = w
        _need_cuda("packed", packed)
        p_dtype = packed.dtype
        if (p_dtype is not torch.int8 and p_dtype is not torch.uint8) or packed.dim() != 2:
            raise TypeError("packed weights must be a 2-D int8 tensor")
        if sc.dtype is not torch.float16 or sc.dim() != 2:
            raise TypeError("scales must be a 2-D float16 tensor")
        N, half_k = packed.shape
        K = half_k * 2
        sc_rows, sc_cols = sc.shape
        if sc_rows != N or sc_cols * groupsize != K:
            raise ValueError(f"scales {tuple(sc.shape)} do not match packed {tuple(packed.shape)}")
        wt, w_stride, w_ptr = _rows16(packed, 1)
        sc_st = sc.stride()
        if sc_st[1] != 1:
            sc = sc.contiguous()
            sc_st = sc.stride()
        return N, K, w_ptr, w_stride, sc.data_ptr(), sc_st[0], (wt, sc)
    _need_cuda("w", w)
    if w.dtype is not torch.float16 or w.dim() != 2:
        raise TypeError("w must be a 2-D float16 tensor or a (packed, scales) tuple")
    N, K = w.shape
    wt, w_stride, w_ptr = _rows16(w, 2)
    return N, K, w_ptr, w_stride, None, 0, wt


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """kernels/rms_norm.py:29-43: ``x * rsqrt(mean(x^2) + eps) * weight`` in fp32, fp16
    out, over the last dimension of ``x [..., hidden]``."""
    _need_cuda("x", x)
    hidden = x.shape[-1]
    if weight.shape != (hidden,):
        raise ValueError(f"weight {tuple(weight.shape)} does not match hidden {hidden}")
    if x.dtype is not torch.float16:
        x = x.to(torch.float16)
    wt = _norm_weight(weight, x)
    x2, x_stride, x_ptr = _rows16(x.reshape(-1, hidden), 2)
    rows = x2.shape[0]
    out = torch.empty(rows, hidden, dtype=torch.float16, device=x.device)
    if rows:
        rc = _lib.load().fi_rmsnorm(x_ptr, x_stride, rows, hidden, wt.data_ptr(), float(eps),
                                    out.data_ptr(), hidden, _lib.tensor_stream(x))
        _lib.check(rc, "rms_norm")
    return out.reshape(x.shape)


def rms_norm_int4_matmul(x: torch.Tensor, norm_weight: torch.Tensor, w, eps: float = 1e-5,
                         groupsize: int = 128, *,
                         workspace: torch.Tensor | None = None) -> torch.Tensor:
    """``int4_matmul(rms_norm(x, norm_weight, eps), w)`` in one call (model.py:82 and the
    QKV projection after it): for few rows the norm is applied inside the GEMM.  Packed
    weights with a group size other than 128 take the fp16 form, as in ``int4_matmul``."""
    _need_cuda("x", x)
    w = _other_group_size(w, groupsize)
    N, K, w_ptr, w_stride, s_ptr, s_stride, _keep = _weight_args(w, groupsize)
    x_shape = x.shape
    if x_shape[-1] != K or norm_weight.shape != (K,):
        raise ValueError(f"x {tuple(x_shape)} / norm weight {tuple(norm_weight.shape)} do not "
                         f"match K = {K}")
    if K % groupsize:
        raise ValueError(f"K ({K}) must be multiple of groupsize ({groupsize})")
    if x.dtype is not torch.float16:
        x = x.to(torch.float16)
    nw = _norm_weight(norm_weight, x)
    x2, x_stride, x_ptr = _rows16(x if len(x_shape) == 2 else x.reshape(-1, K), 2)
    M = x2.shape[0]
    out = torch.empty(M, N, dtype=torch.float16, device=x.device)
    if M == 0 or N == 0:
        return out if len(x_shape) == 2 else out.reshape(*x_shape[:-1], N)
    stream = _lib.tensor_stream(x)
    need = _lib.workspace_size("fi_rmsnorm_int4_matmul_workspace_size", M, N, K)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = _workspace(x.device, stream, need)
    ws_ptr = workspace.data_ptr() if need else None
    ws_bytes = workspace.numel() * workspace.element_size() if need else 0
    rc = _lib.load().fi_rmsnorm_int4_matmul(x_ptr, x_stride, M, K, nw.data_ptr(), float(eps),
                                            w_ptr, w_stride, s_ptr, s_stride, N, groupsize,
                                            out.data_ptr(), N, ws_ptr, ws_bytes, stream)
    _lib.check(rc, "rms_norm_int4_matmul")
    return out if len(x_shape) == 2 else out.reshape(*x_shape[:-1], N)


def quantize_int4_groupwise(w: torch.Tensor, groupsize: int = 128
                            ) -> tuple[torch.Tensor, torch.Tensor]:
    """loader.py:9-41: fp16 ``w [N, K]`` -> (packed int8 ``[N, K/2]``, scales fp16
    ``[N, K/groupsize]``), bit-exact with the reference's arithmetic on a CUDA device;
    ``groupsize`` a power of two from 8 to 512."""
    _need_cuda("w", w)
    if w.dtype != torch.float16 or w.dim() != 2:
        raise TypeError("w must be a 2-D float16 tensor")
    N, K = w.shape
    if K % groupsize:
        raise ValueError(f"K ({K}) must be multiple of groupsize ({groupsize})")
    wt, w_stride, w_ptr = _rows16(w, 2)
    packed = torch.empty(N, K // 2, dtype=torch.int8, device=w.device)
    scales = torch.empty(N, K // groupsize, dtype=torch.float16, device=w.device)
    lib = _lib.load()
    rc = lib.fi_int4_quantize(w_ptr, w_stride, N, K, groupsize, packed.data_ptr(),
                              packed.stride(0), scales.data_ptr(), scales.stride(0),
                              _lib.stream_handle(w.device))
    _lib.check(rc, "quantize_int4_groupwise")
    return packed, scales


def dequantize_int4(packed: torch.Tensor, scales: torch.Tensor,
                    groupsize: int = 128) -> torch.Tensor:
    """kernels/matmul.py:309-326 (``_dequant_storage``): -> fp16 ``[N, K]``, each weight
    fp16(q * scale)."""
    _need_cuda("packed", packed)
    N, K = packed.shape[0], packed.shape[1] * 2
    if scales.shape != (N, K // groupsize):
        raise ValueError(f"scales {tuple(scales.shape)} do not match packed {tuple(packed.shape)}")
    pk = packed if packed.is_contiguous() else packed.contiguous()
    sc = scales if scales.is_contiguous() else scales.contiguous()
    w = torch.empty(N, K, dtype=torch.float16, device=packed.device)
    lib = _lib.load()
    rc = lib.fi_int4_dequantize(pk.data_ptr(), pk.stride(0), sc.data_ptr(), sc.stride(0), N, K,
                                groupsize, w.data_ptr(), w.stride(0),
                                _lib.stream_handle(packed.device))
    _lib.check(rc, "dequantize_int4")
    return w
