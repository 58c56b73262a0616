"""Prefill flash-attention and paged-attention decode on MI355X (drop-in for
``kernels/attention.py``).

Both functions keep the reference's names, positional parameters, defaults, output
allocation (``torch.empty_like(q)``) and the ``num_tokens == 0`` short-circuit.  The
work is done by the hand-written gfx950 kernels in ``csrc/`` behind the C ABI; there
is no other execution path.  Keyword-only extensions, all defaulting to the
reference behaviour:

* ``flash_attention(..., k_cache=, v_cache=, block_table=, block_size=64)`` — also
  write K/V into the paged pool in the same pass (the copy of model.py:176-183).
* ``flash_attention`` accepts ``k``/``v`` with fewer heads than ``q`` (GQA); query
  head ``h`` reads kv head ``h // (H / H_kv)`` — what the reference's expanded call
  (model.py:110-111) computes, without materialising the expansion.
* ``paged_attention(..., context_lens=)`` — per-row context lengths (the reference
  has one shared ``num_tokens``); ``num_tokens`` may also be given as an int32
  tensor of per-row lengths.
"""

from __future__ import annotations

import torch

from . import _lib


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# The wrappers below run once per kernel launch; on the decode path their host time is of
# the order of the GPU time, so they read each tensor's strides and pointer once, compare
# dtypes by identity and devices by index (no torch.device objects).

def _strides_ok(st: tuple, ptr: int) -> bool:
    """Innermost dim contiguous, other strides multiples of 8, 16-byte aligned base."""
    if st[-1] != 1 or ptr % 16:
        return False
    for x in st[:-1]:
        if x % 8:
            return False
    return True


def _rows_ok(t: torch.Tensor) -> bool:
    return _strides_ok(t.stride(), t.data_ptr())


def _prep_rows(t: torch.Tensor) -> tuple[torch.Tensor, tuple, int]:
    """(t or a contiguous copy, its strides, its pointer) with rows the kernels can read."""
    st, ptr = t.stride(), t.data_ptr()
    if not _strides_ok(st, ptr):
        t = t.contiguous()
        st, ptr = t.stride(), t.data_ptr()
    return t, st, ptr


def _check_fp16_cuda(name: str, t: torch.Tensor) -> None:
    if t.dtype is not torch.float16:
        raise TypeError(f"{name} must be float16, got {t.dtype}")
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be on a HIP device (got {t.device}); "
                           "fast_infer_amd has no CPU path")


def _check_table(block_table: torch.Tensor, dev: int) -> torch.Tensor:
    """block_table validated against the device index `dev` of q."""
    if block_table.dtype is not torch.int32:
        raise TypeError(f"block_table must be int32, got {block_table.dtype}")
    if block_table.get_device() != dev:
        raise RuntimeError("block_table must be on the same device as q")
    if block_table.dim() != 2:
        raise ValueError("block_table must be [batch, max_blocks_per_seq]")
    if block_table.stride(-1) != 1:
        block_table = block_table.contiguous()
    return block_table


def flash_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    sm_scale: float = None, *,
                    k_cache: torch.Tensor | None = None,
                    v_cache: torch.Tensor | None = None,
                    block_table: torch.Tensor | None = None,
                    block_size: int = 64) -> torch.Tensor:
    """Causal prefill attention (kernels/attention.py:80-113).

    q: [batch, num_heads, seq_len, head_dim] fp16; k, v: [batch, num_kv_heads,
    seq_len, head_dim] fp16 with num_heads % num_kv_heads == 0.  Returns o with
    q's shape and strides (``torch.empty_like(q)``, :99).  ``sm_scale`` defaults to
    head_dim ** -0.5 (:88-89).  With ``k_cache``/``v_cache`` ([num_blocks, block_size,
    num_kv_heads, head_dim], one layer of the pool) and ``block_table`` the K/V rows
    are also copied into the pool: token t of row b goes to block
    ``block_table[b, t // block_size]``, slot ``t % block_size``.
    """
    batch, num_heads, seq_len, head_dim = q.shape
    if sm_scale is None:
        sm_scale = head_dim ** -0.5
    for name, t in (("q", q), ("k", k), ("v", v)):
        _check_fp16_cuda(name, t)
    if k.dim() != 4 or v.shape != k.shape:
        raise ValueError(f"k and v must share a [batch, kv_heads, seq, dim] shape, got "
                         f"{tuple(k.shape)} / {tuple(v.shape)}")
    if k.shape[0] != batch or k.shape[2] != seq_len or k.shape[3] != head_dim:
        raise ValueError(f"k/v shape {tuple(k.shape)} does not match q {tuple(q.shape)}")
    num_kv_heads = k.shape[1]
    if num_kv_heads == 0 or num_heads % num_kv_heads:
        raise ValueError(f"num_heads {num_heads} is not a multiple of kv heads {num_kv_heads}")
    o = torch.empty_like(q)  # q's strides (:99)
    q, qs, q_ptr = _prep_rows(q)
    k, ks, k_ptr = _prep_rows(k)
    v, vs, v_ptr = _prep_rows(v)
    # the kernel writes 16-byte rows; an output whose strides do not allow that is
    # computed into a contiguous buffer and copied into o at the end
    work = o if _rows_ok(o) else torch.empty(q.shape, dtype=q.dtype, device=q.device)
    ws_ = work.stride()

    kc = vc = bt = None
    n_pool = bt_stride = max_blocks = 0
    if k_cache is not None or v_cache is not None or block_table is not None:
        if k_cache is None or v_cache is None or block_table is None:
            raise ValueError("the fused pool write needs k_cache, v_cache and block_table")
        _check_fp16_cuda("k_cache", k_cache)
        _check_fp16_cuda("v_cache", v_cache)
        expect = (k_cache.shape[0], block_size, num_kv_heads, head_dim)
        if tuple(k_cache.shape) != expect or v_cache.shape != k_cache.shape:
            raise ValueError(f"pool shape {tuple(k_cache.shape)} != {expect}")
        if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
            raise ValueError("pools must be contiguous")
        bt = _check_table(block_table, q.get_device())
        if bt.shape[0] < batch:
            raise ValueError("block_table has fewer rows than the batch")
        kc, vc = k_cache, v_cache
        n_pool, bt_stride, max_blocks = k_cache.shape[0], bt.stride(0), bt.shape[1]

    if batch == 0 or seq_len == 0:
        return o
    lib = _lib.load()
    rc = lib.fi_flash_attention_fwd(
        q_ptr, k_ptr, v_ptr, work.data_ptr(),
        batch, num_heads, num_kv_heads, seq_len, head_dim,
        qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2],
        ws_[0], ws_[1], ws_[2],
        float(sm_scale),
        _ptr(kc), _ptr(vc), n_pool, block_size, _ptr(bt), bt_stride, max_blocks,
        _lib.tensor_stream(q))
    _lib.check(rc, "flash_attention")
    if work is not o:
        o.copy_(work)
    return o


def paged_attention_workspace(batch: int, num_q_heads: int, num_kv_heads: int,
                              num_tokens: int, head_dim: int, device) -> torch.Tensor | None:
    """Device scratch for the split-K partials of one paged_attention call (or None)."""
    nbytes = _lib.load().fi_paged_attention_workspace_size(
        batch, num_q_heads, num_kv_heads, num_tokens, head_dim)
    if nbytes == 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def paged_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                    block_table: torch.Tensor, block_size: int,
                    num_tokens,
                    sm_scale: float = None, *,
                    context_lens: torch.Tensor | None = None,
                    workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Paged-attention decode (kernels/attention.py:191-233).

    q: [batch, num_q_heads, head_dim] fp16; k_cache, v_cache: [num_blocks,
    block_size, num_kv_heads, head_dim] fp16; block_table: int32 [batch,
    max_blocks_per_seq], -1 = unused.  Every row attends to its first ``num_tokens``
    tokens, or to ``context_lens[b]`` tokens when per-row lengths are given (as
    ``context_lens=`` with ``num_tokens`` an upper bound, or as an int32 tensor in
    place of ``num_tokens``, bounded by the table width).  Returns
    ``torch.zeros_like(q)`` for ``num_tokens == 0`` (:205-206); rows of length 0
    give zeros.
    """
    if isinstance(num_tokens, torch.Tensor):
        if context_lens is not None:
            raise ValueError("give per-row lengths either as num_tokens or as context_lens")
        context_lens = num_tokens
        num_tokens = block_table.shape[1] * block_size
    num_tokens = int(num_tokens)
    if context_lens is None and num_tokens == 0:
        return torch.zeros_like(q)
    batch, num_q_heads, head_dim = q.shape
    if sm_scale is None:
        sm_scale = head_dim ** -0.5

    _check_fp16_cuda("q", q)
    _check_fp16_cuda("k_cache", k_cache)
    _check_fp16_cuda("v_cache", v_cache)
    pool_shape = k_cache.shape
    if len(pool_shape) != 4 or v_cache.shape != pool_shape:
        raise ValueError("k_cache/v_cache must be [num_blocks, block_size, kv_heads, dim]")
    num_blocks, pool_bs, num_kv_heads, pool_dim = pool_shape
    if pool_bs != block_size or pool_dim != head_dim:
        raise ValueError(f"pool shape {tuple(pool_shape)} does not match block_size "
                         f"{block_size} / head_dim {head_dim}")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("pools must be contiguous")
    if num_q_heads % num_kv_heads:
        raise ValueError(f"num_q_heads {num_q_heads} not a multiple of kv heads {num_kv_heads}")
    dev = q.get_device()
    block_table = _check_table(block_table, dev)
    bt_rows, bt_cols = block_table.shape
    if bt_rows < batch:
        raise ValueError("block_table has fewer rows than the batch")
    if context_lens is not None:
        if context_lens.dtype is not torch.int32 or context_lens.get_device() != dev:
            context_lens = context_lens.to(device=q.device, dtype=torch.int32)
        if context_lens.numel() < batch:
            raise ValueError("context_lens has fewer entries than the batch")
        if not context_lens.is_contiguous():
            context_lens = context_lens.contiguous()
    o = torch.empty_like(q)  # q's strides (:216)
    q, qs, q_ptr = _prep_rows(q)
    os_, o_ptr = o.stride(), o.data_ptr()
    if _strides_ok(os_, o_ptr):
        work = o
    else:
        work = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        os_, o_ptr = work.stride(), work.data_ptr()
    if batch == 0:
        return o

    lib = _lib.load()
    need = _lib.workspace_size("fi_paged_attention_workspace_size", batch, num_q_heads,
                               num_kv_heads, max(num_tokens, 1), head_dim)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    ws_ptr = workspace.data_ptr() if (need and workspace is not None) else None
    ws_bytes = workspace.numel() * workspace.element_size() if ws_ptr else 0
    rc = lib.fi_paged_attention_fwd(
        q_ptr, qs[0], qs[1],
        k_cache.data_ptr(), v_cache.data_ptr(), num_blocks, block_size, num_kv_heads,
        block_table.data_ptr(), block_table.stride(0), bt_cols,
        _ptr(context_lens), num_tokens,
        o_ptr, os_[0], os_[1],
        batch, num_q_heads, head_dim, float(sm_scale),
        ws_ptr, ws_bytes,
        _lib.tensor_stream(q))
    _lib.check(rc, "paged_attention")
    if work is not o:
        o.copy_(work)
    return o
