"""ctypes binding of ``libfastinfer_hip.so`` (the C ABI in ``include/fast_infer_amd.h``).

The library is loaded lazily, after ``torch`` so that the HIP runtime torch already
loaded (same soname ``libamdhip64.so.7``) is the one the library binds to.  There is
no fallback: if the library is missing or cannot be loaded, every operation raises.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must be imported before the HIP library is loaded)

LIB_PATH = Path(__file__).resolve().parent / "libfastinfer_hip.so"

FI_OK = 0
FI_ERR_INVALID = 1
FI_ERR_UNSUPPORTED = 2
FI_ERR_HIP = 3
FI_ERR_WORKSPACE = 4

_ERROR_NAMES = {
    FI_ERR_INVALID: "FI_ERR_INVALID",
    FI_ERR_UNSUPPORTED: "FI_ERR_UNSUPPORTED",
    FI_ERR_HIP: "FI_ERR_HIP",
    FI_ERR_WORKSPACE: "FI_ERR_WORKSPACE",
}

_i64 = ctypes.c_int64
_ptr = ctypes.c_void_p
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/fast_infer_amd.h
SIGNATURES = {
    "fi_version": (ctypes.c_int, []),
    "fi_last_error": (ctypes.c_char_p, []),
    "fi_flash_attention_fwd": (
        ctypes.c_int,
        [_ptr, _ptr, _ptr, _ptr,                 # q k v o
         _i64, _i64, _i64, _i64, _i64,           # batch Hq Hkv seq D
         _i64, _i64, _i64, _i64, _i64, _i64,     # q / k strides
         _i64, _i64, _i64, _i64, _i64, _i64,     # v / o strides
         _f32,                                   # sm_scale
         _ptr, _ptr, _i64, _i64, _ptr, _i64, _i64,  # pool write
         _ptr],                                  # stream
    ),
    "fi_paged_attention_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64]),
    "fi_paged_attention_fwd": (
        ctypes.c_int,
        [_ptr, _i64, _i64,                       # q, strides
         _ptr, _ptr, _i64, _i64, _i64,           # pools, N, block_size, Hkv
         _ptr, _i64, _i64,                       # block table, stride, max blocks
         _ptr, _i64,                             # context_lens, num_tokens
         _ptr, _i64, _i64,                       # o, strides
         _i64, _i64, _i64,                       # batch Hq D
         _f32,                                   # sm_scale
         _ptr, _sz,                              # workspace
         _ptr],                                  # stream
    ),
    "fi_paged_attention_fwd_noalloc": (
        ctypes.c_int,
        [_ptr, _i64, _i64,                       # q, strides
         _ptr, _ptr, _i64, _i64, _i64,           # pools, N, block_size, Hkv
         _ptr, _i64, _i64,                       # block table, stride, max blocks
         _ptr, _i64,                             # context_lens, num_tokens
         _ptr, _i64, _i64,                       # o, strides
         _i64, _i64, _i64,                       # batch Hq D
         _f32,                                   # sm_scale
         _ptr],                                  # stream
    ),
    "fi_kv_store": (
        ctypes.c_int,
        [_ptr, _i64, _i64, _i64,
         _ptr, _i64, _i64, _i64,
         _ptr, _ptr, _i64, _i64, _i64, _i64,
         _ptr, _i64, _i64,
         _i64, _i64, _i64, _ptr,
         _ptr],
    ),
    "fi_rope_store_kv": (
        ctypes.c_int,
        [_ptr, _i64, _i64, _i64,                 # q, strides
         _ptr, _i64, _i64, _i64,                 # k, strides
         _ptr, _i64, _i64, _i64,                 # v, strides
         _ptr, _ptr, _i64,                       # cos, sin, table rows
         _ptr, _i64, _i64, _i64,                 # q_out, strides
         _ptr, _i64, _i64, _i64,                 # k_out, strides
         _ptr, _ptr, _i64, _i64,                 # pools, N, block_size
         _ptr, _i64, _i64,                       # block table, stride, max blocks
         _i64, _i64, _i64, _i64, _i64,           # batch, tokens, Hq, Hkv, D
         _i64, _ptr,                             # start_pos, start_pos_per_seq
         _ptr],                                  # stream
    ),
    "fi_kv_append": (
        ctypes.c_int,
        [_ptr, _i64, _i64,                       # block table, stride, max blocks
         _ptr, _ptr, _ptr, _ptr,                 # num_alloc, seq_lens, free_queue, state
         _i64, _i64, _i64,                       # num_blocks, block_size, batch
         _ptr, _i64,                             # num_new (per row), num_new_all
         _ptr, _ptr,                             # start_pos_out, context_lens_out
         _ptr],                                  # stream
    ),
    "fi_kv_release": (
        ctypes.c_int,
        [_ptr, _i64, _i64, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _ptr, _ptr],
    ),
    "fi_kv_reset": (
        ctypes.c_int,
        [_ptr, _i64, _i64, _i64, _ptr, _ptr, _ptr, _ptr, _i64, _ptr],
    ),
    "fi_int4_matmul_workspace_size": (_sz, [_i64, _i64, _i64]),
    "fi_int4_matmul": (
        ctypes.c_int,
        [_ptr, _i64, _i64, _i64,                 # x, stride, M, K
         _ptr, _i64, _ptr, _i64,                 # w, stride, scales, stride
         _i64, _i64,                             # N, groupsize
         _ptr, _i64,                             # out, stride
         _ptr, _sz,                              # workspace
         _ptr],                                  # stream
    ),
    "fi_int4_quantize": (
        ctypes.c_int, [_ptr, _i64, _i64, _i64, _i64, _ptr, _i64, _ptr, _i64, _ptr],
    ),
    "fi_int4_dequantize": (
        ctypes.c_int, [_ptr, _i64, _ptr, _i64, _i64, _i64, _i64, _ptr, _i64, _ptr],
    ),
    "fi_rmsnorm": (ctypes.c_int, [_ptr, _i64, _i64, _i64, _ptr, _f32, _ptr, _i64, _ptr]),
    "fi_rmsnorm_int4_matmul_workspace_size": (_sz, [_i64, _i64, _i64]),
    "fi_rmsnorm_int4_matmul": (
        ctypes.c_int,
        [_ptr, _i64, _i64, _i64,                 # x, stride, M, K
         _ptr, _f32,                             # norm weight, eps
         _ptr, _i64, _ptr, _i64,                 # w, stride, scales, stride
         _i64, _i64,                             # N, groupsize
         _ptr, _i64,                             # out, stride
         _ptr, _sz,                              # workspace
         _ptr],                                  # stream
    ),
    "fi_selftest_mfma_f16": (ctypes.c_int, [_ptr, _ptr, _ptr, _ptr]),
}

# status words of the device block manager (state[2])
FI_KV_OK = 0
FI_KV_OUT_OF_BLOCKS = 1
FI_KV_TABLE_FULL = 2
FI_KV_NEGATIVE_COUNT = 3

_lib = None
_lock = threading.Lock()


class FastInferError(RuntimeError):
    """Raised when a fast_infer_amd C-ABI call returns an error code."""


def load() -> ctypes.CDLL:
    """Load the HIP library once and declare every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise FastInferError(
                f"{LIB_PATH.name} is not built; run `python -m fast_infer_amd.build` "
                "(or __graft_entry__.build()) first")
        lib = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_LOCAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != FI_OK:
        msg = load().fi_last_error().decode(errors="replace")
        raise FastInferError(f"{what} failed ({_ERROR_NAMES.get(rc, rc)}): {msg}")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device` (the raw-handle query skips
    building a Stream object: a few microseconds per call on the decode path)."""
    if _raw_stream is not None:
        index = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(index)
    return torch.cuda.current_stream(device).cuda_stream


def tensor_stream(t: torch.Tensor) -> int:
    """hipStream_t of torch's current stream on the device of the HIP tensor `t` (its
    device index read as an int: no torch.device object is built)."""
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


# Workspace sizes depend only on the integer sizes of a call: each distinct query is made
# once.  The wrappers make them on every call, so this saves a foreign call per launch.
_size_cache: dict[tuple, int] = {}


def workspace_size(name: str, *sizes: int) -> int:
    key = (name, sizes)
    n = _size_cache.get(key)
    if n is None:
        n = getattr(load(), name)(*sizes)
        if len(_size_cache) > 4096:
            _size_cache.clear()
        _size_cache[key] = n
    return n
