"""The C-ABI library loads and exports every entry point of include/fast_infer_amd.h.

CPU only: no call here launches a kernel.  The calls made return from argument
validation before any HIP API is used, and check the error codes and messages.
"""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "fast_infer_amd.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fi_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from fast_infer_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} is not built (run __graft_entry__.build())")
    return _lib.load()


def test_header_declares_entry_points():
    names = _declared()
    for n in ("fi_flash_attention_fwd", "fi_paged_attention_fwd", "fi_kv_store",
              "fi_rope_store_kv", "fi_kv_append", "fi_kv_release", "fi_kv_reset",
              "fi_int4_matmul", "fi_int4_matmul_workspace_size", "fi_int4_quantize",
              "fi_int4_dequantize", "fi_rmsnorm", "fi_rmsnorm_int4_matmul",
              "fi_rmsnorm_int4_matmul_workspace_size",
              "fi_paged_attention_workspace_size", "fi_last_error", "fi_version"):
        assert n in names


def test_library_exports_every_declared_symbol(lib):
    from fast_infer_amd import _lib

    for name in _declared():
        assert hasattr(lib, name), f"{name} missing from {_lib.LIB_PATH.name}"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    fi_exported = {s for s in exported if s.startswith("fi_")}
    assert fi_exported == set(_declared()), "exports differ from the header"


def test_version_and_empty_error(lib):
    assert lib.fi_version() == 100
    assert lib.fi_last_error() == b""


def test_unsupported_head_dim(lib):
    """head_dim must be a multiple of 8 up to 128 for the attention kernels (a multiple of
    8 for the KV scatter, of 16 for RoPE); the check comes before any other."""
    from fast_infer_amd import _lib

    for d in (60, 136):
        rc = lib.fi_paged_attention_fwd(8, 0, 0, 16, 16, 1, 64, 1, 16, 1, 1, None, 1, 32, 0, 0,
                                        1, 1, d, 1.0, None, 0, None)
        assert rc == _lib.FI_ERR_UNSUPPORTED
        assert f"head_dim {d}".encode() in lib.fi_last_error()
        rc = lib.fi_flash_attention_fwd(16, 16, 16, 16, 1, 1, 1, 1, d, *([8] * 12), 1.0,
                                        None, None, 0, 64, None, 0, 0, None)
        assert rc == _lib.FI_ERR_UNSUPPORTED
        assert lib.fi_paged_attention_workspace_size(4, 8, 8, 4096, d) == 0
    rc = lib.fi_kv_store(16, 8, 8, 8, 16, 8, 8, 8, 16, 16, 1, 64, 1, 12, 16, 1, 1, 1, 1, 0,
                         None, None)
    assert rc == _lib.FI_ERR_UNSUPPORTED
    assert lib.fi_paged_attention_workspace_size(4, 8, 8, 4096, 64) > 0


def test_invalid_arguments(lib):
    from fast_infer_amd import _lib

    # heads not divisible
    rc = lib.fi_flash_attention_fwd(16, 16, 16, 16, 1, 6, 4, 8, 128, *([8] * 12), 1.0,
                                    None, None, 0, 64, None, 0, 0, None)
    assert rc == _lib.FI_ERR_INVALID
    # misaligned q pointer
    rc = lib.fi_flash_attention_fwd(18, 16, 16, 16, 1, 8, 8, 8, 128, *([8] * 12), 1.0,
                                    None, None, 0, 64, None, 0, 0, None)
    assert rc == _lib.FI_ERR_INVALID and b"aligned" in lib.fi_last_error()
    # fused pool write with block size 0
    rc = lib.fi_flash_attention_fwd(16, 16, 16, 16, 1, 8, 8, 8, 128, *([8] * 12), 1.0,
                                    32, 32, 4, 0, 64, 4, 4, None)
    assert rc == _lib.FI_ERR_INVALID and b"block_size" in lib.fi_last_error()
    # decode block size 0
    rc = lib.fi_paged_attention_fwd(16, 8, 8, 16, 16, 1, 0, 1, 16, 1, 1, None, 1, 32, 8, 8,
                                    1, 1, 128, 1.0, None, 0, None)
    assert rc == _lib.FI_ERR_INVALID
    # block size 1 with partitions whose table entries would not fit the staging area
    rc = lib.fi_paged_attention_fwd(16, 8, 8, 16, 16, 1, 1, 1, 16, 1, 1, None, 4_000_000, 32,
                                    8, 8, 1, 1, 128, 1.0, None, 0, None)
    assert rc == _lib.FI_ERR_UNSUPPORTED and b"block_size 1" in lib.fi_last_error()
    # null pools
    rc = lib.fi_kv_store(16, 8, 8, 8, 16, 8, 8, 8, None, None, 1, 64, 1, 128, 16, 1, 1, 1, 1,
                         0, None, None)
    assert rc == _lib.FI_ERR_INVALID


def test_empty_calls_are_noops(lib):
    from fast_infer_amd import _lib

    assert lib.fi_flash_attention_fwd(None, None, None, None, 0, 8, 8, 8, 128, *([8] * 12),
                                      1.0, None, None, 0, 64, None, 0, 0, None) == _lib.FI_OK
    assert lib.fi_kv_store(None, 8, 8, 8, None, 8, 8, 8, None, None, 1, 64, 1, 128, None, 1,
                           1, 0, 5, 0, None, None) == _lib.FI_OK


def _rope_args(**kw):
    """fi_rope_store_kv's 38 arguments, all valid and 16-byte aligned, with overrides."""
    a = dict(q=16, q_sb=8, q_st=8, q_sh=8, k=16, k_sb=8, k_st=8, k_sh=8, v=16, v_sb=8, v_st=8,
             v_sh=8, cos=16, sin=16, rows=64, q_out=16, qo_sb=8, qo_st=8, qo_sh=8, k_out=16,
             ko_sb=8, ko_st=8, ko_sh=8, k_cache=16, v_cache=16, pool_blocks=4, block_size=64,
             table=16, bt_stride=4, max_blocks=4, batch=1, tokens=1, hq=8, hkv=8, head_dim=128,
             start=0, starts=None, stream=None)
    a.update(kw)
    return list(a.values())


def test_rope_store_kv_validation(lib):
    from fast_infer_amd import _lib

    assert lib.fi_rope_store_kv(*_rope_args(head_dim=72)) == _lib.FI_ERR_UNSUPPORTED
    assert b"head_dim 72" in lib.fi_last_error()
    assert lib.fi_rope_store_kv(*_rope_args(q=18)) == _lib.FI_ERR_INVALID
    assert b"aligned" in lib.fi_last_error()
    assert lib.fi_rope_store_kv(*_rope_args(k_st=12)) == _lib.FI_ERR_INVALID
    assert lib.fi_rope_store_kv(*_rope_args(v=None)) == _lib.FI_ERR_INVALID
    assert b"null" in lib.fi_last_error()
    assert lib.fi_rope_store_kv(*_rope_args(block_size=0)) == _lib.FI_ERR_INVALID
    assert lib.fi_rope_store_kv(*_rope_args(tokens=-1)) == _lib.FI_ERR_INVALID
    # empty calls return before touching any pointer
    assert lib.fi_rope_store_kv(*_rope_args(batch=0, q=None, k=None)) == _lib.FI_OK
    assert lib.fi_rope_store_kv(*_rope_args(tokens=0)) == _lib.FI_OK


def test_block_manager_validation(lib):
    from fast_infer_amd import _lib

    st = (16, 16, 4, 16, 16, 16, 16)   # table, stride, max blocks, num_alloc, lens, queue, state
    assert lib.fi_kv_append(None, *st[1:], 8, 16, 1, None, 1, None, None, None) == \
        _lib.FI_ERR_INVALID
    assert b"null" in lib.fi_last_error()
    assert lib.fi_kv_append(*st, 0, 16, 1, None, 1, None, None, None) == _lib.FI_ERR_INVALID
    assert lib.fi_kv_append(*st, 8, 0, 1, None, 1, None, None, None) == _lib.FI_ERR_INVALID
    assert lib.fi_kv_append(*st, 8, 16, 1, None, -1, None, None, None) == _lib.FI_ERR_INVALID
    # max_blocks_per_seq larger than the table stride
    assert lib.fi_kv_append(16, 2, 4, 16, 16, 16, 16, 8, 16, 1, None, 1, None, None, None) == \
        _lib.FI_ERR_INVALID
    assert lib.fi_kv_release(*st, 8, 1, None, None) == _lib.FI_ERR_INVALID
    assert lib.fi_kv_reset(16, 16, 4, 2, 16, 16, 16, None, 8, None) == _lib.FI_ERR_INVALID
    # empty batches return before any launch
    assert lib.fi_kv_append(*st, 8, 16, 0, None, 1, None, None, None) == _lib.FI_OK
    assert lib.fi_kv_release(*st, 8, 0, None, None) == _lib.FI_OK


def test_int4_validation(lib):
    from fast_infer_amd import _lib

    # groupsize other than 128, K not a multiple of 128, misaligned rows, null pointers
    assert lib.fi_int4_matmul(16, 256, 1, 256, 16, 128, 16, 2, 64, 64, 16, 64, None, 0,
                              None) == _lib.FI_ERR_UNSUPPORTED
    assert b"groupsize 64" in lib.fi_last_error()
    assert lib.fi_int4_matmul(16, 200, 1, 200, 16, 112, 16, 2, 64, 128, 16, 64, None, 0,
                              None) == _lib.FI_ERR_UNSUPPORTED
    assert lib.fi_int4_matmul(18, 256, 1, 256, 16, 128, 16, 2, 64, 128, 16, 64, None, 0,
                              None) == _lib.FI_ERR_INVALID
    assert lib.fi_int4_matmul(None, 256, 1, 256, 16, 128, 16, 2, 64, 128, 16, 64, None, 0,
                              None) == _lib.FI_ERR_INVALID
    # decode-sized rows further apart than one 2^31-byte buffer descriptor covers
    assert lib.fi_int4_matmul(16, 1 << 30, 2, 256, 16, 128, 16, 2, 64, 128, 16, 64, None, 0,
                              None) == _lib.FI_ERR_UNSUPPORTED
    assert b"2^31" in lib.fi_last_error()
    # a split call without its workspace is rejected before launch
    need = lib.fi_int4_matmul_workspace_size(40, 5120, 3072)
    assert need > 0
    assert lib.fi_int4_matmul(16, 3072, 40, 3072, 16, 1536, 16, 24, 5120, 128, 16, 5120, None,
                              0, None) == _lib.FI_ERR_WORKSPACE
    # quantize / dequantize take power-of-two group sizes from 8 to 512
    assert lib.fi_int4_quantize(16, 256, 4, 256, 96, 16, 128, 16, 2, None) == \
        _lib.FI_ERR_UNSUPPORTED
    assert b"groupsize 96" in lib.fi_last_error()
    assert lib.fi_int4_dequantize(16, 128, 16, 4, 4, 256, 1024, 16, 256, None) == \
        _lib.FI_ERR_UNSUPPORTED
    # group size 64 is accepted; here the scale rows are too short for it (4 needed)
    assert lib.fi_int4_quantize(16, 256, 4, 256, 64, 16, 128, 16, 2, None) == \
        _lib.FI_ERR_INVALID
    assert lib.fi_int4_dequantize(16, 128, 16, 2, 4, 100, 128, 16, 256, None) == \
        _lib.FI_ERR_INVALID
    # empty calls return before any launch
    assert lib.fi_int4_matmul(16, 256, 0, 256, 16, 128, 16, 2, 64, 128, 16, 64, None, 0,
                              None) == _lib.FI_OK
    assert lib.fi_int4_quantize(16, 256, 0, 256, 128, 16, 128, 16, 2, None) == _lib.FI_OK


def test_rmsnorm_validation(lib):
    from fast_infer_amd import _lib

    assert lib.fi_rmsnorm(16, 100, 2, 100, 16, 1e-5, 16, 100, None) == _lib.FI_ERR_UNSUPPORTED
    assert lib.fi_rmsnorm(18, 256, 2, 256, 16, 1e-5, 16, 256, None) == _lib.FI_ERR_INVALID
    assert lib.fi_rmsnorm(None, 256, 2, 256, 16, 1e-5, 16, 256, None) == _lib.FI_ERR_INVALID
    assert lib.fi_rmsnorm(16, 256, 0, 256, 16, 1e-5, 16, 256, None) == _lib.FI_OK
    # fused: norm weight missing, misaligned, or the separate-pass workspace missing
    assert lib.fi_rmsnorm_int4_matmul(16, 3072, 1, 3072, None, 1e-5, 16, 1536, 16, 24, 5120,
                                      128, 16, 5120, None, 0, None) == _lib.FI_ERR_INVALID
    assert lib.fi_rmsnorm_int4_matmul(16, 3072, 1, 3072, 24, 1e-5, 16, 1536, 16, 24, 5120,
                                      128, 16, 5120, None, 0, None) == _lib.FI_ERR_INVALID
    assert lib.fi_rmsnorm_int4_matmul_workspace_size(1, 5120, 3072) == 0
    need = lib.fi_rmsnorm_int4_matmul_workspace_size(64, 5120, 3072)
    assert need >= 64 * 3072 * 2
    assert lib.fi_rmsnorm_int4_matmul(16, 3072, 64, 3072, 16, 1e-5, 16, 1536, 16, 24, 5120,
                                      128, 16, 5120, None, 0, None) == _lib.FI_ERR_WORKSPACE


def test_workspace_size(lib):
    # one partition (no workspace) for short contexts, partials for long ones
    assert lib.fi_paged_attention_workspace_size(1, 24, 8, 256, 128) == 0
    n = lib.fi_paged_attention_workspace_size(32, 24, 8, 4096, 128)
    assert n > 0 and n % (32 * 24 * 130 * 4) == 0
    # partials stay 128 columns wide for any supported head_dim; unsupported ones need none
    assert lib.fi_paged_attention_workspace_size(32, 24, 8, 4096, 64) == n
    assert lib.fi_paged_attention_workspace_size(32, 24, 8, 4096, 136) == 0
    rc = lib.fi_paged_attention_fwd(16, 3072, 128, 16, 16, 2048, 64, 8, 16, 64, 64, None,
                                    4096, 32, 3072, 128, 32, 24, 128, 1.0, None, 0, None)
    from fast_infer_amd import _lib

    assert rc == _lib.FI_ERR_WORKSPACE
    assert ctypes.c_size_t(n).value == n
