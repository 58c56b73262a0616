"""Host-side checks of the Python wrappers, on the CPU (no GPU needed).

The wrappers validate their operands before any device work: CPU tensors are rejected (there
is no CPU path) and dtypes are checked, with the same exceptions as the reference's call
sites would see.  Their stride/alignment helpers and the cached workspace-size queries are
pure host logic and are checked against direct computations.
"""

import pytest
import torch

import fast_infer_amd as fi
from fast_infer_amd import _lib, attention, matmul, rope


def _cpu(*shape, dtype=torch.float16):
    return torch.zeros(*shape, dtype=dtype)


def test_attention_wrappers_reject_cpu_and_dtype():
    q, k, v = _cpu(1, 3, 64, 128), _cpu(1, 1, 64, 128), _cpu(1, 1, 64, 128)
    with pytest.raises(RuntimeError, match="HIP device"):
        fi.flash_attention(q, k, v)
    with pytest.raises(TypeError, match="float16"):
        fi.flash_attention(q.float(), k, v)
    pool = _cpu(4, 64, 1, 128)
    table = torch.zeros(1, 4, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="HIP device"):
        fi.paged_attention(_cpu(1, 3, 128), pool, pool, table, 64, 100)
    with pytest.raises(TypeError, match="float16"):
        fi.paged_attention(_cpu(1, 3, 128, dtype=torch.float32), pool, pool, table, 64, 100)
    # num_tokens == 0 short-circuits to zeros before any check (kernels/attention.py:205-206)
    z = fi.paged_attention(_cpu(1, 3, 128), pool, pool, table, 64, 0)
    assert z.shape == (1, 3, 128) and not z.any()


def test_rope_and_int4_wrappers_reject_cpu_and_dtype():
    q, k = _cpu(1, 2, 3, 128), _cpu(1, 2, 1, 128)
    cos = sin = _cpu(16, 128)
    with pytest.raises(RuntimeError, match="HIP device"):
        fi.rope_store_kv(q, k, None, cos, sin)
    with pytest.raises(TypeError, match="float16"):
        fi.rope_store_kv(q.float(), k, None, cos, sin)
    x, w = _cpu(2, 256), _cpu(64, 256)
    with pytest.raises(RuntimeError, match="HIP device"):
        fi.int4_matmul(x, w)
    with pytest.raises(RuntimeError, match="HIP device"):
        fi.rms_norm_int4_matmul(x, _cpu(256), w)


def test_row_helpers():
    t = torch.zeros(2, 3, 16, 128, dtype=torch.float16)
    assert attention._strides_ok(t.stride(), t.data_ptr())
    # a row stride that is not a multiple of 8 elements, or a base 2 bytes past alignment
    odd = torch.zeros(2, 3, 16, 130, dtype=torch.float16)[..., :128]
    assert not attention._strides_ok(odd.stride(), odd.data_ptr())
    flat = torch.zeros(4 * 128 + 8, dtype=torch.float16)
    shifted = flat[1:1 + 4 * 128].view(1, 1, 4, 128)
    assert not attention._strides_ok(shifted.stride(), shifted.data_ptr())
    # _prep_rows: strides and pointer of the tensor it returns, a copy only when needed
    same, st, ptr = attention._prep_rows(t)
    assert same is t and st == t.stride() and ptr == t.data_ptr()
    fixed, st, ptr = attention._prep_rows(odd)
    assert fixed.is_contiguous() and st == fixed.stride() and ptr == fixed.data_ptr()
    assert torch.equal(fixed, odd)
    r, st, ptr = rope._rows(odd)
    assert r.is_contiguous() and st == r.stride() and torch.equal(r, odd)
    # _rows16: 2-D, unit inner stride, 16-byte aligned rows
    m = torch.zeros(5, 256, dtype=torch.float16)
    out, s0, p0 = matmul._rows16(m, 2)
    assert out is m and s0 == 256 and p0 == m.data_ptr()
    strided = torch.zeros(5, 264, dtype=torch.float16)[:, 8:]
    out, s0, p0 = matmul._rows16(strided, 2)
    assert out is strided and s0 == 264
    bad = torch.zeros(5, 257, dtype=torch.float16)[:, 1:]
    out, s0, p0 = matmul._rows16(bad, 2)
    assert out.is_contiguous() and s0 == 256 and torch.equal(out, bad)


def test_workspace_size_cache_matches_direct_queries():
    lib = _lib.load()
    for sizes in ((32, 24, 8, 4096, 128), (1, 24, 8, 256, 128), (64, 24, 8, 1024, 128)):
        direct = lib.fi_paged_attention_workspace_size(*sizes)
        assert _lib.workspace_size("fi_paged_attention_workspace_size", *sizes) == direct
        assert _lib.workspace_size("fi_paged_attention_workspace_size", *sizes) == direct
    for sizes in ((64, 5120, 3072), (1, 3072, 3072), (4096, 5120, 3072)):
        assert (_lib.workspace_size("fi_int4_matmul_workspace_size", *sizes)
                == lib.fi_int4_matmul_workspace_size(*sizes))
        assert (_lib.workspace_size("fi_rmsnorm_int4_matmul_workspace_size", *sizes)
                == lib.fi_rmsnorm_int4_matmul_workspace_size(*sizes))
