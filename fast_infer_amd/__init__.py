"""fast_infer_amd — MI355X-native attention hot path of Fast_Infer.

Drop-in replacements for the reference's ``kernels/attention.py`` (``flash_attention``,
``paged_attention``), ``kv_cache.py`` (``KVCache``) and ``kernels/rope.py``
(``apply_rope``, fused with the pool write in ``rope_store_kv``), plus the K/V pool
writes of ``model.py`` (``store_kv_prefill`` / ``store_kv_decode``) and a device-resident
block allocator with per-sequence lengths (``PagedKVCache``) and the INT4 linear layers
on either side of attention (``int4_matmul``, ``quantize_int4_groupwise``), all running
hand-written gfx950 HIP kernels through the C ABI of ``include/fast_infer_amd.h``.
"""

from .attention import flash_attention, paged_attention, paged_attention_workspace
from .kv_cache import KVCache
from .kv_store import (allocate_decode, allocate_prefill, store_kv, store_kv_decode,
                       store_kv_prefill)
from .matmul import (dequantize_int4, int4_matmul, quantize_int4_groupwise, rms_norm,
                     rms_norm_int4_matmul)
from .paged_cache import PagedKVCache
from .rope import (apply_rope, precompute_freqs, rope_store_kv, rope_store_kv_decode,
                   rope_store_kv_prefill)

__all__ = [
    "flash_attention",
    "paged_attention",
    "paged_attention_workspace",
    "KVCache",
    "PagedKVCache",
    "int4_matmul",
    "quantize_int4_groupwise",
    "dequantize_int4",
    "rms_norm",
    "rms_norm_int4_matmul",
    "store_kv",
    "store_kv_prefill",
    "store_kv_decode",
    "allocate_prefill",
    "allocate_decode",
    "apply_rope",
    "precompute_freqs",
    "rope_store_kv",
    "rope_store_kv_prefill",
    "rope_store_kv_decode",
]
