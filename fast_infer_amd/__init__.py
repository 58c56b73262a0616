"""fast_infer_amd — MI355X-native attention hot path of Fast_Infer.

Drop-in replacements for the reference's ``kernels/attention.py`` (``flash_attention``,
``paged_attention``) and ``kv_cache.py`` (``KVCache``), plus the K/V pool writes of
``model.py`` (``store_kv_prefill`` / ``store_kv_decode``), all running hand-written
gfx950 HIP kernels through the C ABI of ``include/fast_infer_amd.h``.
"""

from .attention import flash_attention, paged_attention, paged_attention_workspace
from .kv_cache import KVCache
from .kv_store import allocate_prefill, store_kv, store_kv_decode, store_kv_prefill

__all__ = [
    "flash_attention",
    "paged_attention",
    "paged_attention_workspace",
    "KVCache",
    "store_kv",
    "store_kv_prefill",
    "store_kv_decode",
    "allocate_prefill",
]
