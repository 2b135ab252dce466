"""ShadowKV cache classes and the method registry (reference: models/kvcache/__init__.py:15-29).

Only the ShadowKV offload class is provided: the other policies of the reference are not on
the sparse-decode path.
"""
from .base import KVCacheBase
from .shadow import ShadowKVCache_CPU

method2kvcache = {
    "shadowkv_cpu": ShadowKVCache_CPU,
}

__all__ = ["KVCacheBase", "ShadowKVCache_CPU", "method2kvcache"]
