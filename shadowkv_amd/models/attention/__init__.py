"""Cache-class -> attention-handler map (reference: models/attention/__init__.py:19-31)."""
from typing import Dict

from ..kvcache import KVCacheBase, ShadowKVCache_CPU
from .base import AttentionBase
from .shadow import ShadowAttention

Cache2Attn: Dict[type, type] = {
    ShadowKVCache_CPU: ShadowAttention,
}

__all__ = ["AttentionBase", "ShadowAttention", "Cache2Attn", "KVCacheBase"]
