"""Abstract KV-cache interface, as in the reference (models/kvcache/base.py:6-34)."""
from abc import ABC, abstractmethod

import torch


class KVCacheBase(ABC):
    """A KV-cache policy: append new entries, move state to the device, report, reset."""

    @abstractmethod
    def update_kv_cache(self, new_k_cache: torch.Tensor, new_v_cache: torch.Tensor, layer_idx: int):
        """Append the new token's keys and values of one layer."""

    @abstractmethod
    def H2D(self):
        """Move the prefill-built state to the device before decoding."""

    @abstractmethod
    def print_stats(self):
        """Print the cache configuration and fill level."""

    @abstractmethod
    def clear(self):
        """Drop all cached state."""

    @abstractmethod
    def get_kv_len(self):
        """Number of tokens represented by the cache (context length)."""
