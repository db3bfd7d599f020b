"""Host-side offload machinery: pinned weight arena, copy streams, checkpoint-to-arena loading, hot-channel
cache. weight_store / stream_manager / load_hf_checkpoint import torch.cuda lazily (pinned memory needs a GPU
context when used, not when imported)."""
from . import hot_cache, load_hf_checkpoint, stream_manager, weight_store

__all__ = ["hot_cache", "load_hf_checkpoint", "stream_manager", "weight_store"]
