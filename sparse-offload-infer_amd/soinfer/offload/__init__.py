"""Hot-channel cache (resident rows of the most frequently selected MLP channels)."""
from . import hot_cache

__all__ = ["hot_cache"]
