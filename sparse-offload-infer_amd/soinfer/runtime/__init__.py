"""Callers of the hot path: the DIP / cache-aware DIP MLP drivers."""
from . import dip

__all__ = ["dip"]
