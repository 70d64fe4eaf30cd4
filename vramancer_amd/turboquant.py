"""Compatibility alias module, as core/turboquant.py:1-4 of the reference."""
from .kv_quantizer import KVCacheCompressor, TurboQuantCompressor  # noqa: F401

__all__ = ["TurboQuantCompressor", "KVCacheCompressor"]
