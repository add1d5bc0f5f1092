"""Paged KV-cache storage and page ownership."""

from .kv_cache import KVCachePool, KVCacheShape
from .page_pool import PagePool

__all__ = ["KVCachePool", "KVCacheShape", "PagePool"]
