"""Streaming caches (reference cortex/cache): the paged LRU embedding cache and the
device event-page cache that streaming decode windows are assembled from."""

from cortex.cache.streaming import EventWindowCache, PageMeta, StreamingKVCache

__all__ = ["EventWindowCache", "PageMeta", "StreamingKVCache"]
