"""StreamingKVCache bookkeeping (reference cortex/cache/streaming.py:79-236) on a CPU
pool: misses, hits, truncation to page_size, overwrite of an existing key, LRU
eviction across sessions, evict_session, hit_rate and pages_used."""

from __future__ import annotations

import torch

from cortex.cache import StreamingKVCache


def _emb(n, v):
    return torch.full((n, 3), float(v))


def test_miss_then_hit_and_truncation():
    c = StreamingKVCache(num_pages=3, page_size=4, hidden_dim=3)
    assert c.read("s", 0) is None and c.hit_rate == 0.0
    c.write("s", 0, _emb(6, 1))  # longer than a page: the first page_size rows are kept
    got = c.read("s", 0)
    assert got.shape == (4, 3) and (got == 1).all()
    assert c.hit_rate == 0.5 and c.pages_used == 1
    c.write("s", 0, _emb(2, 7))  # same key: the page is reused and shrinks to 2 rows
    assert c.pages_used == 1 and c.read("s", 0).shape == (2, 3) and (c.read("s", 0) == 7).all()


def test_lru_eviction_across_sessions():
    c = StreamingKVCache(num_pages=2, page_size=2, hidden_dim=3)
    c.write("a", 0, _emb(1, 1))
    c.write("b", 0, _emb(1, 2))
    assert c.read("a", 0) is not None  # a becomes the most recently used
    c.write("c", 0, _emb(1, 3))  # pool full: evicts b, the least recently used
    assert c.read("b", 0) is None
    assert (c.read("a", 0) == 1).all() and (c.read("c", 0) == 3).all()
    assert c.pages_used == 2


def test_evict_session_frees_its_pages():
    c = StreamingKVCache(num_pages=4, page_size=2, hidden_dim=3)
    for b in (0, 50, 100):
        c.write("x", b, _emb(1, b))
    c.write("y", 0, _emb(1, 9))
    assert c.evict_session("x") == 3 and c.evict_session("x") == 0
    assert c.pages_used == 1 and c.read("x", 50) is None and (c.read("y", 0) == 9).all()
    for b in (0, 50, 100):  # the freed pages are reused without evicting y
        c.write("z", b, _emb(1, 1))
    assert c.read("y", 0) is not None and c.pages_used == 4
