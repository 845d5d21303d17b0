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


def test_native_page_table_follows_the_lru_policy():
    """The native page table of EventWindowCache against the Python page table (the
    reference's bookkeeping) on one random sequence of batched writes, window plans,
    single lookups and session evictions: same page ids, hits, misses, pages in use,
    and the same windows reported missing."""
    import numpy as np

    from cortex.cache.streaming import _NativePageTable, _PagedLRU

    rng = np.random.default_rng(5)
    P, BPP, WIN = 24, 50, 200
    ref, nat_ = _PagedLRU(P), _NativePageTable(P)
    names = [f"s{i}" for i in range(6)]

    def ref_plan(windows):
        items, offsets, row = [], [0], 0
        for sid, w0 in windows:
            pages = [(b, ref._lookup(sid, b)) for b in range(w0, w0 + WIN, BPP)]
            missing = [b for b, p in pages if p is None]
            if missing:
                return None, (sid, missing)
            for _, p in pages:
                n = ref._meta[p].n_events
                if n:
                    items.append((p, n, row, w0))
                    row += n
            offsets.append(row)
        return (np.asarray(items, dtype=np.int64).reshape(-1, 4), np.asarray(offsets)), None

    for step in range(400):
        op = rng.integers(0, 10)
        if op < 5:  # a batch of page writes (keys distinct within the batch)
            keys = {(names[rng.integers(0, 6)], int(rng.integers(0, 12)) * BPP) for _ in range(rng.integers(1, 8))}
            keys = sorted(keys)
            counts = rng.integers(0, 40, len(keys))
            want = []
            for (sid, b0), n in zip(keys, counts):
                p = ref._page_for_write(sid, b0)
                ref._written(p, int(n))
                want.append(p)
            got = nat_.write(np.fromiter((nat_.session(k[0]) for k in keys), dtype=np.int64),
                             np.asarray([k[1] for k in keys], dtype=np.int64), counts.astype(np.int64))
            assert got.tolist() == want, step
        elif op < 8:  # a batch of windows
            windows = [(names[rng.integers(0, 6)], int(rng.integers(0, 9)) * BPP) for _ in range(rng.integers(1, 5))]
            want, miss = ref_plan(windows)
            try:
                items, offsets = nat_.plan([w[0] for w in windows], np.asarray([w[1] for w in windows], dtype=np.int64),
                                           WIN, BPP)
            except KeyError as e:
                assert miss is not None and f"{miss[0]!r}" in str(e) and str(miss[1]) in str(e), (step, e, miss)
            else:
                assert miss is None, step
                np.testing.assert_array_equal(items, want[0])
                np.testing.assert_array_equal(offsets, want[1])
        elif op < 9:  # one lookup
            sid, b0 = names[rng.integers(0, 6)], int(rng.integers(0, 12)) * BPP
            p = ref._lookup(sid, b0)
            got = nat_.lookup(sid, b0)
            assert got == ((-1, 0) if p is None else (p, ref._meta[p].n_events)), step
        else:
            sid = names[rng.integers(0, 6)]
            assert nat_.evict_session(sid) == ref.evict_session(sid), step
        hits, misses, used = nat_.stats()
        assert (hits, misses, used) == (ref._hits, ref._misses, ref.pages_used), step
