"""Paged LRU caches for streaming inference (reference cortex/cache/streaming.py:79-236).

``StreamingKVCache`` keeps the reference's API and bookkeeping exactly -- ``read`` /
``write`` / ``evict_session`` / ``hit_rate`` / ``pages_used``, one page per
``(session_id, bin_start)``, a free list, least-recently-used eviction across
sessions, ``write`` truncating to ``page_size`` rows and overwriting an existing
page -- with the page pool on the GPU.

What it caches is the reference's premise, and that premise does not hold for the
Cortex input: a window's time bins are relative to the window start
(cortex/data/nlb.py:253-256), so the same spike gets a different time embedding in
the next window and cached tokens are not reusable.  ``EventWindowCache`` is the
cache a streaming server can use: pages of RAW events (neuron id, absolute bin,
value) for ``bins_per_page`` consecutive bins, stored once on the device; a decode
window is assembled from its pages by one gather kernel that rewrites the bins
relative to the window start, straight into the forward's input buffer.  Only the
newest stride's events ever cross PCIe, as one pinned copy for all sessions' new
pages plus one scatter launch (``write_many``, or ``write_columns`` for pages already in
columns).  A write's scatter waits on the device for the last gather, so a page reused by
LRU eviction is never overwritten under a window still being assembled on another stream.
Events inside a page keep their arrival order, so a window assembled from time-ordered
pages equals the window built from scratch (events ordered by time bin, as
``np.nonzero`` over (T, N) counts gives).

Neither cache is thread-safe; like the reference, they are meant for the single
inference executor thread.  Prometheus gauges of the reference are not kept.
"""

from __future__ import annotations

import time
import weakref
from collections import OrderedDict
from dataclasses import dataclass
from typing import Any

import numpy as np
import torch

from cortex import _native as nat


@dataclass
class PageMeta:
    """Metadata of one cache page (reference streaming.py:65-76)."""

    page_id: int
    session_id: str
    bin_start: int
    n_events: int
    last_used_at: float


class _PagedLRU:
    """Page table, free list and LRU order shared by both caches."""

    def __init__(self, num_pages: int) -> None:
        if num_pages < 1:
            raise ValueError("num_pages must be >= 1")
        self.num_pages = num_pages
        self._table: dict[tuple[str, int], int] = {}
        self._meta: dict[int, PageMeta] = {}
        self._free: list[int] = list(range(num_pages))
        self._lru: OrderedDict[int, None] = OrderedDict()
        self._hits = 0
        self._misses = 0

    def _lookup(self, session_id: str, bin_start: int) -> int | None:
        """Page of the key, touching LRU and counting a hit; None (a miss) otherwise."""
        page_id = self._table.get((session_id, bin_start))
        if page_id is None:
            self._misses += 1
            return None
        self._lru.move_to_end(page_id)
        self._meta[page_id].last_used_at = time.monotonic()
        self._hits += 1
        return page_id

    def _page_for_write(self, session_id: str, bin_start: int) -> int:
        page_id = self._table.get((session_id, bin_start))
        if page_id is None:
            page_id = self._allocate()
            self._table[(session_id, bin_start)] = page_id
            self._meta[page_id] = PageMeta(page_id, session_id, bin_start, 0, time.monotonic())
            self._lru[page_id] = None
        return page_id

    def _written(self, page_id: int, n: int) -> None:
        self._meta[page_id].n_events = n
        self._meta[page_id].last_used_at = time.monotonic()
        self._lru.move_to_end(page_id)

    def evict_session(self, session_id: str) -> int:
        """Free every page of ``session_id``; returns how many were freed."""
        keys = [k for k in self._table if k[0] == session_id]
        for key in keys:
            self._free_page(self._table.pop(key))
        return len(keys)

    @property
    def hit_rate(self) -> float:
        total = self._hits + self._misses
        return self._hits / total if total > 0 else 0.0

    @property
    def pages_used(self) -> int:
        return len(self._meta)

    def _allocate(self) -> int:
        """A free page id, evicting the least recently used page when none is free."""
        if self._free:
            return self._free.pop()
        lru_id, _ = self._lru.popitem(last=False)
        self._free_page(lru_id)
        return self._free.pop()

    def _free_page(self, page_id: int) -> None:
        meta = self._meta.pop(page_id, None)
        if meta is not None:
            self._table.pop((meta.session_id, meta.bin_start), None)
        self._lru.pop(page_id, None)
        self._free.append(page_id)


class StreamingKVCache(_PagedLRU):
    """Paged embedding cache, API of reference streaming.py:79-236 (pool on ``device``)."""

    def __init__(self, num_pages: int = 128, page_size: int = 64, hidden_dim: int = 512,
                 dtype: torch.dtype = torch.float32, device: str | torch.device = "cpu") -> None:
        super().__init__(num_pages)
        self.page_size = page_size
        self.hidden_dim = hidden_dim
        self.device = torch.device(device)
        self._pool = torch.zeros(num_pages, page_size, hidden_dim, dtype=dtype, device=self.device)

    def read(self, session_id: str, bin_start: int) -> torch.Tensor | None:
        """The cached rows of ``(session_id, bin_start)`` (a view into the pool), or None."""
        page_id = self._lookup(session_id, bin_start)
        if page_id is None:
            return None
        return self._pool[page_id, :self._meta[page_id].n_events, :]

    def write(self, session_id: str, bin_start: int, embeddings: torch.Tensor) -> None:
        """Store the first ``page_size`` rows of ``embeddings`` (E, hidden_dim), replacing
        an existing page of the key; evicts the least recently used page when full."""
        n = min(embeddings.shape[0], self.page_size)
        page_id = self._page_for_write(session_id, bin_start)
        self._pool[page_id, :n, :] = embeddings[:n].detach().to(dtype=self._pool.dtype, device=self.device)
        self._written(page_id, n)


class _NativePageTable:
    """The page table, free list and LRU order of ``EventWindowCache`` in native code
    (``cortex_page_table_*``): the policy of ``_PagedLRU`` with a whole batch of page
    writes or window lookups per call.  Session names map to int64 ids here."""

    def __init__(self, num_pages: int) -> None:
        lib = nat.load()
        box = np.zeros(1, dtype=np.uint64)
        nat.call("cortex_page_table_create", num_pages, box.ctypes.data)
        self._h = int(box[0])
        self._ids: dict[str, int] = {}
        self._finalizer = weakref.finalize(self, lib.cortex_page_table_destroy, self._h)
        self._i64 = np.zeros(3, dtype=np.int64)  # scalar outputs

    def session(self, name: str) -> int:
        sid = self._ids.get(name)
        if sid is None:
            sid = self._ids[name] = len(self._ids)
        return sid

    def write(self, sessions: np.ndarray, bin_starts: np.ndarray, counts: np.ndarray) -> np.ndarray:
        pages = np.empty(sessions.shape[0], dtype=np.int64)
        nat.call("cortex_page_table_write", self._h, sessions.shape[0], sessions.ctypes.data,
                 bin_starts.ctypes.data, counts.ctypes.data, pages.ctypes.data)
        return pages

    def lookup(self, name: str, bin_start: int) -> tuple[int, int]:
        """(page, events) of a key, touched and counted; page -1 (a miss) when absent."""
        out = self._i64
        nat.call("cortex_page_table_lookup", self._h, self.session(name), bin_start, out[0:].ctypes.data,
                 out[1:].ctypes.data)
        return int(out[0]), int(out[1])

    def plan(self, names: list[str], starts: np.ndarray, window_bins: int, bins_per_page: int):
        n = len(names)
        per = window_bins // bins_per_page
        sessions = np.fromiter((self.session(x) for x in names), dtype=np.int64, count=n)
        items = np.empty((max(n * per, 1), 4), dtype=np.int64)
        offsets = np.empty(n + 1, dtype=np.int64)
        missing = np.empty(max(per, 1), dtype=np.int64)
        out = np.zeros(3, dtype=np.int64)  # n_items, missing window, n_missing
        nat.call("cortex_page_table_plan", self._h, n, sessions.ctypes.data, starts.ctypes.data, window_bins,
                 bins_per_page, items.ctypes.data, items.shape[0], out[0:].ctypes.data, offsets.ctypes.data,
                 out[1:].ctypes.data, missing.ctypes.data, out[2:].ctypes.data)
        if out[1] >= 0:
            raise KeyError(f"session {names[int(out[1])]!r}: no page for bins starting at "
                           f"{missing[:int(out[2])].tolist()}")
        return items[:int(out[0])], offsets

    def evict_session(self, name: str) -> int:
        if name not in self._ids:
            return 0
        out = self._i64
        nat.call("cortex_page_table_evict_session", self._h, self._ids[name], out.ctypes.data)
        return int(out[0])

    def stats(self) -> tuple[int, int, int]:
        out = np.zeros(3, dtype=np.int64)
        nat.call("cortex_page_table_stats", self._h, out[0:].ctypes.data, out[1:].ctypes.data, out[2:].ctypes.data)
        return int(out[0]), int(out[1]), int(out[2])


class EventWindowCache:
    """Device pages of raw spike events keyed by ``(session_id, absolute first bin)``.

    Page ``(s, b0)`` holds the events of bins ``[b0, b0 + bins_per_page)``, at most
    ``page_events`` of them, as int64 rows (neuron id, absolute bin, value).  A
    window ``[w0, w0 + window_bins)`` with ``w0`` and ``window_bins`` multiples of
    ``bins_per_page`` is the concatenation of its pages in bin order.  The page table
    (lookups, LRU eviction) is native; its policy is ``StreamingKVCache``'s.
    """

    def __init__(self, num_pages: int = 4096, page_events: int = 1024, bins_per_page: int = 50,
                 device: str | torch.device = "cuda") -> None:
        if num_pages < 1:
            raise ValueError("num_pages must be >= 1")
        self.num_pages = num_pages
        self.page_events = page_events
        self.bins_per_page = bins_per_page
        self.device = torch.device(device)
        nat.require_gpu(torch.empty(0, device=self.device), what="EventWindowCache")
        self._table = _NativePageTable(num_pages)
        self._pool = torch.zeros(num_pages, 3, page_events, dtype=torch.int64, device=self.device)
        self._stage_host = torch.empty(1 << 15, dtype=torch.int64).pin_memory()
        self._stage_dev = torch.empty_like(self._stage_host, device=self.device)
        self._staged = torch.cuda.Event()
        self._gathered: torch.cuda.Event | None = None  # the last gather, on its stream

    @property
    def hit_rate(self) -> float:
        hits, misses, _ = self._table.stats()
        return hits / (hits + misses) if hits + misses > 0 else 0.0

    @property
    def pages_used(self) -> int:
        return self._table.stats()[2]

    def evict_session(self, session_id: str) -> int:
        """Free every page of ``session_id``; returns how many were freed."""
        return self._table.evict_session(session_id)

    def write(self, session_id: str, bin_start: int, neuron_ids: Any, time_bins: Any, values: Any) -> None:
        """Store the events of bins ``[bin_start, bin_start + bins_per_page)``; ``time_bins``
        are absolute.  Raises ValueError for a misaligned page, events outside its bins or
        more than ``page_events`` events (a page never drops events)."""
        self.write_many([(session_id, bin_start, neuron_ids, time_bins, values)])

    def write_many(self, pages: list[tuple[str, int, Any, Any, Any]]) -> None:
        """Several page writes as one pinned host->device copy and one scatter launch, on the
        current stream.  Entries are ``(session_id, bin_start, neuron_ids, time_bins, values)``
        with host integer arrays; a key given twice keeps its last entry.  Every entry is
        checked before any page is written."""
        last: dict[tuple[str, int], tuple[np.ndarray, ...]] = {}
        for session_id, bin_start, nid, tb, val in pages:
            last[(session_id, int(bin_start))] = tuple(
                np.asarray(x.cpu() if torch.is_tensor(x) else x).reshape(-1) for x in (nid, tb, val))
        if not last:
            return
        for c in last.values():
            if not (c[1].shape[0] == c[2].shape[0] == c[0].shape[0]):
                raise ValueError("neuron_ids, time_bins and values must have the same length")
        keys = list(last)
        counts = np.fromiter((c[0].shape[0] for c in last.values()), dtype=np.int64, count=len(keys))
        total = int(counts.sum())
        cols = [np.concatenate([c[f] for c in last.values()]).astype(np.int64, copy=False) if total
                else np.zeros(0, dtype=np.int64) for f in range(3)]
        self._write_pages([k[0] for k in keys], np.fromiter((k[1] for k in keys), dtype=np.int64, count=len(keys)),
                          counts, cols)

    def write_columns(self, session_ids: list[str], bin_starts: Any, counts: Any, neuron_ids: Any,
                      time_bins: Any, values: Any) -> None:
        """``write_many`` for pages already laid out as columns: page i is
        ``(session_ids[i], bin_starts[i])`` and owns the next ``counts[i]`` entries of the
        flat ``neuron_ids`` / ``time_bins`` / ``values`` (absolute bins), pages in order.
        Keys must be distinct.  One pinned copy and one scatter launch, on the current stream."""
        starts = np.asarray(bin_starts, dtype=np.int64).reshape(-1)
        cnt = np.asarray(counts, dtype=np.int64).reshape(-1)
        if not (len(session_ids) == starts.shape[0] == cnt.shape[0]):
            raise ValueError("session_ids, bin_starts and counts must have one entry per page")
        cols = [np.asarray(x.cpu() if torch.is_tensor(x) else x).reshape(-1).astype(np.int64, copy=False)
                for x in (neuron_ids, time_bins, values)]
        if (cnt < 0).any() or not (cols[0].shape[0] == cols[1].shape[0] == cols[2].shape[0] == int(cnt.sum())):
            raise ValueError("neuron_ids, time_bins and values must hold sum(counts) events each")
        if not session_ids:
            return
        self._write_pages(list(session_ids), starts, cnt, cols, distinct=False)

    def _write_pages(self, names: list[str], starts: np.ndarray, counts: np.ndarray, cols: list[np.ndarray],
                     distinct: bool = True) -> None:
        """Check, then write pages ``(names[i], starts[i])`` holding ``counts[i]`` consecutive
        events of ``cols`` each (``distinct``: the keys are known to differ)."""
        P = len(names)
        if P > self.num_pages:
            raise ValueError(f"{P} pages in one write exceed the pool's {self.num_pages}")
        bad = starts % self.bins_per_page != 0
        if bad.any():
            raise ValueError(f"bin_start {int(starts[bad][0])} is not a multiple of "
                             f"bins_per_page={self.bins_per_page}")
        if counts.max() > self.page_events:
            raise ValueError(f"{int(counts.max())} events exceed page_events={self.page_events}")
        total = int(counts.sum())
        if total:
            lo = np.repeat(starts, counts)
            outside = (cols[1] < lo) | (cols[1] >= lo + self.bins_per_page)
            if outside.any():
                i = int(np.argmax(outside))
                k = int(np.searchsorted(np.cumsum(counts), i, side="right"))
                b0 = int(starts[k])
                tb = cols[1][int(counts[:k].sum()):int(counts[:k + 1].sum())]
                raise ValueError(f"time bins [{tb.min()}, {tb.max()}] outside page "
                                 f"[{b0}, {b0 + self.bins_per_page})")
        sessions = np.fromiter((self._table.session(x) for x in names), dtype=np.int64, count=P)
        if not distinct and P > 1:
            order = np.lexsort((starts, sessions))
            same = (sessions[order][1:] == sessions[order][:-1]) & (starts[order][1:] == starts[order][:-1])
            if same.any():
                i = int(order[int(np.argmax(same))])
                raise ValueError(f"page ({names[i]!r}, {int(starts[i])}) is given twice")
        page_ids = self._table.write(sessions, starts, counts)
        nz = counts > 0
        if not nz.any():
            return
        first_row = np.cumsum(counts) - counts
        items = np.stack([page_ids[nz], counts[nz], first_row[nz]], axis=1)
        need = 3 * total + items.size
        self._staged.synchronize()  # the previous write's copy has left the pinned buffer
        if self._stage_host.numel() < need:
            self._stage_host = torch.empty(max(need, 2 * self._stage_host.numel()), dtype=torch.int64).pin_memory()
            self._stage_dev = torch.empty_like(self._stage_host, device=self.device)
        h = self._stage_host.numpy()
        for f in range(3):
            h[f * total:(f + 1) * total] = cols[f]
        h[3 * total:need] = items.reshape(-1)
        dev = self._stage_dev[:need]
        dev.copy_(self._stage_host[:need], non_blocking=True)
        self._staged.record()
        if self._gathered is not None and not self._gathered.query():
            # a gather still queued on another stream may read a page this write reuses
            torch.cuda.current_stream(self.device).wait_event(self._gathered)
        nat.call("cortex_scatter_event_pages", nat.ptr(dev), total, total, nat.ptr(dev[3 * total:]), items.shape[0],
                 nat.ptr(self._pool), self.num_pages, self.page_events, None, nat.stream_of(self.device))

    def read(self, session_id: str, bin_start: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None:
        """(neuron ids, absolute bins, values) views of a page, or None."""
        page_id, n = self._table.lookup(session_id, bin_start)
        if page_id < 0:
            return None
        p = self._pool[page_id]
        return p[0, :n], p[1, :n], p[2, :n]

    def window_pages(self, session_id: str, window_start: int, window_bins: int) -> list[tuple[int, int]]:
        """``[(page_id, n_events)]`` of a window in bin order (touching LRU); KeyError names the
        missing pages."""
        if window_start % self.bins_per_page or window_bins % self.bins_per_page:
            raise ValueError("window_start and window_bins must be multiples of bins_per_page")
        starts = range(window_start, window_start + window_bins, self.bins_per_page)
        pages = [self._table.lookup(session_id, b) for b in starts]
        missing = [b for b, (p, _) in zip(starts, pages) if p < 0]
        if missing:
            raise KeyError(f"session {session_id!r}: no page for bins starting at {missing}")
        return pages

    def plan(self, windows: list[tuple[str, int]], window_bins: int) -> tuple[np.ndarray, np.ndarray]:
        """Gather plan of a batch of windows: ``(items (n, 4) int64, offsets (B+1) int64)``.

        Item = (page id, events, first output row, bin shift = window start); window b
        owns output rows ``[offsets[b], offsets[b+1])``.  KeyError names the first window's
        missing pages.
        """
        if window_bins % self.bins_per_page:
            raise ValueError("window_bins must be a multiple of bins_per_page")
        starts = np.fromiter((w[1] for w in windows), dtype=np.int64, count=len(windows))
        if (starts % self.bins_per_page).any():
            raise ValueError("window starts must be multiples of bins_per_page")
        return self._table.plan([w[0] for w in windows], starts, window_bins, self.bins_per_page)

    def gather(self, items: torch.Tensor, out: torch.Tensor, field_stride: int, out_rows: int,
               err: torch.Tensor | None = None) -> None:
        """Run a device plan (``items`` (n, 4) int64 on the GPU) into ``out``: field f of
        row r at ``out[f * field_stride + r]``, bins relative to each window's start."""
        nat.call("cortex_gather_event_pages", nat.ptr(self._pool), self.num_pages, self.page_events,
                 nat.ptr(items), items.shape[0], nat.ptr(out), field_stride, out_rows, nat.ptr(err),
                 nat.stream_of(self.device))
        if self._gathered is None:
            self._gathered = torch.cuda.Event()
        self._gathered.record(torch.cuda.current_stream(self.device))

    def assemble(self, windows: list[tuple[str, int]], window_bins: int
                 ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
        """Device CSR input of a batch of windows: ``(neuron_ids, time_bins, values, offsets)``
        with bins relative to each window's start."""
        items, offsets = self.plan(windows, window_bins)
        E = int(offsets[-1])
        out = torch.empty(3 * max(E, 1), dtype=torch.int64, device=self.device)
        if items.shape[0]:
            self.gather(torch.from_numpy(items).to(self.device), out, max(E, 1), E)
        S = max(E, 1)
        return out[:E], out[S:S + E], out[2 * S:2 * S + E], torch.from_numpy(offsets).to(self.device)
