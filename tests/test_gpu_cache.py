"""Streaming windows from device event pages (the D7 fix of the reference's
StreamingKVCache premise, cortex/cache/streaming.py:79-236, cortex/data/nlb.py:249-256).

Windows assembled on the device from absolute-bin pages must equal, bit for bit,
the window built from scratch the reference's way (events of the window's (T, N)
counts via np.nonzero, bins relative to the window start); the worker's result for
cached windows must equal its result for the same windows sent as payloads.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
STRIDE, WINDOW = 50, 600


def _events(counts):
    """(T, N) spike counts -> (neuron, bin, value) ordered by bin, then neuron."""
    t, n = np.nonzero(counts)
    return n.astype(np.int64), t.astype(np.int64), np.clip(counts[t, n], 1, 7).astype(np.int64)


def _events_abs(counts, b0):
    nid, tb, val = _events(counts[b0:b0 + STRIDE])
    return nid, tb + b0, val


def _session(seed, T=1200, N=137, rate=0.007):
    return np.random.default_rng(seed).poisson(rate, (T, N))


def _fill(cache, sid, counts, upto):
    for b0 in range(0, upto, STRIDE):
        nid, tb, val = _events(counts[b0:b0 + STRIDE])
        cache.write(sid, b0, nid, tb + b0, val)  # absolute bins


def test_assembled_windows_equal_scratch_windows():
    from cortex.cache import EventWindowCache

    cache = EventWindowCache(num_pages=256, page_events=512, bins_per_page=STRIDE, device=DEV)
    sessions = {f"s{i}": _session(i) for i in range(3)}
    _fill(cache, "s0", sessions["s0"], 1200)  # one page per call
    batch = []
    for sid in ("s1", "s2"):  # every page of two sessions in one batched write
        for b0 in range(0, 1200, STRIDE):
            nid, tb, val = _events(sessions[sid][b0:b0 + STRIDE])
            batch.append((sid, b0, nid, tb + b0, val))
    batch.append(("s1", 0, [5], [3], [2]))  # a key given twice: the last entry is kept ...
    batch.append(("s1", 0, *_events_abs(sessions["s1"], 0)))  # ... so this one
    cache.write_many(batch)
    windows = [("s0", 0), ("s1", 300), ("s2", 600), ("s0", 550), ("s1", 0)]
    nid, tb, val, off = cache.assemble(windows, WINDOW)
    off = off.cpu().numpy()
    for b, (sid, w0) in enumerate(windows):
        ref = _events(sessions[sid][w0:w0 + WINDOW])
        for got, want in zip((nid, tb, val), ref):
            np.testing.assert_array_equal(got[off[b]:off[b + 1]].cpu().numpy(), want, err_msg=f"window {b}")
    assert cache.hit_rate == 1.0 and cache.pages_used == 3 * 24


def test_page_cache_errors_and_eviction():
    from cortex.cache import EventWindowCache

    cache = EventWindowCache(num_pages=4, page_events=8, bins_per_page=STRIDE, device=DEV)
    with pytest.raises(ValueError):
        cache.write("s", 10, [1], [10], [1])  # not aligned to a page
    with pytest.raises(ValueError):
        cache.write("s", 0, [1], [STRIDE], [1])  # bin outside the page
    with pytest.raises(ValueError):
        cache.write("s", 0, np.zeros(9), np.zeros(9), np.ones(9))  # more than page_events
    for b0 in range(0, 5 * STRIDE, STRIDE):  # 5 pages into 4: the first is evicted
        cache.write("s", b0, [b0 // STRIDE], [b0], [1])
    with pytest.raises(KeyError):
        cache.window_pages("s", 0, 2 * STRIDE)
    got = cache.read("s", 4 * STRIDE)
    assert [int(x[0]) for x in got] == [4, 4 * STRIDE, 1]
    assert cache.evict_session("s") == 4 and cache.pages_used == 0


@pytest.mark.parametrize("use_graphs", [True, False])
def test_worker_windows_equal_payloads(use_graphs):
    from cortex.cache import EventWindowCache
    from cortex.models import CortexModel
    from cortex.models.config import CORTEX_S
    from cortex.serve import InferenceWorker

    torch.manual_seed(0)
    model = CortexModel(CORTEX_S).to(DEV).eval()
    w = InferenceWorker(model, CORTEX_S, torch.device(DEV), use_graphs=use_graphs)
    cache = EventWindowCache(num_pages=512, page_events=512, bins_per_page=STRIDE, device=DEV)
    sessions = {f"s{i}": _session(10 + i, rate=0.01) for i in range(4)}
    for step in range(3):  # a stride of new events per session, then one batch of windows
        upto = WINDOW + step * STRIDE
        for sid, counts in sessions.items():
            _fill(cache, sid, counts, upto)
        reqs = [{"request_id": sid, "session_id": sid, "window_start": upto - WINDOW} for sid in sessions]
        got = w.run_windows_sync(reqs, cache, WINDOW)
        payloads = []
        for r in reqs:
            nid, tb, val = _events(sessions[r["session_id"]][r["window_start"]:r["window_start"] + WINDOW])
            payloads.append({"request_id": r["request_id"],
                             "events": {"neuron_id": nid, "time_bin": tb, "value": val}})
        want = w._run_batch_sync(payloads)
        assert [g["request_id"] for g in got] == [x["request_id"] for x in want]
        assert [g["behavior"] for g in got] == [x["behavior"] for x in want]
    w.shutdown()


def _stride_columns(sessions, names, b0):
    """One stride of every session as page columns: counts per page, then the events."""
    parts = [_events_abs(sessions[s], b0) for s in names]
    cnt = np.array([p[0].shape[0] for p in parts], dtype=np.int64)
    return cnt, *(np.concatenate([p[f] for p in parts]) for f in range(3))


def test_write_columns_equals_write_many():
    from cortex.cache import EventWindowCache

    names = [f"s{i}" for i in range(5)]
    sessions = {s: _session(40 + i) for i, s in enumerate(names)}
    a = EventWindowCache(num_pages=256, page_events=512, bins_per_page=STRIDE, device=DEV)
    b = EventWindowCache(num_pages=256, page_events=512, bins_per_page=STRIDE, device=DEV)
    for b0 in range(0, 900, STRIDE):
        cnt, nid, tb, val = _stride_columns(sessions, names, b0)
        a.write_columns(names, np.full(len(names), b0), cnt, nid, tb, val)
        b.write_many([(s, b0, *_events_abs(sessions[s], b0)) for s in names])
    windows = [(s, w0) for s in names for w0 in (0, 150, 300)]
    got, want = a.assemble(windows, WINDOW), b.assemble(windows, WINDOW)
    for x, y in zip(got, want):
        assert torch.equal(x, y)
    cnt, nid, tb, val = _stride_columns(sessions, names[:2], 900)
    with pytest.raises(ValueError):  # a key given twice
        a.write_columns([names[0], names[0]], [900, 900], cnt, nid, tb, val)
    with pytest.raises(ValueError):  # counts do not cover the events
        a.write_columns(names[:2], [900, 900], cnt + 1, nid, tb, val)
    with pytest.raises(ValueError):  # a bin outside its page
        a.write_columns(names[:2], [950, 900], cnt, nid, tb, val)
    a.write_columns([], [], [], [], [], [])


@pytest.mark.parametrize("use_graphs", [True, False])
def test_pipelined_windows_equal_sync(use_graphs):
    """submit_windows / collect with the next stride written while a batch runs: the same
    results as the synchronous path, with LRU eviction on every step, and with a third
    submission settling the oldest uncollected batch."""
    from cortex.cache import EventWindowCache
    from cortex.models import CortexModel
    from cortex.models.config import CORTEX_S
    from cortex.serve import InferenceWorker

    torch.manual_seed(0)
    model = CortexModel(CORTEX_S).to(DEV).eval()
    w = InferenceWorker(model, CORTEX_S, torch.device(DEV), use_graphs=use_graphs)
    names = [f"s{i}" for i in range(6)]
    sessions = {s: _session(60 + i, T=1600, rate=0.01) for i, s in enumerate(names)}
    per = WINDOW // STRIDE
    piped = EventWindowCache(num_pages=(per + 1) * len(names), page_events=512, bins_per_page=STRIDE, device=DEV)
    sync = EventWindowCache(num_pages=(per + 1) * len(names), page_events=512, bins_per_page=STRIDE, device=DEV)
    for b0 in range(0, WINDOW - STRIDE, STRIDE):
        cnt, nid, tb, val = _stride_columns(sessions, names, b0)
        piped.write_columns(names, np.full(len(names), b0), cnt, nid, tb, val)
        for s in names:
            sync.write(s, b0, *_events_abs(sessions[s], b0))
    steps = 8
    reqs = [[{"request_id": f"{s}:{k}", "session_id": s, "window_start": k * STRIDE} for s in names]
            for k in range(steps)]
    got, pending = [], None
    for k in range(steps):
        cnt, nid, tb, val = _stride_columns(sessions, names, WINDOW - STRIDE + k * STRIDE)
        piped.write_columns(names, np.full(len(names), WINDOW - STRIDE + k * STRIDE), cnt, nid, tb, val)
        nxt = w.submit_windows(reqs[k], piped, WINDOW)
        if pending is not None:
            got.append(w.collect(pending))
        pending = nxt
    got.append(w.collect(pending))
    want = []
    for k in range(steps):
        for s in names:
            sync.write(s, WINDOW - STRIDE + k * STRIDE, *_events_abs(sessions[s], WINDOW - STRIDE + k * STRIDE))
        want.append(w.run_windows_sync(reqs[k], sync, WINDOW))
    assert [[r["behavior"] for r in g] for g in got] == [[r["behavior"] for r in x] for x in want]
    assert [[r["request_id"] for r in g] for g in got] == [[r["request_id"] for r in x] for x in want]
    # three in flight: the third submission settles the first, results unchanged
    b0 = WINDOW + (steps - 1) * STRIDE
    last = [[{"request_id": s, "session_id": s, "window_start": w0} for s in names]
            for w0 in (b0 - WINDOW, b0 - WINDOW - STRIDE, b0 - WINDOW)]  # pages still in the pool
    ps = [w.submit_windows(r, sync, WINDOW) for r in last]
    outs = [w.collect(p) for p in ps]
    assert [r["behavior"] for r in outs[0]] == [r["behavior"] for r in want[-1]]
    for r, o in zip(last, outs):
        assert [x["behavior"] for x in o] == [x["behavior"] for x in w.run_windows_sync(r, sync, WINDOW)]
    w.shutdown()
