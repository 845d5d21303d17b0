"""Host side of the serving worker (reference cortex/serve/worker.py:160-249): the
payload -> CSR packing and the event buckets.  Runs without a GPU."""

from __future__ import annotations

import numpy as np
import pytest

from cortex.serve.worker import batch_bucket, event_bucket, pack_payloads


def _payload(i, n, rng):
    return {"request_id": f"r{i}", "events": [{"neuron_id": int(rng.integers(0, 512)),
                                                "time_bin": int(rng.integers(0, 1024)),
                                                "value": int(rng.integers(0, 8))} for _ in range(n)]}


def test_event_bucket_bounds():
    prev = 0
    for n in list(range(0, 3000, 7)) + [16383, 16384, 16385, 100000, 131072, 262145]:
        b = event_bucket(n)
        assert b >= n and b >= prev
        if n > 256:
            assert b < 2 * n if n <= 16384 else b - n < 4096
        prev = b
    assert event_bucket(1) == 256 and event_bucket(257) == 512 and event_bucket(16385) == 20480


@pytest.mark.parametrize("bucket", [True, False])
def test_pack_payloads_matches_flat_contract(bucket):
    """Same flat events and sample order as the reference's list building
    (worker.py:166-177), as CSR offsets instead of batch indices."""
    rng = np.random.default_rng(3)
    counts = [5, 0, 300, 1, 0, 0]
    payloads = [_payload(i, n, rng) for i, n in enumerate(counts)]
    flat, B, E, Eb = pack_payloads(payloads, bucket)
    ref_nid, ref_tb, ref_val, ref_bidx = [], [], [], []
    for b, p in enumerate(payloads):
        for ev in p["events"]:
            ref_nid.append(ev["neuron_id"]); ref_tb.append(ev["time_bin"]); ref_val.append(ev["value"])
            ref_bidx.append(b)
    assert B == max(ref_bidx) + 1 == 4 and E == len(ref_nid)
    assert Eb == (event_bucket(E) if bucket else E)
    for f, ref in enumerate((ref_nid, ref_tb, ref_val)):
        np.testing.assert_array_equal(flat[f * Eb:f * Eb + E], ref)
        assert (flat[f * Eb + E:(f + 1) * Eb] == 0).all()
    off = flat[3 * Eb:3 * Eb + B + 1]
    np.testing.assert_array_equal(off, np.concatenate([[0], np.cumsum(np.bincount(ref_bidx, minlength=B))]))


def test_pack_payloads_columnar_and_buffer_reuse():
    rng = np.random.default_rng(4)
    lists = [_payload(i, n, rng) for i, n in enumerate([7, 70])]
    cols = [{"request_id": p["request_id"],
             "events": {k: np.array([ev[k] for ev in p["events"]]) for k in ("neuron_id", "time_bin", "value")}}
            for p in lists]
    a, *ma = pack_payloads(lists)
    buf = np.full(4096, -1, dtype=np.int64)
    b, *mb = pack_payloads(cols, out=buf)
    assert ma == mb and np.shares_memory(b, buf)
    np.testing.assert_array_equal(a, b)
    small = np.zeros(3, dtype=np.int64)
    c, *_ = pack_payloads(cols, out=small)  # too small: a fresh array
    assert not np.shares_memory(c, small)
    np.testing.assert_array_equal(a, c)
    with pytest.raises(ValueError):
        pack_payloads([{"request_id": "x", "events": {"neuron_id": [1, 2], "time_bin": [1], "value": [1, 1]}}])


def test_pack_payloads_no_events():
    flat, B, E, Eb = pack_payloads([{"request_id": "a", "events": []}, {"request_id": "b"}])
    assert (B, E, Eb) == (0, 0, 0)


def test_batch_bucket_bounds():
    """At most 25 % padding samples, monotone, and few distinct sizes (four per doubling)."""
    prev = 0
    for b in range(1, 2049):
        bb = batch_bucket(b)
        assert bb >= b and bb >= prev and (bb == b if b <= 8 else bb <= 1.25 * b)
        prev = bb
    assert len({batch_bucket(b) for b in range(1, 257)}) <= 8 + 4 * 5
    assert [batch_bucket(b) for b in (8, 9, 11, 17, 33, 100, 256, 257)] == [8, 10, 12, 20, 40, 112, 256, 320]


def test_pack_payloads_batch_pad_appends_empty_samples():
    rng = np.random.default_rng(6)
    payloads = [_payload(i, n, rng) for i, n in enumerate([3, 0, 9, 4, 1, 1, 2, 5, 7, 2, 0])]
    a, B, E, Eb = pack_payloads(payloads)
    b, B2, E2, Eb2 = pack_payloads(payloads, batch_pad=True)
    assert (B, E, Eb) == (B2, E2, Eb2) == (10, 34, 256)
    Bb = batch_bucket(B)
    assert Bb == 10 and b.shape[0] == 3 * Eb + Bb + 1
    np.testing.assert_array_equal(b[:3 * Eb + B + 1], a)
    payloads.append(_payload(11, 3, rng))  # B = 12 -> bucket 12; B = 9 below pads to 10
    c, B3, E3, _ = pack_payloads(payloads[:9], batch_pad=True)
    assert B3 == 9 and c.shape[0] == 3 * 256 + 10 + 1
    assert c[-1] == c[-2] == E3
