"""The serving worker on the GPU (reference cortex/serve/worker.py:95-249): its
results equal the model's own forward on the same events, with and without the
captured graphs, for the reference's payload contract and the columnar extension.

Tolerance: the worker runs the same kernels on the same rows; the event buckets
only add padding rows past offsets[B], which no kernel attends.  Outputs must agree
to 1e-5 of the largest |output| (in practice bit-identical).
"""

from __future__ import annotations

import asyncio

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _model():
    from cortex.models import CortexModel
    from cortex.models.config import CORTEX_S
    from cortex.quantization.calibrate import (attach_calibration_hooks, convert_model, derive_scales,
                                               remove_calibration_hooks)

    torch.manual_seed(0)
    model = CortexModel(CORTEX_S).to(DEV).eval()
    rng = np.random.default_rng(1)
    nid = torch.from_numpy(rng.integers(0, 512, 1024)).to(DEV)
    tb = torch.from_numpy(rng.integers(0, 1024, 1024)).to(DEV)
    val = torch.from_numpy(rng.integers(0, 8, 1024)).to(DEV)
    bidx = torch.arange(1024, device=DEV) // 512
    hooks = attach_calibration_hooks(model)
    with torch.no_grad():
        model(nid, tb, val, bidx)
    remove_calibration_hooks(hooks)
    return convert_model(model, derive_scales(model, hooks), inplace=True)


@pytest.fixture(scope="module")
def model():
    return _model()


def _payloads(counts, seed, columnar=False):
    rng = np.random.default_rng(seed)
    out = []
    for i, n in enumerate(counts):
        nid, tb, val = rng.integers(0, 512, n), rng.integers(0, 1024, n), rng.integers(0, 8, n)
        if columnar:
            ev = {"neuron_id": nid, "time_bin": tb, "value": val}
        else:
            ev = [{"neuron_id": int(a), "time_bin": int(b), "value": int(c)} for a, b, c in zip(nid, tb, val)]
        out.append({"request_id": f"req{i}", "events": ev})
    return out


def _expected(model, payloads, dim=2):
    nid, tb, val, bidx = [], [], [], []
    for b, p in enumerate(payloads):
        ev = p["events"]
        if isinstance(ev, dict):
            nid += list(ev["neuron_id"]); tb += list(ev["time_bin"]); val += list(ev["value"])
            bidx += [b] * len(ev["neuron_id"])
        else:
            for e in ev:
                nid.append(e["neuron_id"]); tb.append(e["time_bin"]); val.append(e["value"]); bidx.append(b)
    if not nid:
        return np.zeros((len(payloads), dim))
    t = [torch.tensor(x, dtype=torch.int64, device=DEV) for x in (nid, tb, val, bidx)]
    with torch.no_grad():
        out = model(*t)["behavior"].float().cpu().numpy()
    full = np.zeros((len(payloads), dim))
    full[:out.shape[0]] = out
    return full


def _check(results, payloads, want):
    assert [r["request_id"] for r in results] == [p["request_id"] for p in payloads]
    got = np.array([r["behavior"] for r in results])
    assert got.shape == want.shape
    tol = 1e-5 * max(np.abs(want).max(), 1e-6)
    assert np.abs(got - want).max() <= tol, np.abs(got - want).max()
    assert all(r["inference_ms"] > 0 for r in results)


@pytest.mark.parametrize("use_graphs", [True, False])
def test_worker_matches_model_forward(model, use_graphs):
    from cortex.models.config import CORTEX_S
    from cortex.serve import InferenceWorker

    w = InferenceWorker(model, CORTEX_S, torch.device(DEV), max_batch_size=32, use_graphs=use_graphs)
    w.warmup(2)
    assert w.ready
    # empty payloads inside and at the end; a batch repeated (graph reuse) with new data
    for counts, seed in [([512, 0, 77, 1, 300, 0], 1), ([512, 5, 77, 1, 300, 0], 2), ([64] * 9, 3), ([2048], 4)]:
        p = _payloads(counts, seed)
        _check(w._run_batch_sync(p), p, _expected(model, p))
    w.shutdown()


def test_worker_columnar_payloads_and_async(model):
    from cortex.models.config import CORTEX_S
    from cortex.serve import InferenceWorker

    w = InferenceWorker(model, CORTEX_S, torch.device(DEV))
    p_list = _payloads([100, 600, 3], seed=5)
    p_col = _payloads([100, 600, 3], seed=5, columnar=True)
    a = w._run_batch_sync(p_list)
    b = asyncio.run(w.run_batch(p_col))
    assert [r["behavior"] for r in a] == [r["behavior"] for r in b]
    _check(b, p_col, _expected(model, p_list))
    assert asyncio.run(w.run_batch([])) == []
    none = w._run_batch_sync([{"request_id": "x", "events": []}])
    assert none[0]["behavior"] == [0.0, 0.0]
    w.shutdown()


def test_worker_pipelined_batches_equal_sync(model):
    """submit_batch / collect with the next batch packed while one runs (and a third
    submission settling the oldest uncollected batch): the same result dicts as
    _run_batch_sync, including trailing and all-empty payloads."""
    from cortex.models.config import CORTEX_S
    from cortex.serve import InferenceWorker

    w = InferenceWorker(model, CORTEX_S, torch.device(DEV))
    batches = [_payloads([100, 600, 3], seed=5), _payloads([50, 0, 700, 0], seed=6, columnar=True),
               [{"request_id": "e", "events": []}], _payloads([300] * 8, seed=7)]
    want = [w._run_batch_sync(b) for b in batches]
    got, pending = [], None
    for b in batches:
        nxt = w.submit_batch(b)
        if pending is not None:
            got.append(w.collect(pending))
        pending = nxt
    got.append(w.collect(pending))
    ps = [w.submit_batch(b) for b in batches[:3]]  # three in flight: the first is settled early
    got3 = [w.collect(p) for p in ps]
    for g, x in zip(got + got3, want + want[:3]):
        assert [r["request_id"] for r in g] == [r["request_id"] for r in x]
        assert [r["behavior"] for r in g] == [r["behavior"] for r in x]
    w.shutdown()


def test_worker_rejects_out_of_range_events(model):
    from cortex.models.config import CORTEX_S
    from cortex.serve import InferenceWorker

    w = InferenceWorker(model, CORTEX_S, torch.device(DEV))
    p = _payloads([40, 40], seed=6)
    p[1]["events"][3]["neuron_id"] = 100_000
    with pytest.raises(IndexError):
        w._run_batch_sync(p)
    ok = _payloads([40, 40], seed=6)  # the next batch on the same graph is clean again
    _check(w._run_batch_sync(ok), ok, _expected(model, ok))
    # pipelined: the bad batch raises at its collect, the batches around it are unaffected
    first, bad, last = w.submit_batch(ok), w.submit_batch(p), w.submit_batch(ok)
    _check(w.collect(first), ok, _expected(model, ok))
    with pytest.raises(IndexError):
        w.collect(bad)
    _check(w.collect(last), ok, _expected(model, ok))
    w.shutdown()


def test_forward_csr_equals_forward(model):
    """The pre-grouped entry (no pack plan) against the batch_indices entry."""
    rng = np.random.default_rng(9)
    counts = np.array([30, 0, 700, 64])
    E = int(counts.sum())
    nid, tb, val = (torch.from_numpy(rng.integers(0, hi, E)).to(DEV) for hi in (512, 1024, 8))
    off = torch.from_numpy(np.concatenate([[0], np.cumsum(counts)])).to(DEV)
    bidx = torch.repeat_interleave(torch.arange(4, device=DEV), torch.from_numpy(counts).to(DEV))
    pad = 100  # rows past offsets[B] are ignored
    z = torch.zeros(pad, dtype=torch.int64, device=DEV)
    with torch.no_grad():
        a = model.forward_csr(torch.cat([nid, z]), torch.cat([tb, z]), torch.cat([val, z]), off)
        b = model(nid, tb, val, bidx, batch_size=4)["behavior"]
    torch.testing.assert_close(a, b, rtol=0, atol=1e-5 * float(b.abs().max()))
