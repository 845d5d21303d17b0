"""Batched inference worker on gfx950 (reference cortex/serve/worker.py:92-253).

Same surface as the reference's ``InferenceWorker``: ``run_batch`` (async, one
single-thread executor so forward passes never overlap), ``_run_batch_sync``,
``warmup``, ``ready``, ``shutdown``, and the payload and result dicts of its
contract (worker.py:22-32).  What changes is the way a batch reaches the GPU:

* The payloads are already grouped by request, so the batch is CSR by
  construction: the host writes the events sample after sample plus the (B+1)
  offsets; the device never sorts ``batch_indices``.
* Neuron ids, time bins, values and offsets go into ONE pinned host buffer laid
  out like the device input buffer, and cross in one asynchronous copy.
* The forward for a given (batch bucket, event bucket) is captured once as a HIP
  graph and replayed (about 60 launches become one).  Event counts are rounded up
  to a bucket, the padding events lie past ``offsets[B]`` and are never attended;
  batch sizes are rounded up to a bucket too (at most 25 % more samples), the extra
  samples are empty (their offsets repeat ``offsets[B]``) and their rows are dropped,
  so a dynamic batcher's mix of sizes reuses a few dozen graphs instead of
  capturing one per exact size.
* The (B, behavior_dim) result comes back through a pinned buffer; the only host
  synchronisation is the one wait for that copy.

Payload ``events`` may be the reference's list of ``{"neuron_id", "time_bin",
"value"}`` dicts or, as an extension, a mapping of three equal-length integer
arrays ``{"neuron_id": ..., "time_bin": ..., "value": ...}`` (no per-event Python
work).  Request metrics (the reference's Prometheus gauges) are not kept here.
"""

from __future__ import annotations

import asyncio
import time
from collections import OrderedDict
from concurrent.futures import ThreadPoolExecutor
from typing import Any

import numpy as np
import torch
from torch import nn

from cortex.models.config import CortexConfig

_FIELDS = ("neuron_id", "time_bin", "value")


def load_model(config: CortexConfig, checkpoint_path: str | None = None,
               device: torch.device | None = None) -> nn.Module:
    """``CortexModel`` on ``device`` (reference worker.py:61-89).

    A checkpoint is read with ``torch.load(weights_only=True)``: plain tensors and
    containers only.  The reference's ``{"model_state_dict": ...}`` wrapper and a bare
    state dict are both accepted; missing or unexpected keys are tolerated
    (``strict=False``) as there.
    """
    from cortex.models.cortex import CortexModel

    if device is None:
        if not torch.cuda.is_available():
            raise RuntimeError("the Cortex gfx950 forward needs a ROCm device")
        device = torch.device("cuda")
    model = CortexModel(config).to(device).eval()
    if checkpoint_path:
        try:
            payload = torch.load(checkpoint_path, map_location=device, weights_only=True)
        except FileNotFoundError:
            return model
        state = payload.get("model_state_dict", payload)
        model.load_state_dict(state, strict=False)
    return model


def event_bucket(n: int, fine: int = 4096) -> int:
    """Padded event count of a batch: the next power of two up to 16384 (at least
    256), then the next multiple of ``fine``; the padding costs at most 2x of the
    event-side work (tokenizer, kv projection) for small batches and < ``fine``
    rows for large ones, and bounds the number of distinct captured graphs."""
    if n <= 256:
        return 256
    if n <= 16384:
        return 1 << (n - 1).bit_length()
    return -(-n // fine) * fine


def batch_bucket(b: int) -> int:
    """Batch size a captured graph is built for: ``b`` itself up to 8, then ``b`` rounded up
    to a quarter of its power of two (8, 10, 12, 14, 16, 20, 24, 28, 32, 40, ...): at
    most 25 % padding samples, four graphs per doubling of the batch."""
    if b <= 8:
        return b
    step = 1 << (b.bit_length() - 3)
    return -(-b // step) * step


def _as_columns(events: Any) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    if isinstance(events, dict):
        cols = [np.asarray(events[f], dtype=np.int64).reshape(-1) for f in _FIELDS]
        if not (cols[0].shape == cols[1].shape == cols[2].shape):
            raise ValueError("columnar events need equal-length neuron_id, time_bin and value arrays")
        return cols[0], cols[1], cols[2]
    n = len(events)
    out = np.empty((3, n), dtype=np.int64)
    for i, ev in enumerate(events):
        out[0, i] = int(ev["neuron_id"])
        out[1, i] = int(ev["time_bin"])
        out[2, i] = int(ev["value"])
    return out[0], out[1], out[2]


def pack_payloads(payloads: list[dict[str, Any]], bucket: bool = True,
                  out: np.ndarray | None = None, *, batch_pad: bool = False) -> tuple[np.ndarray, int, int, int]:
    """Payloads -> the flat int64 input ``[nid (Eb) | tb (Eb) | val (Eb) | offsets (Bb+1)]``.

    Returns ``(flat, B, E, Eb)``: B ends at the last payload with events (the
    reference's ``max(batch_indices) + 1``, worker.py:171-177,238 and cortex.py:140), E is
    the number of real events, Eb the padded count (``event_bucket(E)`` when
    ``bucket``, else E).  Events keep the payload order, so sample b owns rows
    ``[offsets[b], offsets[b+1])``; padding rows are zeros.  Bb is ``batch_bucket(B)``
    with ``batch_pad`` (empty samples B..Bb-1: their offsets are E), else B.  B = 0
    when no payload has an event.  ``out`` receives the data when it is long enough
    (``3 Eb + Bb + 1``).
    """
    cols = [_as_columns(p.get("events", [])) for p in payloads]
    counts = np.array([c[0].shape[0] for c in cols], dtype=np.int64)
    nonempty = np.flatnonzero(counts)
    if nonempty.size == 0:
        return np.zeros(1, dtype=np.int64), 0, 0, 0
    B = int(nonempty[-1]) + 1
    Bb = batch_bucket(B) if batch_pad else B
    E = int(counts[:B].sum())
    Eb = event_bucket(E) if bucket else E
    n = 3 * Eb + Bb + 1
    h = out[:n] if out is not None and out.shape[0] >= n else np.empty(n, dtype=np.int64)
    for f in range(3):
        np.concatenate([c[f] for c in cols[:B]], out=h[f * Eb:f * Eb + E])
        h[f * Eb + E:(f + 1) * Eb] = 0  # padding events: valid table rows, never attended
    h[3 * Eb] = 0
    np.cumsum(counts[:B], out=h[3 * Eb + 1:3 * Eb + B + 1])
    h[3 * Eb + B + 1:n] = E  # padding samples: empty
    return h, B, E, Eb


class _CsrGraph:
    """The forward for one (batch, event bucket), captured on ``stream``.

    ``inp`` is the device input buffer ``[nid (E) | tb (E) | val (E) | offsets (B+1)]``.
    """

    def __init__(self, model: nn.Module, batch: int, events: int, device: torch.device,
                 stream: torch.cuda.Stream, pool: Any) -> None:
        self.batch, self.events = batch, events
        self.inp = torch.zeros(3 * events + batch + 1, dtype=torch.int64, device=device)  # empty samples
        self.err = torch.zeros(1, dtype=torch.int32, device=device)
        E = events
        self._args = (self.inp[:E], self.inp[E:2 * E], self.inp[2 * E:3 * E], self.inp[3 * E:])
        self.model = model
        with torch.cuda.stream(stream), torch.inference_mode():
            for _ in range(2):  # weights images, batch-invariant projections, allocator warm
                self._run()
        stream.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, pool=pool, stream=stream), torch.inference_mode():
            self.out = self._run()

    def _run(self) -> torch.Tensor:
        nid, tb, val, off = self._args
        return self.model.forward_csr(nid, tb, val, off, err_flag=self.err)


class _Slot:
    """Pinned host buffers of one batch in flight (input staging, result, error flag) and
    the event after its last copy; two slots let the host prepare one batch while the GPU
    runs the other."""

    def __init__(self) -> None:
        self.host_in = torch.empty(1 << 16, dtype=torch.int64).pin_memory()
        self.host_out = torch.empty(1024, dtype=torch.float32).pin_memory()
        self.host_err = torch.zeros(1, dtype=torch.int32).pin_memory()
        self.done = torch.cuda.Event()
        self.pending: PendingBatch | None = None


class PendingBatch:
    """A batch in flight, from ``InferenceWorker.submit_batch`` (payloads) or
    ``submit_windows`` (cached streaming windows); pass it to ``collect`` for the result
    dicts.  Its result stays in its pinned slot until collected, or until a later
    submission needs the slot (then it moves to host memory)."""

    def __init__(self, slot: _Slot, requests: list[dict[str, Any]], batch: int, dim: int, t0: float) -> None:
        self._slot, self.requests, self._B, self._dim, self._t0 = slot, requests, batch, dim, t0
        self._rows: np.ndarray | None = None
        self._error: Exception | None = None
        self._ms = 0.0

    def _settle(self) -> None:
        """Wait for the batch and move its result out of the pinned slot."""
        if self._rows is not None or self._error is not None:
            return
        slot = self._slot
        slot.done.synchronize()
        e = int(slot.host_err[0])
        if e & 4:  # the host plan and the device pool disagree: a bug, not bad input
            self._error = RuntimeError("event page gather got a malformed plan item")
        elif e:
            self._error = IndexError("event index out of range (neuron_id, time_bin or value outside its "
                                     "embedding table)")
        else:
            self._rows = slot.host_out[:self._B * self._dim].view(self._B, self._dim).numpy().copy()
        self._ms = (time.perf_counter() - self._t0) * 1000
        if slot.pending is self:
            slot.pending = None


class InferenceWorker:
    """Batched inference worker (reference worker.py:92-253); one model, one GPU.

    ``use_graphs`` replays a captured graph per (batch bucket, event bucket), keeping at
    most ``max_graphs`` of them (least recently used evicted); all share one memory pool,
    which is safe because batches never overlap.  ``captures`` counts the graphs
    captured so far.
    """

    def __init__(self, model: nn.Module, config: CortexConfig, device: torch.device, max_batch_size: int = 32,
                 *, use_graphs: bool = True, max_graphs: int = 128) -> None:
        device = torch.device(device)
        if device.type != "cuda":
            raise RuntimeError("InferenceWorker runs the gfx950 forward; it needs a ROCm device")
        if device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        self.model = model
        self.config = config
        self.device = device
        self.max_batch_size = max_batch_size
        self.use_graphs = use_graphs
        self.max_graphs = max_graphs
        self._executor = ThreadPoolExecutor(max_workers=1, thread_name_prefix="inference")
        self._stream = torch.cuda.Stream(device=device)  # default priority
        self._graphs: OrderedDict[tuple[int, int], _CsrGraph] = OrderedDict()
        self._pool = torch.cuda.graph_pool_handle() if use_graphs else None
        self._slots = (_Slot(), _Slot())
        self._next_slot = 0
        self._plan_dev: torch.Tensor | None = None
        self._loaded = False
        self.captures = 0

    # ------------------------------------------------------------------ API

    def warmup(self, n_iters: int = 3) -> None:
        """Dummy batches of 64 events each (reference worker.py:135-147)."""
        dummy = [{"request_id": f"warmup_{i}", "events": [{"neuron_id": 0, "time_bin": 0, "value": 0}] * 64}
                 for i in range(min(n_iters, self.max_batch_size))]
        for _ in range(n_iters):
            self._run_batch_sync(dummy)
        self._loaded = True

    @property
    def ready(self) -> bool:
        return self._loaded

    async def run_batch(self, payloads: list[dict[str, Any]]) -> list[dict[str, Any]]:
        """Async entry point: the batch runs on the worker's executor thread."""
        if not payloads:
            return []
        loop = asyncio.get_running_loop()
        return await loop.run_in_executor(self._executor, self._run_batch_sync, payloads)

    def shutdown(self) -> None:
        self._executor.shutdown(wait=False)

    # ------------------------------------------------------------------ batch

    def submit_batch(self, payloads: list[dict[str, Any]]) -> PendingBatch:
        """``_run_batch_sync`` without the wait: packs the payloads into a pinned slot, queues
        the copy, the forward and the result copy on the worker stream and returns at once,
        so the host can pack the next batch while this one runs (two in flight, as
        ``submit_windows``).  ``collect`` gives the result dicts.  Not thread-safe."""
        t0 = time.perf_counter()
        slot = self._acquire_slot()
        flat, B, E, Eb = pack_payloads(payloads, self.use_graphs, slot.host_in.numpy(), batch_pad=self.use_graphs)
        dim = self.config.behavior_dim
        pending = PendingBatch(slot, payloads, B, dim, t0)
        if B == 0:
            pending._rows = np.zeros((0, dim), dtype=np.float32)
            pending._ms = (time.perf_counter() - t0) * 1000
            return pending
        src = self._stage(slot, flat, 3 * Eb + self._bb(B) + 1)
        self._launch(slot, B, Eb, lambda inp, err: inp.copy_(src, non_blocking=True))
        slot.pending = pending
        return pending

    def _run_batch_sync(self, payloads: list[dict[str, Any]]) -> list[dict[str, Any]]:
        """One synchronous forward over ``payloads`` (runs on the executor thread).

        As in the reference, the model batch ends at the last payload that has
        events (``max(batch_indices) + 1``); later payloads get zeros.
        """
        t0 = time.perf_counter()
        dim = self.config.behavior_dim
        slot = self._acquire_slot()
        flat, B, E, Eb = pack_payloads(payloads, self.use_graphs, slot.host_in.numpy(), batch_pad=self.use_graphs)
        if B == 0:
            ms = (time.perf_counter() - t0) * 1000
            return [{"request_id": p["request_id"], "behavior": [0.0] * dim, "inference_ms": ms} for p in payloads]
        src = self._stage(slot, flat, 3 * Eb + self._bb(B) + 1)
        behavior = self._forward(slot, B, Eb, lambda inp, err: inp.copy_(src, non_blocking=True))
        ms = (time.perf_counter() - t0) * 1000
        rows = behavior.tolist()
        return [{"request_id": p["request_id"], "behavior": rows[i] if i < B else [0.0] * dim, "inference_ms": ms}
                for i, p in enumerate(payloads)]

    def run_windows_sync(self, requests: list[dict[str, Any]], cache: Any, window_bins: int = 600
                         ) -> list[dict[str, Any]]:
        """Streaming batch: each request ``{"request_id", "session_id", "window_start"}`` names a
        decode window whose event pages are already in ``cache`` (an ``EventWindowCache`` on this
        device).  The window inputs are gathered on the device into the forward's input buffer;
        only the gather plan and the offsets cross PCIe.  Same result dicts as ``run_batch``."""
        if not requests:
            return []
        return self.collect(self.submit_windows(requests, cache, window_bins))

    def submit_windows(self, requests: list[dict[str, Any]], cache: Any, window_bins: int = 600) -> PendingBatch:
        """``run_windows_sync`` without the wait: plans the batch, queues the page gather,
        the forward and the result copy on the worker stream, and returns at once.  While it
        runs the host can write the next stride's pages and submit the next batch (two
        batches in flight; submitting a third first settles the oldest).  ``collect`` gives
        the result dicts.  Not thread-safe, like the cache."""
        t0 = time.perf_counter()
        if not requests:
            raise ValueError("submit_windows needs at least one request")
        items, offsets = cache.plan([(r["session_id"], int(r["window_start"])) for r in requests], window_bins)
        B, E = len(requests), int(offsets[-1])
        Bb = self._bb(B)
        Eb = event_bucket(E) if self.use_graphs else max(E, 1)
        n_host = Bb + 1 + items.size
        slot = self._acquire_slot()
        if slot.host_in.numel() < n_host:
            slot.host_in = torch.empty(max(n_host, 2 * slot.host_in.numel()), dtype=torch.int64).pin_memory()
        h = slot.host_in.numpy()
        h[:B + 1] = offsets
        h[B + 1:Bb + 1] = E  # padding samples: empty
        h[Bb + 1:n_host] = items.reshape(-1)
        have = 0 if self._plan_dev is None else self._plan_dev.numel()
        if have < max(items.size, 4):
            self._stream.synchronize()  # the old plan buffer may still be read by a queued gather
            self._plan_dev = torch.empty(max(items.size, 4, 2 * have), dtype=torch.int64, device=self.device)
        plan_dev = self._plan_dev[:items.size].view(-1, 4)
        off_host, plan_host = slot.host_in[:Bb + 1], slot.host_in[Bb + 1:n_host]

        def fill(inp: torch.Tensor, err: torch.Tensor) -> None:
            inp[3 * Eb:3 * Eb + Bb + 1].copy_(off_host, non_blocking=True)
            if items.shape[0]:
                plan_dev.view(-1).copy_(plan_host, non_blocking=True)
                cache.gather(plan_dev, inp, Eb, E, err)

        self._stream.wait_stream(torch.cuda.current_stream(self.device))  # page writes issued on it
        self._launch(slot, B, Eb, fill)
        pending = PendingBatch(slot, requests, B, self.config.behavior_dim, t0)
        slot.pending = pending
        return pending

    def collect(self, pending: PendingBatch) -> list[dict[str, Any]]:
        """Result dicts of a submitted batch (waits for it).  As in ``_run_batch_sync``,
        requests past the model batch (no events) get zeros."""
        pending._settle()
        if pending._error is not None:
            raise pending._error
        rows = pending._rows.tolist()
        zero = [0.0] * self.config.behavior_dim
        return [{"request_id": r["request_id"], "behavior": rows[i] if i < len(rows) else zero,
                 "inference_ms": pending._ms} for i, r in enumerate(pending.requests)]

    def _acquire_slot(self) -> _Slot:
        """The next pinned slot, once the batch that used it last is off the GPU (its result,
        if nobody collected it yet, moves to host memory first)."""
        slot = self._slots[self._next_slot]
        self._next_slot ^= 1
        if slot.pending is not None:
            slot.pending._settle()
        slot.done.synchronize()
        return slot

    def _bb(self, B: int) -> int:
        """Samples the forward runs for B real ones (the graph's batch bucket)."""
        return batch_bucket(B) if self.use_graphs else B

    @staticmethod
    def _stage(slot: _Slot, flat: np.ndarray, n_in: int) -> torch.Tensor:
        """The first ``n_in`` words of the packed batch in the slot's pinned buffer."""
        if flat.ctypes.data != slot.host_in.data_ptr():  # did not fit: grow the pinned buffer
            slot.host_in = torch.empty(max(n_in, 2 * slot.host_in.numel()), dtype=torch.int64).pin_memory()
            slot.host_in.numpy()[:n_in] = flat[:n_in]
        return slot.host_in[:n_in]

    def _launch(self, slot: _Slot, B: int, Eb: int, fill) -> None:
        """``fill(inp, err)`` writes the (Bb, Eb) input buffer on the worker stream (Bb =
        ``_bb(B)``); then the forward runs and the first B rows of the behaviour are copied
        into ``slot`` (no host wait)."""
        dim = self.config.behavior_dim
        Bb = self._bb(B)
        if slot.host_out.numel() < B * dim:
            slot.host_out = torch.empty(max(B * dim, 2 * slot.host_out.numel()), dtype=torch.float32).pin_memory()
        with torch.cuda.device(self.device), torch.cuda.stream(self._stream):
            if self.use_graphs:
                g = self._graph(Bb, Eb)
                g.err.zero_()
                fill(g.inp, g.err)
                g.graph.replay()
                out, err = g.out[:B], g.err
            else:
                inp = torch.empty(3 * Eb + B + 1, dtype=torch.int64, device=self.device)
                err = torch.zeros(1, dtype=torch.int32, device=self.device)
                fill(inp, err)
                with torch.inference_mode():
                    out = self.model.forward_csr(inp[:Eb], inp[Eb:2 * Eb], inp[2 * Eb:3 * Eb], inp[3 * Eb:],
                                                 err_flag=err)
            slot.host_out[:B * dim].view(B, dim).copy_(out, non_blocking=True)
            slot.host_err.copy_(err, non_blocking=True)
            slot.done.record(self._stream)

    def _forward(self, slot: _Slot, B: int, Eb: int, fill) -> np.ndarray:
        """``_launch`` and wait: the (B, dim) behaviour on the host."""
        pending = PendingBatch(slot, [], B, self.config.behavior_dim, time.perf_counter())
        slot.pending = pending
        self._launch(slot, B, Eb, fill)
        pending._settle()
        if pending._error is not None:
            raise pending._error
        return pending._rows

    def _graph(self, B: int, Eb: int) -> _CsrGraph:
        key = (B, Eb)
        g = self._graphs.get(key)
        if g is None:
            if len(self._graphs) >= self.max_graphs:
                self._stream.synchronize()  # the evicted graph may still be replaying
                self._graphs.popitem(last=False)
            g = _CsrGraph(self.model, B, Eb, self.device, self._stream, self._pool)
            self._graphs[key] = g
            self.captures += 1
        else:
            self._graphs.move_to_end(key)
        return g
