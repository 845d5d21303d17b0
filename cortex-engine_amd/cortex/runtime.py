"""HIP-graph capture of the Cortex forward for a fixed (batch_size, n_events).

The forward is a fixed sequence of ~45 kernel launches once B and the total event
count are known (the pack plan and every per-sample length live on the device).
Capturing it once and replaying removes the host launch cost, which dominates at
small batches (serving latency at B = 1).
"""

from __future__ import annotations

import torch

from cortex.models.cortex import CortexModel, _raise_on_flag


class CapturedForward:
    """Replayable ``model(neuron_ids, time_bins, values, batch_indices)["behavior"]``.

    The graph reads its events from four static int64 device buffers of length
    ``n_events``.  By default they are allocated here and ``cap(nid, tb, val, bidx)`` copies
    the caller's tensors into them before each replay.  A caller whose events already live in
    device buffers it owns can pass them as ``inputs=(nid, tb, val, bidx)``: the graph is then
    captured on those buffers, and ``cap()`` replays on whatever they hold, with no copies.
    Writing new events into them (``cap.neuron_ids.copy_(...)``, an H2D straight from pinned
    memory, ...) before ``cap()`` serves the next request.

    The returned tensor is the graph's static output (clone it to keep it past the next call).
    ``err_flag`` is cleared at the start of every replay (by the pack plan's first kernel), so
    after a call it holds that call's index-range violations only; with
    ``check_indices=True`` each call reads it back (one synchronisation) and raises
    ``IndexError`` as ``CortexModel.forward`` does.
    """

    def __init__(self, model: CortexModel, batch_size: int, n_events: int, warmup: int = 2, *,
                 check_indices: bool = False, inputs: tuple[torch.Tensor, ...] | None = None) -> None:
        if n_events < 1 or batch_size < 1:
            raise ValueError("need batch_size >= 1 and n_events >= 1")
        dev = next(model.parameters()).device
        if dev.type != "cuda":
            raise RuntimeError("CapturedForward needs the model on a ROCm device")
        self.model = model
        self.check_indices = check_indices
        self.batch_size = batch_size
        self.n_events = n_events
        if inputs is None:
            self.neuron_ids = torch.zeros(n_events, dtype=torch.int64, device=dev)
            self.time_bins = torch.zeros(n_events, dtype=torch.int64, device=dev)
            self.values = torch.zeros(n_events, dtype=torch.int64, device=dev)
            self.batch_indices = (torch.arange(n_events, device=dev) * batch_size) // n_events
        else:
            if len(inputs) != 4:
                raise ValueError("inputs must be (neuron_ids, time_bins, values, batch_indices)")
            for t in inputs:
                if (t.device != dev or t.dtype != torch.int64 or t.dim() != 1 or t.shape[0] != n_events
                        or not t.is_contiguous()):
                    raise ValueError(f"inputs must be contiguous int64 ({n_events},) tensors on {dev}")
            self.neuron_ids, self.time_bins, self.values, self.batch_indices = inputs
        self.err_flag = torch.zeros(1, dtype=torch.int32, device=dev)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side), torch.inference_mode():
            for _ in range(warmup):
                self._run()
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph), torch.inference_mode():
            self.output = self._run()

    def _run(self) -> torch.Tensor:
        # the pack plan zeroes the flag in its first launch (no fill kernel, no memset node)
        return self.model(self.neuron_ids, self.time_bins, self.values, self.batch_indices,
                          batch_size=self.batch_size, err_flag=self.err_flag, clear_err=True)["behavior"]

    def __call__(self, *events: torch.Tensor) -> torch.Tensor:
        """Replay on the static buffers; with four tensors, copy them in first."""
        if events:
            if len(events) != 4:
                raise ValueError("pass (neuron_ids, time_bins, values, batch_indices) or nothing")
            if events[0].shape[0] != self.n_events:
                raise ValueError(f"captured for {self.n_events} events, got {events[0].shape[0]}")
            for dst, src in zip((self.neuron_ids, self.time_bins, self.values, self.batch_indices), events):
                if src.data_ptr() != dst.data_ptr():
                    dst.copy_(src, non_blocking=True)
        self.graph.replay()
        if self.check_indices:
            _raise_on_flag(self.err_flag)
        return self.output
