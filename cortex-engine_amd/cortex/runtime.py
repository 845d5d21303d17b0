"""HIP-graph capture of the Cortex forward for a fixed (batch_size, n_events).

The forward is a fixed sequence of ~60 kernel launches once B and the total event
count are known (the pack plan and every per-sample length live on the device).
Capturing it once and replaying removes the host launch cost, which dominates at
small batches (serving latency at B = 1).
"""

from __future__ import annotations

import torch

from cortex.models.cortex import CortexModel, _raise_on_flag


class CapturedForward:
    """Replayable ``model(neuron_ids, time_bins, values, batch_indices)["behavior"]``.

    Inputs are copied into static device buffers before each replay; the returned
    tensor is the graph's static output (clone it to keep it past the next call).
    ``err_flag`` is cleared before every replay, so after a call it holds that call's
    index-range violations only; with ``check_indices=True`` each call reads it back
    (one synchronisation) and raises ``IndexError`` as ``CortexModel.forward`` does.
    """

    def __init__(self, model: CortexModel, batch_size: int, n_events: int, warmup: int = 2, *,
                 check_indices: bool = False) -> None:
        if n_events < 1 or batch_size < 1:
            raise ValueError("need batch_size >= 1 and n_events >= 1")
        dev = next(model.parameters()).device
        if dev.type != "cuda":
            raise RuntimeError("CapturedForward needs the model on a ROCm device")
        self.model = model
        self.check_indices = check_indices
        self.batch_size = batch_size
        self.n_events = n_events
        self.neuron_ids = torch.zeros(n_events, dtype=torch.int64, device=dev)
        self.time_bins = torch.zeros(n_events, dtype=torch.int64, device=dev)
        self.values = torch.zeros(n_events, dtype=torch.int64, device=dev)
        self.batch_indices = (torch.arange(n_events, device=dev) * batch_size) // n_events
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
        return self.model(self.neuron_ids, self.time_bins, self.values, self.batch_indices,
                          batch_size=self.batch_size, err_flag=self.err_flag)["behavior"]

    def __call__(self, neuron_ids, time_bins, values, batch_indices) -> torch.Tensor:
        if neuron_ids.shape[0] != self.n_events:
            raise ValueError(f"captured for {self.n_events} events, got {neuron_ids.shape[0]}")
        self.neuron_ids.copy_(neuron_ids, non_blocking=True)
        self.time_bins.copy_(time_bins, non_blocking=True)
        self.values.copy_(values, non_blocking=True)
        self.batch_indices.copy_(batch_indices, non_blocking=True)
        self.err_flag.zero_()  # a fill kernel, outside the graph
        self.graph.replay()
        if self.check_indices:
            _raise_on_flag(self.err_flag)
        return self.output
