"""Spike tokenizer module (reference cortex/models/tokenizer.py:39-93).

Three embeddings (neuron id, time bin, value bucket) created and re-initialised
N(0, 0.02) in the reference's order; on a ROCm device the forward is the fused HIP
gather-add kernel.
"""

from __future__ import annotations

import torch
from torch import nn

from cortex.kernels import ops
from cortex.models.config import CortexConfig


class SpikeTokenizer(nn.Module):
    """Embed spike events as tokens: ``(N[nid] + T[tb]) + V[val]``."""

    def __init__(self, config: CortexConfig) -> None:
        super().__init__()
        self.config = config
        self.neuron_emb = nn.Embedding(config.max_neurons, config.hidden_dim)
        self.time_emb = nn.Embedding(config.max_time_bins, config.hidden_dim)
        self.value_emb = nn.Embedding(config.spike_value_buckets, config.hidden_dim)
        self._init_weights()

    def _init_weights(self) -> None:
        for emb in (self.neuron_emb, self.time_emb, self.value_emb):
            nn.init.normal_(emb.weight, std=0.02)

    def forward(self, neuron_ids: torch.Tensor, time_bins: torch.Tensor, values: torch.Tensor) -> torch.Tensor:
        """``(E,)`` int64 indices -> ``(E, hidden_dim)`` tokens in the tables' dtype."""
        if not (neuron_ids.shape == time_bins.shape == values.shape):
            raise ValueError(
                f"shape mismatch: neuron_ids={neuron_ids.shape}, "
                f"time_bins={time_bins.shape}, values={values.shape}"
            )
        E = neuron_ids.shape[0]
        if E == 0:
            return torch.empty((0, self.config.hidden_dim), dtype=self.neuron_emb.weight.dtype,
                               device=self.neuron_emb.weight.device)
        return ops.tokenize(self.neuron_emb.weight, self.time_emb.weight, self.value_emb.weight,
                            neuron_ids, time_bins, values)
