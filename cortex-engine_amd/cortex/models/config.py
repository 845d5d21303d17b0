"""Model configuration (reference cortex/models/config.py:14-103).

Same fields, validation and the three reference sizes.  ``dtype`` -- declared but
never read by the reference -- selects the MFMA input dtype of the HIP forward:
``"bfloat16"`` (default; bf16 operands, fp32 accumulation, fp32 residual stream)
or ``"float32"`` (fp32 operands on fp32 MFMA).
"""

from __future__ import annotations

import torch
from pydantic import BaseModel, Field, model_validator


class CortexConfig(BaseModel):
    """Configuration of the Cortex model family (all architecture fields required)."""

    hidden_dim: int = Field(..., gt=0, description="width of the token and latent vectors")
    num_layers: int = Field(..., gt=0, description="self-attention blocks over the latents")
    num_heads: int = Field(..., gt=0, description="heads of each self-attention block")
    head_dim: int = Field(..., gt=0, description="width of one head (num_heads x head_dim = hidden_dim)")
    mlp_ratio: float = Field(4.0, gt=0, description="hidden width of a block's MLP, as a multiple of hidden_dim")
    dropout: float = Field(0.0, ge=0, lt=1)

    num_latents: int = Field(..., gt=0, description="number of learned latent queries")
    latent_dim: int = Field(..., gt=0, description="width of a latent query")
    cross_attn_heads: int = Field(..., gt=0)

    max_neurons: int = Field(..., gt=0, description="rows of the neuron-id embedding table")
    max_time_bins: int = Field(..., gt=0, description="rows of the time-bin embedding table")
    spike_value_buckets: int = Field(8, gt=0, description="rows of the spike-count embedding table")

    behavior_dim: int = Field(..., gt=0, description="values decoded per sample (2: x and y velocity)")
    use_masked_spike_head: bool = True

    dtype: str = Field("bfloat16", pattern="^(float32|float16|bfloat16)$")

    # Kept for configuration compatibility: on a ROCm device every op of this
    # package runs on the HIP kernels regardless of this flag.
    use_kernels: bool = False

    @model_validator(mode="after")
    def _check_head_consistency(self) -> CortexConfig:
        d, h, w = self.hidden_dim, self.num_heads, self.head_dim
        if d % h:
            raise ValueError(f"{h} heads do not split hidden_dim {d} evenly")
        if h * w != d:
            # the phrase "must equal hidden_dim" is what callers match on
            raise ValueError(f"{h} heads x head_dim {w} = {h * w}: the product must equal hidden_dim ({d})")
        return self

    @property
    def compute_dtype(self) -> torch.dtype:
        """MFMA operand dtype of the HIP forward."""
        if self.dtype == "float16":
            raise NotImplementedError("the Cortex HIP forward computes in bfloat16 or float32, not float16")
        return torch.float32 if self.dtype == "float32" else torch.bfloat16


def _cfg(d: int, layers: int, heads: int, latents: int) -> CortexConfig:
    return CortexConfig(hidden_dim=d, num_layers=layers, num_heads=heads, head_dim=64, num_latents=latents,
                        latent_dim=d, cross_attn_heads=heads, max_neurons=512, max_time_bins=1024,
                        behavior_dim=2)


CORTEX_XS = _cfg(256, 5, 4, 128)
CORTEX_S = _cfg(512, 7, 8, 256)
CORTEX_M = _cfg(768, 11, 12, 384)
