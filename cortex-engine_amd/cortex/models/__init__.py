"""Cortex model modules (reference cortex/models)."""

from cortex.models.config import CortexConfig
from cortex.models.cortex import CortexModel
from cortex.models.tokenizer import SpikeTokenizer

__all__ = ["CortexConfig", "CortexModel", "SpikeTokenizer"]
