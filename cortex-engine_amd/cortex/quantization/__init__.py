"""INT8 weight-only post-training quantisation (reference cortex/quantization)."""
