"""gfx950 HIP kernels of the Cortex-S forward, behind the reference's kernel API.

Modules keep the reference's import paths and signatures:
``cortex.kernels.tokenizer`` (fused_tokenizer), ``cortex.kernels.sparse_xattn``
(sparse_cross_attention, build_temporal_block_mask) and
``cortex.kernels.fused_rmsnorm`` (rms_norm_linear), plus ``cortex.kernels.pack``
(device-side ragged-event pack) and ``cortex.kernels.ops`` (functional layer).
"""
