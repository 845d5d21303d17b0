"""Fused RMSNorm (or LayerNorm) + linear on gfx950.

Drop-in for ``cortex.kernels.fused_rmsnorm`` of the reference
(cortex/kernels/fused_rmsnorm.py:86-301).  ``rms_norm_linear`` keeps the reference
signature (``w`` pre-transposed ``(K, N)``) and semantics
``((x_f32 / rms) * gamma).to(x.dtype) @ w (+ bias)``: per-row statistics in fp32,
the normalised row rounded to x's dtype while it is staged into LDS, the contraction
on MFMA (bf16 for bf16 inputs, fp32 for fp32 inputs) with fp32 accumulation.
``norm_linear_int8`` is the same kernel on QuantizedLinear's int8 ``(N, K)``
weights with the per-channel scale applied in the epilogue.
"""

from __future__ import annotations

import torch

from cortex import _native as nat
from cortex.kernels import ops


def rms_norm_linear_reference(x, gamma, w, bias=None, eps: float = 1e-6):
    """PyTorch formulation (reference fused_rmsnorm.py:86-108): what ``rms_norm_linear`` returns
    for rows that are not on a ROCm device, as the reference dispatcher does.  GPU tensors
    never reach it."""
    x_f32 = x.float()
    rms = torch.sqrt(x_f32.pow(2).mean(dim=-1, keepdim=True) + eps)
    x_norm = (x_f32 / rms) * gamma.float()
    out = x_norm.to(x.dtype) @ w
    if bias is not None:
        out = out + bias
    return out


def rms_norm_linear(x: torch.Tensor, gamma: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None = None,
                    eps: float = 1e-6) -> torch.Tensor:
    """Fused RMSNorm + linear, output ``(..., N)`` in x's dtype (reference :239-301).

    Rows on a ROCm device run the HIP kernel; on any other device the call returns
    ``rms_norm_linear_reference`` over the flattened rows (reference :266-269)."""
    if x.device.type != "cuda":
        lead, K = x.shape[:-1], x.shape[-1]
        return rms_norm_linear_reference(x.reshape(-1, K), gamma, w, bias, eps).reshape(*lead, w.shape[1])
    nat.require_gpu(x, gamma, w, bias, what="rms_norm_linear")
    if w.dtype != x.dtype:
        raise RuntimeError(f"rms_norm_linear: w dtype {w.dtype} differs from x dtype {x.dtype}")
    compute = torch.bfloat16 if x.dtype == torch.bfloat16 else torch.float32
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise RuntimeError(f"rms_norm_linear: dtype {x.dtype} not supported (bfloat16 or float32)")
    return ops.norm_linear(x, weight=w, w_layout="kn", norm="rms", gamma=gamma, eps=eps, bias=bias,
                           out_dtype=x.dtype, compute_dtype=compute)


def norm_linear_int8(x: torch.Tensor, weight_int8: torch.Tensor, weight_scale: torch.Tensor, *,
                     norm: str | None = "rms", gamma: torch.Tensor | None = None,
                     beta: torch.Tensor | None = None, eps: float = 1e-6, bias: torch.Tensor | None = None,
                     act: str | None = None, residual: torch.Tensor | None = None,
                     out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Norm (``'rms'``, ``'layer'`` or None) + INT8 per-channel linear (+GELU, +residual).

    ``weight_int8`` is ``(N, K)`` int8 and ``weight_scale`` ``(N,)`` fp32 as stored by
    QuantizedLinear (reference calibrate.py:192-193).  bf16 inputs use bf16 MFMA,
    fp32 inputs fp32 MFMA; the int8 weights are widened exactly.
    """
    nat.require_gpu(x, weight_int8, weight_scale, gamma, beta, bias, residual, what="norm_linear_int8")
    compute = torch.bfloat16 if x.dtype == torch.bfloat16 else torch.float32
    return ops.norm_linear(x, weight_int8=weight_int8, weight_scale=weight_scale, norm=norm, gamma=gamma,
                           beta=beta, eps=eps, bias=bias, act=act, residual=residual,
                           out_dtype=out_dtype or x.dtype, compute_dtype=compute)
