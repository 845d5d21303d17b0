"""Module-level glue between nn.Linear / QuantizedLinear / nn.LayerNorm and the
fused HIP ops (norm prologue, dequant + bias + GELU + residual epilogue)."""

from __future__ import annotations

import torch
from torch import nn

from cortex.kernels import ops


def linear_weights(lin: nn.Module) -> dict:
    """Weight arguments of ``ops.norm_linear`` for an nn.Linear or a QuantizedLinear."""
    if hasattr(lin, "weight_int8"):
        return {"weight_int8": lin.weight_int8, "weight_scale": lin.weight_scale, "bias": lin.bias}
    return {"weight": lin.weight, "bias": lin.bias}


def apply_linear(lin: nn.Module, x: torch.Tensor, *, norm: nn.LayerNorm | None = None, stats=None,
                 act: str | None = None, residual: torch.Tensor | None = None, res_rows: int = 0,
                 out_dtype: torch.dtype, compute: torch.dtype, out: torch.Tensor | None = None) -> torch.Tensor:
    """``act(lin(norm(x))) + residual`` as one fused kernel.

    When the linear carries forward pre-hooks (calibration), its input is
    materialised first and handed to the hooks exactly as ``nn.Module.__call__``
    would, then the linear runs on it.
    """
    if lin._forward_pre_hooks:
        xin = x if norm is None else ops.layer_norm(x, norm.weight, norm.bias, norm.eps, out_dtype=x.dtype)
        for hook in list(lin._forward_pre_hooks.values()):
            hook(lin, (xin,))
        return ops.norm_linear(xin, **linear_weights(lin), act=act, residual=residual, res_rows=res_rows,
                               out_dtype=out_dtype, compute_dtype=compute, out=out)
    kw = {}
    if norm is not None:
        kw = {"norm": "layer", "gamma": norm.weight, "beta": norm.bias, "eps": norm.eps, "stats": stats}
    return ops.norm_linear(x, **linear_weights(lin), **kw, act=act, residual=residual, res_rows=res_rows,
                           out_dtype=out_dtype, compute_dtype=compute, out=out)
