"""Opt-in W8A8 execution of the self-attention MLPs (int8 activations x int8 weights).

The reference derives a per-tensor activation scale for every linear during
calibration (``derive_scales``, cortex/quantization/calibrate.py:145-150: the
99th-percentile absmax of the linear's input over the calibration batches, / 127)
and never uses it: ``QuantizedLinear.forward`` dequantises the weight and multiplies
the float activations (calibrate.py:225-228).  This module uses those scales:

    xq = clamp(rint(x * (1 / act_scale)), -127, 127)          (int8, round half to even)
    y  = act_scale * weight_scale[n] * sum_k xq[k] weight_int8[n, k] + bias[n]

with the sum exact in int32 on the gfx950 int8 MFMA.  In each self-attention block
the out-projection kernel writes ``norm_mlp(x)`` straight as int8 at mlp.0's scale,
mlp.0 writes ``GELU(.)`` as int8 at mlp.2's scale, and mlp.2 adds its fp32 result to
the residual stream.  When qkv_proj and out_proj are quantised with scales too, the
attention half runs the same way: ``norm_attn(x)`` as int8 at qkv_proj's scale, the
fused qkv projection + attention on int8 operands writing its output as int8 at
out_proj's scale, and out_proj on int8 operands.  The attention itself (softmax, P V)
stays bf16, and everything outside the self-attention blocks keeps the default path.

This is NOT the reference's arithmetic: activations lose precision to 8 bits (the
saturation at the calibrated absmax included).  It is off unless ``enable_w8a8`` is
called, and the state_dict is unchanged (the scales live on the modules as plain
attributes).
"""

from __future__ import annotations

import torch.nn as nn

from cortex.quantization.calibrate import LayerScales, QuantizedLinear

_ATTR = "_cortex_w8a8"


def enable_w8a8(model: nn.Module, scales: dict[str, LayerScales]) -> int:
    """Switch to W8A8 every self-attention block whose ``mlp.0`` and ``mlp.2`` are
    ``QuantizedLinear`` with calibrated scales in ``scales`` (module name -> LayerScales,
    as ``derive_scales`` returns for the float model): its MLP, and also its attention half
    when ``qkv_proj`` and ``out_proj`` are quantised with scales too.  Returns the number of
    blocks switched."""
    from cortex.models.perceiver import SelfAttentionBlock

    def scale(name: str, lin: nn.Module) -> float | None:
        s = scales.get(name)
        ok = isinstance(lin, QuantizedLinear) and s is not None and s.act_scale > 0
        return float(s.act_scale) if ok else None

    n = 0
    for name, mod in model.named_modules():
        if not isinstance(mod, SelfAttentionBlock):
            continue
        s_up, s_down = scale(f"{name}.mlp.0", mod.mlp[0]), scale(f"{name}.mlp.2", mod.mlp[2])
        if s_up is None or s_down is None:
            continue
        s_qkv, s_out = scale(f"{name}.qkv_proj", mod.qkv_proj), scale(f"{name}.out_proj", mod.out_proj)
        attn = (s_qkv, s_out) if s_qkv is not None and s_out is not None else None
        mod.__dict__[_ATTR] = (s_up, s_down, attn)
        n += 1
    return n


def disable_w8a8(model: nn.Module) -> None:
    """Back to the default (bf16-activation) path everywhere."""
    for mod in model.modules():
        mod.__dict__.pop(_ATTR, None)


def w8a8_scales(block: nn.Module) -> tuple | None:
    """``(act_scale of mlp.0, act_scale of mlp.2, attn)`` when ``block`` runs its MLP as W8A8;
    ``attn`` is ``(act_scale of qkv_proj, act_scale of out_proj)`` when its attention half
    does too, else None."""
    return block.__dict__.get(_ATTR)
