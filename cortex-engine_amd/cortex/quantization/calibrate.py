"""INT8 per-channel weight quantisation with calibration, on gfx950.

Drop-in for ``cortex.quantization.calibrate`` of the reference
(cortex/quantization/calibrate.py:55-362): the same public names, buffers and
state_dict keys (``weight_int8`` int8 (N, K), ``weight_scale`` fp32 (N,),
``bias``).  What changes is where the arithmetic runs:

* the weight scale ``max(|W[n,:]|, 1e-8) / 127`` and the quantise step
  ``clamp(round_half_even(W / scale), -127, 127)`` run in one HIP kernel, bit-exact
  with the reference formula (IEEE division, round half to even);
* ``QuantizedLinear.forward`` never materialises a dequantised weight: the int8
  weight is widened exactly inside the MFMA GEMM and the per-channel scale is
  applied to the fp32 accumulator in the epilogue.

Calibration bookkeeping (hooks, percentiles, conversion, save/load) is host logic
and keeps the reference behaviour.  Weight arithmetic requires the model on a
ROCm device.
"""

from __future__ import annotations

import copy
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

import torch
import torch.nn as nn

from cortex import _native as nat
from cortex.kernels import ops

# ---------------------------------------------------------------- calibration


@dataclass
class ActivationStats:
    """Per-layer activation abs-max history (reference calibrate.py:55-83)."""

    abs_max_history: list[float] = field(default_factory=list)

    def update(self, x: torch.Tensor) -> None:
        self.abs_max_history.append(float(x.detach().abs().max().item()))

    @property
    def percentile_99(self) -> float:
        """Element ``max(0, int(0.99 n) - 1)`` of the sorted history; 1.0 when empty."""
        if not self.abs_max_history:
            return 1.0
        vals = sorted(self.abs_max_history)
        return vals[max(0, int(len(vals) * 0.99) - 1)]

    @property
    def n_batches(self) -> int:
        return len(self.abs_max_history)


class CalibrationHook:
    """Forward pre-hook recording the input of a linear layer (reference :86-97)."""

    def __init__(self) -> None:
        self.stats = ActivationStats()
        self._handle: Any = None

    def __call__(self, module: nn.Module, args: tuple[Any, ...]) -> None:
        if args:
            self.stats.update(args[0])

    def remove(self) -> None:
        if self._handle is not None:
            self._handle.remove()
            self._handle = None


def attach_calibration_hooks(model: nn.Module) -> dict[str, CalibrationHook]:
    """Attach a pre-hook to every ``nn.Linear``; return ``name -> hook``."""
    hooks: dict[str, CalibrationHook] = {}
    for name, module in model.named_modules():
        if isinstance(module, nn.Linear):
            hook = CalibrationHook()
            hook._handle = module.register_forward_pre_hook(hook)
            hooks[name] = hook
    return hooks


def remove_calibration_hooks(hooks: dict[str, CalibrationHook]) -> None:
    for hook in hooks.values():
        hook.remove()


# ---------------------------------------------------------------- scales


@dataclass
class LayerScales:
    """Quantisation scales of one linear layer."""

    weight_scale: torch.Tensor  # (out_features,) fp32
    act_scale: float


def weight_scale(weight: torch.Tensor) -> torch.Tensor:
    """Per-output-channel scale ``max(max_k |W[n,k]|, 1e-8) / 127`` (HIP kernel)."""
    w = weight.detach().float()
    dev = nat.require_gpu(w, what="weight_scale")
    w = ops._row_major_2d(w)
    N, K = w.shape
    s = torch.empty(N, dtype=torch.float32, device=dev)
    nat.call("cortex_quantize_int8", nat.ptr(w), N, K, w.stride(0) if N > 1 else K, None, nat.ptr(s), None, K,
             nat.stream_of(dev))
    return s


def derive_scales(model: nn.Module, hooks: dict[str, CalibrationHook]) -> dict[str, LayerScales]:
    """Scales for every ``nn.Linear`` whose hook saw at least one batch (reference :127-164)."""
    scales: dict[str, LayerScales] = {}
    for name, module in model.named_modules():
        if not isinstance(module, nn.Linear) or name not in hooks:
            continue
        hook = hooks[name]
        if hook.stats.n_batches == 0:
            continue
        ws = weight_scale(module.weight)
        act_scale = max(hook.stats.percentile_99, 1e-8) / 127.0
        scales[name] = LayerScales(weight_scale=ws.cpu(), act_scale=act_scale)
    return scales


# ---------------------------------------------------------------- QuantizedLinear


class QuantizedLinear(nn.Module):
    """``nn.Linear`` replacement holding int8 per-channel weights (reference :170-235).

    ``forward`` runs the HIP INT8 GEMM: int8 weights widened exactly inside the
    kernel, fp32 accumulation, ``* weight_scale[n] (+ bias[n])`` in the epilogue;
    output in ``x.dtype`` (bf16 inputs use bf16 MFMA, fp32 inputs fp32 MFMA).
    """

    in_features: int
    out_features: int
    weight_int8: torch.Tensor
    weight_scale: torch.Tensor
    bias: torch.Tensor | None

    def __init__(self, weight_int8: torch.Tensor, weight_scale: torch.Tensor, bias: torch.Tensor | None) -> None:
        super().__init__()
        self.in_features = weight_int8.shape[1]
        self.out_features = weight_int8.shape[0]
        self.register_buffer("weight_int8", weight_int8)
        self.register_buffer("weight_scale", weight_scale)
        self.register_buffer("bias", bias)

    @classmethod
    def from_linear(cls, linear: nn.Linear, scales: LayerScales) -> QuantizedLinear:
        """Quantise a float ``nn.Linear`` with pre-computed scales (HIP kernel)."""
        w = linear.weight.detach().float()
        s = scales.weight_scale.to(w.device)
        q, s = ops.quantize_int8(w, s)
        bias = linear.bias.detach().clone() if linear.bias is not None else None
        return cls(q, s, bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        compute = torch.bfloat16 if x.dtype == torch.bfloat16 else torch.float32
        return ops.norm_linear(x, weight_int8=self.weight_int8, weight_scale=self.weight_scale, bias=self.bias,
                               out_dtype=x.dtype, compute_dtype=compute)

    def extra_repr(self) -> str:
        return (
            f"in_features={self.in_features}, out_features={self.out_features}, "
            f"bias={self.bias is not None}, quantized=INT8"
        )


# ---------------------------------------------------------------- conversion


def convert_model(model: nn.Module, scales: dict[str, LayerScales], inplace: bool = True) -> nn.Module:
    """Replace every ``nn.Linear`` that has scales by a ``QuantizedLinear`` (reference :240-264)."""
    if not inplace:
        model = copy.deepcopy(model)
    _replace_linears(model, scales, prefix="")
    return model


def _replace_linears(module: nn.Module, scales: dict[str, LayerScales], prefix: str) -> None:
    for name, child in list(module.named_children()):
        full_name = f"{prefix}.{name}".lstrip(".")
        if isinstance(child, nn.Linear) and full_name in scales:
            setattr(module, name, QuantizedLinear.from_linear(child, scales[full_name]))
        else:
            _replace_linears(child, scales, full_name)


def model_weight_bytes(model: nn.Module) -> int:
    """Bytes of all parameters and buffers."""
    total = sum(p.numel() * p.element_size() for p in model.parameters())
    return total + sum(b.numel() * b.element_size() for b in model.buffers())


def count_quantized_linears(model: nn.Module) -> tuple[int, int]:
    """``(n_quantized, n_total)`` linear-type layers."""
    n_quant = sum(1 for m in model.modules() if isinstance(m, QuantizedLinear))
    n_float = sum(1 for m in model.modules() if isinstance(m, nn.Linear))
    return n_quant, n_quant + n_float


# ---------------------------------------------------------------- save / load


def save_quantized(model: nn.Module, path: Path, meta: dict[str, Any] | None = None) -> None:
    """``torch.save({'state_dict': ..., 'meta': ...})`` (reference :305-318)."""
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    torch.save({"state_dict": model.state_dict(), "meta": meta or {}}, path)


def load_quantized(path: Path, model: nn.Module) -> nn.Module:
    """Load into an already converted skeleton (reference :321-338); weights_only load."""
    payload = torch.load(path, map_location="cpu", weights_only=True)
    model.load_state_dict(payload["state_dict"])
    return model


def calibration_summary(hooks: dict[str, CalibrationHook], scales: dict[str, LayerScales]) -> list[dict[str, Any]]:
    """Per-layer calibration statistics (reference :344-362)."""
    rows = []
    for name, hook in hooks.items():
        s = scales.get(name)
        rows.append(
            {
                "layer": name,
                "calib_batches": hook.stats.n_batches,
                "act_abs_max_p99": round(hook.stats.percentile_99, 6),
                "act_scale": round(s.act_scale, 8) if s else None,
                "weight_scale_min": round(float(s.weight_scale.min()), 8) if s else None,
                "weight_scale_max": round(float(s.weight_scale.max()), 8) if s else None,
            }
        )
    return rows
