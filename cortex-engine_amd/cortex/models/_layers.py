"""Module-level glue between nn.Linear / QuantizedLinear / nn.LayerNorm and the HIP ops.

bf16 compute (the default):
  * ``norm -> linear`` runs as one LayerNorm row kernel writing bf16 rows
    (``cortex_ln_rows``) followed by the pipelined MFMA GEMM on bf16 operands;
  * the GEMM reads the weight's bf16 execution image, built once per weight tensor
    on the device and cached on the module (rebuilt when the weight's storage or
    version changes).  For a QuantizedLinear the image holds the int8 values
    themselves -- every int8 value is exactly a bf16 value -- and the per-channel
    scale is applied to the fp32 accumulator in the epilogue, so results are
    identical to widening the int8 weight inside the kernel.  With
    ``CORTEX_INT8_WEIGHTS=widen`` no image is kept: every kernel (the GEMMs, the fused
    QKV projection + attention, the residual linear + LayerNorm) streams the int8
    weight and widens it on chip, bit-identical results with a third of the resident
    weight bytes, at some cost in time (the images are the measured-faster default).
    ``CORTEX_INT8_WEIGHTS=window`` keeps only the int8 weights resident as well, plus one
    shared bf16 window per weight group (the cross-attention block; every self-attention
    block in turn): a group is widened into its window by extra workgroups of the row kernel
    that feeds it (the tokenizer + LayerNorm for the cross-attention and the first block,
    each block's own LayerNorm rows after that), so the GEMMs run on bf16 weights at the
    image speed and no launch is added (``WeightWindow``).
    For a float nn.Linear the image is the weight rounded to bf16, as ``F.linear`` on
    bf16 inputs would use it.
fp32 compute: int8 or fp32 weights, fp32 operands, fused norm prologue.
"""

from __future__ import annotations

import os

import torch
from torch import nn

from cortex.kernels import ops

INT8_WEIGHTS = os.environ.get("CORTEX_INT8_WEIGHTS", "image")
_LN_ROWS_K = (256, 512, 768, 1024)


def linear_weights(lin: nn.Module) -> dict:
    """Weight arguments of ``ops.norm_linear`` in their stored form."""
    if hasattr(lin, "weight_int8"):
        return {"weight_int8": lin.weight_int8, "weight_scale": lin.weight_scale, "bias": lin.bias}
    return {"weight": lin.weight, "bias": lin.bias}


class WeightWindow:
    """bf16 windows for INT8-resident weights (``CORTEX_INT8_WEIGHTS=window``).

    Each region is one bf16 buffer that the QuantizedLinears of several groups (modules whose
    linears run together) share in turn: the group last widened into it is resident.  The
    forward hands a group's ``pairs`` (int8 weight, bf16 view) to the row kernel launched just
    before the group runs, which widens them in extra workgroups; a linear of a group that is
    not resident when its weights are asked for is widened on a launch of its own first, so
    every path stays correct.  The resident set is tracked on the host in launch order (graph
    capture records the same sequence); forwards that share a model must run on one stream,
    as its activation buffers already require.

    A linear with a ``role`` ("ln": the residual linear + LayerNorm kernel; "res": the residual
    GEMM) is widened in MFMA fragment order (``ops.frag_weight``'s layout) when the direct-weight
    kernel of that role takes the forward's row count, as the bf16 images are in the default
    mode; the layout is part of what is resident."""

    def __init__(self, regions: dict, device: torch.device, roles: dict | None = None) -> None:
        # regions: name -> [(owner module, [QuantizedLinear, ...]), ...]; roles: id(linear) -> role
        self._views = {}      # id(linear) -> bf16 (N, K) view of its region
        self._owner = {}      # id(linear) -> (region, owner)
        self._pairs = {}      # id(owner) -> [(int8, view), ...]
        self._linears = {}    # id(owner) -> [linear, ...]
        self._held = {}       # region -> (id(owner), version key, layout per linear) resident now
        self._roles = dict(roles or {})
        self.bytes = 0
        for region, groups in regions.items():
            size = max(sum(l.weight_int8.numel() for l in lins) for _, lins in groups)
            buf = torch.empty(size, dtype=torch.bfloat16, device=device)
            self.bytes += buf.numel() * buf.element_size()
            for owner, lins in groups:
                off, pairs = 0, []
                for lin in lins:
                    q = lin.weight_int8
                    view = buf[off:off + q.numel()].view(q.shape)
                    off += q.numel()
                    self._views[id(lin)] = view
                    self._owner[id(lin)] = (region, owner)
                    pairs.append((q, view))
                    lin.__dict__["_cortex_window"] = self
                self._pairs[id(owner)] = pairs
                self._linears[id(owner)] = lins
                owner.__dict__["_cortex_window"] = self

    def _key(self, owner) -> tuple:
        return tuple((l.weight_int8.data_ptr(), l.weight_int8._version) for l in self._linears[id(owner)])

    def reset(self) -> None:
        """Nothing resident: a new forward widens every group it reads."""
        self._held.clear()

    def layout(self, lin: nn.Module, rows: int | None) -> int:
        """K when ``lin`` is to be widened in fragment order for a forward of ``rows`` rows (its
        role's direct-weight kernel takes that shape), else 0."""
        role = self._roles.get(id(lin))
        if role is None or rows is None:
            return 0
        N, K = lin.weight_int8.shape
        if K < 64 or K & (K - 1):
            return 0
        dev = lin.weight_int8.device
        ok = ops.frag_ok(rows, N, K, dev) if role == "ln" else ops.frag_res_ok(rows, N, K, dev)
        return K if ok else 0

    def take(self, owner, rows: int | None = None, plain=None) -> list:
        """The (int8, bf16 view, K) items of ``owner``'s group for a rider launched now, which
        makes it resident (in the layouts for ``rows``; the linear ``plain`` in plain rows);
        empty when it already is."""
        if owner is None or id(owner) not in self._pairs:
            return []
        lins = self._linears[id(owner)]
        region = self._owner[id(lins[0])][0]
        ks = tuple(0 if lin is plain else self.layout(lin, rows) for lin in lins)
        key = (id(owner), self._key(owner), ks)
        if self._held.get(region) == key:
            return []
        self._held[region] = key
        return [(q, v, k) for (q, v), k in zip(self._pairs[id(owner)], ks)]

    def view(self, lin: nn.Module, rows: int | None = None, plain: bool = False) -> torch.Tensor:
        """bf16 weight of ``lin``, its group widened first on a launch of its own unless resident:
        ``lin`` in plain (N, K) rows with ``plain``, else in the layout for ``rows`` rows when
        given (``is_frag`` tells which); the rest of a group widened here is laid out for ``rows``."""
        region, owner = self._owner[id(lin)]
        held = self._held.get(region)
        want = 0 if plain else (self.layout(lin, rows) if rows is not None else None)
        if (held is None or held[:2] != (id(owner), self._key(owner))
                or (want is not None and held[2][self._linears[id(owner)].index(lin)] != want)):
            pairs = self.take(owner, rows, plain=lin if plain else None)
            if pairs:
                ops.widen_int8(pairs)
        return self._views[id(lin)]

    def is_frag(self, lin: nn.Module) -> bool:
        """Whether ``lin``'s resident window holds it in fragment order."""
        region, owner = self._owner[id(lin)]
        held = self._held.get(region)
        return held is not None and held[0] == id(owner) and held[2][self._linears[id(owner)].index(lin)] != 0


def weight_window(owner: nn.Module) -> WeightWindow | None:
    """The window that ``owner``'s group belongs to, in window mode."""
    return owner.__dict__.get("_cortex_window") if INT8_WEIGHTS == "window" else None


def rider(*owners, rows: int | None = None) -> list | None:
    """The weight items that the next row kernel should widen so that ``owners``' groups are
    resident in their window, laid out for a forward of ``rows`` rows (None outside window mode
    or when nothing is to widen)."""
    pairs = []
    for o in owners:
        win = weight_window(o) if o is not None else None
        if win is not None:
            pairs += win.take(o, rows)
    return pairs or None


def build_weight_window(regions: dict, device: torch.device, roles: dict | None = None) -> WeightWindow | None:
    """A ``WeightWindow`` over the QuantizedLinears of ``regions`` (name -> [(owner, [linear])])
    in window mode, None otherwise or when a group holds no int8 weight; ``roles``: id(linear)
    -> "ln" / "res" for the linears whose kernels take a fragment-order weight."""
    if INT8_WEIGHTS != "window":
        return None
    groups = {r: [(o, [l for l in lins if hasattr(l, "weight_int8")]) for o, lins in g] for r, g in regions.items()}
    groups = {r: [(o, lins) for o, lins in g if lins] for r, g in groups.items()}
    groups = {r: g for r, g in groups.items() if g}
    if not groups:
        return None
    for g in groups.values():
        for _, lins in g:
            for lin in lins:
                q = lin.weight_int8
                if not q.is_contiguous() or q.numel() % 16 or q.device != device:
                    return None
    return WeightWindow(groups, device, roles)


def exec_weights(lin: nn.Module, compute: torch.dtype, rows: int | None = None) -> dict:
    """Weight arguments for the GEMM at ``compute`` precision (bf16 image when bf16; in window
    mode the window in plain rows, ``rows`` laying out the rest of a group widened here)."""
    quant = hasattr(lin, "weight_int8")
    if compute != torch.bfloat16 or (quant and INT8_WEIGHTS != "image"):
        win = lin.__dict__.get("_cortex_window") if compute == torch.bfloat16 and INT8_WEIGHTS == "window" else None
        if win is not None:
            return {"weight": win.view(lin, rows, plain=True), "weight_scale": lin.weight_scale, "bias": lin.bias}
        return linear_weights(lin)
    src = lin.weight_int8 if quant else lin.weight
    key = (src.data_ptr(), src._version, tuple(src.shape), src.device)
    cached = lin.__dict__.get("_cortex_exec")
    if cached is None or cached[0] != key:
        if ops.capturing_graph():  # only recorded now: the graph converts on every replay, nothing cached
            return {"weight": ops.convert(src, torch.bfloat16), "weight_scale": lin.weight_scale if quant else None,
                    "bias": lin.bias}
        cached = (key, ops.convert(src, torch.bfloat16))
        lin.__dict__["_cortex_exec"] = cached
    return {"weight": cached[1], "weight_scale": lin.weight_scale if quant else None, "bias": lin.bias}


def fused_weight(lin: nn.Module, rows: int | None = None) -> tuple:
    """``(weight, weight_scale, bias)`` for the fused bf16 kernels (QKV + attention, residual
    linear + LayerNorm): the bf16 image, or with ``CORTEX_INT8_WEIGHTS=widen`` the int8 weight
    itself, which those kernels widen on chip (with ``window``, the bf16 window in plain rows
    when the linear has one; ``rows`` lays out the rest of a group widened here)."""
    if hasattr(lin, "weight_int8") and INT8_WEIGHTS != "image":
        win = lin.__dict__.get("_cortex_window") if INT8_WEIGHTS == "window" else None
        if win is not None:
            return win.view(lin, rows, plain=True), lin.weight_scale, lin.bias
        return lin.weight_int8, lin.weight_scale, lin.bias
    w = exec_weights(lin, torch.bfloat16)
    return w["weight"], w["weight_scale"], w["bias"]


def frag_image(lin: nn.Module) -> torch.Tensor:
    """The linear's weight as bf16 in MFMA fragment order (``ops.frag_weight``), built once per
    weight state and cached on the module like the bf16 image (the direct-weight residual
    LayerNorm kernel streams it; same values as the image)."""
    src = lin.weight_int8 if hasattr(lin, "weight_int8") else lin.weight
    key = (src.data_ptr(), src._version, tuple(src.shape), src.device)
    cached = lin.__dict__.get("_cortex_frag")
    if cached is None or cached[0] != key:
        if ops.capturing_graph():  # only recorded now: the graph rebuilds it on every replay, nothing cached
            return ops.frag_weight(src)
        cached = (key, ops.frag_weight(src))
        lin.__dict__["_cortex_frag"] = cached
    return cached[1]


def bf16_weight(lin: nn.Module) -> tuple:
    """``(bf16 weight, weight_scale)`` for one-time preparation kernels that read bf16 rows:
    the cached image, or in the widen and window modes a temporary widened copy (not kept)."""
    if hasattr(lin, "weight_int8") and INT8_WEIGHTS != "image":
        return ops.convert(lin.weight_int8, torch.bfloat16), lin.weight_scale
    w = exec_weights(lin, torch.bfloat16)
    return w["weight"], w["weight_scale"]


def resident_weight_bytes(model: nn.Module) -> dict:
    """Device bytes the model holds for weights: its parameters and buffers (int8 weights and
    scales, embeddings, norms, latents) and the bf16 execution images cached on its linears."""
    own = sum(t.numel() * t.element_size() for t in list(model.parameters()) + list(model.buffers()))
    images = 0
    for m in model.modules():
        for name in ("_cortex_exec", "_cortex_frag"):
            c = m.__dict__.get(name)
            if c is not None:
                images += c[1].numel() * c[1].element_size()
    windows = {id(w): w.bytes for m in model.modules() if (w := m.__dict__.get("_cortex_window")) is not None}
    window = sum(windows.values())
    int8 = sum(b.numel() for n, b in model.named_buffers() if n.endswith("weight_int8"))
    return {"total": own + images + window, "parameters_and_buffers": own, "int8_weights": int8,
            "bf16_images": images, "bf16_windows": window}


def _state_key(tensors) -> tuple:
    return tuple((t.data_ptr(), t._version, tuple(t.shape), t.dtype) for t in tensors if t is not None)


def _param_tensors(mod: nn.Module) -> list:
    return [t for t in list(mod.parameters(recurse=False)) + list(mod.buffers(recurse=False))]


def batch_invariant(owner: nn.Module, name: str, inputs: list, mods: list, fn):
    """``fn()`` computed once and kept on ``owner`` while ``inputs`` and the parameters and
    buffers of ``mods`` are unchanged (same storage, same version counter).

    For results that depend on weights only (the learned latent queries after their
    norm and projection, the behaviour queries after theirs): a forward then reads
    them instead of recomputing them.  Never cached while a module carries forward
    pre-hooks, so that calibration still sees every input, nor from inside a HIP graph
    capture (the graph then recomputes it on every replay).
    """
    if any(m._forward_pre_hooks for m in mods):
        return fn()
    tensors = list(inputs)
    for m in mods:
        tensors += _param_tensors(m)
    key = _state_key(tensors)
    slot = owner.__dict__.setdefault("_cortex_invariant", {})
    hit = slot.get(name)
    if hit is not None and hit[0] == key:
        return hit[1]
    val = fn()
    if not ops.capturing_graph():  # under capture fn() was only recorded: recomputed per replay
        slot[name] = (key, val)
    return val


def ln_params(norm: nn.LayerNorm):
    """``(weight, bias, eps)`` of a LayerNorm, as the row kernels take it."""
    return (norm.weight, norm.bias, norm.eps)


def fused_tokens_ok(tables, norm: nn.LayerNorm) -> bool:
    """Whether the tokenizer + LayerNorm kernel covers these embedding tables and norm."""
    D = tables[0].shape[1]
    if D not in _LN_ROWS_K or any(t.dtype != torch.float32 or t.stride(-1) != 1 or t.data_ptr() % 16
                                  or t.stride(0) % 4 for t in tables):
        return False
    return all(p is not None and p.dtype == torch.float32 and p.data_ptr() % 16 == 0 for p in (norm.weight, norm.bias))


def ln_rows_ok(x: torch.Tensor, *norms: nn.LayerNorm) -> bool:
    """Whether the register-resident LayerNorm row kernel covers this input."""
    if x.dtype != torch.float32 or x.shape[-1] not in _LN_ROWS_K:
        return False
    for n in norms:
        for p in (n.weight, n.bias):
            if p is None or p.dtype != torch.float32 or p.data_ptr() % 16:
                return False
    return True


def normalize_bf16(x: torch.Tensor, norm: nn.LayerNorm, norm2: nn.LayerNorm | None = None,
                   widen: list | None = None) -> torch.Tensor:
    """``norm2(norm(x))`` (or ``norm(x)``) as bf16 rows (one launch; ``widen``: weight pairs that
    ride along, see ``WeightWindow``)."""
    x2 = x.reshape(-1, x.shape[-1])
    if x2.data_ptr() % 16 or (x2.shape[0] > 1 and x2.stride(0) % 4) or x2.stride(-1) != 1:
        x2 = x2.contiguous()
    return ops.ln_rows(x2, ln_params(norm), ln_params(norm2) if norm2 is not None else None, widen=widen)


def residual_ln_ok(lin: nn.Module, norm: nn.LayerNorm, consumer: nn.Module, x: torch.Tensor,
                   compute: torch.dtype) -> bool:
    """Whether ``residual + lin(a)`` followed by ``norm`` (feeding ``consumer``) can run as
    one ``cortex_linear_residual_ln`` launch: bf16 compute, no calibration hooks on the
    linear, the norm's consumer or the norm, D in {256, 512}, fp32 aligned norm parameters."""
    if compute != torch.bfloat16 or lin._forward_pre_hooks or consumer._forward_pre_hooks or norm._forward_pre_hooks:
        return False
    D = x.shape[-1]
    src = lin.weight_int8 if hasattr(lin, "weight_int8") else lin.weight
    if D not in (256, 512) or src.shape[0] != D or src.shape[1] % 64 or x.dtype != torch.float32:
        return False
    if x.data_ptr() % 16 or x.stride(-1) != 1 or (x.dim() > 1 and x.stride(0) % 4):
        return False
    if lin.bias is not None and (lin.bias.dtype != torch.float32 or lin.bias.data_ptr() % 16):
        return False
    return ln_rows_ok(x, norm)


def linear_residual_ln(lin: nn.Module, a: torch.Tensor, residual: torch.Tensor, norm: nn.LayerNorm, *,
                       res_rows: int = 0, out: torch.Tensor | None = None, xq_scale: float | None = None):
    """``x = residual + lin(a)`` (fp32) and ``norm(x)`` (bf16; int8 at ``xq_scale`` when given)
    in one launch (see ``residual_ln_ok``).  Returns ``(x, norm(x))``.  With bf16 images (the
    default INT8 mode) the weight goes in MFMA fragment order where the direct-weight kernel
    takes it (``ops.frag_ok``)."""
    src = lin.weight_int8 if hasattr(lin, "weight_int8") else lin.weight
    win = lin.__dict__.get("_cortex_window") if hasattr(lin, "weight_int8") and INT8_WEIGHTS == "window" else None
    if win is not None:  # the window, in fragment order when this shape takes it
        w = win.view(lin, rows=a.shape[0])
        return ops.linear_residual_ln(a, w, lin.weight_scale, lin.bias, residual=residual, ln=ln_params(norm),
                                      res_rows=res_rows, out=out, xq_scale=xq_scale, frag=win.is_frag(lin))
    if (not (hasattr(lin, "weight_int8") and INT8_WEIGHTS != "image")
            and ops.frag_ok(a.shape[0], src.shape[0], src.shape[1], a.device)):
        return ops.linear_residual_ln(a, frag_image(lin), lin.weight_scale if hasattr(lin, "weight_int8") else None,
                                      lin.bias, residual=residual, ln=ln_params(norm), res_rows=res_rows, out=out,
                                      xq_scale=xq_scale, frag=True)
    w, scale, bias = fused_weight(lin)
    return ops.linear_residual_ln(a, w, scale, bias, residual=residual, ln=ln_params(norm), res_rows=res_rows,
                                  out=out, xq_scale=xq_scale)


def apply_linear(lin: nn.Module, x: torch.Tensor, *, norm: nn.LayerNorm | None = None, stats=None,
                 act: str | None = None, residual: torch.Tensor | None = None, res_rows: int = 0,
                 out_dtype: torch.dtype, compute: torch.dtype, out: torch.Tensor | None = None) -> torch.Tensor:
    """``act(lin(norm(x))) + residual`` on the HIP kernels.

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
    if (residual is not None and norm is None and act is None and compute == torch.bfloat16
            and x.dtype == torch.bfloat16 and residual.dtype == torch.float32 and out_dtype == torch.float32
            and not (hasattr(lin, "weight_int8") and INT8_WEIGHTS != "image")
            and (lin.bias is None or lin.bias.dtype == torch.float32)):
        src = lin.weight_int8 if hasattr(lin, "weight_int8") else lin.weight
        M = x.numel() // x.shape[-1]
        if (src.dim() == 2 and src.shape[1] == x.shape[-1] and residual.shape[-1] == src.shape[0]
                and ops.frag_res_ok(M, src.shape[0], src.shape[1], x.device)):
            # the direct-weight residual GEMM on the fragment-order weight (MLP-down)
            return ops.linear_residual_frag(x, frag_image(lin), lin.weight_scale if hasattr(lin, "weight_int8")
                                            else None, lin.bias, residual=residual, res_rows=res_rows, out=out)
    win = lin.__dict__.get("_cortex_window") if hasattr(lin, "weight_int8") and INT8_WEIGHTS == "window" else None
    if (win is not None and residual is not None and norm is None and act is None and compute == torch.bfloat16
            and x.dtype == torch.bfloat16 and residual.dtype == torch.float32 and out_dtype == torch.float32
            and (lin.bias is None or lin.bias.dtype == torch.float32)):
        w = win.view(lin, rows=x.numel() // x.shape[-1])
        if win.is_frag(lin):  # the window in fragment order: the direct-weight residual GEMM
            return ops.linear_residual_frag(x, w, lin.weight_scale, lin.bias, residual=residual, res_rows=res_rows,
                                            out=out)
    w = exec_weights(lin, compute)
    if norm is not None and compute == torch.bfloat16 and stats is None and ln_rows_ok(x, norm):
        lead = x.shape[:-1]
        xn = normalize_bf16(x, norm).reshape(*lead, x.shape[-1])
        return ops.norm_linear(xn, **w, act=act, residual=residual, res_rows=res_rows, out_dtype=out_dtype,
                               compute_dtype=compute, out=out)
    kw = {}
    if norm is not None:
        kw = {"norm": "layer", "gamma": norm.weight, "beta": norm.bias, "eps": norm.eps, "stats": stats}
    return ops.norm_linear(x, **w, **kw, act=act, residual=residual, res_rows=res_rows, out_dtype=out_dtype,
                           compute_dtype=compute, out=out)
