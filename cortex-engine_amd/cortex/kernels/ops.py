"""Functional wrappers over the gfx950 kernels (one Python call -> one or two launches).

These are the building blocks of the drop-in APIs (``cortex.kernels.*``,
``cortex.quantization``) and of the model forward (``cortex.models``).  Every
function takes GPU tensors, allocates its outputs with torch's caching allocator
(unless ``out=`` is given), launches on torch's current stream and never
synchronises the host.
"""

from __future__ import annotations

import ctypes
import math
import os
from collections import OrderedDict

import torch

from cortex import _native as nat

NORM = {None: 0, "none": 0, "layer": 1, "rms": 2}
_CU_COUNT: dict[int, int] = {}


def splitk_splits(M: int, N: int, K: int, device: torch.device) -> int:
    """K slabs for a residual linear with few rows (0: no split).  Split when the 128 x 128
    output tiles fill at most a quarter of the CUs: the largest of 2, 4, 8 slabs that keeps
    tiles x slabs within one workgroup per CU and K a multiple of 64 per slab."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    cus = _CU_COUNT.get(idx)
    if cus is None:
        cus = _CU_COUNT[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    tiles = math.ceil(M / 128) * math.ceil(N / 128)
    if M < 1 or tiles * 4 > cus or K < 128:
        return 0
    s = 1
    while s < 8 and tiles * s * 2 <= cus and K % (64 * s * 2) == 0:
        s *= 2
    return s if s > 1 else 0
ACT = {None: 0, "none": 0, "gelu": 1}


def _row_major_2d(x: torch.Tensor) -> torch.Tensor:
    if x.dim() != 2:
        raise ValueError(f"expected a 2-D tensor, got shape {tuple(x.shape)}")
    if x.stride(1) != 1 or (x.size(0) > 1 and x.stride(0) < x.size(1)):
        x = x.contiguous()
    return x


# --------------------------------------------------------------------------- pack


def pack_plan(batch_indices: torch.Tensor, batch_size: int, err: torch.Tensor | None = None, *,
              with_rank: bool = True, identity: bool = False, clear_err: bool = False, widen=None):
    """Stable CSR plan of ragged events: ``(offsets (B+1), order (E), rank (E))``.

    offsets/order/rank are int64 device tensors; see ``cortex_pack_plan``.  With
    ``with_rank=False`` the rank is not written and ``None`` is returned in its place.
    With ``identity=True`` a fourth value is returned, the plan's int32 identity flag: a
    plan of sorted indices sets it and leaves ``order`` unwritten, so ``order`` may only be
    handed on together with the flag (``tokenize`` / ``tokenize_ln`` take both).
    ``clear_err=True`` zeroes ``err`` inside the plan's first launch before anything ORs into it.
    ``widen``: (int8, bf16) weight pairs widened by extra workgroups of the plan's first launch
    (``widen_int8``).
    """
    dev = nat.require_gpu(batch_indices, what="pack_plan")
    if batch_indices.dtype != torch.int64 or batch_indices.dim() != 1:
        raise ValueError("batch_indices must be a 1-D int64 tensor")
    E = batch_indices.shape[0]
    B = int(batch_size)
    offsets = torch.empty(B + 1, dtype=torch.int64, device=dev)
    order = torch.empty(E, dtype=torch.int64, device=dev)
    rank = torch.empty(E, dtype=torch.int64, device=dev) if with_rank else None
    ident = torch.empty(1, dtype=torch.int32, device=dev) if identity else None
    ws_bytes = nat.load().cortex_pack_workspace_bytes(E, B)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    args = (nat.ptr(batch_indices), batch_indices.stride(0) if E else 1, E, B, nat.ptr(offsets), nat.ptr(order), None,
            nat.ptr(rank), nat.ptr(ws), ws_bytes, nat.ptr(err), nat.ptr(ident), 1 if clear_err else 0)
    if widen:
        nat.call("cortex_pack_plan_widen", *args, *_widen_args(widen, dev), nat.stream_of(dev))
    else:
        nat.call("cortex_pack_plan", *args, nat.stream_of(dev))
    return (offsets, order, rank, ident) if identity else (offsets, order, rank)


def tokenize(neuron_emb, time_emb, value_emb, neuron_ids, time_bins, values, *, order=None, offsets=None,
             csr_offsets=None, batch_size: int = 0, max_events: int = 0, out=None, mask=None, err=None,
             identity=None):
    """Fused gather-add ``(N[nid] + T[tb]) + V[val]`` into CSR rows (``offsets`` None) or
    the padded ``(B, max_events, D)`` layout with its mask (``offsets`` given).

    In CSR mode pass the plan's offsets as ``csr_offsets``: rows past
    ``offsets[B]`` (events dropped for an invalid batch index) are then zeroed.
    ``identity``: the plan's identity flag (``pack_plan(..., identity=True)``), when ``order``
    came from such a plan.
    """
    dev = nat.require_gpu(neuron_emb, time_emb, value_emb, neuron_ids, time_bins, values, what="tokenize")
    D = neuron_emb.shape[1]
    E = neuron_ids.shape[0]
    padded = offsets is not None
    if out is None:
        shape = (batch_size, max_events, D) if padded else (E, D)
        out = torch.empty(shape, dtype=neuron_emb.dtype, device=dev)
    if padded and mask is None:
        mask = torch.empty((batch_size, max_events), dtype=torch.bool, device=dev)
    ld_out = out.stride(-2) if out.dim() >= 2 and out.shape[-2] > 1 else D
    st = [t.stride(0) if t.numel() else 1 for t in (neuron_ids, time_bins, values)]
    nat.call("cortex_tokenize", nat.code(neuron_emb.dtype), D,
             nat.ptr(neuron_emb), neuron_emb.shape[0], neuron_emb.stride(0),
             nat.ptr(time_emb), time_emb.shape[0], time_emb.stride(0),
             nat.ptr(value_emb), value_emb.shape[0], value_emb.stride(0),
             nat.ptr(neuron_ids), st[0], nat.ptr(time_bins), st[1], nat.ptr(values), st[2], E,
             nat.ptr(order), _end_ptr(csr_offsets), nat.ptr(offsets), batch_size, max_events, nat.ptr(out),
             ld_out, nat.ptr(mask) if padded else None, nat.ptr(identity), nat.ptr(err), nat.stream_of(dev))
    return (out, mask) if padded else out


WIDEN_MAX = 8  # arrays per widening rider (WR_MAX in the kernels)


def _widen_args(pairs, dev) -> tuple:
    """``(n, src, dst, count, frag_k)`` C arrays of the (int8 source, bf16 destination[, K]) items
    of a widening rider: contiguous tensors of equal element counts (multiples of 16) on ``dev``;
    a third item K > 0 writes the (N, K) destination in MFMA fragment order (``frag_weight``'s
    layout; K a power of two from 64)."""
    pairs = [tuple(p) if len(p) == 3 else (p[0], p[1], 0) for p in pairs]
    if len(pairs) > WIDEN_MAX:
        raise ValueError(f"at most {WIDEN_MAX} arrays widen in one launch (got {len(pairs)})")
    for src, dst, _ in pairs:
        if src.dtype != torch.int8 or dst.dtype != torch.bfloat16:
            raise ValueError("widening takes int8 sources and bf16 destinations")
        if src.numel() != dst.numel() or src.numel() % 16 or not (src.is_contiguous() and dst.is_contiguous()):
            raise ValueError("widening needs contiguous arrays of equal size, a multiple of 16 elements")
        if src.device != dev or dst.device != dev:
            raise RuntimeError("widening arrays must be on the launching device")
    n = len(pairs)
    src = (ctypes.c_void_p * max(n, 1))(*[p[0].data_ptr() for p in pairs])
    dst = (ctypes.c_void_p * max(n, 1))(*[p[1].data_ptr() for p in pairs])
    cnt = (ctypes.c_int64 * max(n, 1))(*[p[0].numel() for p in pairs])
    fk = (ctypes.c_int64 * max(n, 1))(*[int(p[2]) for p in pairs])
    return n, src, dst, cnt, fk


def widen_int8(pairs) -> None:
    """``dst.copy_(src)`` (int8 -> bf16, exact) for each ``(src, dst)`` pair in one launch
    (``cortex_widen_int8``); a ``(src, dst, K)`` item writes dst in MFMA fragment order."""
    pairs = list(pairs)
    if not pairs:
        return
    dev = nat.require_gpu(*[t for p in pairs for t in p[:2]], what="widen_int8")
    nat.call("cortex_widen_int8", *_widen_args(pairs, dev), nat.stream_of(dev))


def tokenize_ln(neuron_emb, time_emb, value_emb, neuron_ids, time_bins, values, ln, *, order=None,
                csr_offsets=None, err=None, out=None, identity=None, widen=None) -> torch.Tensor:
    """``LN((N[nid] + T[tb]) + V[val])`` as bf16 CSR rows (one launch, fp32 tokens never stored).

    ``ln`` is ``(weight, bias, eps)``; rows follow ``order`` (the pack plan, with its identity
    flag when it has one) and rows past ``csr_offsets[B]`` come out as ``LN(0)``.  ``widen``:
    (int8, bf16) weight pairs widened by extra workgroups of the same launch (``widen_int8``)."""
    dev = nat.require_gpu(neuron_emb, time_emb, value_emb, neuron_ids, time_bins, values, order, err,
                          what="tokenize_ln")
    for t in (neuron_emb, time_emb, value_emb):
        if t.dtype != torch.float32 or t.stride(-1) != 1:
            raise ValueError("tokenize_ln needs fp32 tables with unit column stride")
    E, D = neuron_ids.shape[0], neuron_emb.shape[1]
    g, b, eps = ln
    if out is None:
        out = torch.empty((E, D), dtype=torch.bfloat16, device=dev)
    args = (D, nat.ptr(neuron_emb), neuron_emb.shape[0], neuron_emb.stride(0),
            nat.ptr(time_emb), time_emb.shape[0], time_emb.stride(0), nat.ptr(value_emb), value_emb.shape[0],
            value_emb.stride(0), nat.ptr(neuron_ids), neuron_ids.stride(0) if E else 1, nat.ptr(time_bins),
            time_bins.stride(0) if E else 1, nat.ptr(values), values.stride(0) if E else 1, E, nat.ptr(order),
            nat.ptr(identity), _end_ptr(csr_offsets), nat.ptr(g), nat.ptr(b), float(eps), nat.ptr(out),
            out.stride(0), nat.ptr(err))
    if widen:
        nat.call("cortex_tokenize_ln_widen", *args, *_widen_args(widen, dev), nat.stream_of(dev))
    else:
        nat.call("cortex_tokenize_ln", *args, nat.stream_of(dev))
    return out


def _end_ptr(offsets) -> int | None:
    """Device address of offsets[B] (the number of valid CSR rows)."""
    if offsets is None:
        return None
    return offsets.data_ptr() + (offsets.numel() - 1) * offsets.element_size()


def pack_rows(src, order, offsets, batch_size: int, max_events: int):
    """Padded ``(B, max_events, D)`` copy of CSR-ordered rows plus the bool mask."""
    dev = nat.require_gpu(src, order, offsets, what="pack_rows")
    src = _row_major_2d(src)
    E, D = src.shape
    out = torch.empty((batch_size, max_events, D), dtype=src.dtype, device=dev)
    mask = torch.empty((batch_size, max_events), dtype=torch.bool, device=dev)
    nat.call("cortex_pack_rows", nat.code(src.dtype), D, nat.ptr(src), src.stride(0) if E > 1 else D, E,
             nat.ptr(order), None, nat.ptr(offsets), batch_size, max_events, nat.ptr(out), D, nat.ptr(mask),
             nat.stream_of(dev))
    return out, mask


# --------------------------------------------------------------------------- quantise


def quantize_int8(weight: torch.Tensor, scale: torch.Tensor | None = None):
    """INT8 per-row quantisation of a 2-D fp32 weight: ``(q int8 (N,K), scale fp32 (N,))``."""
    dev = nat.require_gpu(weight, scale, what="quantize_int8")
    w = _row_major_2d(weight.detach().float())
    N, K = w.shape
    q = torch.empty((N, K), dtype=torch.int8, device=dev)
    s_out = None
    if scale is None:
        s_out = torch.empty(N, dtype=torch.float32, device=dev)
    else:
        scale = scale.detach().to(device=dev, dtype=torch.float32).contiguous()
    nat.call("cortex_quantize_int8", nat.ptr(w), N, K, w.stride(0) if N > 1 else K, nat.ptr(scale),
             nat.ptr(s_out), nat.ptr(q), K, nat.stream_of(dev))
    return q, (s_out if scale is None else scale)


# --------------------------------------------------------------------------- norms


def row_stats(x: torch.Tensor, norm: str, eps: float, out=None) -> torch.Tensor:
    """(M, 2) fp32 per-row statistics: LayerNorm (mean, rstd) or RMSNorm (0, rms)."""
    dev = nat.require_gpu(x, what="row_stats")
    x = _row_major_2d(x)
    M, K = x.shape
    if out is None:
        out = torch.empty((M, 2), dtype=torch.float32, device=dev)
    nat.call("cortex_row_stats", M, K, nat.code(x.dtype), nat.ptr(x), x.stride(0) if M > 1 else K, NORM[norm],
             float(eps), nat.ptr(out), nat.stream_of(dev))
    return out


def layer_norm(x: torch.Tensor, weight, bias, eps: float, out_dtype=None, out=None) -> torch.Tensor:
    """LayerNorm over the last dim, written out (any leading shape)."""
    dev = nat.require_gpu(x, weight, bias, what="layer_norm")
    K = x.shape[-1]
    x2 = _row_major_2d(x.reshape(-1, K))
    M = x2.shape[0]
    out_dtype = out_dtype or x.dtype
    if out is None:
        out = torch.empty(x.shape, dtype=out_dtype, device=dev)
    gdt = nat.code(weight.dtype) if weight is not None else nat.F32
    nat.call("cortex_layer_norm", M, K, nat.code(x2.dtype), nat.ptr(x2), x2.stride(0) if M > 1 else K,
             nat.ptr(weight), nat.ptr(bias), gdt, float(eps), nat.code(out.dtype), nat.ptr(out), K,
             nat.stream_of(dev))
    return out


_LN_ROWS_K = (256, 512, 768, 1024)


def norm_rows(x: torch.Tensor, norm: str, gamma=None, beta=None, eps: float = 1e-6) -> torch.Tensor:
    """RMSNorm (``norm='rms'``) or LayerNorm (``'layer'``) of the rows of ``x`` (fp32 or
    bf16, K in {256, 512, 768, 1024}) as bf16 rows (``cortex_norm_rows``)."""
    dev = nat.require_gpu(x, gamma, beta, what="norm_rows")
    x2 = _row_major_2d(x.reshape(-1, x.shape[-1]))
    M, K = x2.shape
    out = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
    gdt = nat.code(gamma.dtype) if gamma is not None else (nat.code(beta.dtype) if beta is not None else nat.F32)
    nat.call("cortex_norm_rows", M, K, nat.code(x2.dtype), nat.ptr(x2), x2.stride(0) if M > 1 else K, NORM[norm],
             nat.ptr(gamma), nat.ptr(beta), gdt, float(eps), nat.ptr(out), K, nat.stream_of(dev))
    return out


def transpose_bf16(w: torch.Tensor) -> torch.Tensor:
    """``w.T`` of a bf16 (R, C) matrix as contiguous (C, R) rows (``cortex_transpose_bf16``)."""
    dev = nat.require_gpu(w, what="transpose_bf16")
    w2 = _row_major_2d(w)
    R, C = w2.shape
    out = torch.empty((C, R), dtype=torch.bfloat16, device=dev)
    nat.call("cortex_transpose_bf16", R, C, nat.ptr(w2), w2.stride(0) if R > 1 else C, nat.ptr(out), R,
             nat.stream_of(dev))
    return out


def ln_rows(x: torch.Tensor, ln1, ln2=None, out_bf16: bool = True, out_f32: bool = False, widen=None):
    """LayerNorm over rows of fp32 ``x`` (K in {256, 512, 768, 1024}); ``ln1``/``ln2``
    are ``(weight, bias, eps)`` triples (``ln2`` applied after ``ln1`` when given).
    Returns the bf16 and/or fp32 result(s).  ``widen``: (int8, bf16) weight pairs widened by
    extra workgroups of the same launch (``widen_int8``)."""
    dev = nat.require_gpu(x, what="ln_rows")
    x2 = _row_major_2d(x.reshape(-1, x.shape[-1]))
    M, K = x2.shape
    ob = torch.empty((M, K), dtype=torch.bfloat16, device=dev) if out_bf16 else None
    of = torch.empty((M, K), dtype=torch.float32, device=dev) if out_f32 else None
    g1, b1, e1 = ln1
    g2, b2, e2 = ln2 if ln2 is not None else (None, None, 0.0)
    args = (M, K, nat.ptr(x2), x2.stride(0) if M > 1 else K, nat.ptr(g1), nat.ptr(b1), float(e1), nat.ptr(g2),
            nat.ptr(b2), float(e2), nat.ptr(ob), K, nat.ptr(of), K)
    if widen:
        nat.call("cortex_ln_rows_widen", *args, *_widen_args(widen, dev), nat.stream_of(dev))
    else:
        nat.call("cortex_ln_rows", *args, nat.stream_of(dev))
    if out_bf16 and out_f32:
        return ob, of
    return ob if out_bf16 else of


def qkv_attention(xn: torch.Tensor, weight: torch.Tensor, weight_scale, bias, batch: int, length: int,
                  heads: int, scale: float | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Self-attention with its QKV projection fused (``cortex_qkv_attention``): ``xn`` (B*L, D)
    bf16 rows, ``weight`` the (3D, D) bf16 image or the int8 weight itself (widened in the
    kernel); returns the merged-head (B*L, D) bf16 output."""
    dev = nat.require_gpu(xn, weight, weight_scale, bias, out, what="qkv_attention")
    M, D = xn.shape
    if out is None:
        out = torch.empty((M, D), dtype=torch.bfloat16, device=dev)
    s = float(scale) if scale is not None else (D // heads) ** -0.5
    nat.call("cortex_qkv_attention", batch, length, D, heads, nat.ptr(xn), xn.stride(0), nat.code(weight.dtype),
             nat.ptr(weight), weight.stride(0), nat.ptr(weight_scale), nat.ptr(bias), s, nat.ptr(out), out.stride(0),
             nat.stream_of(dev))
    return out


def frag_weight(weight: torch.Tensor) -> torch.Tensor:
    """The (N, K) weight (int8, bf16 or fp32) as bf16 in MFMA fragment order
    (``cortex_frag_weight``), shape (N, K) but not row-major: only ``linear_residual_ln(...,
    frag=True)`` reads it.  Values exactly those of ``convert(weight, torch.bfloat16)``."""
    dev = nat.require_gpu(weight, what="frag_weight")
    w2 = _row_major_2d(weight)
    N, K = w2.shape
    out = torch.empty((N, K), dtype=torch.bfloat16, device=dev)
    nat.call("cortex_frag_weight", N, K, nat.ptr(w2), nat.code(w2.dtype), w2.stride(0), nat.ptr(out),
             nat.stream_of(dev))
    return out


def frag_ok(M: int, N: int, K: int, device: torch.device) -> bool:
    """Whether ``linear_residual_ln`` takes a fragment-order weight at this shape (the
    direct-weight kernel: K 256 or 512, and rows enough that no K split applies)."""
    return N in (256, 512) and K in (256, 512) and not splitk_splits(M, N, K, device)


def frag_res_ok(M: int, N: int, K: int, device: torch.device) -> bool:
    """Whether ``linear_residual_frag`` applies: the direct-weight residual GEMM (N a multiple
    of 128, K 1024 / 2048 / 3072) while its 128 x 128 tiles fit one per CU and no K split
    across workgroups applies (larger grids keep the (N, K) image and the taller tiles)."""
    if M < 1 or N % 128 or K not in (1024, 2048, 3072) or splitk_splits(M, N, K, device):
        return False
    idx = device.index if device.index is not None else torch.cuda.current_device()
    cus = _CU_COUNT.get(idx)
    if cus is None:
        cus = _CU_COUNT[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return math.ceil(M / 128) * (N // 128) <= cus


def linear_residual_frag(x: torch.Tensor, weight_frag: torch.Tensor, weight_scale=None, bias=None, *,
                         residual: torch.Tensor, res_rows: int = 0, out: torch.Tensor | None = None) -> torch.Tensor:
    """``out = residual + x @ (W * scale)^T + bias`` (fp32; ``out`` may be ``residual``) with the
    weight in MFMA fragment order (``frag_weight``), on the direct-weight residual GEMM (see
    ``frag_res_ok``).  Bit-identical to the same call with the bf16 image."""
    dev = nat.require_gpu(x, weight_frag, weight_scale, bias, residual, out, what="linear_residual_frag")
    x2 = _row_major_2d(x.reshape(-1, x.shape[-1]))
    M, K = x2.shape
    N = weight_frag.shape[0]
    if not frag_res_ok(M, N, K, dev):
        raise ValueError(f"the direct-weight residual GEMM does not apply at M={M}, N={N}, K={K}")
    res2 = _row_major_2d(residual.reshape(-1, N))
    if out is None:
        out = torch.empty((*x.shape[:-1], N), dtype=torch.float32, device=dev)
    out2 = out.reshape(-1, N)
    nat.call("cortex_norm_linear", M, N, K, nat.BF16, nat.ptr(x2), x2.stride(0), 0, None, None, None, nat.F32,
             nat.BF16, nat.BF16_FRAG, 0, nat.ptr(weight_frag), K, nat.ptr(weight_scale), nat.F32, nat.ptr(bias), 0,
             nat.F32, nat.ptr(res2), res2.stride(0), int(res_rows), nat.F32, nat.ptr(out2), out2.stride(0),
             nat.stream_of(dev))
    return out


def linear_residual_ln(x: torch.Tensor, weight: torch.Tensor, weight_scale=None, bias=None, *,
                       residual: torch.Tensor, ln, res_rows: int = 0, out: torch.Tensor | None = None,
                       xq_scale: float | None = None, frag: bool = False):
    """``out = residual + x @ (weight * scale)^T + bias`` (fp32) and ``LN(out)`` (bf16) in one
    kernel; ``x`` (M, K) bf16, ``weight`` (N, K) the bf16 image, the int8 weight itself
    (widened in the kernel) or, with ``frag``, ``frag_weight``'s fragment-order bf16 copy (see
    ``frag_ok``), N in {256, 512}.  ``out`` may be ``residual`` itself.  Returns ``(out, xn)``.
    With ``xq_scale`` (the W8A8 mode) ``xn`` is int8:
    ``clamp(rint(LN(out) * (1 / xq_scale)), -127, 127)``."""
    dev = nat.require_gpu(x, weight, weight_scale, bias, residual, out, what="linear_residual_ln")
    M, K = x.shape
    N = weight.shape[0]
    if frag and not frag_ok(M, N, K, dev):
        raise ValueError(f"a fragment-order weight does not apply at M={M}, N={N}, K={K}")
    w_code = nat.BF16_FRAG if frag else nat.code(weight.dtype)
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=dev)
    g, b, eps = ln
    if xq_scale is not None:
        xq = torch.empty((M, N), dtype=torch.int8, device=dev)
        nat.call("cortex_linear_residual_ln_i8", M, N, K, nat.ptr(x), x.stride(0), w_code,
                 nat.ptr(weight), weight.stride(0),
                 nat.ptr(weight_scale), nat.ptr(bias), nat.ptr(residual), residual.stride(0), int(res_rows),
                 nat.ptr(out), out.stride(0), nat.ptr(g), nat.ptr(b), float(eps), nat.ptr(xq), xq.stride(0),
                 float(xq_scale), nat.stream_of(dev))
        return out, xq
    xn = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    splits = splitk_splits(M, N, K, dev) if weight.dtype == torch.bfloat16 and not frag else 0
    if splits:  # few rows: K split across workgroups, slabs summed in order, then the LayerNorm
        ws_t = torch.empty(nat.load().cortex_splitk_workspace_bytes(M, N, splits), dtype=torch.uint8, device=dev)
        nat.call("cortex_linear_residual_ln_splitk", M, N, K, nat.ptr(x), x.stride(0), nat.ptr(weight),
                 weight.stride(0), nat.ptr(weight_scale), nat.ptr(bias), nat.ptr(residual), residual.stride(0),
                 int(res_rows), nat.ptr(out), out.stride(0), nat.ptr(g), nat.ptr(b), float(eps), nat.ptr(xn),
                 xn.stride(0), splits, nat.ptr(ws_t), ws_t.numel(), nat.stream_of(dev))
        return out, xn
    nat.call("cortex_linear_residual_ln", M, N, K, nat.ptr(x), x.stride(0), w_code, nat.ptr(weight),
             weight.stride(0),
             nat.ptr(weight_scale), nat.ptr(bias), nat.ptr(residual), residual.stride(0), int(res_rows),
             nat.ptr(out), out.stride(0), nat.ptr(g), nat.ptr(b), float(eps), nat.ptr(xn), xn.stride(0),
             nat.stream_of(dev))
    return out, xn


def linear_w8a8(xq: torch.Tensor, a_scale: float, weight_int8: torch.Tensor, weight_scale=None, bias=None, *,
                act: str | None = None, residual: torch.Tensor | None = None, res_rows: int = 0,
                out_dtype: torch.dtype = torch.float32, out_scale: float | None = None,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """The opt-in W8A8 linear (``cortex_linear_w8a8``): int8 activations ``xq`` (M, K) at
    per-tensor scale ``a_scale`` times the int8 weight (N, K), exact int32 sums, then
    ``* a_scale * weight_scale + bias`` (and GELU).  ``out_dtype`` float32 (optionally plus
    ``residual``; ``out`` may be the residual) or int8 at ``out_scale``."""
    dev = nat.require_gpu(xq, weight_int8, weight_scale, bias, residual, out, what="linear_w8a8")
    if xq.dtype != torch.int8 or weight_int8.dtype != torch.int8:
        raise ValueError("linear_w8a8 takes int8 activations and an int8 weight")
    x2 = _row_major_2d(xq.reshape(-1, xq.shape[-1]))
    w2 = _row_major_2d(weight_int8)
    M, K = x2.shape
    N = w2.shape[0]
    if w2.shape[1] != K:
        raise ValueError(f"inner dims differ: x has K={K}, weight has K={w2.shape[1]}")
    if out_dtype not in (torch.float32, torch.int8):
        raise ValueError("out_dtype must be float32 or int8")
    if out is None:
        out = torch.empty((*xq.shape[:-1], N), dtype=out_dtype, device=dev)
    out2 = out.reshape(-1, N)
    res2 = None if residual is None else _row_major_2d(residual.reshape(-1, N))
    nat.call("cortex_linear_w8a8", M, N, K, nat.ptr(x2), x2.stride(0) if M > 1 else K, float(a_scale), nat.ptr(w2),
             w2.stride(0) if N > 1 else K, nat.ptr(weight_scale), nat.ptr(bias), ACT[act], nat.ptr(res2),
             (res2.stride(0) if res2.shape[0] > 1 else N) if res2 is not None else 0, int(res_rows), nat.ptr(out2),
             nat.code(out_dtype), float(out_scale or 0.0), out2.stride(0) if M > 1 else N, nat.stream_of(dev))
    return out


def qkv_attention_w8a8(xq: torch.Tensor, a_scale: float, w_int8: torch.Tensor, w_scale, bias, batch: int,
                       length: int, heads: int, *, out_dtype: torch.dtype = torch.bfloat16,
                       out_scale: float | None = None) -> torch.Tensor:
    """``qkv_attention`` in the W8A8 mode: int8 ``xq`` rows at ``a_scale`` and the int8 qkv
    weight; the merged-head output as bf16 or, with ``out_dtype=torch.int8``, int8 at
    ``out_scale``."""
    dev = nat.require_gpu(xq, w_int8, w_scale, bias, what="qkv_attention_w8a8")
    M, D = xq.shape
    out = torch.empty((M, D), dtype=out_dtype, device=dev)
    nat.call("cortex_qkv_attention_w8a8", int(batch), int(length), D, int(heads), nat.ptr(xq), xq.stride(0),
             float(a_scale), nat.ptr(w_int8), w_int8.stride(0), nat.ptr(w_scale), nat.ptr(bias),
             1.0 / math.sqrt(D // int(heads)), nat.ptr(out), nat.code(out_dtype), float(out_scale or 0.0),
             out.stride(0), nat.stream_of(dev))
    return out


def linear_residual_ln_w8a8(xq: torch.Tensor, a_scale: float, w_int8: torch.Tensor, w_scale=None, bias=None, *,
                            residual: torch.Tensor, ln, res_rows: int = 0, out: torch.Tensor | None = None,
                            xn_dtype: torch.dtype = torch.bfloat16, xn_scale: float | None = None):
    """``linear_residual_ln`` with int8 ``xq`` rows at ``a_scale`` and the int8 weight (W8A8);
    ``LN(out)`` as bf16 or, with ``xn_dtype=torch.int8``, int8 at ``xn_scale``."""
    dev = nat.require_gpu(xq, w_int8, w_scale, bias, residual, out, what="linear_residual_ln_w8a8")
    M, K = xq.shape
    N = w_int8.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=dev)
    xn = torch.empty((M, N), dtype=xn_dtype, device=dev)
    g, b, eps = ln
    nat.call("cortex_linear_residual_ln_w8a8", M, N, K, nat.ptr(xq), xq.stride(0), float(a_scale), nat.ptr(w_int8),
             w_int8.stride(0), nat.ptr(w_scale), nat.ptr(bias), nat.ptr(residual), residual.stride(0), int(res_rows),
             nat.ptr(out), out.stride(0), nat.ptr(g), nat.ptr(b), float(eps), nat.ptr(xn), nat.code(xn_dtype),
             float(xn_scale or 0.0), xn.stride(0), nat.stream_of(dev))
    return out, xn


def ln_rows_i8(x: torch.Tensor, gamma, beta, eps: float, scale: float) -> torch.Tensor:
    """``clamp(rint(LayerNorm(x) * (1 / scale)), -127, 127)`` as int8 rows (W8A8 operand)."""
    dev = nat.require_gpu(x, gamma, beta, what="ln_rows_i8")
    M, K = x.shape
    out = torch.empty((M, K), dtype=torch.int8, device=dev)
    nat.call("cortex_ln_rows_i8", M, K, nat.ptr(x), x.stride(0), nat.ptr(gamma), nat.ptr(beta), float(eps),
             nat.ptr(out), out.stride(0), float(scale), nat.stream_of(dev))
    return out


def head_prep(q: torch.Tensor, kv_weight: torch.Tensor, kv_scale, out_weight: torch.Tensor, out_scale,
              num_heads: int) -> torch.Tensor:
    """Folded behaviour-head matrix (32, D) bf16 (see ``cortex_head_prep``) from the projected
    queries ``q`` (Q, D) bf16 and the bf16 weight images of kv_proj (2D, D) and out_proj (1, D)
    with their optional per-row scales."""
    dev = nat.require_gpu(q, kv_weight, out_weight, kv_scale, out_scale, what="head_prep")
    Q, D = q.shape
    for t in (q, kv_weight, out_weight):
        if t.dtype != torch.bfloat16 or t.stride(-1) != 1:
            raise ValueError("head_prep needs bf16 operands with unit column stride")
    ac = torch.empty((32, D), dtype=torch.bfloat16, device=dev)
    nat.call("cortex_head_prep", nat.ptr(q), q.stride(0), Q, int(num_heads), D, nat.ptr(kv_weight),
             nat.ptr(kv_scale), kv_weight.stride(0), nat.ptr(out_weight), nat.ptr(out_scale), nat.ptr(ac),
             nat.stream_of(dev))
    return ac


def behavior_head(x: torch.Tensor, batch: int, ln1, ln2, ac: torch.Tensor, num_queries: int, num_heads: int,
                  out: torch.Tensor | None = None) -> torch.Tensor:
    """Fused behaviour head: ``(B, Q)`` fp32 from the (B*L, D) fp32 latents, the two
    LayerNorms ``ln1`` then ``ln2`` (``(weight, bias, eps)``) and the folded matrix ``ac``."""
    dev = nat.require_gpu(x, ac, out, what="behavior_head")
    x2 = _row_major_2d(x.reshape(-1, x.shape[-1]))
    M, D = x2.shape
    L = M // batch
    if out is None:
        out = torch.empty((batch, num_queries), dtype=torch.float32, device=dev)
    (g1, b1, e1), (g2, b2, e2) = ln1, ln2
    ws_bytes = int(nat.load().cortex_behavior_head_workspace_bytes(batch, L))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    nat.call("cortex_behavior_head", nat.ptr(x2), x2.stride(0) if M > 1 else D, batch, L, D, int(num_queries),
             int(num_heads), nat.ptr(g1), nat.ptr(b1), float(e1), nat.ptr(g2), nat.ptr(b2), float(e2), nat.ptr(ac),
             nat.ptr(out), nat.ptr(ws), ws_bytes, nat.stream_of(dev))
    return out


def pooled_linear(x: torch.Tensor, batch: int, ln=None, weight: torch.Tensor | None = None,
                  weight_scale: torch.Tensor | None = None, bias: torch.Tensor | None = None, *,
                  pooled: bool = False):
    """Masked-spike head: the mean over each sample's L rows of ``x`` (B*L, D) fp32, after the
    LayerNorm ``ln`` = ``(weight, bias, eps)`` when given, then ``mean @ weight^T (* scale) + bias``
    with ``weight`` (N, D) fp32, or int8 with its per-row ``weight_scale``.  Returns
    ``(B, N)`` fp32, or ``(out, mean)`` with ``pooled=True``; ``weight=None`` returns the
    (B, D) mean alone (see ``cortex_pooled_linear``)."""
    dev = nat.require_gpu(x, weight, weight_scale, bias, what="pooled_linear")
    x2 = _row_major_2d(x.reshape(-1, x.shape[-1]))
    if x2.dtype != torch.float32:
        raise ValueError("pooled_linear takes fp32 rows")
    if x2.data_ptr() % 16 or (x2.shape[0] > 1 and x2.stride(0) % 4):
        x2 = x2.contiguous()
    M, D = x2.shape
    if batch < 1 or M % batch:
        raise ValueError(f"{M} rows do not split into {batch} samples")
    L = M // batch
    g = b = None
    eps = 0.0
    if ln is not None:
        g, b, eps = ln
        g, b = g.detach().float().contiguous(), b.detach().float().contiguous()
    N = 0
    w = None
    if weight is not None:
        if weight.dtype not in (torch.float32, torch.int8) or weight.shape[1] != D:
            raise ValueError("pooled_linear weight must be (N, D) fp32 or int8")
        if weight.dtype == torch.int8 and weight_scale is None:
            raise ValueError("an int8 weight needs its per-row scale")
        w = weight.detach().contiguous()
        N = w.shape[0]
    out = torch.empty((batch, N), dtype=torch.float32, device=dev)
    mean = torch.empty((batch, D), dtype=torch.float32, device=dev) if (pooled or w is None) else None
    sc = weight_scale.detach().float().contiguous() if weight_scale is not None and w is not None else None
    bs = bias.detach().float().contiguous() if bias is not None and w is not None else None
    nat.call("cortex_pooled_linear", nat.ptr(x2), x2.stride(0) if M > 1 else D, batch, L, D, nat.ptr(g),
             nat.ptr(b), float(eps), N, nat.code(w.dtype) if w is not None else nat.F32, nat.ptr(w),
             w.stride(0) if w is not None else D, nat.ptr(sc), nat.ptr(bs), nat.ptr(mean), nat.ptr(out),
             nat.stream_of(dev))
    if w is None:
        return mean
    return (out, mean) if pooled else out


def convert(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Elementwise dtype conversion on the GPU (int8/f32/bf16/f16 -> f32/bf16)."""
    dev = nat.require_gpu(t, what="convert")
    src = t.detach().contiguous()
    out = torch.empty(src.shape, dtype=dtype, device=dev)
    nat.call("cortex_convert", nat.code(src.dtype), nat.ptr(src), nat.code(dtype), nat.ptr(out), src.numel(),
             nat.stream_of(dev))
    return out


# --------------------------------------------------------------------------- linear


# "image" (default): the RMS gain folded into a cached bf16 copy of an int8 weight, which the
# fused norm + linear kernel reads; "widen": that kernel streams the int8 weight itself and
# normalises the rows (bit-for-bit the model's CORTEX_INT8_WEIGHTS switch, same variable)
INT8_WEIGHTS = os.environ.get("CORTEX_INT8_WEIGHTS", "image")

_KN_CACHE: "OrderedDict[tuple, tuple]" = OrderedDict()
_KN_CACHE_SIZE = 16
# keys whose rows a captured HIP graph reads: never evicted (the graph holds their address)
_KN_PINNED: set = set()
_KN_RETIRED: list = []  # rows of pinned entries rebuilt since their capture


def capturing_graph() -> bool:
    """Whether torch's current stream is capturing a HIP graph: kernels launched now are only
    recorded, so their outputs must not be cached for eager use."""
    return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


def _cached_rows(key: tuple, holds: tuple, versions: tuple, build):
    """A derived weight tensor kept in ``_KN_CACHE``: ``holds`` are the source tensors (their
    storages are kept alive, so their addresses are not reused while cached) and ``versions``
    their version counters (an in-place update rebuilds the entry).

    Under HIP graph capture the build kernel is only recorded, not run, so a miss builds a
    temporary that the graph recomputes on every replay and is not cached (a later eager call
    would otherwise read rows that were never written); a hit is pinned, since the graph keeps
    reading that tensor's address on every replay."""
    capturing = capturing_graph()
    hit = _KN_CACHE.get(key)
    if hit is not None and hit[1] == versions:
        _KN_CACHE.move_to_end(key)
        if capturing:
            _KN_PINNED.add(key)
        return hit[2]
    if capturing:
        return build()
    rows = build()
    if hit is not None and key in _KN_PINNED:  # a graph still reads the old rows: keep them alive
        _KN_RETIRED.append(hit[2])
        _KN_PINNED.discard(key)
    _KN_CACHE[key] = (tuple(t.untyped_storage() for t in holds), versions, rows)
    _KN_CACHE.move_to_end(key)
    for k in list(_KN_CACHE):
        if len(_KN_CACHE) - len(_KN_PINNED & _KN_CACHE.keys()) <= _KN_CACHE_SIZE:
            break
        if k not in _KN_PINNED and k != key:
            del _KN_CACHE[k]
    return rows


def derived_weight_bytes() -> int:
    """Device bytes held by the cached derived weights (folded-gain and transposed rows)."""
    rows = [e[2] for e in _KN_CACHE.values()] + _KN_RETIRED
    return sum(t.numel() * t.element_size() for t in rows)


def _tensor_key(t: torch.Tensor) -> tuple:
    return (t.untyped_storage().data_ptr(), t.storage_offset(), tuple(t.shape), tuple(t.stride()), t.dtype, t.device)


def kn_weight_rows(w: torch.Tensor) -> torch.Tensor:
    """The (N, K) bf16 rows of a (K, N) weight (``rms_norm_linear``'s layout), cached per weight
    and rebuilt when the weight changes in place."""
    return _cached_rows(("kn", _tensor_key(w)), (w,), (w._version,),
                        lambda: transpose_bf16(w if w.dtype == torch.bfloat16 else w.to(torch.bfloat16)))


def fold_gain(w: torch.Tensor, gamma: torch.Tensor, kn: bool = False) -> torch.Tensor:
    """bf16 (N, K) rows ``w[n, k] * gamma[k]`` (``cortex_fold_gain``) of an (N, K) weight, or of a
    (K, N) weight with ``kn``: int8, bf16 or fp32 weights, fp32 or bf16 gamma."""
    dev = nat.require_gpu(w, gamma, what="fold_gain")
    w = _row_major_2d(w)
    g = gamma.detach().contiguous()
    N, K = (w.shape[1], w.shape[0]) if kn else (w.shape[0], w.shape[1])
    if g.numel() != K:
        raise ValueError(f"gamma has {g.numel()} values, the weight's K is {K}")
    out = torch.empty((N, K), dtype=torch.bfloat16, device=dev)
    ld_w = w.stride(0) if w.shape[0] > 1 else w.shape[1]
    nat.call("cortex_fold_gain", N, K, nat.ptr(w), nat.code(w.dtype), int(kn), ld_w, nat.ptr(g), nat.code(g.dtype),
             nat.ptr(out), K, nat.stream_of(dev))
    return out


def folded_weight_rows(w: torch.Tensor, gamma: torch.Tensor, kn: bool = False) -> torch.Tensor:
    """``fold_gain(w, gamma, kn)``, cached per (weight, gamma) pair and rebuilt when either changes
    in place: RMSNorm's gain carried by the weight, so the fused kernel applies only 1 / rms."""
    key = ("fold", _tensor_key(w), _tensor_key(gamma), kn)
    return _cached_rows(key, (w, gamma), (w._version, gamma._version), lambda: fold_gain(w, gamma, kn))


def norm_linear_fused(x: torch.Tensor, w: torch.Tensor, w_scale=None, *, norm: str = "rms", gamma, beta=None,
                      eps: float = 1e-6, bias=None, act: str | None = None,
                      out: torch.Tensor | None = None, out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """``act(norm(x) @ w^T * w_scale + bias)`` in one launch (``cortex_norm_linear_fused``): x (M, K)
    bf16 rows (K a multiple of 64 up to 512), w (N, K) bf16 or int8, the RMS / LayerNorm
    statistics computed in the kernel from the staged rows.  ``gamma=None`` with RMS: no gain
    (a weight from ``folded_weight_rows`` carries it); 1 / rms scales the accumulator."""
    dev = nat.require_gpu(x, w, w_scale, gamma, beta, bias, out, what="norm_linear_fused")
    M, K = x.shape
    N = w.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=dev)
    g = gamma.detach().contiguous() if gamma is not None else None
    b = beta.detach().contiguous() if (beta is not None and norm == "layer") else None
    g_code = nat.code(g.dtype if g is not None else torch.float32)
    nat.call("cortex_norm_linear_fused", M, N, K, nat.ptr(x), x.stride(0) if M > 1 else K, NORM[norm], nat.ptr(g),
             nat.ptr(b), g_code, float(eps), nat.code(w.dtype), nat.ptr(w), w.stride(0) if N > 1 else K,
             nat.ptr(w_scale), nat.ptr(bias), ACT[act], nat.code(out.dtype), nat.ptr(out),
             out.stride(0) if M > 1 else N, nat.stream_of(dev))
    return out


def norm_linear(x: torch.Tensor, *, weight: torch.Tensor | None = None, weight_int8: torch.Tensor | None = None,
                weight_scale: torch.Tensor | None = None, w_layout: str = "nk", norm: str | None = None,
                gamma=None, beta=None, eps: float = 1e-5, stats=None, bias=None, act: str | None = None,
                residual: torch.Tensor | None = None, res_rows: int = 0, out_dtype=None,
                compute_dtype=torch.bfloat16, out: torch.Tensor | None = None) -> torch.Tensor:
    """``act(norm(x) @ W^T * scale + bias) + residual`` over the last dim of ``x``.

    ``weight`` is a float (N, K) (``w_layout='nk'``, nn.Linear) or (K, N)
    (``'kn'``, rms_norm_linear) matrix; ``weight_int8``/``weight_scale`` is the
    QuantizedLinear form.  ``compute_dtype`` is the MFMA input dtype (bf16 or fp32).
    """
    w = weight if weight is not None else weight_int8
    dev = nat.require_gpu(x, w, weight_scale, gamma, beta, bias, residual, out, what="norm_linear")
    K = x.shape[-1]
    lead = x.shape[:-1]
    x2 = _row_major_2d(x.reshape(-1, K))
    M = x2.shape[0]
    if weight_int8 is not None:
        if weight_int8.dtype != torch.int8 or weight_scale is None:
            raise ValueError("weight_int8 must be int8 and come with weight_scale")
        w2 = _row_major_2d(weight_int8)
        N, Kw = w2.shape
        layout = 0
        ws = weight_scale.contiguous()
    else:
        w2 = _row_major_2d(weight.detach())
        layout = 0 if w_layout == "nk" else 1
        N, Kw = (w2.shape if layout == 0 else (w2.shape[1], w2.shape[0]))
        ws = weight_scale.contiguous() if weight_scale is not None else None
    if Kw != K:
        raise ValueError(f"inner dims differ: x has K={K}, weight has K={Kw}")
    if compute_dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"compute dtype {compute_dtype} not supported (bfloat16 or float32)")
    if x2.dtype == torch.bfloat16 and compute_dtype != torch.bfloat16:
        raise ValueError("bf16 activations need bf16 compute")
    out_dtype = out_dtype or x.dtype
    if out is None:
        out = torch.empty((*lead, N), dtype=out_dtype, device=dev)
    out2 = out.reshape(-1, N)
    if out2.data_ptr() != out.data_ptr() or (M > 1 and out2.stride(0) < N) or out2.stride(-1) != 1:
        raise ValueError("out must be row-major contiguous over its last dim")
    nrm = NORM[norm]
    if (nrm and stats is None and residual is None and compute_dtype == torch.bfloat16 and x2.dtype == torch.bfloat16
            and K % 64 == 0 and K <= 512 and N % 8 == 0 and out_dtype in (torch.bfloat16, torch.float32)
            and (weight_int8 is not None or w2.dtype == torch.bfloat16 or layout == 1 or nrm == NORM["rms"])
            and gamma is not None
            and gamma.dtype in (torch.float32, torch.bfloat16) and (beta is None or beta.dtype == gamma.dtype)
            and (bias is None or bias.dtype == torch.float32)
            and x2.data_ptr() % 16 == 0 and (M == 1 or x2.stride(0) % 8 == 0)
            and (layout == 1 or (w2.data_ptr() % 16 == 0 and (N == 1 or w2.stride(0) % 16 == 0)))
            and all(t is None or t.data_ptr() % 16 == 0 for t in (ws, bias, out2, gamma, beta))
            and gamma.is_contiguous() and (beta is None or beta.is_contiguous())):
        # one launch: the statistics from the staged rows, the contraction on (N, K) rows.  RMS:
        # the gain is folded once into a cached bf16 copy of the weight (cortex_fold_gain) and
        # the kernel scales the accumulator by 1 / rms; with CORTEX_INT8_WEIGHTS=widen an int8
        # weight is streamed as it is and the kernel normalises the rows instead
        if nrm == NORM["rms"] and not (weight_int8 is not None and INT8_WEIGHTS == "widen"):
            w2 = folded_weight_rows(w2, gamma, kn=layout == 1)
            gamma = None
        elif weight_int8 is None and layout == 1:
            w2 = kn_weight_rows(w2)
        return norm_linear_fused(x2, w2, ws, norm=norm, gamma=gamma, beta=beta, eps=eps, bias=bias, act=act,
                                 out=out2).reshape(out.shape)
    if (nrm and stats is None and compute_dtype == torch.bfloat16 and K in _LN_ROWS_K
            and x2.dtype in (torch.bfloat16, torch.float32) and x2.data_ptr() % 16 == 0
            and (M == 1 or x2.stride(0) % 4 == 0)
            and (gamma is None or beta is None or gamma.dtype == beta.dtype)
            and all(p is None or (p.dtype in (torch.float32, torch.bfloat16) and p.is_contiguous())
                    for p in (gamma, beta))):
        # the normalised rows once as bf16 rows (the MFMA operand is that rounding either way),
        # then the bf16 GEMM streaming (N, K) weight rows
        xn = norm_rows(x2, norm, gamma, beta, eps)
        if weight_int8 is not None:
            kw = {"weight": convert(w2, torch.bfloat16), "weight_scale": ws}
        elif layout == 1:
            kw = {"weight": transpose_bf16(w2.to(torch.bfloat16) if w2.dtype != torch.bfloat16 else w2),
                  "weight_scale": ws}
        else:
            kw = {"weight": w2, "weight_scale": ws}
        return norm_linear(xn, **kw, bias=bias, act=act, residual=residual, res_rows=res_rows,
                           out_dtype=out_dtype, compute_dtype=compute_dtype, out=out)
    if nrm and stats is None:
        stats = row_stats(x2, "layer" if nrm == 1 else "rms", eps)
    res2 = None
    if residual is not None:
        res2 = residual.reshape(-1, N) if residual.dim() != 2 else residual
        res2 = _row_major_2d(res2)
    ld_w = w2.stride(0) if w2.shape[0] > 1 else w2.shape[1]
    if (res2 is not None and not nrm and not ACT[act] and layout == 0 and weight is not None
            and w2.dtype == torch.bfloat16 and x2.dtype == torch.bfloat16 and res2.dtype == torch.float32
            and out2.dtype == torch.float32 and (bias is None or bias.dtype == torch.float32)
            and all(t is None or t.data_ptr() % 16 == 0 for t in (x2, w2, ws, bias, res2, out2))
            and (M == 1 or (x2.stride(0) % 8 == 0 and out2.stride(0) % 4 == 0))
            and (w2.shape[0] == 1 or w2.stride(0) % 8 == 0) and (res2.shape[0] == 1 or res2.stride(0) % 4 == 0)):
        splits = splitk_splits(M, N, K, dev)
        if splits:  # few rows: K split across workgroups, slabs summed in order
            ws_t = torch.empty(nat.load().cortex_splitk_workspace_bytes(M, N, splits), dtype=torch.uint8, device=dev)
            nat.call("cortex_linear_residual_splitk", M, N, K, nat.ptr(x2), x2.stride(0) if M > 1 else K,
                     nat.ptr(w2), ld_w, nat.ptr(ws), nat.ptr(bias), nat.ptr(res2),
                     res2.stride(0) if res2.shape[0] > 1 else N, int(res_rows), nat.ptr(out2),
                     out2.stride(0) if M > 1 else N, splits, nat.ptr(ws_t), ws_t.numel(), nat.stream_of(dev))
            return out
    gdt = nat.code(gamma.dtype) if gamma is not None else nat.F32
    nat.call("cortex_norm_linear", M, N, K, nat.code(x2.dtype), nat.ptr(x2), x2.stride(0) if M > 1 else K, nrm,
             nat.ptr(stats), nat.ptr(gamma), nat.ptr(beta), gdt, nat.code(compute_dtype),
             nat.code(w2.dtype), layout, nat.ptr(w2), ld_w, nat.ptr(ws),
             nat.code(bias.dtype) if bias is not None else nat.F32, nat.ptr(bias), ACT[act],
             nat.code(res2.dtype) if res2 is not None else nat.F32, nat.ptr(res2),
             (res2.stride(0) if res2.shape[0] > 1 else N) if res2 is not None else 0, int(res_rows),
             nat.code(out2.dtype), nat.ptr(out2), out2.stride(0) if M > 1 else N, nat.stream_of(dev))
    return out


# --------------------------------------------------------------------------- attention


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, scale: float | None = None,
              kv_offsets: torch.Tensor | None = None, kv_lengths: torch.Tensor | None = None,
              key_mask: torch.Tensor | None = None, block_mask: torch.Tensor | None = None,
              block_l: int = 64, block_e: int = 64, out: torch.Tensor | None = None,
              batch: int | None = None) -> torch.Tensor:
    """``softmax(scale q k^T | allowed) v`` for (B, H, L, Dh) views (any strides, Dh contiguous).

    ``q`` may have batch stride 0 (batch-invariant queries, ``expand``-ed).  With
    ``kv_offsets`` (B+1) ``k``/``v`` are (1, H, E_total, Dh) CSR views and sample b
    uses rows [kv_offsets[b], kv_offsets[b+1]).
    """
    # the tile mask is a small host-side structure (the reference builds it on the CPU)
    dev = nat.require_gpu(q, k, v, kv_offsets, kv_lengths, key_mask, out, what="attention")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError("q, k, v must share a dtype")
    if q.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"attention dtype {q.dtype} not supported (bfloat16 or float32)")
    for t in (q, k, v):
        if t.stride(-1) != 1:
            raise ValueError("attention inputs need a contiguous last (head) dim")
    B = q.shape[0] if batch is None else batch
    H, Lq, Dh = q.shape[1], q.shape[2], q.shape[3]
    Lk = k.shape[2]
    if out is None:
        out = torch.empty((B, H, Lq, Dh), dtype=q.dtype, device=dev)
    s = float(scale) if scale is not None else Dh ** -0.5
    km_sb = 0
    if key_mask is not None:
        key_mask = key_mask.to(torch.uint8) if key_mask.dtype == torch.bool else key_mask
        key_mask = key_mask.contiguous()
        km_sb = key_mask.stride(0) if key_mask.dim() == 2 else 0
    bm_sb = n_qt = n_kt = 0
    if block_mask is not None:
        block_mask = block_mask.to(device=dev)
        block_mask = (block_mask.view(torch.uint8) if block_mask.dtype == torch.bool
                      else block_mask.to(torch.uint8)).contiguous()
        if block_mask.dim() not in (2, 3) or (block_mask.dim() == 3 and block_mask.shape[0] != B):
            raise ValueError(f"block_mask must be (n_q, n_k) or ({B}, n_q, n_k), got {tuple(block_mask.shape)}")
        n_qt, n_kt = block_mask.shape[-2], block_mask.shape[-1]
        bm_sb = block_mask.stride(0) if block_mask.dim() == 3 else 0
    qsb = q.stride(0) if q.shape[0] > 1 else 0
    nat.call("cortex_attention", nat.code(q.dtype), B, H, Lq, Lk, Dh,
             nat.ptr(q), qsb, q.stride(1), q.stride(2),
             nat.ptr(k), k.stride(0), k.stride(1), k.stride(2),
             nat.ptr(v), v.stride(0), v.stride(1), v.stride(2),
             nat.ptr(kv_offsets), nat.ptr(kv_lengths), nat.ptr(key_mask), km_sb,
             nat.ptr(block_mask), bm_sb, n_qt, n_kt, int(block_l), int(block_e), s,
             nat.ptr(out), out.stride(0), out.stride(1), out.stride(2), nat.stream_of(dev))
    return out


def temporal_block_mask(event_times: torch.Tensor, n_latents: int, max_time_bins: int, window_bins: int = 30,
                        block_l: int = 64, block_e: int = 64, *, offsets: torch.Tensor | None = None,
                        n_k: int | None = None) -> torch.Tensor:
    """Device tile mask of reference sparse_xattn.py:152-200, as a bool tensor on the GPU.

    Without ``offsets``: ``(n_q, ceil(E / block_e))`` over the E events, as the
    reference.  With (B+1) CSR ``offsets``: ``(B, n_q, n_k)`` per-sample masks whose key
    tiles start at each sample's first event; ``n_k`` defaults to ``ceil(E / block_e)``
    (no host read of the per-sample counts) and tiles past a sample's end are False.
    """
    dev = nat.require_gpu(event_times, offsets, what="temporal_block_mask")
    t = event_times.reshape(-1)
    if t.dtype != torch.int64:
        t = t.to(torch.int64)
    E = t.shape[0]
    n_q = math.ceil(n_latents / block_l)
    if n_k is None:
        n_k = math.ceil(E / block_e)
    if offsets is None:
        out = torch.empty((n_q, n_k), dtype=torch.bool, device=dev)
        B, out_sb = 1, 0
    else:
        offsets = offsets.to(torch.int64).contiguous()
        B = offsets.shape[0] - 1
        out = torch.empty((B, n_q, n_k), dtype=torch.bool, device=dev)
        out_sb = n_q * n_k
    nat.call("cortex_temporal_block_mask", nat.ptr(t), t.stride(0) if E > 0 else 1, E, nat.ptr(offsets), B,
             int(n_latents), int(max_time_bins), int(window_bins), int(block_l), int(block_e), n_q, n_k,
             nat.ptr(out), out_sb, nat.stream_of(dev))
    return out


def heads_view(x2d: torch.Tensor, batch: int, length: int, heads: int, col0: int = 0, width: int | None = None):
    """(B*L, C) row-major buffer -> (B, H, L, Dh) view of columns [col0, col0+width)."""
    C = x2d.shape[-1]
    width = width if width is not None else C - col0
    dh = width // heads
    return x2d.as_strided((batch, heads, length, dh), (length * x2d.stride(0), dh, x2d.stride(0), 1),
                          x2d.storage_offset() + col0)


def merge_heads_out(batch: int, length: int, heads: int, dh: int, dtype, device):
    """Allocate a (B*L, H*Dh) buffer and its (B, H, L, Dh) view for attention output."""
    buf = torch.empty((batch * length, heads * dh), dtype=dtype, device=device)
    return buf, heads_view(buf, batch, length, heads)


def ceil_div(a: int, b: int) -> int:
    return -(-a // b)


__all__ = [
    "pack_plan", "tokenize", "pack_rows", "quantize_int8", "row_stats", "layer_norm", "norm_linear",
    "attention", "heads_view", "merge_heads_out", "ceil_div", "math",
]
