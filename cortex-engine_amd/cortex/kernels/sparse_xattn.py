"""Block-sparse Perceiver cross-attention on gfx950.

Drop-in for ``cortex.kernels.sparse_xattn`` of the reference
(cortex/kernels/sparse_xattn.py:96-434).  ``sparse_cross_attention`` keeps the
reference signature and its tile-mask semantics -- element (l, e) is attended iff
``block_mask[l // BLOCK_L, e // BLOCK_E]`` -- and runs one HIP kernel that streams
64-key tiles through LDS with an online softmax, skipping tiles that hold no
allowed element; rows with no allowed key are 0 (the l=0 guard of the reference
Triton kernel, :325-328).  Keyword-only extensions: a per-sample tile mask
``(B, n_q, n_k)``, per-sample ``kv_lengths`` (the padding of ragged events) and a
``(B, E)`` ``key_padding_mask`` (the model's SDPA mask, perceiver.py:75-80).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from cortex import _native as nat
from cortex.kernels import ops


def sparse_cross_attention_reference(q, k, v, block_mask=None, BLOCK_L: int = 64, BLOCK_E: int = 64,
                                     scale: float | None = None):
    """PyTorch formulation (reference sparse_xattn.py:96-146): what ``sparse_cross_attention``
    returns for queries that are not on a ROCm device, as the reference dispatcher does.

    Dense SDPA when ``block_mask`` is None; otherwise the tile mask expanded to
    elements, -inf outside it, softmax in fp32.  GPU tensors never reach it.
    """
    L, Dh = q.shape[-2], q.shape[-1]
    E = k.shape[-2]
    s = scale if scale is not None else Dh ** -0.5
    if block_mask is None:
        return F.scaled_dot_product_attention(q, k, v, scale=s)
    n_q, n_k = math.ceil(L / BLOCK_L), math.ceil(E / BLOCK_E)
    assert block_mask.shape == (n_q, n_k), f"block_mask shape {block_mask.shape} != expected ({n_q}, {n_k})"
    li = torch.arange(L, device=q.device) // BLOCK_L
    ei = torch.arange(E, device=q.device) // BLOCK_E
    allowed = block_mask.to(q.device)[li[:, None], ei[None, :]]
    bias = torch.zeros(L, E, device=q.device, dtype=q.dtype).masked_fill(~allowed, float("-inf"))
    scores = torch.matmul(q, k.transpose(-2, -1)) * s + bias
    attn = torch.softmax(scores.float(), dim=-1).to(q.dtype)
    return torch.matmul(attn, v)


def build_temporal_block_mask(event_times: torch.Tensor, n_latents: int, max_time_bins: int,
                              window_bins: int = 30, BLOCK_L: int = 64, BLOCK_E: int = 64) -> torch.Tensor:
    """Conservative ``(n_q, n_k)`` CPU bool tile mask from latent time centres.

    Same definition as reference sparse_xattn.py:152-200: latent i sits at
    ``i / L * T`` (fp32); a latent tile covers ``[int(min) - w, int(max) + w]``; an
    event tile covers the [min, max] time of its events; keep the pair iff the
    intervals overlap.  Event times on a GPU are reduced there
    (``ops.temporal_block_mask``, one kernel) and only the small mask is copied back;
    host event times, as in the reference, are reduced on the host, vectorised over
    tiles (the centres increase with i, so a tile's min/max are its first/last centre).
    """
    if event_times.is_cuda:
        return ops.temporal_block_mask(event_times, n_latents, max_time_bins, window_bins, BLOCK_L,
                                       BLOCK_E).cpu()
    t = event_times.detach().to("cpu", torch.int64).reshape(-1)
    E = t.shape[0]
    n_q = math.ceil(n_latents / BLOCK_L)
    n_k = math.ceil(E / BLOCK_E)
    if n_k == 0:
        return torch.zeros(n_q, 0, dtype=torch.bool)
    pad = n_k * BLOCK_E - E
    tmin = torch.cat([t, t[-1:].expand(pad)]).reshape(n_k, BLOCK_E).amin(dim=1)
    tmax = torch.cat([t, t[-1:].expand(pad)]).reshape(n_k, BLOCK_E).amax(dim=1)
    centres = torch.arange(n_latents, dtype=torch.float32) / n_latents * max_time_bins
    first = torch.arange(n_q) * BLOCK_L
    last = torch.clamp(first + BLOCK_L - 1, max=n_latents - 1)
    lo = centres[first].to(torch.int64) - window_bins  # int() truncation; centres >= 0
    hi = centres[last].to(torch.int64) + window_bins
    return (tmin[None, :] <= hi[:, None]) & (tmax[None, :] >= lo[:, None])


def sparse_cross_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, block_mask=None,
                           BLOCK_L: int = 64, BLOCK_E: int = 64, scale: float | None = None, *,
                           kv_lengths: torch.Tensor | None = None,
                           key_padding_mask: torch.Tensor | None = None) -> torch.Tensor:
    """Block-sparse cross-attention ``(B, H, L, Dh)`` in q's dtype (bf16 or fp32).

    Signature of reference sparse_xattn.py:340-348.  ``block_mask`` may be
    ``(n_q, n_k)`` (shared by every (b, h), as in the reference) or ``(B, n_q, n_k)``;
    ``None`` is dense attention (also on the HIP kernel).  Queries on a ROCm device run the
    HIP kernel; on any other device the call returns ``sparse_cross_attention_reference``
    (reference :366-368), which has no keyword-only extensions.
    """
    if q.device.type != "cuda":
        if kv_lengths is not None or key_padding_mask is not None or (
                block_mask is not None and block_mask.dim() != 2):
            raise ValueError("kv_lengths, key_padding_mask and per-sample tile masks need ROCm GPU tensors")
        return sparse_cross_attention_reference(q, k, v, block_mask, BLOCK_L, BLOCK_E, scale)
    nat.require_gpu(q, k, v, what="sparse_cross_attention")
    B, H, L, Dh = q.shape
    E = k.shape[2]
    if block_mask is not None:
        n_q, n_k = math.ceil(L / BLOCK_L), math.ceil(E / BLOCK_E)
        if block_mask.dim() == 2:
            assert block_mask.shape == (n_q, n_k), (
                f"block_mask shape {block_mask.shape} != expected ({n_q}, {n_k})")
        else:
            assert block_mask.shape == (B, n_q, n_k), (
                f"block_mask shape {block_mask.shape} != expected ({B}, {n_q}, {n_k})")
    if kv_lengths is not None:
        kv_lengths = kv_lengths.to(device=q.device, dtype=torch.int64).contiguous()
    if key_padding_mask is not None:
        key_padding_mask = key_padding_mask.to(device=q.device)
    return ops.attention(q, k, v, scale=scale, kv_lengths=kv_lengths, key_mask=key_padding_mask,
                         block_mask=block_mask, block_l=BLOCK_L, block_e=BLOCK_E)
