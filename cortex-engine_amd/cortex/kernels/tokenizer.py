"""Fused spike tokenizer on gfx950.

Drop-in for ``cortex.kernels.tokenizer`` of the reference
(cortex/kernels/tokenizer.py:68-249): the same ``fused_tokenizer`` signature and
argument checks, executed by one HIP kernel that gathers the three embedding rows
of every event and adds them in the reference's order,
``(neuron_emb[nid] + time_emb[tb]) + value_emb[val]``, with 16-byte coalesced row
stores.  ``tokenize_and_pack`` additionally fuses the ragged-event pack (CSR rows +
offsets, or the padded layout + mask) with a device-side stable counting sort.
"""

from __future__ import annotations

import torch

from cortex import _native as nat
from cortex.kernels import ops


def fused_tokenizer_reference(neuron_emb, time_emb, value_emb, neuron_ids, time_bins, values):
    """PyTorch formulation (reference tokenizer.py:68-81): what ``fused_tokenizer`` returns for
    tables that are not on a ROCm device, as the reference dispatcher does for non-CUDA
    devices.  GPU tensors never reach it."""
    return neuron_emb[neuron_ids] + time_emb[time_bins] + value_emb[values]


def _check(neuron_emb, time_emb, value_emb, neuron_ids, time_bins, values) -> int:
    if not (neuron_emb.is_contiguous() and time_emb.is_contiguous() and value_emb.is_contiguous()):
        raise ValueError("embedding tables must be contiguous (call .contiguous() first)")
    if not (neuron_ids.shape == time_bins.shape == values.shape):
        raise ValueError(
            f"index tensors must have identical shapes, got "
            f"{neuron_ids.shape}, {time_bins.shape}, {values.shape}"
        )
    D = neuron_emb.shape[1]
    if time_emb.shape[1] != D or value_emb.shape[1] != D:
        raise ValueError("all embedding tables must have the same hidden dim D")
    if not (neuron_emb.dtype == time_emb.dtype == value_emb.dtype):
        raise ValueError("all embedding tables must share a dtype")
    for t in (neuron_ids, time_bins, values):
        if t.dtype != torch.int64:
            raise ValueError("index tensors must be int64")
    return D


def fused_tokenizer(neuron_emb: torch.Tensor, time_emb: torch.Tensor, value_emb: torch.Tensor,
                    neuron_ids: torch.Tensor, time_bins: torch.Tensor, values: torch.Tensor, *,
                    check_indices: bool = False) -> torch.Tensor:
    """Fused spike tokenizer: ``(E, D)`` tokens in the tables' dtype.

    Same contract as reference cortex/kernels/tokenizer.py:177-249 (ValueError on
    non-contiguous tables, mismatched index shapes or hidden dims; ``E == 0``
    returns an empty ``(0, D)`` tensor; indices may be strided).  Tables on a ROCm
    device run the HIP kernel (a missing library raises ``NativeLibraryError``);
    tables on any other device take ``fused_tokenizer_reference``, as the reference
    dispatcher does (tokenizer.py:201-206).  On the GPU, out-of-range indices never
    touch memory outside the tables: the row is written as zeros; with
    ``check_indices=True`` an ``IndexError`` is raised (this synchronises the host,
    like the reference's eager CPU path).
    """
    if neuron_emb.device.type != "cuda":
        return fused_tokenizer_reference(neuron_emb, time_emb, value_emb, neuron_ids, time_bins, values)
    D = _check(neuron_emb, time_emb, value_emb, neuron_ids, time_bins, values)
    dev = nat.require_gpu(neuron_emb, time_emb, value_emb, neuron_ids, time_bins, values,
                          what="fused_tokenizer")
    E = neuron_ids.shape[0]
    if E == 0:
        return torch.empty((0, D), dtype=neuron_emb.dtype, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev) if check_indices else None
    out = ops.tokenize(neuron_emb, time_emb, value_emb, neuron_ids.reshape(-1), time_bins.reshape(-1),
                       values.reshape(-1), err=err)
    if check_indices and int(err.item()) != 0:
        raise IndexError("fused_tokenizer: index out of range for an embedding table")
    return out


def tokenize_and_pack(neuron_emb, time_emb, value_emb, neuron_ids, time_bins, values, batch_indices, *,
                      batch_size: int | None = None, layout: str = "csr", max_events: int | None = None,
                      err: torch.Tensor | None = None):
    """Tokenize and pack ragged events in one pass over the tables.

    ``layout='csr'``: returns ``(tokens (E, D), offsets (B+1,))`` with rows in stable
    batch order -- the ``sorted_tokens`` / cumulative counts of the reference pack
    (cortex/models/cortex.py:149-160).  ``layout='padded'``: returns
    ``(tokens (B, E_max, D), mask (B, E_max))`` exactly like ``_pack_events``
    (cortex.py:125-165).  ``batch_size`` / ``max_events`` given by the caller avoid
    the reference's host synchronisations; when omitted they are read back.
    """
    _check(neuron_emb, time_emb, value_emb, neuron_ids, time_bins, values)
    dev = nat.require_gpu(neuron_emb, neuron_ids, batch_indices, what="tokenize_and_pack")
    E = neuron_ids.shape[0]
    if batch_size is None:
        batch_size = int(batch_indices.max().item()) + 1 if E > 0 else 1
    # sorted batch indices (the collate order): the plan only flags the identity, no order array
    offsets, order, _, ident = ops.pack_plan(batch_indices, batch_size, err=err, with_rank=False, identity=True)
    if layout == "csr":
        tok = ops.tokenize(neuron_emb, time_emb, value_emb, neuron_ids, time_bins, values, order=order,
                           csr_offsets=offsets, err=err, identity=ident)
        return tok, offsets
    if layout == "padded":
        if max_events is None:
            max_events = int((offsets[1:] - offsets[:-1]).max().item()) if E > 0 else 0
        return ops.tokenize(neuron_emb, time_emb, value_emb, neuron_ids, time_bins, values, order=order,
                            offsets=offsets, batch_size=batch_size, max_events=max_events, err=err,
                            identity=ident)
    raise ValueError(f"layout must be 'csr' or 'padded', got {layout!r}")
