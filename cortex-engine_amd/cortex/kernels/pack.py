"""Ragged-event pack on gfx950 (reference cortex/models/cortex.py:125-165).

The reference sorts the flat events by batch index with a stable argsort and
scatters them into a zero-padded ``(B, E_max, D)`` tensor, reading ``B`` and
``E_max`` back to the host.  Here a device-side stable counting sort produces the
CSR plan (offsets, order) without host synchronisation; the padded copy is a
second launch that writes every output row (data or zeros) exactly once.
"""

from __future__ import annotations

import torch

from cortex import _native as nat
from cortex.kernels import ops


def pack_plan(batch_indices: torch.Tensor, batch_size: int, err: torch.Tensor | None = None):
    """``(offsets (B+1), order (E), rank (E))`` int64 device tensors (stable order)."""
    return ops.pack_plan(batch_indices, batch_size, err=err)


def pack_events(flat_tokens: torch.Tensor, batch_indices: torch.Tensor, *, batch_size: int | None = None,
                max_events: int | None = None):
    """Pack flat ``(E, D)`` tokens into ``(B, E_max, D)`` plus a ``(B, E_max)`` bool mask.

    Same result as the reference ``_pack_events``; pass ``batch_size`` and
    ``max_events`` to skip the two host read-backs it performs.
    """
    nat.require_gpu(flat_tokens, batch_indices, what="pack_events")
    E = batch_indices.shape[0]
    if flat_tokens.shape[0] != E:
        raise ValueError("flat_tokens and batch_indices disagree on the number of events")
    if batch_size is None:
        batch_size = int(batch_indices.max().item()) + 1 if E > 0 else 1
    offsets, order, _ = ops.pack_plan(batch_indices, batch_size, with_rank=False)
    if max_events is None:
        max_events = int((offsets[1:] - offsets[:-1]).max().item()) if E > 0 else 0
    return ops.pack_rows(flat_tokens.reshape(E, flat_tokens.shape[-1]), order, offsets, batch_size, max_events)


def pack_csr(flat_tokens: torch.Tensor, batch_indices: torch.Tensor, batch_size: int):
    """CSR form: ``(rows (E, D) in stable batch order, offsets (B+1,))``."""
    nat.require_gpu(flat_tokens, batch_indices, what="pack_csr")
    offsets, order, _ = ops.pack_plan(batch_indices, batch_size, with_rank=False)
    E = batch_indices.shape[0]
    dev = flat_tokens.device
    out = torch.empty_like(flat_tokens.reshape(E, flat_tokens.shape[-1]))
    if E:
        src = ops._row_major_2d(flat_tokens.reshape(E, flat_tokens.shape[-1]))
        nat.call("cortex_pack_rows", nat.code(src.dtype), src.shape[1], nat.ptr(src),
                 src.stride(0) if E > 1 else src.shape[1], E, nat.ptr(order), ops._end_ptr(offsets), None, 0, 0,
                 nat.ptr(out), out.shape[1], None, nat.stream_of(dev))
    return out, offsets
