"""Top-level Cortex model (reference cortex/models/cortex.py:15-165).

``CortexModel.forward`` on a ROCm device runs the whole Cortex-S inference path on
the gfx950 kernels without padding the events:

1. device-side stable pack plan of ``batch_indices`` -> CSR offsets + row order
   (no host read-back when ``batch_size`` is given);
2. fused tokenizer writing the tokens directly in CSR order;
3. ``norm_kv`` + ``kv_proj`` on the E_total real event rows only;
4. cross-attention of the batch-invariant latent queries (projected once, not
   once per sample) against each sample's CSR key/value rows -- padded tiles do
   not exist, so they are never visited;
5. ``out_proj`` with the learned latents as a broadcast residual, 7 fused
   self-attention blocks, ``final_norm``;
6. behaviour head in one kernel: both LayerNorms, then the weights folded into the
   2 batch-invariant queries and into ``out_proj`` (once per parameter state), so
   only 32 dot products per latent row remain.

Results equal the reference forward (padded SDPA with a key-padding mask) up to
floating-point rounding; with ``config.dtype='float32'`` every operand is fp32.
"""

from __future__ import annotations

import torch
from torch import nn

from cortex.kernels import ops
from cortex.kernels.pack import pack_events as _device_pack_events
from cortex.models._layers import (apply_linear, batch_invariant, bf16_weight, exec_weights, fused_tokens_ok,
                                   linear_residual_ln, linear_weights, ln_params, ln_rows_ok, normalize_bf16,
                                   residual_ln_ok, rider)
from cortex.models.config import CortexConfig
from cortex.models.perceiver import PerceiverEncoder
from cortex.models.tokenizer import SpikeTokenizer


class BehaviorDecoder(nn.Module):
    """Learned behaviour queries cross-attending to the latents (reference :15-53)."""

    def __init__(self, config: CortexConfig) -> None:
        super().__init__()
        self.config = config
        self.query = nn.Parameter(torch.randn(config.behavior_dim, config.latent_dim) * 0.02)
        self.q_proj = nn.Linear(config.latent_dim, config.latent_dim, bias=False)
        self.kv_proj = nn.Linear(config.latent_dim, 2 * config.latent_dim, bias=False)
        self.out_proj = nn.Linear(config.latent_dim, 1, bias=False)
        self.norm = nn.LayerNorm(config.latent_dim)
        self.num_heads = config.num_heads
        self.head_dim = config.head_dim

    def forward_rows(self, lat: torch.Tensor, batch: int, pre_norm: nn.LayerNorm | None = None) -> torch.Tensor:
        """(B*L, D) latents -> (B, behavior_dim) fp32.

        ``pre_norm`` (the encoder's final norm) is applied to ``lat`` first.  With bf16
        compute the whole head is one kernel (``cortex_behavior_head``): both LayerNorms,
        then the weights folded into the queries and the output projection -- scores
        ``(W_k^T q) . n`` and values ``(W_v^T w_out) . n`` -- so the kv projection, the
        attention and ``out_proj`` are never materialised.  Otherwise (fp32, calibration
        hooks, shapes outside the kernel) the head runs as written.
        """
        compute = self.config.compute_dtype
        L = self.config.num_latents
        D = lat.shape[1]
        H = self.num_heads
        Q = self.query.shape[0]
        if pre_norm is not None and self._fused_ok(lat, pre_norm):
            return ops.behavior_head(lat, batch, ln_params(pre_norm), ln_params(self.norm), self._folded(), Q, H)
        if (pre_norm is not None and compute == torch.bfloat16 and not self.kv_proj._forward_pre_hooks
                and ln_rows_ok(lat, pre_norm, self.norm)):
            kv = ops.norm_linear(normalize_bf16(lat, pre_norm, self.norm), **exec_weights(self.kv_proj, compute),
                                 out_dtype=compute, compute_dtype=compute)
        else:
            if pre_norm is not None:
                lat = ops.layer_norm(lat, pre_norm.weight, pre_norm.bias, pre_norm.eps)
            kv = apply_linear(self.kv_proj, lat, norm=self.norm, out_dtype=compute, compute=compute)
        q = batch_invariant(self, f"q_{compute}", [self.query], [self.q_proj],  # (Q, D), batch-invariant
                            lambda: apply_linear(self.q_proj, self.query, out_dtype=compute, compute=compute))
        o_buf, o = ops.merge_heads_out(batch, Q, H, D // H, compute, lat.device)
        ops.attention(ops.heads_view(q, 1, Q, H), ops.heads_view(kv, batch, L, H, 0, D),
                      ops.heads_view(kv, batch, L, H, D, D), out=o, batch=batch)
        out = apply_linear(self.out_proj, o_buf, out_dtype=torch.float32, compute=compute)
        return out.reshape(batch, Q)

    def _fused_ok(self, lat: torch.Tensor, pre_norm: nn.LayerNorm) -> bool:
        """Whether the fused head kernel covers this call: bf16 compute, no calibration hooks,
        no biases on the folded projections, Q*H <= 16 and D in {256, 512, 768}."""
        mods = (self.q_proj, self.kv_proj, self.out_proj, self.norm, pre_norm)
        return (self.config.compute_dtype == torch.bfloat16 and not any(m._forward_pre_hooks for m in mods)
                and self.kv_proj.bias is None and self.out_proj.bias is None
                and self.query.shape[0] * self.num_heads <= 16 and lat.shape[1] in (256, 512, 768)
                and lat.shape[1] % self.num_heads == 0 and ln_rows_ok(lat, pre_norm, self.norm)
                and lat.data_ptr() % 16 == 0 and lat.stride(0) % 4 == 0)

    def _folded(self) -> torch.Tensor:
        """The (32, D) folded query / value-output matrix, once per parameter state."""
        compute = torch.bfloat16

        def build():
            q = apply_linear(self.q_proj, self.query, out_dtype=compute, compute=compute)
            (kv, kv_s), (ow, ow_s) = bf16_weight(self.kv_proj), bf16_weight(self.out_proj)
            return ops.head_prep(q, kv, kv_s, ow, ow_s, self.num_heads)

        return batch_invariant(self, "head_folded", [self.query], [self.q_proj, self.kv_proj, self.out_proj], build)

    def forward(self, latents: torch.Tensor) -> torch.Tensor:
        """latents (B, L, D) -> behaviour (B, behavior_dim)."""
        B, L, D = latents.shape
        return self.forward_rows(latents.reshape(B * L, D).contiguous(), B).to(latents.dtype)


class MaskedSpikeHead(nn.Module):
    """Masked-spike logits: ``proj(latents.mean(dim=1))`` (reference :56-69).

    One kernel (``cortex_pooled_linear``): the mean over each sample's latent rows, with the
    encoder's final LayerNorm applied to every row first when it is passed, then the
    N = spike_value_buckets projection with bias, fp32 throughout.  ``proj`` may be an
    ``nn.Linear`` or a ``QuantizedLinear`` (int8 weight widened with its per-row scale in
    fp32, as ``QuantizedLinear.forward`` does on fp32 latents).
    """

    def __init__(self, config: CortexConfig) -> None:
        super().__init__()
        self.proj = nn.Linear(config.latent_dim, config.spike_value_buckets)

    def forward(self, latents: torch.Tensor) -> torch.Tensor:
        """latents (B, L, D) -> (B, spike_value_buckets) fp32."""
        B, L, D = latents.shape
        return self.forward_rows(latents.reshape(B * L, D).float(), B)

    def forward_rows(self, lat: torch.Tensor, batch: int, pre_norm: nn.LayerNorm | None = None) -> torch.Tensor:
        """(B*L, D) fp32 latent rows (``pre_norm`` applied to each row first) -> (B, N) fp32."""
        ln = ln_params(pre_norm) if pre_norm is not None else None
        if self.proj._forward_pre_hooks:  # calibration: the hooks see the pooled rows, as in the reference
            mean = ops.pooled_linear(lat, batch, ln)
            return apply_linear(self.proj, mean, out_dtype=torch.float32, compute=torch.float32)
        w = linear_weights(self.proj)
        return ops.pooled_linear(lat, batch, ln, w.get("weight_int8", w.get("weight")), w.get("weight_scale"),
                                 w.get("bias"))


class CortexModel(nn.Module):
    """Perceiver-style neural decoder (reference :72-122)."""

    def __init__(self, config: CortexConfig) -> None:
        super().__init__()
        self.config = config
        self.tokenizer = SpikeTokenizer(config)
        self.encoder = PerceiverEncoder(config)
        self.behavior_head = BehaviorDecoder(config)
        self.masked_spike_head = MaskedSpikeHead(config) if config.use_masked_spike_head else None

    def forward(self, neuron_ids: torch.Tensor, time_bins: torch.Tensor, values: torch.Tensor,
                batch_indices: torch.Tensor, return_aux: bool = False, *, batch_size: int | None = None,
                err_flag: torch.Tensor | None = None, check_indices: bool = False,
                clear_err: bool = False) -> dict[str, torch.Tensor]:
        """Spike events -> ``{"behavior": (B, behavior_dim)}``, plus ``"masked_spike_logits"``
        (B, spike_value_buckets) when ``return_aux`` is set and the model has that head.

        ``batch_size`` (keyword-only) avoids reading ``max(batch_indices)+1`` back to the
        host; ``err_flag`` (int32 device tensor) collects index-range violations
        without a synchronisation.  By default an event index outside its table gives a
        zero token row and a batch index outside [0, B) drops the event, flagged in
        ``err_flag`` only; ``check_indices=True`` reads the flag back after the forward
        (one synchronisation) and raises ``IndexError`` as the eager embedding lookup
        of the reference does (cortex/models/tokenizer.py:90-93).  ``clear_err=True`` zeroes
        ``err_flag`` first, inside the pack plan's first launch.
        """
        if not (neuron_ids.shape == time_bins.shape == values.shape == batch_indices.shape):
            raise ValueError(
                f"shape mismatch: neuron_ids={neuron_ids.shape}, time_bins={time_bins.shape}, "
                f"values={values.shape}, batch_indices={batch_indices.shape}"
            )
        E = neuron_ids.shape[0]
        if batch_size is None:
            batch_size = int(batch_indices.max().item()) + 1 if E > 0 else 1
        if check_indices and err_flag is None:
            err_flag = torch.empty(1, dtype=torch.int32, device=neuron_ids.device)
        # INT8-resident window mode: the cross-attention's and the first block's weights widen into
        # their windows in the plan's first launch, on the CUs its few workgroups leave idle
        widen = self._window_rider(rows=int(batch_size) * self.config.num_latents)
        offsets, order, _, ident = ops.pack_plan(batch_indices, int(batch_size), err=err_flag, with_rank=False,
                                                 identity=True, clear_err=clear_err or check_indices, widen=widen)
        out = self._forward_planned(neuron_ids, time_bins, values, offsets, order, int(batch_size), err_flag,
                                    aux=return_aux, identity=ident)
        if check_indices:
            _raise_on_flag(err_flag)
        return out

    def forward_csr(self, neuron_ids: torch.Tensor, time_bins: torch.Tensor, values: torch.Tensor,
                    offsets: torch.Tensor, *, err_flag: torch.Tensor | None = None,
                    check_indices: bool = False) -> torch.Tensor:
        """Events already grouped by sample -> behaviour ``(B, behavior_dim)`` fp32.

        Sample b owns events ``[offsets[b], offsets[b+1])`` (``offsets``: (B+1,) int64 on
        the device, non-decreasing from 0).  Events past ``offsets[B]`` (padding of a
        fixed-size buffer) are ignored.  Skips the pack plan: a server that builds the
        batch sample by sample has the CSR layout for free.  ``check_indices`` as in
        ``forward``.
        """
        if not (neuron_ids.shape == time_bins.shape == values.shape):
            raise ValueError(
                f"shape mismatch: neuron_ids={neuron_ids.shape}, time_bins={time_bins.shape}, values={values.shape}")
        err_flag = _checked_flag(err_flag, check_indices, neuron_ids.device)
        self._window_rider(take=False)
        out = self._forward_planned(neuron_ids, time_bins, values, offsets, None, offsets.shape[0] - 1,
                                    err_flag)["behavior"]
        if check_indices:
            _raise_on_flag(err_flag)
        return out

    def _forward_planned(self, neuron_ids, time_bins, values, offsets, order, B: int, err_flag,
                         aux: bool = False, identity: torch.Tensor | None = None) -> dict[str, torch.Tensor]:
        """The forward from a CSR plan: row r of the packed events is event ``order[r]``
        (``r`` itself when ``order`` is None or the plan's ``identity`` flag is set); rows past
        ``offsets[B]`` are ignored."""
        enc = self.encoder
        tokens = self._token_rows(neuron_ids, time_bins, values, offsets, order, err_flag, identity,
                                  rows=B * self.config.num_latents)
        x, xn = self._cross_rows(tokens, offsets, B)
        x = self._encode(x, B, xn)
        out = {"behavior": self.behavior_head.forward_rows(x, B, pre_norm=enc.final_norm)}
        if aux and self.masked_spike_head is not None:
            out["masked_spike_logits"] = self.masked_spike_head.forward_rows(x, B, pre_norm=enc.final_norm)
        return out

    def _window_rider(self, take: bool = True, rows: int | None = None) -> list | None:
        """Start of a forward in the INT8-resident window mode: nothing is resident yet (every
        weight group this forward reads is widened again), and with ``take`` the weight items of
        the cross-attention and the first block (laid out for ``rows`` latent rows), for the
        forward's first launch to widen."""
        win = self.encoder.weight_window()
        if win is None:
            return None
        win.reset()
        if not take:
            return None
        blocks = self.encoder.self_attn_blocks
        return rider(self.encoder.cross_attn, blocks[0] if len(blocks) else None, rows=rows)

    def _token_rows(self, neuron_ids, time_bins, values, offsets, order, err_flag,
                    identity: torch.Tensor | None = None, rows: int | None = None) -> tuple[torch.Tensor, bool]:
        """The event rows in CSR order: ``(norm_kv(tokens) as bf16 rows, True)`` in one pass over the
        tables when the fused tokenizer + LayerNorm applies (the fp32 tokens are never stored),
        else ``(tokens, False)``.  ``rows``: the latent rows of the forward (B L), for the window
        layouts of the weights widened in the same launch."""
        cfg = self.config
        tok, xa = self.tokenizer, self.encoder.cross_attn
        tables = (tok.neuron_emb.weight, tok.time_emb.weight, tok.value_emb.weight)
        if (cfg.compute_dtype == torch.bfloat16 and not xa.kv_proj._forward_pre_hooks
                and fused_tokens_ok(tables, xa.norm_kv)):
            # the cross-attention's and the first block's weights widen into their windows in the
            # same launch (INT8-resident window mode), unless the pack plan carried them
            blocks = self.encoder.self_attn_blocks
            widen = rider(xa, blocks[0] if len(blocks) else None, rows=rows)
            return ops.tokenize_ln(*tables, neuron_ids, time_bins, values, ln_params(xa.norm_kv), order=order,
                                   csr_offsets=offsets, err=err_flag, identity=identity, widen=widen), True
        return ops.tokenize(*tables, neuron_ids, time_bins, values, order=order, csr_offsets=offsets,
                            err=err_flag, identity=identity), False

    def _cross_rows(self, tokens: tuple[torch.Tensor, bool], offsets: torch.Tensor, B: int):
        """Cross-attention of the latents into each sample's CSR event rows: ``kv_proj`` on the real
        events, the batch-invariant latent queries against them, ``out_proj`` with the latents as a
        broadcast residual.  Returns the fp32 residual rows ``x`` (B*L, D) and, when computed in
        the same launch, the first block's ``norm_attn(x)`` (else None)."""
        cfg = self.config
        compute = cfg.compute_dtype
        enc = self.encoder
        xa = enc.cross_attn
        D, L, H = cfg.latent_dim, cfg.num_latents, xa.num_heads
        rows, normed = tokens
        E = rows.shape[0]
        if normed:
            kv = ops.norm_linear(rows, **exec_weights(xa.kv_proj, compute), out_dtype=compute, compute_dtype=compute)
        else:
            kv = apply_linear(xa.kv_proj, rows, norm=xa.norm_kv, out_dtype=compute, compute=compute)  # (E, 2D)
        q = xa.project_queries(enc.latents, compute)  # (L, D), shared by every sample
        o_buf, o = ops.merge_heads_out(B, L, H, D // H, compute, kv.device)
        ops.attention(ops.heads_view(q, 1, L, H), ops.heads_view(kv, 1, E, H, 0, D),
                      ops.heads_view(kv, 1, E, H, D, D), kv_offsets=offsets, out=o, batch=B)
        first = enc.self_attn_blocks[0] if len(enc.self_attn_blocks) else None
        if first is not None and residual_ln_ok(xa.out_proj, first.norm_attn, first.qkv_proj, enc.latents, compute):
            # latents + out_proj(attn) and the first block's norm_attn in one launch
            return linear_residual_ln(xa.out_proj, o_buf, enc.latents, first.norm_attn, res_rows=L,
                                      out=torch.empty(B * L, D, dtype=torch.float32, device=kv.device))
        x = apply_linear(xa.out_proj, o_buf, residual=enc.latents, res_rows=L, out_dtype=torch.float32,
                         compute=compute)  # (B*L, D) fp32 residual stream
        return x, None

    def _encode(self, x: torch.Tensor, B: int, xn: torch.Tensor | None = None) -> torch.Tensor:
        """The self-attention stack on the fresh residual buffer ``x`` (updated in place)."""
        return self.encoder.encode_rows(x, B, final_norm=False, inplace=True, xn=xn)


def _checked_flag(err_flag: torch.Tensor | None, check: bool, device: torch.device) -> torch.Tensor | None:
    """The error flag a checked forward reads back: the caller's (cleared), or a fresh one."""
    if not check:
        return err_flag
    if err_flag is None:
        return torch.zeros(1, dtype=torch.int32, device=device)
    err_flag.zero_()
    return err_flag


def _raise_on_flag(err_flag: torch.Tensor) -> None:
    e = int(err_flag.item())
    if e & 2:
        raise IndexError("batch index outside [0, batch_size)")
    if e:
        raise IndexError("event index out of range (neuron_id, time_bin or value outside its embedding table)")


def _pack_events(flat_tokens: torch.Tensor, batch_indices: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Pack flat (E, D) tokens into (B, E_max, D) with a (B, E_max) bool mask.

    Same contract as reference cortex/models/cortex.py:125-165 (B and E_max read
    back from the device); runs the device-side stable pack.
    """
    return _device_pack_events(flat_tokens, batch_indices)
