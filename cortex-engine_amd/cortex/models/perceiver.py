"""Perceiver encoder modules (reference cortex/models/perceiver.py:35-158).

Parameters, names and construction order follow the reference so that seeded
initialisation and state_dicts are identical.  On a ROCm device each block runs as
fused HIP kernels: LayerNorm folded into the following linear's A-tile staging,
INT8/float weights on MFMA with dequant / GELU / residual in the epilogue, and the
attention kernel reading heads straight out of the projection buffers (no
rearrange copies).  The residual stream stays fp32; linear operands use the
config's compute dtype.
"""

from __future__ import annotations

import torch
from torch import nn

from cortex.kernels import ops
from cortex.models import _layers
from cortex.models._layers import (apply_linear, batch_invariant, build_weight_window, exec_weights, fused_weight,
                                   linear_residual_ln, ln_rows_ok, normalize_bf16, residual_ln_ok, rider)
from cortex.models.config import CortexConfig


class CrossAttentionBlock(nn.Module):
    """Cross-attention from input tokens into the latent array (reference :35-82)."""

    def __init__(self, config: CortexConfig) -> None:
        super().__init__()
        self.config = config
        self.num_heads = config.cross_attn_heads
        self.head_dim = config.latent_dim // config.cross_attn_heads
        if self.head_dim * self.num_heads != config.latent_dim:
            raise ValueError("latent_dim must be divisible by cross_attn_heads")
        self.q_proj = nn.Linear(config.latent_dim, config.latent_dim, bias=False)
        self.kv_proj = nn.Linear(config.hidden_dim, 2 * config.latent_dim, bias=False)
        self.out_proj = nn.Linear(config.latent_dim, config.latent_dim, bias=False)
        self.norm_q = nn.LayerNorm(config.latent_dim)
        self.norm_kv = nn.LayerNorm(config.hidden_dim)

    def project_queries(self, latents: torch.Tensor, compute: torch.dtype) -> torch.Tensor:
        """``q_proj(norm_q(latents))`` for (L, D) batch-invariant latents -> (L, D).

        Depends on parameters only, so it is computed once per parameter state."""
        return batch_invariant(
            self, f"q_{compute}", [latents], [self.q_proj, self.norm_q],
            lambda: apply_linear(self.q_proj, latents, norm=self.norm_q, out_dtype=compute, compute=compute))

    def forward(self, latents: torch.Tensor, tokens: torch.Tensor,
                token_mask: torch.Tensor | None = None) -> torch.Tensor:
        """latents (B, L, D), tokens (B, E, D), token_mask (B, E) bool -> (B, L, D)."""
        compute = self.config.compute_dtype
        B, L, D = latents.shape
        E = tokens.shape[1]
        H = self.num_heads
        q = apply_linear(self.q_proj, latents, norm=self.norm_q, out_dtype=compute, compute=compute)
        kv = apply_linear(self.kv_proj, tokens, norm=self.norm_kv, out_dtype=compute, compute=compute)
        q2, kv2 = q.reshape(B * L, D), kv.reshape(B * E, 2 * D)
        o_buf, o = ops.merge_heads_out(B, L, H, D // H, compute, latents.device)
        ops.attention(ops.heads_view(q2, B, L, H), ops.heads_view(kv2, B, E, H, 0, D),
                      ops.heads_view(kv2, B, E, H, D, D), key_mask=token_mask, out=o)
        return apply_linear(self.out_proj, o_buf, residual=latents.reshape(B * L, D).contiguous(),
                            out_dtype=latents.dtype, compute=compute).reshape(B, L, D)


class SelfAttentionBlock(nn.Module):
    """Pre-norm self-attention + GELU MLP over the latents (reference :85-126)."""

    def __init__(self, config: CortexConfig) -> None:
        super().__init__()
        self.config = config
        self.num_heads = config.num_heads
        self.head_dim = config.head_dim
        self.qkv_proj = nn.Linear(config.latent_dim, 3 * config.latent_dim, bias=False)
        self.out_proj = nn.Linear(config.latent_dim, config.latent_dim, bias=False)
        self.norm_attn = nn.LayerNorm(config.latent_dim)
        self.norm_mlp = nn.LayerNorm(config.latent_dim)
        mlp_hidden = int(config.latent_dim * config.mlp_ratio)
        self.mlp = nn.Sequential(
            nn.Linear(config.latent_dim, mlp_hidden, bias=False),
            nn.GELU(),
            nn.Linear(mlp_hidden, config.latent_dim, bias=False),
        )

    def forward_rows(self, x: torch.Tensor, batch: int, length: int, inplace: bool = False,
                     xn: torch.Tensor | None = None) -> torch.Tensor:
        """Block on a (B*L, D) fp32 residual buffer; returns the new residual buffer
        (``x`` itself, updated in place, when ``inplace``).  ``xn``: ``norm_attn(x)`` as bf16
        rows when the producer of ``x`` already wrote it.

        With bf16 compute, ``x + out_proj(attn)`` and ``norm_mlp`` of the result run as one
        kernel (``ops.linear_residual_ln``); the LayerNorm'd rows feed ``mlp.0`` directly.
        """
        compute = self.config.compute_dtype
        D = x.shape[1]
        H = self.num_heads
        w8 = self._w8a8(x, compute)
        if w8 is not None and w8[2] is not None and self._fused_attention_ok(x, length):
            return self._forward_rows_w8a8(x, batch, length, inplace, w8)
        if self._fused_attention_ok(x, length):
            # qkv projection + attention per (head, sample) on chip: qkv never reaches HBM
            if xn is None:  # this block's weights widen into their window in the same launch
                xn = normalize_bf16(x, self.norm_attn, widen=rider(self, rows=x.numel() // x.shape[-1]))
            o_buf = ops.qkv_attention(xn, *fused_weight(self.qkv_proj, rows=batch * length), batch, length, H)
        else:
            if xn is not None:
                qkv = ops.norm_linear(xn, **exec_weights(self.qkv_proj, compute), out_dtype=compute,
                                      compute_dtype=compute)
            else:
                qkv = apply_linear(self.qkv_proj, x, norm=self.norm_attn, out_dtype=compute, compute=compute)
            o_buf, o = ops.merge_heads_out(batch, length, H, D // H, compute, x.device)
            ops.attention(ops.heads_view(qkv, batch, length, H, 0, D), ops.heads_view(qkv, batch, length, H, D, D),
                          ops.heads_view(qkv, batch, length, H, 2 * D, D), out=o)
        # each residual element is read and then written by the same lane: in place is safe
        if w8 is not None:  # opt-in W8A8 MLP (cortex.quantization.w8a8): int8 activations end to end
            up, down = self.mlp[0], self.mlp[2]
            x, xq = linear_residual_ln(self.out_proj, o_buf, x, self.norm_mlp, out=x if inplace else None,
                                       xq_scale=w8[0])
            hq = ops.linear_w8a8(xq, w8[0], up.weight_int8, up.weight_scale, up.bias, act="gelu",
                                 out_dtype=torch.int8, out_scale=w8[1])
            return ops.linear_w8a8(hq, w8[1], down.weight_int8, down.weight_scale, down.bias, residual=x, out=x)
        if residual_ln_ok(self.out_proj, self.norm_mlp, self.mlp[0], x, compute):
            x, hn = linear_residual_ln(self.out_proj, o_buf, x, self.norm_mlp, out=x if inplace else None)
            h = ops.norm_linear(hn, **exec_weights(self.mlp[0], compute), act="gelu", out_dtype=compute,
                                compute_dtype=compute)
        else:
            x = apply_linear(self.out_proj, o_buf, residual=x, out_dtype=x.dtype, compute=compute,
                             out=x if inplace else None)
            h = apply_linear(self.mlp[0], x, norm=self.norm_mlp, act="gelu", out_dtype=compute, compute=compute)
        return apply_linear(self.mlp[2], h, residual=x, out_dtype=x.dtype, compute=compute,
                            out=x if inplace else None)

    def _w8a8(self, x: torch.Tensor, compute: torch.dtype) -> tuple | None:
        """``(s_up, s_down, attn)`` activation scales when this block runs its MLP as W8A8
        (enabled, bf16 compute, no calibration hooks, int8 weights with K a multiple of 128,
        fp32 biases); ``attn`` = ``(s_qkv, s_out)`` when the attention half qualifies too
        (int8 qkv / out weights, D = 512, no hooks on them or on norm_attn), else None."""
        from cortex.quantization.w8a8 import w8a8_scales

        w8 = w8a8_scales(self)
        if w8 is None or not residual_ln_ok(self.out_proj, self.norm_mlp, self.mlp[0], x, compute):
            return None
        up, down = self.mlp[0], self.mlp[2]
        if up._forward_pre_hooks or down._forward_pre_hooks or not hasattr(up, "weight_int8"):
            return None
        if up.weight_int8.shape[1] % 128 or down.weight_int8.shape[1] % 128 or up.weight_int8.shape[0] % 8:
            return None
        lins = (up, down, self.qkv_proj, self.out_proj)
        if any(getattr(m, "bias", None) is not None and m.bias.dtype != torch.float32 for m in lins):
            return None
        attn = w8[2]
        if attn is not None:
            qkv, out = self.qkv_proj, self.out_proj
            if (x.shape[1] != 512 or qkv._forward_pre_hooks or out._forward_pre_hooks
                    or self.norm_attn._forward_pre_hooks or not hasattr(qkv, "weight_int8")
                    or not hasattr(out, "weight_int8")):
                attn = None
        return (w8[0], w8[1], attn)

    def _forward_rows_w8a8(self, x: torch.Tensor, batch: int, length: int, inplace: bool, w8: tuple) -> torch.Tensor:
        """The whole block on int8 activations (W8A8 mode): norm_attn -> int8, qkv projection +
        attention on int8 operands -> int8 output, out_proj + residual + norm_mlp -> int8, the
        MLP as in forward_rows.  The fp32 residual stream and the softmax stay as they are."""
        s_up, s_down, (s_qkv, s_out) = w8
        qkv, outp, up, down = self.qkv_proj, self.out_proj, self.mlp[0], self.mlp[2]
        na, nm = self.norm_attn, self.norm_mlp
        xq = ops.ln_rows_i8(x, na.weight, na.bias, na.eps, s_qkv)
        oq = ops.qkv_attention_w8a8(xq, s_qkv, qkv.weight_int8, qkv.weight_scale, qkv.bias, batch, length,
                                    self.num_heads, out_dtype=torch.int8, out_scale=s_out)
        x, hq_in = ops.linear_residual_ln_w8a8(oq, s_out, outp.weight_int8, outp.weight_scale, outp.bias, residual=x,
                                               ln=(nm.weight, nm.bias, nm.eps), out=x if inplace else None,
                                               xn_dtype=torch.int8, xn_scale=s_up)
        hq = ops.linear_w8a8(hq_in, s_up, up.weight_int8, up.weight_scale, up.bias, act="gelu",
                             out_dtype=torch.int8, out_scale=s_down)
        return ops.linear_w8a8(hq, s_down, down.weight_int8, down.weight_scale, down.bias, residual=x, out=x)

    def _fused_attention_ok(self, x: torch.Tensor, length: int) -> bool:
        """Whether ``cortex_qkv_attention`` covers this block: bf16 compute, no calibration
        hooks on qkv_proj or norm_attn, head dim 64, at most 256 latents, an fp32 bias (or none)."""
        lin = self.qkv_proj
        D = x.shape[1]
        return (self.config.compute_dtype == torch.bfloat16 and not lin._forward_pre_hooks
                and not self.norm_attn._forward_pre_hooks and D == 64 * self.num_heads and D % 64 == 0
                and 1 <= length <= 256
                and (lin.bias is None or (lin.bias.dtype == torch.float32 and lin.bias.data_ptr() % 16 == 0))
                and ln_rows_ok(x, self.norm_attn))

    def forward(self, latents: torch.Tensor) -> torch.Tensor:
        """(B, L, D) -> (B, L, D)."""
        B, L, D = latents.shape
        x = latents.reshape(B * L, D).contiguous()
        return self.forward_rows(x, B, L).reshape(B, L, D)


class PerceiverEncoder(nn.Module):
    """Cross-attention into learned latents, then N self-attention blocks (reference :129-158)."""

    def __init__(self, config: CortexConfig) -> None:
        super().__init__()
        self.config = config
        self.latents = nn.Parameter(torch.randn(config.num_latents, config.latent_dim) * 0.02)
        self.cross_attn = CrossAttentionBlock(config)
        self.self_attn_blocks = nn.ModuleList([SelfAttentionBlock(config) for _ in range(config.num_layers)])
        self.final_norm = nn.LayerNorm(config.latent_dim)

    def weight_window(self):
        """The ``WeightWindow`` of the INT8-resident mode (``CORTEX_INT8_WEIGHTS=window``) over the
        cross-attention's kv / out projections and, in a second region shared block by block, the
        self-attention blocks' four linears; built on first use, rebuilt when a weight is replaced.
        None in the other modes."""
        if _layers.INT8_WEIGHTS != "window":
            return None
        xa = self.cross_attn
        regions = {"cross": [(xa, [xa.kv_proj, xa.out_proj])],
                   "block": [(b, [b.qkv_proj, b.out_proj, b.mlp[0], b.mlp[2]]) for b in self.self_attn_blocks]}
        # the residual linear + LayerNorm and the residual GEMM read fragment-order weights
        roles = {id(xa.out_proj): "ln"}
        for b in self.self_attn_blocks:
            roles[id(b.out_proj)] = "ln"
            roles[id(b.mlp[2])] = "res"
        lins = [lin for g in regions.values() for _, ls in g for lin in ls if hasattr(lin, "weight_int8")]
        sig = tuple((lin.weight_int8.data_ptr(), tuple(lin.weight_int8.shape)) for lin in lins)
        cached = self.__dict__.get("_cortex_window_sig")
        if cached is not None and cached[0] == sig:
            return cached[1]
        win = build_weight_window(regions, lins[0].weight_int8.device, roles) if lins else None
        self.__dict__["_cortex_window_sig"] = (sig, win)
        return win

    def encode_rows(self, x: torch.Tensor, batch: int, final_norm: bool = True, inplace: bool = False,
                    xn: torch.Tensor | None = None) -> torch.Tensor:
        """Self-attention stack (+ final norm) on the (B*L, D) residual after cross-attention;
        ``xn`` is the first block's ``norm_attn(x)`` when already computed."""
        L = self.config.num_latents
        for i, block in enumerate(self.self_attn_blocks):
            x = block.forward_rows(x, batch, L, inplace=inplace, xn=xn if i == 0 else None)
        if not final_norm:
            return x
        return ops.layer_norm(x, self.final_norm.weight, self.final_norm.bias, self.final_norm.eps)

    def forward(self, tokens: torch.Tensor, token_mask: torch.Tensor | None = None) -> torch.Tensor:
        """tokens (B, E, D), token_mask (B, E) bool -> latents (B, L, D)."""
        B = tokens.shape[0]
        L, D = self.latents.shape
        win = self.weight_window()
        if win is not None:
            win.reset()
        lat = self.latents.unsqueeze(0).expand(B, -1, -1)
        x = self.cross_attn(lat, tokens, token_mask)
        return self.encode_rows(x.reshape(B * L, D), B).reshape(B, L, D)
