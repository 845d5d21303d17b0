"""bf16 / head-dim-64 attention (the forward's self-, cross- and behaviour-head
attention) on the GPU vs the float64 oracle, and vs the general kernel (a3, a4).

Tolerance: the probabilities and the output are rounded to bf16 once each
(relative step 2^-8), so outputs agree with the float64 result of the same bf16
inputs to 1e-2 of the largest output magnitude.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import cortex_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
H, DH = 8, 64


def _close(got: np.ndarray, ref: np.ndarray, frac: float = 1e-2):
    tol = frac * max(float(np.abs(ref).max()), 1e-6)
    err = float(np.abs(got - ref).max())
    assert err <= tol, f"max |err| {err:.3e} > {tol:.3e}"


@pytest.mark.parametrize("lens", [[512, 300, 1, 0, 63, 64, 65, 640], [128] * 4, [7, 700, 129], [2048, 5, 1500, 0]])
def test_csr_cross_attention_bf16(lens):
    """Batch-invariant latent queries (q batch stride 0) against ragged CSR keys."""
    from cortex.kernels import ops

    lens = np.asarray(lens)
    B, L = len(lens), 256
    off = np.concatenate([[0], np.cumsum(lens)])
    g = torch.Generator().manual_seed(int(lens.sum()))
    q = (torch.randn(1, H, L, DH, generator=g) / 4).bfloat16()
    kv = torch.randn(max(int(off[-1]), 1), 2 * H * DH, generator=g).bfloat16()
    kd = kv.to(DEV)
    E = int(off[-1])
    out = ops.attention(q.to(DEV), ops.heads_view(kd, 1, E, H, 0, H * DH), ops.heads_view(kd, 1, E, H, H * DH, H * DH),
                        kv_offsets=torch.from_numpy(off).to(DEV), batch=B).float().cpu().numpy()
    for b in range(B):
        if lens[b] == 0:
            assert (out[b] == 0).all()
            continue
        kb = kv[off[b]:off[b + 1], :H * DH].float().reshape(-1, H, DH).permute(1, 0, 2)[None]
        vb = kv[off[b]:off[b + 1], H * DH:].float().reshape(-1, H, DH).permute(1, 0, 2)[None]
        ref = O.attention_bruteforce_f64(q.float(), kb, vb)
        _close(out[b:b + 1], ref)


@pytest.mark.parametrize("B,L", [(4, 256), (2, 200), (3, 64), (1, 129)])
def test_self_attention_from_qkv_buffer_bf16(B, L):
    """Heads read in place from a fused (B*L, 3*H*DH) projection buffer, merged-head output."""
    from cortex.kernels import ops

    g = torch.Generator().manual_seed(B * 1000 + L)
    qkv = (torch.randn(B * L, 3 * H * DH, generator=g) / 3).bfloat16()
    qd = qkv.to(DEV)
    D = H * DH
    o_buf, o = ops.merge_heads_out(B, L, H, DH, torch.bfloat16, qd.device)
    ops.attention(ops.heads_view(qd, B, L, H, 0, D), ops.heads_view(qd, B, L, H, D, D),
                  ops.heads_view(qd, B, L, H, 2 * D, D), out=o)
    got = o_buf.float().cpu().numpy().reshape(B, L, H, DH).transpose(0, 2, 1, 3)
    t = qkv.float().reshape(B, L, 3, H, DH).permute(2, 0, 3, 1, 4)
    ref = O.attention_bruteforce_f64(t[0], t[1], t[2])
    _close(got, ref)


def test_broadcast_two_queries_bf16():
    """The behaviour head's form: 2 shared queries against each sample's 256 latents."""
    from cortex.kernels import ops

    B, L, Q = 6, 256, 2
    g = torch.Generator().manual_seed(77)
    q = (torch.randn(Q, H * DH, generator=g) / 2).bfloat16()
    kv = torch.randn(B * L, 2 * H * DH, generator=g).bfloat16()
    qd, kd = q.to(DEV), kv.to(DEV)
    o_buf, o = ops.merge_heads_out(B, Q, H, DH, torch.bfloat16, kd.device)
    ops.attention(ops.heads_view(qd, 1, Q, H), ops.heads_view(kd, B, L, H, 0, H * DH),
                  ops.heads_view(kd, B, L, H, H * DH, H * DH), out=o, batch=B)
    got = o_buf.float().cpu().numpy().reshape(B, Q, H, DH).transpose(0, 2, 1, 3)
    qq = q.float().reshape(1, Q, H, DH).permute(0, 2, 1, 3).expand(B, -1, -1, -1)
    t = kv.float().reshape(B, L, 2, H, DH).permute(2, 0, 3, 1, 4)
    ref = O.attention_bruteforce_f64(qq, t[0], t[1])
    _close(got, ref)


def test_fast_and_general_kernels_agree():
    """The same inputs through the fast path (lengths only) and through the general kernel
    (forced by an all-true block mask) agree to bf16 resolution."""
    from cortex.kernels.sparse_xattn import sparse_cross_attention

    g = torch.Generator().manual_seed(5)
    B, L, E = 4, 256, 512
    q, k, v = ((torch.randn(B, H, n, DH, generator=g) / 4).bfloat16().to(DEV) for n in (L, E, E))
    lens = torch.tensor([512, 17, 300, 64], device=DEV)
    fast = sparse_cross_attention(q, k, v, kv_lengths=lens).float()
    mask = torch.ones(L // 64, E // 64, dtype=torch.bool)
    kpm = torch.arange(E, device=DEV)[None, :] < lens[:, None]
    general = sparse_cross_attention(q, k, v, mask, BLOCK_L=64, BLOCK_E=64, key_padding_mask=kpm).float()
    err = float((fast - general).abs().max())
    assert err <= 1e-2 * float(general.abs().max())


@pytest.mark.parametrize("B,L,D", [(3, 256, 512), (2, 200, 512), (4, 64, 256), (2, 1, 512), (33, 256, 512)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_fused_qkv_attention(B, L, D, with_bias):
    """QKV projection + self-attention in one kernel: against a float64 projection of the
    same bf16/int8 operands (rounded to bf16, as the projection's output is) followed by the
    float64 attention oracle; 1e-2 of the largest output."""
    from cortex.kernels import ops

    Hh = D // 64
    g = torch.Generator().manual_seed(B * 7 + L + D)
    xn = torch.randn(B * L, D, generator=g).bfloat16()
    w = torch.randn(3 * D, D, generator=g) * 0.04
    q8, s = O.quantize_int8(w.numpy())
    q8, s = torch.from_numpy(q8), torch.from_numpy(s)
    bias = 0.05 * torch.randn(3 * D, generator=g) if with_bias else None
    img = ops.convert(q8.to(DEV), torch.bfloat16)
    out = ops.qkv_attention(xn.to(DEV), img, s.to(DEV), bias.to(DEV) if with_bias else None, B, L, Hh)
    # the int8 weight itself, widened in the kernel: bit-identical to its bf16 image
    out8 = ops.qkv_attention(xn.to(DEV), q8.to(DEV), s.to(DEV), bias.to(DEV) if with_bias else None, B, L, Hh)
    torch.testing.assert_close(out8, out, rtol=0, atol=0)
    qkv = xn.double() @ q8.double().T * s.double()
    if with_bias:
        qkv = qkv + bias.double()
    qkv = qkv.bfloat16().float().reshape(B, L, 3, Hh, 64)
    q, k, v = (qkv[:, :, i].permute(0, 2, 1, 3) for i in range(3))
    ref = O.attention_bruteforce_f64(q, k, v)  # (B, H, L, 64)
    got = out.float().cpu().reshape(B, L, Hh, 64).permute(0, 2, 1, 3).numpy()
    _close(got, ref)
