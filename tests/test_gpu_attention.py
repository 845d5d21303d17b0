"""Attention on the GPU vs the float64 oracle (a3, a4)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import cortex_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _qkv(B, H, L, E, Dh, dtype=torch.float32, seed=123, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return tuple((torch.randn(B, H, n, Dh, generator=g) * scale).to(dtype) for n in (L, E, E))


def _close(got: np.ndarray, ref: np.ndarray, frac: float = 1e-2) -> float:
    """max |got - ref| <= frac * max |ref| (scale-relative: near-uniform attention over
    hundreds of keys gives outputs far below 1, where a fixed absolute bound says nothing)."""
    tol = frac * max(float(np.abs(ref).max()), 1e-6)
    err = float(np.abs(got - ref).max())
    assert err <= tol, f"max |err| {err:.3e} > {tol:.3e}"
    return tol


def _dense(L, E, bl, be):
    return torch.ones(math.ceil(L / bl), math.ceil(E / be), dtype=torch.bool)


@pytest.mark.parametrize("B,H,L,E,Dh", [(1, 1, 32, 64, 16), (2, 4, 64, 128, 32), (1, 8, 128, 256, 64),
                                        (2, 8, 256, 512, 64), (1, 2, 33, 71, 64), (1, 2, 40, 50, 128)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_dense_mask_matches_oracle(B, H, L, E, Dh, dtype):
    from cortex.kernels.sparse_xattn import sparse_cross_attention

    q, k, v = _qkv(B, H, L, E, Dh, dtype)
    mask = _dense(L, E, 32, 32)
    out = sparse_cross_attention(q.to(DEV), k.to(DEV), v.to(DEV), mask, BLOCK_L=32, BLOCK_E=32,
                                 scale=Dh ** -0.5)
    ref = O.sparse_cross_attention(q.float(), k.float(), v.float(), mask.numpy(), 32, 32, Dh ** -0.5)
    assert out.shape == q.shape and out.dtype == dtype
    got = out.float().cpu().numpy()
    if dtype == torch.float32:
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)
        assert np.abs(got - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())
    else:
        _close(got, ref)


def test_checkerboard_sparse_mask_fp32():
    from cortex.kernels.sparse_xattn import sparse_cross_attention

    B, H, L, E, Dh = 1, 4, 64, 128, 32
    q, k, v = _qkv(B, H, L, E, Dh)
    n_q, n_k = 2, 4
    mask = torch.tensor([[(i + j) % 2 == 0 for j in range(n_k)] for i in range(n_q)])
    out = sparse_cross_attention(q.to(DEV), k.to(DEV), v.to(DEV), mask, BLOCK_L=32, BLOCK_E=32)
    ref = O.sparse_cross_attention(q, k, v, mask.numpy(), 32, 32)
    np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-4, atol=1e-5)


def test_all_masked_rows_are_zero_and_partial_tiles():
    from cortex.kernels.sparse_xattn import sparse_cross_attention

    q, k, v = _qkv(1, 2, 48, 100, 64)
    mask = torch.tensor([[True, False, True, False, False, True, False],
                         [False, False, False, False, False, False, False],
                         [False, True, False, False, False, False, True]])  # BLOCK_L 16, BLOCK_E 16
    out = sparse_cross_attention(q.to(DEV), k.to(DEV), v.to(DEV), mask, BLOCK_L=16, BLOCK_E=16)
    ref = O.sparse_cross_attention(q, k, v, mask.numpy(), 16, 16)
    np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-4, atol=1e-5)
    assert (out[:, :, 16:32].cpu() == 0).all()


def test_config1_ragged_lengths_bf16():
    """Config 1: B=32, L=256, E_pad=512, Dh=64, bf16, true lengths U[128,512], N(0,1)/sqrt(64)."""
    from cortex.kernels.sparse_xattn import sparse_cross_attention

    rng = np.random.default_rng(1)
    lens = rng.integers(128, 513, 32)
    q, k, v = _qkv(32, 8, 256, 512, 64, torch.bfloat16, seed=1, scale=1 / 8)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    ref = O.sparse_cross_attention(q.float(), k.float(), v.float(), kv_lengths=lens)
    out = sparse_cross_attention(qd, kd, vd, kv_lengths=torch.from_numpy(lens).to(DEV))
    tol = _close(out.float().cpu().numpy(), ref)
    # the bound discriminates: one 64-event tile more or less, or one key more, is out of it
    for delta in (-64, 64, 1):
        wrong = O.sparse_cross_attention(q.float(), k.float(), v.float(), kv_lengths=np.clip(lens + delta, 1, 512))
        assert float(np.abs(wrong - ref).max()) > tol, delta
    # the same padding as a per-batch 64-event tile mask (whole tiles) + key padding mask
    kpm = torch.arange(512)[None, :] < torch.from_numpy(lens)[:, None]
    tiles = torch.stack([torch.ones(4, 8, dtype=torch.bool) & (torch.arange(8) * 64 < int(n))[None, :]
                         for n in lens])
    out2 = sparse_cross_attention(qd, kd, vd, tiles, BLOCK_L=64, BLOCK_E=64, key_padding_mask=kpm.to(DEV))
    _close(out2.float().cpu().numpy(), ref)


def test_csr_offsets_cross_attention_fp32():
    """Batch-invariant queries against ragged CSR keys (the model's cross-attention layout)."""
    from cortex.kernels import ops

    rng = np.random.default_rng(4)
    lens = rng.integers(1, 300, 5)
    lens[2] = 0
    off = np.concatenate([[0], np.cumsum(lens)])
    H, L, Dh = 8, 256, 64
    g = torch.Generator().manual_seed(4)
    q = torch.randn(1, H, L, Dh, generator=g) / 8
    kv = torch.randn(int(off[-1]), 2 * H * Dh, generator=g)
    kd = kv.to(DEV)
    out = ops.attention(q.to(DEV), ops.heads_view(kd, 1, int(off[-1]), H, 0, H * Dh),
                        ops.heads_view(kd, 1, int(off[-1]), H, H * Dh, H * Dh),
                        kv_offsets=torch.from_numpy(off).to(DEV), batch=5)
    for b in range(5):
        kb = kv[off[b]:off[b + 1], :H * Dh].reshape(-1, H, Dh).permute(1, 0, 2)[None]
        vb = kv[off[b]:off[b + 1], H * Dh:].reshape(-1, H, Dh).permute(1, 0, 2)[None]
        ref = O.attention_bruteforce_f64(q, kb, vb) if lens[b] else np.zeros((1, H, L, Dh))
        np.testing.assert_allclose(out[b:b + 1].cpu().numpy(), ref, rtol=1e-4, atol=1e-5)


