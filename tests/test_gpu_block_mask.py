"""Temporal tile mask on the device and tile-masked attention on the bf16 fast path
(reference sparse_xattn.py:152-200 and :340-434).

The mask is integer work and must equal the oracle bit for bit (the oracle is pinned
by the reference's known answers and a brute-force definition in test_oracle.py).
Masked attention: bf16 inputs, fp32 softmax, outputs within 1e-2 of the largest
output magnitude of the float64 oracle on the same bf16 inputs; rows with no
allowed key are exactly 0.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import cortex_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _close(got: np.ndarray, ref: np.ndarray, frac: float = 1e-2):
    tol = frac * max(float(np.abs(ref).max()), 1e-6)
    err = float(np.abs(got - ref).max())
    assert err <= tol, f"max |err| {err:.3e} > {tol:.3e}"


@pytest.mark.parametrize("seed", range(6))
def test_temporal_mask_single_sample_matches_oracle(seed):
    from cortex.kernels import ops
    from cortex.kernels.sparse_xattn import build_temporal_block_mask

    rng = np.random.default_rng(100 + seed)
    for _ in range(6):
        E = int(rng.integers(1, 3000))
        L = int(rng.integers(1, 400))
        T = int(rng.choice([600, 7, 1000003, int(rng.integers(1, 5000))]))
        w = int(rng.integers(0, 80))
        bl, be = int(rng.choice([16, 32, 64])), int(rng.choice([32, 64, 128]))
        t = np.sort(rng.integers(0, max(T, 1), E)) if rng.random() < 0.7 else rng.integers(0, max(T, 1), E)
        ref = O.temporal_block_mask(t, L, T, w, bl, be)
        td = torch.from_numpy(t).to(DEV)
        got = ops.temporal_block_mask(td, L, T, w, bl, be)
        assert got.dtype == torch.bool and got.shape == ref.shape
        np.testing.assert_array_equal(got.cpu().numpy(), ref, err_msg=f"E={E} L={L} T={T} w={w} bl={bl} be={be}")
        cpu = build_temporal_block_mask(td, L, T, w, bl, be)  # the reference API on device times
        assert cpu.device.type == "cpu"
        np.testing.assert_array_equal(cpu.numpy(), ref)


def test_temporal_mask_known_answers():
    """The reference test's cases: a full window allows everything, window 0 does not."""
    from cortex.kernels import ops

    t = torch.arange(64, device=DEV) % 120
    assert ops.temporal_block_mask(t, 32, 120, window_bins=120, block_l=32, block_e=32).all()
    z = torch.zeros(128, dtype=torch.int64, device=DEV)
    m = ops.temporal_block_mask(z, 64, 120, window_bins=0, block_l=32, block_e=32).cpu()
    assert not m.all() and m[0].all()
    assert ops.temporal_block_mask(torch.zeros(0, dtype=torch.int64, device=DEV), 64, 120).shape == (1, 0)


def test_temporal_mask_per_sample_csr():
    from cortex.kernels import ops

    rng = np.random.default_rng(7)
    lens = np.array([0, 1, 63, 64, 65, 700, 130, 0, 2000])
    off = np.concatenate([[0], np.cumsum(lens)])
    T, L, w = 600, 256, 25
    t = np.concatenate([np.sort(rng.integers(0, T, n)) for n in lens])
    got = ops.temporal_block_mask(torch.from_numpy(t).to(DEV), L, T, w, 64, 64,
                                  offsets=torch.from_numpy(off).to(DEV)).cpu().numpy()
    n_k = math.ceil(off[-1] / 64)
    assert got.shape == (len(lens), math.ceil(L / 64), n_k)
    for b, n in enumerate(lens):
        ref = np.zeros((math.ceil(L / 64), n_k), dtype=bool)
        if n:
            r = O.temporal_block_mask(t[off[b]:off[b + 1]], L, T, w, 64, 64)
            ref[:, :r.shape[1]] = r
        np.testing.assert_array_equal(got[b], ref, err_msg=f"sample {b}")


def _masked_case(B, H, L, E, bl, be, mask_kind, seed, lens=None):
    from cortex.kernels import ops

    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, H, L, 64, generator=g) / 4).bfloat16()
    k = torch.randn(B, H, E, 64, generator=g).bfloat16()
    v = torch.randn(B, H, E, 64, generator=g).bfloat16()
    n_q, n_k = math.ceil(L / bl), math.ceil(E / be)
    rng = np.random.default_rng(seed)
    if mask_kind == "temporal":
        t = np.sort(rng.integers(0, 600, E))
        bm = O.temporal_block_mask(t, L, 600, 40, bl, be)
    elif mask_kind == "per_sample":
        bm = rng.random((B, n_q, n_k)) < 0.4
        bm[0] = False  # a sample with no allowed tile at all
    else:
        bm = rng.random((n_q, n_k)) < 0.3
        bm[0] = False  # a query tile with no allowed key tile
    kl = None if lens is None else torch.tensor(lens, dtype=torch.int64)
    out = ops.attention(q.to(DEV), k.to(DEV), v.to(DEV), block_mask=torch.from_numpy(bm).to(DEV),
                        block_l=bl, block_e=be, kv_lengths=None if kl is None else kl.to(DEV))
    ref = O.sparse_cross_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), bm, bl, be,
                                   kv_lengths=lens)
    got = out.float().cpu().numpy()
    _close(got, ref)
    em = O.expand_block_mask(bm, L, E, bl, be)
    if em.ndim == 2:
        em = np.broadcast_to(em, (B, L, E))
    if lens is not None:
        em = em & (np.arange(E)[None, None, :] < np.asarray(lens)[:, None, None])
    empty = ~em.any(-1)  # (B, L)
    assert (got.transpose(0, 2, 1, 3)[empty] == 0).all()


@pytest.mark.parametrize("B,H,L,E,bl,be,kind", [
    (2, 8, 256, 512, 64, 64, "temporal"),       # 16-query groups per wave, shared mask
    (32, 8, 256, 512, 64, 64, "temporal"),      # 32-query waves (B*H >= 256)
    (3, 8, 200, 700, 32, 64, "random"),         # partial query and key tiles
    (32, 8, 256, 384, 16, 64, "random"),        # two query tiles inside one wave
    (2, 4, 256, 5000, 64, 128, "random"),       # > 64 key tiles: schedule window advances
    (4, 8, 256, 600, 64, 64, "per_sample"),     # (B, n_q, n_k) masks, one all-false sample
])
def test_masked_fast_attention_matches_oracle(B, H, L, E, bl, be, kind):
    _masked_case(B, H, L, E, bl, be, kind, seed=B * 31 + E)


def test_masked_attention_with_lengths():
    """Tile mask and per-sample lengths together (the last allowed tile is partial)."""
    _masked_case(3, 8, 256, 640, 64, 64, "random", seed=5, lens=[640, 130, 1])


def test_masked_attention_general_tile_shape():
    """block_e = 32 is outside the fast path's 64-key tiles: the general kernel runs."""
    _masked_case(2, 8, 128, 300, 64, 32, "random", seed=9)
