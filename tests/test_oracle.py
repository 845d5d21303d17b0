"""Pin the CPU oracle before trusting it (CPU only).

Each oracle function is checked against something independent of its own
formula: goldens written by importing the reference (tests/golden/make_golden.py),
pure-Python brute force on tiny inputs, reference known-answer tests, library
routines, or invariants that a dropped term / swapped index / wrong rounding mode
would break.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import cortex_oracle as O

# ----------------------------------------------------------------- model goldens


def _product_model(name: str, seed: int):
    from cortex.models import CortexModel
    from cortex.models.config import CORTEX_S, CORTEX_XS

    torch.manual_seed(seed)
    return CortexModel({"xs": CORTEX_XS, "s": CORTEX_S}[name]).eval()


@pytest.mark.parametrize("name", ["xs", "s"])
def test_seeded_init_matches_reference_checksums(golden, name):
    """Construction order of the models equals the reference's RNG consumption."""
    meta, _ = golden
    case = meta["cases"][name]
    sd = _product_model(name, case["seed"]).state_dict()
    assert set(sd) == set(case["state_dict"]), set(sd) ^ set(case["state_dict"])
    for k, ref in case["state_dict"].items():
        t = sd[k].detach().double()
        assert list(t.shape) == ref["shape"], k
        assert float(t.sum()) == pytest.approx(ref["sum"], rel=1e-9, abs=1e-9), k
        assert float(t.abs().sum()) == pytest.approx(ref["abs_sum"], rel=1e-9, abs=1e-9), k
        np.testing.assert_array_equal(sd[k].flatten()[:8].numpy(), np.float32(ref["head"]), err_msg=k)


@pytest.mark.parametrize("name", ["xs", "s"])
@pytest.mark.parametrize("inputs", ["sorted", "shuffled"])
def test_oracle_forward_fp32_matches_reference(golden, name, inputs):
    meta, arr = golden
    sd = _product_model(name, meta["cases"][name]["seed"]).state_dict()
    shape = O.CORTEX_XS_SHAPE if name == "xs" else O.CORTEX_S_SHAPE
    p = f"{name}_{inputs}_"
    beh = O.forward(sd, shape, arr[p + "neuron_ids"], arr[p + "time_bins"], arr[p + "values"],
                    arr[p + "batch_indices"])
    np.testing.assert_allclose(beh.numpy(), arr[p + "behavior_fp32"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("name", ["xs", "s"])
def test_oracle_quantization_matches_reference_convert_model(golden, name):
    """Every int8 weight / scale of the reference's convert_model, bit for bit in sum form."""
    meta, arr = golden
    case = meta["cases"][name]
    sd = O.quantize_state_dict(_product_model(name, case["seed"]).state_dict())
    qkeys = {k for k in sd if k.endswith(("weight_int8", "weight_scale"))}
    assert qkeys == set(case["int8_state_dict"])
    assert len(qkeys) == 2 * case["n_quantized"] == 2 * 34 if name == "s" else True
    for k, ref in case["int8_state_dict"].items():
        t = sd[k]
        if t.dtype == torch.int8:
            assert int(t.long().sum()) == ref["sum"], k
            assert int(t.long().abs().sum()) == ref["abs_sum"], k
            assert int((t.long() ** 2).sum()) == ref["sq_sum"], k
        else:
            assert float(t.double().sum()) == ref["sum"], k
            np.testing.assert_array_equal(t[:8].numpy(), np.float32(ref["head"]), err_msg=k)
    for key in ("encoder.cross_attn.q_proj.weight_int8", "encoder.self_attn_blocks.0.mlp.2.weight_int8",
                "behavior_head.out_proj.weight_int8", "encoder.cross_attn.q_proj.weight_scale",
                "behavior_head.out_proj.weight_scale"):
        ref = arr[f"{name}_slice_{key}"]
        np.testing.assert_array_equal(sd[key][: ref.shape[0]].numpy(), ref, err_msg=key)


@pytest.mark.parametrize("name", ["xs", "s"])
@pytest.mark.parametrize("inputs", ["sorted", "shuffled"])
def test_oracle_forward_int8_matches_reference(golden, name, inputs):
    meta, arr = golden
    sd = O.quantize_state_dict(_product_model(name, meta["cases"][name]["seed"]).state_dict())
    shape = O.CORTEX_XS_SHAPE if name == "xs" else O.CORTEX_S_SHAPE
    p = f"{name}_{inputs}_"
    beh = O.forward(sd, shape, arr[p + "neuron_ids"], arr[p + "time_bins"], arr[p + "values"],
                    arr[p + "batch_indices"])
    np.testing.assert_allclose(beh.numpy(), arr[p + "behavior_int8"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("name", ["xs", "s"])
@pytest.mark.parametrize("inputs", ["sorted", "shuffled"])
@pytest.mark.parametrize("quant", ["fp32", "int8"])
def test_oracle_masked_spike_logits_match_reference(golden, name, inputs, quant):
    """``return_aux`` output of the reference (masked_spike_head.proj stays float in the INT8
    model: calibration forwards never reach it)."""
    meta, arr = golden
    sd = _product_model(name, meta["cases"][name]["seed"]).state_dict()
    if quant == "int8":
        sd = O.quantize_state_dict(sd)
    shape = O.CORTEX_XS_SHAPE if name == "xs" else O.CORTEX_S_SHAPE
    p = f"{name}_{inputs}_"
    aux: dict = {}
    O.forward(sd, shape, arr[p + "neuron_ids"], arr[p + "time_bins"], arr[p + "values"], arr[p + "batch_indices"],
              aux=aux)
    np.testing.assert_allclose(aux["masked_spike_logits"].numpy(), arr[p + f"aux_{quant}"], rtol=1e-5, atol=1e-6)


def test_golden_int8_differs_from_fp32(golden):
    """The INT8 goldens are a different model from the fp32 ones (guards a no-op convert)."""
    _, arr = golden
    d = np.abs(arr["s_sorted_behavior_int8"] - arr["s_sorted_behavior_fp32"]).max()
    assert 1e-6 < d < 5e-2


# ----------------------------------------------------------------- tokenizer


def test_tokenize_bruteforce_fp32_bitexact():
    rng = np.random.default_rng(1)
    n, t, v = (rng.normal(0, 0.02, (s, 8)).astype(np.float32) for s in (5, 7, 3))
    nid, tb, val = rng.integers(0, 5, 11), rng.integers(0, 7, 11), rng.integers(0, 3, 11)
    out = O.tokenize(n, t, v, nid, tb, val)
    for e in range(11):
        for d in range(8):
            want = np.float32(np.float32(n[nid[e], d] + t[tb[e], d]) + v[val[e], d])
            assert out[e, d].tobytes() == want.tobytes()


def test_tokenize_add_order_matters_and_is_left_to_right():
    """(n + t) + v differs from n + (t + v) for these values; the oracle must give the former."""
    n = np.array([[1.0]], np.float32)
    t = np.array([[-1.0]], np.float32)
    v = np.array([[1e-8]], np.float32)
    z = np.zeros(1, np.int64)
    assert O.tokenize(n, t, v, z, z, z)[0, 0] == np.float32(1e-8)  # (1 - 1) + 1e-8
    assert np.float32(1.0) + (np.float32(-1.0) + np.float32(1e-8)) == 0.0  # right to left loses it


def test_tokenize_reference_known_answers():
    torch.manual_seed(42)
    n, t, v = (torch.randn(s, 32) for s in (8, 16, 4))
    one = O.tokenize(n.numpy(), t.numpy(), v.numpy(), [3], [7], [1])
    np.testing.assert_array_equal(one[0], (n[3] + t[7] + v[1]).numpy())
    same = O.tokenize(n.numpy(), t.numpy(), v.numpy(), [0] * 100, [0] * 100, [0] * 100)
    assert (same == same[0:1]).all()
    assert O.tokenize(n.numpy(), t.numpy(), v.numpy(), [], [], []).shape == (0, 32)
    with pytest.raises(IndexError):
        O.tokenize(n.numpy(), t.numpy(), v.numpy(), [8], [0], [0])


# ----------------------------------------------------------------- pack


def _pack_bruteforce(x, b):
    B = max(b) + 1 if len(b) else 1
    rows = [[] for _ in range(B)]
    for i, bi in enumerate(b):
        rows[bi].append(x[i])
    emax = max((len(r) for r in rows), default=0)
    out = np.zeros((B, emax, x.shape[1]), x.dtype)
    mask = np.zeros((B, emax), bool)
    for bi, r in enumerate(rows):
        for j, row in enumerate(r):
            out[bi, j] = row
            mask[bi, j] = True
    return out, mask


@pytest.mark.parametrize("seed", range(5))
def test_pack_bruteforce_and_invariants(seed):
    rng = np.random.default_rng(seed)
    E = int(rng.integers(0, 40))
    b = rng.integers(0, 6, E)
    x = rng.normal(size=(E, 3)).astype(np.float32)
    p = O.pack_events(x, b)
    out, mask = _pack_bruteforce(x, list(b))
    np.testing.assert_array_equal(p.padded, out)
    np.testing.assert_array_equal(p.mask, mask)
    assert p.offsets[-1] == E and (np.diff(p.offsets) >= 0).all()
    np.testing.assert_array_equal(p.csr, x[p.order])
    # stability: inside a sample, source order increases
    for s in range(len(p.offsets) - 1):
        seg = p.order[p.offsets[s]:p.offsets[s + 1]]
        assert (np.diff(seg) > 0).all()
        assert (b[seg] == s).all()


def test_pack_empty_is_one_empty_sample():
    p = O.pack_events(np.zeros((0, 4), np.float32), np.zeros(0, np.int64))
    assert p.padded.shape == (1, 0, 4) and p.mask.shape == (1, 0)


# ----------------------------------------------------------------- quantisation


def test_quantize_error_bound_and_range():
    rng = np.random.default_rng(3)
    w = rng.normal(0, 0.02, (64, 96)).astype(np.float32)
    q, s = O.quantize_int8(w)
    assert q.dtype == np.int8 and q.min() >= -127 and q.max() <= 127
    err = np.abs(w - q.astype(np.float32) * s[:, None])
    assert (err <= 0.5 * s[:, None] * (1 + 1e-5)).all()
    # the row max maps to +-127 exactly
    idx = np.abs(w).argmax(axis=1)
    np.testing.assert_array_equal(np.abs(q[np.arange(64), idx]), 127)


def test_quantize_round_half_even_ties():
    """Weights constructed to land exactly on k + 0.5 after division round to even."""
    s = np.float32(1.0 / 127.0)  # row max 1.0 -> scale = 1/127 exactly as computed in fp32
    row = np.array([1.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5], np.float32)
    w = row.copy()
    w[1:] = (row[1:] * s).astype(np.float32)
    q, sc = O.quantize_int8(w[None, :])
    assert sc[0] == np.float32(1.0) / np.float32(127.0)
    scaled = (w / sc[0]).astype(np.float32)
    ties = np.abs(scaled - np.round(scaled)) == 0.5
    if ties[1:].any():  # where the quotient is exactly .5, the result is the even neighbour
        assert (q[0][1:][ties[1:]] % 2 == 0).all()
    assert q[0][0] == 127


def test_quantize_zero_row_and_special_scale():
    w = np.zeros((2, 8), np.float32)
    w[1, 3] = -4.0
    q, s = O.quantize_int8(w)
    assert s[0] == np.float32(np.float32(1e-8) / np.float32(127.0)) and (q[0] == 0).all()
    assert q[1, 3] == -127 and s[1] == np.float32(4.0) / np.float32(127.0)


# ----------------------------------------------------------------- attention


def test_attention_bruteforce_matches_sdpa():
    torch.manual_seed(123)
    q, k, v = torch.randn(2, 3, 17, 16), torch.randn(2, 3, 29, 16), torch.randn(2, 3, 29, 16)
    ref = F.scaled_dot_product_attention(q.double(), k.double(), v.double())
    np.testing.assert_allclose(O.attention_bruteforce_f64(q, k, v), ref.numpy(), rtol=1e-10, atol=1e-12)


def test_sparse_oracle_dense_mask_and_lengths():
    torch.manual_seed(5)
    q, k, v = torch.randn(2, 2, 32, 8), torch.randn(2, 2, 64, 8), torch.randn(2, 2, 64, 8)
    dense = O.sparse_cross_attention(q, k, v, np.ones((1, 2), bool), 32, 32)
    np.testing.assert_allclose(dense, F.scaled_dot_product_attention(q, k, v).numpy(), rtol=1e-5, atol=1e-6)
    lens = np.array([10, 64])
    got = O.sparse_cross_attention(q, k, v, kv_lengths=lens)
    mask = torch.arange(64)[None, :] < torch.tensor(lens)[:, None]
    ref = F.scaled_dot_product_attention(q, k, v, attn_mask=mask[:, None, None, :])
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-5, atol=1e-6)


def test_sparse_oracle_masked_tile_changes_output_and_empty_rows():
    torch.manual_seed(6)
    q, k, v = torch.randn(1, 1, 32, 8), torch.randn(1, 1, 64, 8), torch.randn(1, 1, 64, 8)
    full = O.sparse_cross_attention(q, k, v, np.array([[True, True]]), 32, 32)
    half = O.sparse_cross_attention(q, k, v, np.array([[True, False]]), 32, 32)
    assert not np.allclose(full, half, atol=1e-3)
    ref_half = F.scaled_dot_product_attention(q, k[:, :, :32], v[:, :, :32])
    np.testing.assert_allclose(half, ref_half.numpy(), rtol=1e-5, atol=1e-6)
    none = O.sparse_cross_attention(q, k, v, np.array([[False, False]]), 32, 32)
    assert (none == 0).all()
    assert np.isnan(O.sparse_cross_attention(q, k, v, np.array([[False, False]]), 32, 32, empty_rows="nan")).all()


# ----------------------------------------------------------------- temporal mask


def test_temporal_mask_reference_known_answers():
    rng = np.random.default_rng(0)
    t = rng.integers(0, 120, 64)
    assert O.temporal_block_mask(t, 32, 120, window_bins=120, BLOCK_L=32, BLOCK_E=32).all()
    z = np.zeros(128, np.int64)
    m = O.temporal_block_mask(z, 64, 120, window_bins=0, BLOCK_L=32, BLOCK_E=32)
    assert m.shape == (2, 4) and not m.all()


@pytest.mark.parametrize("seed", range(4))
def test_temporal_mask_bruteforce_definition(seed):
    rng = np.random.default_rng(seed)
    E, L, T, w = int(rng.integers(1, 200)), int(rng.integers(1, 130)), 600, int(rng.integers(0, 40))
    t = np.sort(rng.integers(0, T, E))
    bl, be = 16, 32
    m = O.temporal_block_mask(t, L, T, w, bl, be)
    for qi in range(math.ceil(L / bl)):
        cs = [np.float32(np.float32(i) / np.float32(L)) * np.float32(T) for i in range(qi * bl, min(L, qi * bl + bl))]
        lo, hi = int(min(cs)) - w, int(max(cs)) + w
        for kj in range(math.ceil(E / be)):
            seg = t[kj * be:(kj + 1) * be]
            assert m[qi, kj] == (seg.min() <= hi and seg.max() >= lo)


# ----------------------------------------------------------------- rms_norm_linear


def test_rms_norm_linear_oracle_matches_library_rms_norm():
    torch.manual_seed(17)
    x, g, w, b = torch.randn(33, 70), torch.randn(70), torch.randn(70, 97), torch.randn(97)
    ref = F.rms_norm(x, (70,), g, 1e-6) @ w + b
    torch.testing.assert_close(O.rms_norm_linear(x, g, w, b), ref, rtol=1e-5, atol=1e-5)


def test_rms_norm_linear_oracle_known_answers():
    x = torch.full((8, 64), 1e4)
    w = torch.randn(64, 32)
    assert torch.isfinite(O.rms_norm_linear(x, torch.ones(64), w)).all()
    # gamma = 1, constant rows normalise to +-1
    x = torch.tensor([[2.0, 2.0], [-3.0, -3.0]])
    out = O.rms_norm_linear(x, torch.ones(2), torch.eye(2), eps=0.0)
    torch.testing.assert_close(out, torch.tensor([[1.0, 1.0], [-1.0, -1.0]]))


def test_flops_per_sample_matches_published_figure():
    """13.56 GFLOP per Cortex-S sample at 512 events (closed-form count)."""
    assert O.flops_per_sample(O.CORTEX_S_SHAPE, 512) / 1e9 == pytest.approx(13.56, abs=0.01)
