"""Host-side logic of the package (CPU only): config, calibration bookkeeping,
save/load, temporal tile mask, and the CPU-device fallback of the three kernel
dispatchers."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

from oracle import cortex_oracle as O


def test_config_validation_and_compute_dtype():
    from cortex.models.config import CORTEX_M, CORTEX_S, CORTEX_XS, CortexConfig

    with pytest.raises(ValueError, match="must equal hidden_dim"):
        CortexConfig(hidden_dim=128, num_layers=2, num_heads=2, head_dim=32, num_latents=32, latent_dim=128,
                     cross_attn_heads=2, max_neurons=256, max_time_bins=512, behavior_dim=2)
    assert CORTEX_S.compute_dtype == torch.bfloat16
    assert CortexConfig(**{**CORTEX_XS.model_dump(), "dtype": "float32"}).compute_dtype == torch.float32
    with pytest.raises(NotImplementedError):
        _ = CortexConfig(**{**CORTEX_XS.model_dump(), "dtype": "float16"}).compute_dtype
    assert (CORTEX_M.hidden_dim, CORTEX_M.num_layers, CORTEX_M.num_latents) == (768, 11, 384)


def test_activation_stats_percentile():
    from cortex.quantization.calibrate import ActivationStats

    s = ActivationStats()
    assert s.percentile_99 == 1.0
    s.update(torch.tensor([1.0, -2.0, 3.0]))
    assert s.n_batches == 1 and s.percentile_99 == pytest.approx(3.0)
    s = ActivationStats()
    for _ in range(99):
        s.update(torch.ones(10))
    s.update(torch.full((10,), 100.0))
    assert s.n_batches == 100 and s.percentile_99 < 50.0
    s = ActivationStats()
    s.update(torch.tensor([-5.0, 1.0]))
    assert s.percentile_99 == pytest.approx(5.0)


def test_hooks_attach_count_and_remove():
    from cortex.quantization.calibrate import attach_calibration_hooks, remove_calibration_hooks

    model = nn.Sequential(nn.Linear(16, 32), nn.ReLU(), nn.Linear(32, 8))
    hooks = attach_calibration_hooks(model)
    assert len(hooks) == 2
    with torch.no_grad():
        for _ in range(5):
            model(torch.randn(4, 16))
    remove_calibration_hooks(hooks)
    with torch.no_grad():
        model(torch.randn(4, 16))
    assert all(h.stats.n_batches == 5 for h in hooks.values())


def test_quantized_linear_buffers_save_load_roundtrip(tmp_path):
    from cortex.quantization.calibrate import (QuantizedLinear, calibration_summary, count_quantized_linears,
                                               load_quantized, model_weight_bytes, save_quantized)

    q, s = O.quantize_int8(np.random.default_rng(0).normal(0, 0.02, (8, 16)).astype(np.float32))
    m = nn.Sequential(QuantizedLinear(torch.from_numpy(q), torch.from_numpy(s), None), nn.Linear(8, 4))
    assert count_quantized_linears(m) == (1, 2)
    assert model_weight_bytes(m) == 8 * 16 + 8 * 4 + (4 * 8 + 4) * 4
    assert "INT8" in m[0].extra_repr()
    assert set(m[0].state_dict()) == {"weight_int8", "weight_scale"}
    save_quantized(m, tmp_path / "q.pt", meta={"note": "x"})
    m2 = nn.Sequential(QuantizedLinear(torch.zeros(8, 16, dtype=torch.int8), torch.zeros(8), None),
                       nn.Linear(8, 4))
    load_quantized(tmp_path / "q.pt", m2)
    assert torch.equal(m2[0].weight_int8, m[0].weight_int8) and torch.equal(m2[0].weight_scale, m[0].weight_scale)
    assert calibration_summary({}, {}) == []


def test_temporal_block_mask_matches_oracle():
    from cortex.kernels.sparse_xattn import build_temporal_block_mask

    rng = np.random.default_rng(8)
    for _ in range(8):
        E, L = int(rng.integers(1, 700)), int(rng.integers(1, 300))
        t = np.sort(rng.integers(0, 600, E))
        w = int(rng.integers(0, 60))
        got = build_temporal_block_mask(torch.from_numpy(t), L, 600, w, 32, 64)
        np.testing.assert_array_equal(got.numpy(), O.temporal_block_mask(t, L, 600, w, 32, 64))
    assert build_temporal_block_mask(torch.arange(64) % 120, 32, 120, window_bins=120, BLOCK_L=32,
                                     BLOCK_E=32).all()


def test_reference_formulations_are_exported():
    """The *_reference functions of the reference API stay importable (torch formulations)."""
    from cortex.kernels.fused_rmsnorm import rms_norm_linear_reference
    from cortex.kernels.sparse_xattn import sparse_cross_attention_reference
    from cortex.kernels.tokenizer import fused_tokenizer_reference

    torch.manual_seed(0)
    x, g, w = torch.randn(4, 8), torch.ones(8), torch.randn(8, 3)
    torch.testing.assert_close(rms_norm_linear_reference(x, g, w), O.rms_norm_linear(x, g, w))
    n = torch.randn(5, 4)
    i = torch.tensor([1, 2])
    assert torch.equal(fused_tokenizer_reference(n, n, n, i, i, i), (n[i] + n[i]) + n[i])
    q = torch.randn(1, 1, 8, 4)
    assert sparse_cross_attention_reference(q, q, q).shape == q.shape


def test_dispatchers_fall_back_on_cpu_tensors():
    """The three kernel dispatchers return the reference's PyTorch formulation for tensors on a
    non-ROCm device, as the reference's dispatchers do (tokenizer.py:201-206,
    sparse_xattn.py:366-368, fused_rmsnorm.py:266-269); checked against the oracle."""
    from cortex.kernels.fused_rmsnorm import rms_norm_linear
    from cortex.kernels.sparse_xattn import sparse_cross_attention
    from cortex.kernels.tokenizer import fused_tokenizer

    g = torch.Generator().manual_seed(42)
    n, t, v = (torch.randn(r, 16, generator=g) * 0.02 for r in (37, 60, 8))
    nid, tb = torch.randint(0, 37, (50,), generator=g), torch.randint(0, 60, (50,), generator=g)
    val = torch.randint(0, 8, (50,), generator=g)
    got = fused_tokenizer(n, t, v, nid, tb, val)
    np.testing.assert_array_equal(got.numpy(), O.tokenize(n.numpy(), t.numpy(), v.numpy(), nid, tb, val))
    # the reference's own known answers: the manual sum and a single event
    assert torch.equal(fused_tokenizer(n, t, v, nid[:1], tb[:1], val[:1]), (n[nid[:1]] + t[tb[:1]]) + v[val[:1]])

    x, gm, w, b = torch.randn(3, 5, 32, generator=g), 1 + 0.02 * torch.randn(32, generator=g), \
        torch.randn(32, 24, generator=g), torch.randn(24, generator=g)
    got = rms_norm_linear(x, gm, w, b)
    assert got.shape == (3, 5, 24)
    torch.testing.assert_close(got.reshape(15, 24), O.rms_norm_linear(x.reshape(15, 32), gm, w, b),
                               rtol=1e-5, atol=1e-5)

    q, k, vv = (torch.randn(2, 2, s, 16, generator=g) for s in (40, 70, 70))
    dense = sparse_cross_attention(q, k, vv)
    np.testing.assert_allclose(dense.numpy(), O.sparse_cross_attention(q.numpy(), k.numpy(), vv.numpy()),
                               rtol=1e-5, atol=1e-5)
    mask = torch.tensor([[True, False, True], [False, True, True]])
    got = sparse_cross_attention(q, k, vv, mask, BLOCK_L=32, BLOCK_E=32)
    want = O.sparse_cross_attention(q.numpy(), k.numpy(), vv.numpy(), mask.numpy(), 32, 32, empty_rows="nan")
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-5, atol=1e-5)
    with pytest.raises(AssertionError, match="block_mask shape"):
        sparse_cross_attention(q, k, vv, mask[:, :2], BLOCK_L=32, BLOCK_E=32)
    with pytest.raises(ValueError, match="ROCm GPU"):
        sparse_cross_attention(q, k, vv, kv_lengths=torch.tensor([3, 4]))


def test_model_and_extensions_refuse_cpu_tensors():
    """Everything beyond the three reference dispatchers (the fused model forward, the pack and
    tokenize + pack extensions) runs on ROCm tensors only and says so."""
    from cortex.kernels import ops
    from cortex.kernels.tokenizer import tokenize_and_pack
    from cortex.models import CortexModel
    from cortex.models.config import CORTEX_XS

    n = torch.randn(4, 8)
    i = torch.zeros(3, dtype=torch.int64)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        tokenize_and_pack(n, n, n, i, i, i, i, batch_size=1)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.pack_plan(i, 1)
    model = CortexModel(CORTEX_XS)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        model(i, i, i, i)
    with pytest.raises(ValueError, match="shape mismatch"):
        model.tokenizer(i, i[:-1], i)


def test_w8a8_enable_disable_bookkeeping():
    """enable_w8a8 switches exactly the blocks whose two MLP linears are QuantizedLinear with
    positive calibrated scales, keeps the state_dict unchanged, and disable_w8a8 undoes it."""
    from cortex.models import CortexModel
    from cortex.models.config import CORTEX_XS
    from cortex.quantization.calibrate import LayerScales, QuantizedLinear
    from cortex.quantization.w8a8 import disable_w8a8, enable_w8a8, w8a8_scales

    model = CortexModel(CORTEX_XS)
    blocks = list(model.encoder.self_attn_blocks)
    scales = {}
    for i, blk in enumerate(blocks):
        for j in (0, 2):
            lin = blk.mlp[j]
            q, s = O.quantize_int8(lin.weight.detach().numpy())
            bias = None if lin.bias is None else lin.bias.detach().clone()
            blk.mlp[j] = QuantizedLinear(torch.from_numpy(q), torch.from_numpy(s), bias)
            scales[f"encoder.self_attn_blocks.{i}.mlp.{j}"] = LayerScales(torch.from_numpy(s), 0.01 * (i + 1) + j)
    for name in ("qkv_proj", "out_proj"):  # block 0's attention linears too: its attention half goes int8
        lin = getattr(blocks[0], name)
        q, s = O.quantize_int8(lin.weight.detach().numpy())
        bias = None if lin.bias is None else lin.bias.detach().clone()
        setattr(blocks[0], name, QuantizedLinear(torch.from_numpy(q), torch.from_numpy(s), bias))
        scales[f"encoder.self_attn_blocks.0.{name}"] = LayerScales(torch.from_numpy(s), 0.5 if name == "qkv_proj" else 0.25)
    keys = set(model.state_dict())
    del scales["encoder.self_attn_blocks.1.mlp.2"]  # no calibration data for one linear: that block stays
    scales["encoder.self_attn_blocks.2.mlp.0"] = LayerScales(torch.ones(1), 0.0)  # a zero scale: stays too
    assert enable_w8a8(model, scales) == len(blocks) - 2
    assert w8a8_scales(blocks[0]) == (0.01, 2.01, (0.5, 0.25)) and w8a8_scales(blocks[1]) is None
    assert w8a8_scales(blocks[3]) == (0.04, 2.04, None)  # float attention linears: MLP only
    assert w8a8_scales(blocks[2]) is None
    assert set(model.state_dict()) == keys
    disable_w8a8(model)
    assert all(w8a8_scales(b) is None for b in blocks)
