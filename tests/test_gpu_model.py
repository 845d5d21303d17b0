"""Full Cortex forward on the GPU vs the reference goldens and the oracle (a3, a5, a8, a9)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import cortex_oracle as O
from tests._bars import check_forward

pytestmark = pytest.mark.gpu
DEV = "cuda"
INPUT_KEYS = ("neuron_ids", "time_bins", "values", "batch_indices")


def _cfg(name: str, dtype: str):
    from cortex.models.config import CORTEX_S, CORTEX_XS, CortexConfig

    base = {"xs": CORTEX_XS, "s": CORTEX_S}[name]
    return CortexConfig(**{**base.model_dump(), "dtype": dtype})


def _model(name: str, dtype: str, seed: int = 0):
    from cortex.models import CortexModel

    torch.manual_seed(seed)
    return CortexModel(_cfg(name, dtype)).to(DEV).eval()


def _inputs(arr, prefix):
    return [torch.from_numpy(arr[prefix + k]).to(DEV) for k in INPUT_KEYS]


def _int8(model, inputs):
    from cortex.quantization.calibrate import (attach_calibration_hooks, convert_model, derive_scales,
                                               remove_calibration_hooks)

    hooks = attach_calibration_hooks(model)
    with torch.no_grad():
        model(*inputs)
    remove_calibration_hooks(hooks)
    assert all(h.stats.n_batches == 1 for n, h in hooks.items() if not n.startswith("masked_spike_head"))
    return convert_model(model, derive_scales(model, hooks), inplace=True)


@pytest.mark.parametrize("name", ["xs", "s"])
@pytest.mark.parametrize("inputs", ["sorted", "shuffled"])
def test_fp32_forward_matches_reference_golden(golden, name, inputs):
    """float32 compute: <= 1e-5 relative (to the largest |output|) vs the reference forward."""
    _, arr = golden
    model = _model(name, "float32")
    with torch.no_grad():
        beh = model(*_inputs(arr, f"{name}_{inputs}_"))["behavior"].cpu().numpy()
    ref = arr[f"{name}_{inputs}_behavior_fp32"]
    assert beh.shape == ref.shape
    assert np.abs(beh - ref).max() <= 1e-5 * np.abs(ref).max()


@pytest.mark.parametrize("name", ["xs", "s"])
@pytest.mark.parametrize("dtype,tol", [("float32", "rel1e-5"), ("bfloat16", 2e-2)])
def test_int8_forward_matches_reference_golden(golden, name, dtype, tol):
    """INT8 weights (quantised on the GPU): fp32 compute <= 1e-5 relative; bf16 compute <= 2e-2 max-abs."""
    _, arr = golden
    model = _int8(_model(name, dtype), _inputs(arr, f"{name}_sorted_"))
    for inputs in ("sorted", "shuffled"):
        with torch.no_grad():
            beh = model(*_inputs(arr, f"{name}_{inputs}_"))["behavior"].cpu().numpy()
        ref = arr[f"{name}_{inputs}_behavior_int8"]
        if tol == "rel1e-5":
            assert np.abs(beh - ref).max() <= 1e-5 * np.abs(ref).max(), np.abs(beh - ref).max()
        else:
            check_forward(beh, ref, 4e-3 if name == "s" else 1.5e-3, f"golden {name} {inputs} int8 bf16")


def _config3_inputs(B=32, per=512, seed=0):
    rng = np.random.default_rng(seed)
    E = B * per
    nid = rng.integers(0, 137, E)
    tb = rng.integers(0, 600, E)
    val = np.clip(rng.poisson(1.0, E) + 1, 0, 7)
    bidx = np.repeat(np.arange(B), per)
    return nid, tb, val, bidx


def test_config3_int8_bf16_forward_vs_oracle():
    """Config 3 shape (B=32 x 512 events, CORTEX_S, INT8): decoded velocity within 2e-2 max-abs."""
    arrs = _config3_inputs()
    inputs = [torch.from_numpy(a).to(DEV) for a in arrs]
    model = _int8(_model("s", "bfloat16"), [t[:2048] for t in inputs])
    with torch.no_grad():
        beh = model(*inputs, batch_size=32)["behavior"].cpu().numpy()
    sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    torch.set_num_threads(max(1, torch.get_num_threads()))
    ref = O.forward(sd, O.CORTEX_S_SHAPE, *arrs).numpy()
    assert beh.shape == (32, 2)
    check_forward(beh, ref, 5e-3, "config 3 B=32x512")


@pytest.mark.parametrize("B,lo,hi,seed", [(1, 1, 1, 11), (1, 2048, 2048, 12), (3, 64, 2048, 13), (17, 1, 700, 14),
                                         (64, 64, 900, 15)])
def test_ragged_batches_int8_bf16_vs_oracle(B, lo, hi, seed):
    """Serving-shaped batches: B samples with U[lo, hi] events each (a single event, a
    2048-event sample, 17 ragged samples ...), events in random order; the INT8 bf16
    forward (graph-free) is within 2e-2 max-abs of the float32 oracle."""
    rng = np.random.default_rng(seed)
    counts = rng.integers(lo, hi + 1, B)
    E = int(counts.sum())
    bidx = np.repeat(np.arange(B), counts)
    perm = rng.permutation(E)
    arrs = (rng.integers(0, 137, E), rng.integers(0, 600, E), np.clip(rng.poisson(1.0, E) + 1, 0, 7), bidx[perm])
    inputs = [torch.from_numpy(np.ascontiguousarray(a)).to(DEV) for a in arrs]
    model = _int8(_model("s", "bfloat16"), inputs)
    with torch.no_grad():
        beh = model(*inputs, batch_size=B)["behavior"].cpu().numpy()
    sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    ref = O.forward(sd, O.CORTEX_S_SHAPE, *arrs, batch_size=B).numpy()
    assert beh.shape == (B, 2) and np.isfinite(beh).all()
    check_forward(beh, ref, 5e-3, f"ragged B={B} U[{lo},{hi}]")


def test_cortex_m_int8_bf16_forward_vs_oracle():
    """CORTEX_M (D=768, 12 heads, 384 latents) runs the general kernels wherever the fused ones
    do not apply (384 latents, 12 heads x 2 behaviour queries, N=768 rows): INT8, bf16 compute,
    decoded velocity within 2e-2 max-abs of the float32 oracle."""
    from cortex.models import CortexModel
    from cortex.models.config import CORTEX_M

    arrs = _config3_inputs(B=2, per=200, seed=4)
    inputs = [torch.from_numpy(a).to(DEV) for a in arrs]
    torch.manual_seed(0)
    model = _int8(CortexModel(CORTEX_M).to(DEV).eval(), inputs)
    with torch.no_grad():
        beh = model(*inputs, batch_size=2)["behavior"].cpu().numpy()
    sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    shape = O.ModelShape(768, 11, 12, 384, 768, 12)
    ref = O.forward(sd, shape, *arrs).numpy()
    assert beh.shape == (2, 2) and np.isfinite(beh).all()
    check_forward(beh, ref, 1e-3, "CORTEX_M")


def test_module_path_equals_fused_csr_path_fp32():
    """tokenizer -> _pack_events -> encoder -> behavior_head (padded modules) == fused CSR forward."""
    from cortex.models.cortex import _pack_events

    arrs = _config3_inputs(B=3, per=100, seed=3)
    nid, tb, val, bidx = (torch.from_numpy(a).to(DEV) for a in arrs)
    bidx = bidx[torch.randperm(bidx.shape[0], device=DEV)]
    model = _model("xs", "float32")
    with torch.no_grad():
        fused = model(nid, tb, val, bidx)["behavior"]
        tokens, mask = _pack_events(model.tokenizer(nid, tb, val), bidx)
        lat = model.encoder(tokens, mask)
        modular = model.behavior_head(lat)
    torch.testing.assert_close(modular, fused, rtol=1e-5, atol=1e-6)


def test_captured_graph_replays_match_eager():
    from cortex.runtime import CapturedForward

    model = _int8(_model("s", "bfloat16"), [torch.from_numpy(a).to(DEV) for a in _config3_inputs(2, 64)])
    cap = CapturedForward(model, batch_size=4, n_events=4 * 300)
    for seed in range(3):
        inputs = [torch.from_numpy(a).to(DEV) for a in _config3_inputs(4, 300, seed=10 + seed)]
        got = cap(*inputs).clone()
        with torch.no_grad():
            want = model(*inputs, batch_size=4)["behavior"]
        torch.cuda.synchronize()
        torch.testing.assert_close(got, want, rtol=0, atol=0)


def test_captured_graph_on_caller_buffers():
    """A graph captured on the caller's event buffers replays whatever they hold (no copies), and
    the error flag is cleared inside every replay: an out-of-range call leaves it set, the next
    valid call clears it."""
    from cortex.runtime import CapturedForward

    model = _int8(_model("s", "bfloat16"), [torch.from_numpy(a).to(DEV) for a in _config3_inputs(2, 64)])
    bufs = tuple(torch.from_numpy(a).to(DEV) for a in _config3_inputs(4, 300, seed=30))
    cap = CapturedForward(model, batch_size=4, n_events=4 * 300, inputs=bufs)
    assert cap.neuron_ids.data_ptr() == bufs[0].data_ptr()
    for seed in range(3):
        new = [torch.from_numpy(a).to(DEV) for a in _config3_inputs(4, 300, seed=40 + seed)]
        for dst, src in zip(bufs, new):
            dst.copy_(src)
        got = cap().clone()
        with torch.no_grad():
            want = model(*new, batch_size=4)["behavior"]
        torch.cuda.synchronize()
        torch.testing.assert_close(got, want, rtol=0, atol=0)
    good = bufs[0].clone()
    bufs[0][5] = 10_000
    cap()
    assert int(cap.err_flag.item()) & 1
    bufs[0].copy_(good)
    cap()
    assert int(cap.err_flag.item()) == 0
    with pytest.raises(ValueError):
        CapturedForward(model, batch_size=4, n_events=4 * 300, inputs=bufs[:3])


def test_invalid_token_index_sets_error_flag():
    model = _model("xs", "bfloat16")
    nid, tb, val, bidx = (torch.from_numpy(a).to(DEV) for a in _config3_inputs(2, 50))
    nid[7] = 10_000
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    with torch.no_grad():
        out = model(nid, tb, val, bidx, batch_size=2, err_flag=err)["behavior"]
    assert torch.isfinite(out).all() and int(err.item()) & 1


def test_batch_invariant_queries_follow_parameter_updates():
    """The cached latent/behaviour query projections are rebuilt when a parameter changes in place."""
    model = _int8(_model("xs", "bfloat16"), [torch.from_numpy(a).to(DEV) for a in _config3_inputs(2, 64)])
    inputs = [torch.from_numpy(a).to(DEV) for a in _config3_inputs(3, 80, seed=21)]
    with torch.no_grad():
        a = model(*inputs, batch_size=3)["behavior"].clone()
        b = model(*inputs, batch_size=3)["behavior"].clone()
        torch.testing.assert_close(a, b, rtol=0, atol=0)
        model.encoder.latents.mul_(1.5)
        model.behavior_head.query.add_(0.05)
        c = model(*inputs, batch_size=3)["behavior"].clone()
        model.encoder.__dict__.pop("_cortex_invariant", None)
        model.encoder.cross_attn.__dict__.pop("_cortex_invariant", None)
        model.behavior_head.__dict__.pop("_cortex_invariant", None)
        d = model(*inputs, batch_size=3)["behavior"].clone()
    assert not torch.equal(a, c)
    torch.testing.assert_close(c, d, rtol=0, atol=0)


@pytest.mark.parametrize("name", ["xs", "s"])
def test_fused_behavior_head_matches_oracle_and_unfused(name):
    """The folded one-kernel head (both LayerNorms, folded query/value-output rows) against
    the float32 oracle head on the same latents and against the head run as written
    (forced by a calibration-style pre-hook).  Bar: the decoded-velocity 2e-2 max-abs."""
    arrs = _config3_inputs(2, 64)
    model = _int8(_model(name, "bfloat16"), [torch.from_numpy(a).to(DEV) for a in arrs])
    cfg = model.config
    B, L, D = 5, cfg.num_latents, cfg.latent_dim
    g = torch.Generator().manual_seed(3)
    lat = (torch.randn(B * L, D, generator=g) * 1.5 + 0.2).to(DEV)
    head, fn = model.behavior_head, model.encoder.final_norm
    with torch.no_grad():
        fused = head.forward_rows(lat, B, pre_norm=fn)
        hook = head.q_proj.register_forward_pre_hook(lambda m, a: None)
        try:
            plain = head.forward_rows(lat, B, pre_norm=fn)
        finally:
            hook.remove()
        again = head.forward_rows(lat, B, pre_norm=fn)  # the folded rows come from the cache
    sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    shape = O.CORTEX_S_SHAPE if name == "s" else O.CORTEX_XS_SHAPE
    x = torch.nn.functional.layer_norm(lat.cpu().reshape(B, L, D), (D,), sd["encoder.final_norm.weight"],
                                       sd["encoder.final_norm.bias"], fn.eps)
    ref = O.behavior_head(sd, shape, x).numpy()
    f, p = fused.cpu().numpy(), plain.cpu().numpy()
    assert f.shape == (B, 2) and np.isfinite(f).all()
    check_forward(f, ref, 5e-4, f"fused head {name} vs oracle")
    check_forward(f, p, 5e-4, f"fused head {name} vs the head as written")
    assert torch.equal(fused, again)


@pytest.mark.parametrize("D,L,B", [(512, 256, 3), (512, 100, 2), (256, 77, 4), (512, 1, 1), (768, 70, 2)])
def test_behavior_head_kernel_latent_counts(D, L, B):
    """``cortex_behavior_head`` on latent counts that are not multiples of its 16-latent split
    (partials per 16 latents, merged per sample by the second launch) against float64: both
    LayerNorms, rows rounded to bf16 as the kernel's MFMA operand, the exp2-domain softmax over
    latents of the folded score rows, the weighted value rows summed over heads."""
    import torch.nn.functional as F
    from cortex.kernels import ops

    g = torch.Generator().manual_seed(D + L + B)
    Q, H = 2, 8
    QH = Q * H
    x = torch.randn(B * L, D, generator=g) * 1.3 + 0.1
    g1, g2 = (1 + 0.1 * torch.randn(D, generator=g) for _ in range(2))
    b1, b2 = (0.1 * torch.randn(D, generator=g) for _ in range(2))
    ac = torch.zeros(32, D)
    ac[:QH] = torch.randn(QH, D, generator=g) * (3.0 / D ** 0.5)
    ac[16:16 + QH] = torch.randn(QH, D, generator=g) * 0.05
    ac = ac.bfloat16()
    out = ops.behavior_head(x.to(DEV), B, (g1.to(DEV), b1.to(DEV), 1e-5), (g2.to(DEV), b2.to(DEV), 1e-5),
                            ac.to(DEV), Q, H).cpu().double()
    n = F.layer_norm(F.layer_norm(x.double(), (D,), g1.double(), b1.double(), 1e-5), (D,), g2.double(),
                     b2.double(), 1e-5)
    n = n.to(torch.bfloat16).double().reshape(B, L, D)
    a = ac.double()
    sc, tv = n @ a[:QH].T, n @ a[16:16 + QH].T  # (B, L, QH)
    wts = torch.softmax(sc * np.log(2.0), dim=1)
    ref = (wts * tv).sum(1).reshape(B, Q, H).sum(-1)
    err = float((out - ref).abs().max())
    assert err <= 2e-3 * float(ref.abs().max()) + 1e-5, (err, float(ref.abs().max()))


def test_widen_mode_streams_int8_weights_through_the_fused_path(monkeypatch):
    """CORTEX_INT8_WEIGHTS=widen: no bf16 weight image is built; the GEMMs, the fused QKV +
    attention and the residual linear + LayerNorm read the int8 weights and widen them on chip.
    Config-3 shape (B=32 x 512 events): bit-identical to the image mode (the same int8 values
    reach the MFMAs, with the same tiles and K order) and within 2e-2 of the float32 oracle; the resident weight bytes drop to the int8 weights,
    their scales and the float parameters."""
    from cortex.kernels import ops
    from cortex.models import _layers

    arrs = _config3_inputs(seed=7)
    inputs = [torch.from_numpy(a).to(DEV) for a in arrs]
    monkeypatch.setattr(_layers, "INT8_WEIGHTS", "widen")
    model = _int8(_model("s", "bfloat16"), [t[:2048] for t in inputs])
    calls = {"qkv_attention": 0, "linear_residual_ln": 0}
    for name in calls:
        orig = getattr(ops, name)

        def spy(*a, _orig=orig, _name=name, **k):
            calls[_name] += 1
            assert a[1].dtype == torch.int8, (_name, a[1].dtype)  # the weight argument
            return _orig(*a, **k)
        monkeypatch.setattr(ops, name, spy)
    with torch.no_grad():
        widen = model(*inputs, batch_size=32)["behavior"]
        widen2 = model(*inputs, batch_size=32)["behavior"]
    assert calls["qkv_attention"] == 2 * 7 and calls["linear_residual_ln"] >= 2 * 7
    wb = _layers.resident_weight_bytes(model)
    assert wb["bf16_images"] == 0 and 20e6 < wb["int8_weights"] < 30e6
    monkeypatch.undo()
    with torch.no_grad():
        image = model(*inputs, batch_size=32)["behavior"]
    # (the batch-invariant query projections and the folded head stay cached from the widen run)
    assert 1.5 * wb["int8_weights"] < _layers.resident_weight_bytes(model)["bf16_images"] <= 2 * wb["int8_weights"]
    torch.testing.assert_close(widen, widen2, rtol=0, atol=0)
    # the same int8 values reach the MFMAs in both modes and the tiles and K order agree
    torch.testing.assert_close(widen, image, rtol=0, atol=0)
    sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    ref = O.forward(sd, O.CORTEX_S_SHAPE, *arrs).numpy()
    assert np.abs(widen.cpu().numpy() - ref).max() <= 2e-2


def test_window_mode_widens_each_block_in_the_row_kernel_ahead_of_it(monkeypatch):
    """CORTEX_INT8_WEIGHTS=window: only the int8 weights stay resident, plus two bf16 windows (the
    cross-attention's kv / out projections; one self-attention block's four linears, which the
    blocks take in turn).  In a forward the pack plan's first launch widens the cross-attention's
    and the first block's weights (the tokenizer + LayerNorm launch does when the caller hands
    over a CSR plan) and each later block's LayerNorm row launch its own, with no widening launch
    of its own.  Config-3 shape: bit-identical to the image mode
    (the same bf16 weight values reach the same kernels), eager and replayed from a graph."""
    from cortex.kernels import ops
    from cortex.models import _layers
    from cortex.runtime import CapturedForward

    arrs = _config3_inputs(seed=9)
    inputs = [torch.from_numpy(a).to(DEV) for a in arrs]
    monkeypatch.setattr(_layers, "INT8_WEIGHTS", "window")
    model = _int8(_model("s", "bfloat16"), [t[:2048] for t in inputs])
    seen = {"alone": 0, "pack_plan": [], "tokenize_ln": [], "ln_rows": []}
    orig_w, orig_t, orig_l, orig_p = ops.widen_int8, ops.tokenize_ln, ops.ln_rows, ops.pack_plan

    def widen_spy(pairs):
        seen["alone"] += 1
        return orig_w(pairs)

    def tok_spy(*a, widen=None, **k):
        seen["tokenize_ln"].append(len(widen or []))
        return orig_t(*a, widen=widen, **k)

    def ln_spy(*a, widen=None, **k):
        seen["ln_rows"].append(len(widen or []))
        return orig_l(*a, widen=widen, **k)

    def plan_spy(*a, widen=None, **k):
        seen["pack_plan"].append(len(widen or []))
        return orig_p(*a, widen=widen, **k)
    monkeypatch.setattr(ops, "widen_int8", widen_spy)
    monkeypatch.setattr(ops, "pack_plan", plan_spy)
    monkeypatch.setattr(ops, "tokenize_ln", tok_spy)
    monkeypatch.setattr(ops, "ln_rows", ln_spy)
    with torch.no_grad():
        model(*inputs, batch_size=32)  # caches the batch-invariant query projections
        seen.update(alone=0, pack_plan=[], tokenize_ln=[], ln_rows=[])
        win = model(*inputs, batch_size=32)["behavior"].clone()
        win2 = model(*inputs, batch_size=32)["behavior"].clone()
        assert seen["alone"] == 0, seen
        assert seen["pack_plan"] == [2 + 4] * 2 and seen["tokenize_ln"] == [0] * 2, seen
        assert seen["ln_rows"] == [4] * 12, seen
        # a caller-built CSR plan (the serving path): the tokenizer launch carries them instead
        offs = torch.arange(0, 32 * 512 + 1, 512, device=DEV)
        seen.update(alone=0, pack_plan=[], tokenize_ln=[], ln_rows=[])
        csr = model.forward_csr(*inputs[:3], offs).clone()
        assert seen["alone"] == 0 and seen["pack_plan"] == [] and seen["tokenize_ln"] == [2 + 4], seen
    wb = _layers.resident_weight_bytes(model)
    D = 512
    assert wb["bf16_images"] == 0
    assert wb["bf16_windows"] == 2 * (3 * D * D) + 2 * (12 * D * D), wb
    cap = CapturedForward(model, batch_size=32, n_events=32 * 512)
    graph = cap(*inputs).clone()
    # blocks run outside the model forward: one normalising its own rows carries its weights in
    # that launch; one handed its normalised rows widens them on a launch of its own first
    blk, blk2 = model.encoder.self_attn_blocks[3], model.encoder.self_attn_blocks[5]
    x = torch.randn(32 * 256, D, device=DEV)
    with torch.no_grad():
        xn2 = _layers.normalize_bf16(x, blk2.norm_attn)
        seen.update(alone=0, ln_rows=[])
        y_win = blk.forward_rows(x.clone(), 32, 256)
        assert seen["ln_rows"] == [4] and seen["alone"] == 0, seen
        y2_win = blk2.forward_rows(x.clone(), 32, 256, xn=xn2)
        assert seen["alone"] == 1, seen
        # other batch shapes take other kernels on the same windows: B = 1 (K split across
        # workgroups), B = 64 (persistent and three-stage tiles), ragged and shuffled events
        other = [[torch.from_numpy(a).to(DEV) for a in _config3_inputs(B, per, seed=20 + B)]
                 for B, per in ((1, 700), (64, 160))]
        other[1][3] = other[1][3][torch.randperm(other[1][3].shape[0], device=DEV)]
        other_win = [model(*o, batch_size=o[3].max().item() + 1)["behavior"].clone() for o in other]
    monkeypatch.undo()
    with torch.no_grad():
        image = model(*inputs, batch_size=32)["behavior"]
        y_img = blk.forward_rows(x.clone(), 32, 256)
        y2_img = blk2.forward_rows(x.clone(), 32, 256, xn=xn2)
        other_img = [model(*o, batch_size=o[3].max().item() + 1)["behavior"] for o in other]
    for w, i in zip(other_win, other_img):
        torch.testing.assert_close(w, i, rtol=0, atol=0)
    assert _layers.resident_weight_bytes(model)["bf16_images"] > 2 * wb["bf16_windows"]
    torch.testing.assert_close(win, win2, rtol=0, atol=0)
    torch.testing.assert_close(win, image, rtol=0, atol=0)
    torch.testing.assert_close(csr, image, rtol=0, atol=0)
    torch.testing.assert_close(graph, image, rtol=0, atol=0)
    torch.testing.assert_close(y_win, y_img, rtol=0, atol=0)
    torch.testing.assert_close(y2_win, y2_img, rtol=0, atol=0)
