"""Serving-shaped batches against the oracle (config 4): CortexModel.forward and the
InferenceWorker (reference cortex/serve/worker.py:160-249, cortex/models/cortex.py:90-122)
on B in {8, 128, 256} samples of clip(Poisson(512), 64, 2048) events, CORTEX_S with INT8
weights and bf16 compute.  Decoded velocity within 2e-2 max-abs of the float32 oracle on
the same events.  B = 256 holds about 131k events: past the one-launch pack plan's 65,536,
so the three-launch plan runs, and the block GEMMs see M = 65,536 rows.

Also here: the ``return_aux`` output (masked_spike_logits) against the reference goldens
and the oracle, and the opt-in index check of the forward and of a captured forward.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import cortex_oracle as O
from tests._bars import check_forward

pytestmark = pytest.mark.gpu
DEV = "cuda"
INPUT_KEYS = ("neuron_ids", "time_bins", "values", "batch_indices")


def _int8_model(dtype: str = "bfloat16"):
    from cortex.models import CortexModel
    from cortex.models.config import CORTEX_S, CortexConfig
    from cortex.quantization.calibrate import (attach_calibration_hooks, convert_model, derive_scales,
                                               remove_calibration_hooks)

    torch.manual_seed(0)
    model = CortexModel(CortexConfig(**{**CORTEX_S.model_dump(), "dtype": dtype})).to(DEV).eval()
    rng = np.random.default_rng(1)
    t = [torch.from_numpy(a).to(DEV) for a in (rng.integers(0, 137, 2048), rng.integers(0, 600, 2048),
                                                np.clip(rng.poisson(1.0, 2048) + 1, 0, 7),
                                                np.repeat(np.arange(4), 512))]
    hooks = attach_calibration_hooks(model)
    with torch.no_grad():
        model(*t)
    remove_calibration_hooks(hooks)
    return convert_model(model, derive_scales(model, hooks), inplace=True)


@pytest.fixture(scope="module")
def model():
    return _int8_model()


@pytest.fixture(scope="module")
def oracle_sd(model):
    return {k: v.detach().cpu() for k, v in model.state_dict().items()}


def _serving_events(B: int, seed: int):
    """B samples, E_b = clip(Poisson(512), 64, 2048), ids as config 0; per-sample columns."""
    rng = np.random.default_rng(seed)
    counts = np.clip(rng.poisson(512, B), 64, 2048)
    cols = []
    for n in counts:
        cols.append((rng.integers(0, 137, n), rng.integers(0, 600, n), np.clip(rng.poisson(1.0, n) + 1, 0, 7)))
    return counts, cols


def _flat(counts, cols, seed):
    """Events of all samples with batch indices, in a shuffled order."""
    nid = np.concatenate([c[0] for c in cols])
    tb = np.concatenate([c[1] for c in cols])
    val = np.concatenate([c[2] for c in cols])
    bidx = np.repeat(np.arange(len(counts)), counts)
    perm = np.random.default_rng(seed).permutation(nid.shape[0])
    return nid[perm], tb[perm], val[perm], bidx[perm]


_CASES = [(8, 41), (128, 42), (256, 43)]
_ORACLE: dict = {}


def _oracle(oracle_sd, B, seed):
    """Oracle behaviour for one case (computed once per module)."""
    if (B, seed) not in _ORACLE:
        counts, cols = _serving_events(B, seed)
        arrs = _flat(counts, cols, seed)
        torch.set_num_threads(max(1, torch.get_num_threads()))
        _ORACLE[(B, seed)] = O.forward(oracle_sd, O.CORTEX_S_SHAPE, *arrs, batch_size=B).numpy()
    return _ORACLE[(B, seed)]


@pytest.mark.parametrize("B,seed", _CASES)
def test_serving_batches_forward_vs_oracle(model, oracle_sd, B, seed):
    counts, cols = _serving_events(B, seed)
    arrs = _flat(counts, cols, seed)
    print(f"config4 forward B={B} E={int(counts.sum())} seed={seed}", flush=True)
    inputs = [torch.from_numpy(np.ascontiguousarray(a)).to(DEV) for a in arrs]
    with torch.no_grad():
        beh = model(*inputs, batch_size=B, check_indices=True)["behavior"].cpu().numpy()
    ref = _oracle(oracle_sd, B, seed)
    assert beh.shape == (B, 2) and np.isfinite(beh).all()
    check_forward(beh, ref, 5e-3, f"config 4 forward B={B}")


@pytest.mark.parametrize("B,seed", _CASES)
@pytest.mark.parametrize("mode", ["sync", "pipelined"])
def test_serving_batches_worker_vs_oracle(model, oracle_sd, B, seed, mode):
    """The worker on columnar payloads (captured graph per batch / event bucket) against the
    oracle on the same events; "pipelined" submits the batch behind another one."""
    from cortex.models.config import CORTEX_S
    from cortex.serve import InferenceWorker

    counts, cols = _serving_events(B, seed)
    print(f"config4 worker B={B} E={int(counts.sum())} mode={mode}", flush=True)
    payloads = [{"request_id": f"r{i}", "events": {"neuron_id": c[0], "time_bin": c[1], "value": c[2]}}
                for i, c in enumerate(cols)]
    w = InferenceWorker(model, CORTEX_S, torch.device(DEV), max_batch_size=B)
    if mode == "sync":
        res = w._run_batch_sync(payloads)
    else:
        first = w.submit_batch(payloads[: max(1, B // 2)])
        pend = w.submit_batch(payloads)
        w.collect(first)
        res = w.collect(pend)
    assert [r["request_id"] for r in res] == [p["request_id"] for p in payloads]
    got = np.array([r["behavior"] for r in res])
    ref = _oracle(oracle_sd, B, seed)
    assert got.shape == (B, 2) and np.isfinite(got).all()
    check_forward(got, ref, 5e-3, f"config 4 worker B={B} {mode}")


def test_worker_batch_buckets_reuse_graphs(model):
    """A dynamic batcher's sizes B = 1..32: graphs are captured per (batch bucket, event
    bucket), the padding samples are dropped, and each result equals the graph-free forward."""
    from cortex.models.config import CORTEX_S
    from cortex.serve import InferenceWorker, batch_bucket

    w = InferenceWorker(model, CORTEX_S, torch.device(DEV), max_batch_size=32)
    ref_w = InferenceWorker(model, CORTEX_S, torch.device(DEV), max_batch_size=32, use_graphs=False)
    rng = np.random.default_rng(9)
    sizes = [1, 9, 10, 3, 31, 32, 25, 9, 17, 32, 1]
    for i, B in enumerate(sizes):
        payloads = [{"request_id": f"b{i}_{j}", "events": {"neuron_id": rng.integers(0, 137, 64),
                                                             "time_bin": rng.integers(0, 600, 64),
                                                             "value": rng.integers(0, 8, 64)}} for j in range(B)]
        got = np.array([r["behavior"] for r in w._run_batch_sync(payloads)])
        want = np.array([r["behavior"] for r in ref_w._run_batch_sync(payloads)])
        assert got.shape == (B, 2)
        assert np.abs(got - want).max() <= 1e-5 * max(np.abs(want).max(), 1e-6)
    keys = {(batch_bucket(B), 256 if 64 * B <= 256 else 1 << (64 * B - 1).bit_length()) for B in sizes}
    assert w.captures == len(keys) < len(sizes)


@pytest.mark.parametrize("name", ["xs", "s"])
@pytest.mark.parametrize("dtype,quant", [("float32", "fp32"), ("float32", "int8"), ("bfloat16", "int8")])
def test_return_aux_matches_reference_golden(golden, name, dtype, quant):
    """masked_spike_logits (return_aux) against the reference: fp32 compute within 1e-5 of
    the largest |logit| (float and INT8 models), bf16 compute within 2e-2 max-abs."""
    from cortex.models import CortexModel
    from cortex.models.config import CORTEX_S, CORTEX_XS, CortexConfig
    from cortex.quantization.calibrate import (attach_calibration_hooks, convert_model, derive_scales,
                                               remove_calibration_hooks)

    _, arr = golden
    base = {"xs": CORTEX_XS, "s": CORTEX_S}[name]
    torch.manual_seed(0)
    model = CortexModel(CortexConfig(**{**base.model_dump(), "dtype": dtype})).to(DEV).eval()
    if quant == "int8":
        calib = [torch.from_numpy(arr[f"{name}_sorted_{k}"]).to(DEV) for k in INPUT_KEYS]
        hooks = attach_calibration_hooks(model)
        with torch.no_grad():
            model(*calib)
        remove_calibration_hooks(hooks)
        convert_model(model, derive_scales(model, hooks), inplace=True)
        assert not hasattr(model.masked_spike_head.proj, "weight_int8")  # never calibrated, stays float
    for inputs in ("sorted", "shuffled"):
        t = [torch.from_numpy(arr[f"{name}_{inputs}_{k}"]).to(DEV) for k in INPUT_KEYS]
        with torch.no_grad():
            out = model(*t, return_aux=True)
        ref = arr[f"{name}_{inputs}_aux_{quant}"]
        got = out["masked_spike_logits"].cpu().numpy()
        assert got.shape == ref.shape and got.dtype == np.float32
        np.testing.assert_array_equal(out["behavior"].shape, arr[f"{name}_{inputs}_behavior_{quant}"].shape)
        if dtype == "float32":
            assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max(), np.abs(got - ref).max()
        else:
            check_forward(got, ref, 7e-3, f"return_aux golden {name} {inputs} {quant}")
        with torch.no_grad():
            assert "masked_spike_logits" not in model(*t)


def test_return_aux_quantized_head_vs_oracle(model, oracle_sd):
    """A masked-spike head that was converted too (int8 weight, per-row scale, bias): the
    widened fp32 weight as QuantizedLinear.forward uses it, against the oracle."""
    from cortex.quantization.calibrate import LayerScales, QuantizedLinear, weight_scale

    head = model.masked_spike_head.proj
    qhead = QuantizedLinear.from_linear(head, LayerScales(weight_scale=weight_scale(head.weight), act_scale=1.0))
    model.masked_spike_head.proj = qhead
    try:
        counts, cols = _serving_events(5, 50)
        arrs = _flat(counts, cols, 50)
        inputs = [torch.from_numpy(np.ascontiguousarray(a)).to(DEV) for a in arrs]
        with torch.no_grad():
            got = model(*inputs, return_aux=True)["masked_spike_logits"].cpu().numpy()
        sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
        assert "masked_spike_head.proj.weight_int8" in sd
        aux: dict = {}
        O.forward(sd, O.CORTEX_S_SHAPE, *arrs, batch_size=5, aux=aux)
        ref = aux["masked_spike_logits"].numpy()
        check_forward(got, ref, 7e-3, "masked-spike logits")
    finally:
        model.masked_spike_head.proj = head


def test_pooled_linear_kernel_vs_float64():
    """The pooled-head kernel alone: LayerNorm per row, mean over L rows, N = 8 outputs with
    bias; fp32 and int8 weights; D = 256 / 512 / 768 / 1024; within 1e-5 of a float64 restatement."""
    from cortex.kernels import ops

    g = torch.Generator().manual_seed(3)
    for D, L, B in ((256, 7, 3), (512, 256, 4), (768, 33, 2), (1024, 5, 1)):
        x = torch.randn(B * L, D, generator=g) * 2 + 0.5
        gm, bt = 1 + 0.1 * torch.randn(D, generator=g), 0.1 * torch.randn(D, generator=g)
        w = torch.randn(8, D, generator=g) * 0.05
        bias = torch.randn(8, generator=g)
        xd = x.double()
        mu = xd.mean(1, keepdim=True)
        var = ((xd - mu) ** 2).mean(1, keepdim=True)
        xn = (xd - mu) / torch.sqrt(var + 1e-5) * gm.double() + bt.double()
        m = xn.reshape(B, L, D).mean(1)
        ref = m @ w.double().T + bias.double()
        got = ops.pooled_linear(x.to(DEV), B, (gm.to(DEV), bt.to(DEV), 1e-5), w.to(DEV), None, bias.to(DEV))
        assert float((got.cpu().double() - ref).abs().max()) <= 1e-5 * float(ref.abs().max())
        mean = ops.pooled_linear(x.to(DEV), B, None)
        assert float((mean.cpu().double() - xd.reshape(B, L, D).mean(1)).abs().max()) <= 1e-5 * float(xd.abs().max())
        q, s = O.quantize_int8(w.numpy())
        wq = torch.from_numpy(q).double() * torch.from_numpy(s).double()[:, None]
        ref_q = m @ wq.T
        got_q = ops.pooled_linear(x.to(DEV), B, (gm.to(DEV), bt.to(DEV), 1e-5), torch.from_numpy(q).to(DEV),
                                  torch.from_numpy(s).to(DEV))
        assert float((got_q.cpu().double() - ref_q).abs().max()) <= 1e-5 * float(ref_q.abs().max())


def test_check_indices_raises_index_error(model):
    counts, cols = _serving_events(3, 60)
    arrs = [np.ascontiguousarray(a) for a in _flat(counts, cols, 60)]
    good = [torch.from_numpy(a).to(DEV) for a in arrs]
    with torch.no_grad():
        ref = model(*good, batch_size=3)["behavior"]
        again = model(*good, batch_size=3, check_indices=True)["behavior"]
    torch.testing.assert_close(again, ref, rtol=0, atol=0)
    for field, bad in ((0, 512), (1, 1024), (2, 8), (0, -1)):
        t = [x.clone() for x in good]
        t[field][5] = bad
        with torch.no_grad(), pytest.raises(IndexError):
            model(*t, batch_size=3, check_indices=True)
        with torch.no_grad():  # unchecked: no exception, the flag alone records it
            flag = torch.zeros(1, dtype=torch.int32, device=DEV)
            model(*t, batch_size=3, err_flag=flag)
            assert int(flag.item()) & 1
    t = [x.clone() for x in good]
    t[3][0] = 3  # batch index outside [0, 3)
    with torch.no_grad(), pytest.raises(IndexError, match="batch index"):
        model(*t, batch_size=3, check_indices=True)


def test_captured_forward_clears_flag_per_replay(model):
    from cortex.runtime import CapturedForward

    counts, cols = _serving_events(2, 61)
    arrs = [torch.from_numpy(np.ascontiguousarray(a)).to(DEV) for a in _flat(counts, cols, 61)]
    cap = CapturedForward(model, 2, arrs[0].shape[0], check_indices=True)
    want = cap(*arrs).clone()
    bad = [x.clone() for x in arrs]
    bad[1][3] = 5000
    with pytest.raises(IndexError):
        cap(*bad)
    torch.testing.assert_close(cap(*arrs), want, rtol=0, atol=0)  # flag cleared: no stale error
    assert int(cap.err_flag.item()) == 0
