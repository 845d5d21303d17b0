"""INT8 weight quantisation on the GPU: bit-exact vs the oracle and the reference goldens (a7)."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

from oracle import cortex_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("N,K", [(1536, 512), (2048, 512), (512, 2048), (1, 512), (17, 33)])
def test_quantize_bitexact(N, K):
    from cortex.kernels import ops

    rng = np.random.default_rng(N * 7 + K)
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    w[0, :] = 0.0  # all-zero row -> scale 1e-8/127, q = 0
    q, s = ops.quantize_int8(torch.from_numpy(w).to(DEV))
    qo, so = O.quantize_int8(w)
    np.testing.assert_array_equal(s.cpu().numpy(), so)
    np.testing.assert_array_equal(q.cpu().numpy(), qo)


def test_quantize_half_way_ties_round_to_even():
    from cortex.kernels import ops

    # quotients exactly k + 0.5 with a power-of-two scale (row max 127 * 2^-7 -> scale 2^-7)
    s = np.float32(2.0 ** -7)
    vals = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5], np.float32) * s
    q, sc = ops.quantize_int8(torch.from_numpy(vals[None, :]).to(DEV))
    qo, so = O.quantize_int8(vals[None, :])
    assert sc.item() == so[0] == s
    np.testing.assert_array_equal(q.cpu().numpy(), qo)
    np.testing.assert_array_equal(qo[0], [127, 0, 2, 2, 0, -2, -2, 126, -126])


def test_quantized_linear_api_and_forward():
    from cortex.quantization.calibrate import LayerScales, QuantizedLinear, weight_scale

    torch.manual_seed(0)
    lin = nn.Linear(64, 32, bias=True).to(DEV)
    nn.init.normal_(lin.weight, std=1.0)
    ws = weight_scale(lin.weight)
    np.testing.assert_array_equal(ws.cpu().numpy(), O.weight_scale(lin.weight.detach().cpu().numpy()))
    ql = QuantizedLinear.from_linear(lin, LayerScales(weight_scale=ws.cpu(), act_scale=0.01))
    assert ql.weight_int8.dtype == torch.int8 and ql.weight_scale.shape == (32,)
    assert "INT8" in ql.extra_repr() and "weight_int8" in ql.state_dict()
    x = torch.randn(16, 64, device=DEV)
    out = ql(x)
    wdq = torch.from_numpy(O.dequantize(ql.weight_int8.cpu().numpy(), ql.weight_scale.cpu().numpy()))
    ref = x.cpu() @ wdq.T + lin.bias.detach().cpu()
    torch.testing.assert_close(out.cpu(), ref, rtol=1e-5, atol=1e-5)
    assert (out.cpu() - lin(x).detach().cpu()).abs().max() < 1.0
    xb = x.bfloat16()
    assert ql(xb).dtype == torch.bfloat16


@pytest.mark.parametrize("name", ["xs", "s"])
def test_convert_model_matches_reference_int8_checksums(golden, name):
    """Full calibrate -> derive_scales -> convert_model flow on the GPU equals the reference's int8 model."""
    from cortex.models import CortexModel
    from cortex.models.config import CORTEX_S, CORTEX_XS
    from cortex.quantization.calibrate import (attach_calibration_hooks, convert_model, count_quantized_linears,
                                               derive_scales, remove_calibration_hooks)

    meta, arr = golden
    case = meta["cases"][name]
    torch.manual_seed(case["seed"])
    model = CortexModel({"xs": CORTEX_XS, "s": CORTEX_S}[name]).to(DEV).eval()
    hooks = attach_calibration_hooks(model)
    p = f"{name}_sorted_"
    inp = [torch.from_numpy(arr[p + k]).to(DEV) for k in ("neuron_ids", "time_bins", "values", "batch_indices")]
    with torch.no_grad():
        model(*inp)
    remove_calibration_hooks(hooks)
    scales = derive_scales(model, hooks)
    assert len(scales) == case["n_quantized"]
    qmodel = convert_model(model, scales, inplace=False)
    n_q, n_tot = count_quantized_linears(qmodel)
    assert n_q == case["n_quantized"] and n_tot == n_q + 1
    sd = qmodel.state_dict()
    for k, ref in case["int8_state_dict"].items():
        t = sd[k].cpu()
        if t.dtype == torch.int8:
            assert int(t.long().sum()) == ref["sum"], k
            assert int((t.long() ** 2).sum()) == ref["sq_sum"], k
        else:
            assert float(t.double().sum()) == ref["sum"], k
            np.testing.assert_array_equal(t[:8].numpy(), np.float32(ref["head"]), err_msg=k)
