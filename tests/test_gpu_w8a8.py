"""The opt-in W8A8 mode (cortex.quantization.w8a8): int8 activations x int8 weights.

Kernel level: the int8 GEMM sums exactly in int32, so its fp32 results are checked
against an exact int64 contraction of the same operands (then the documented fp32
epilogue), and its int8 outputs against the quantisation formula of the documented
interface; the int8 LayerNorm output against torch's LayerNorm of the kernel's own fp32
rows.  Model level: CORTEX_S with W8A8 MLPs stays within the 2e-2 parity bar of the
oracle's fp32 INT8-weight forward (the reference's arithmetic), which the W8A8 mode does
not reproduce exactly: its activations carry 8 bits.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import cortex_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _q(y: np.ndarray, scale: float) -> np.ndarray:
    inv = np.float32(1.0) / np.float32(scale)
    return np.clip(np.rint(y.astype(np.float32) * inv), -127, 127).astype(np.int8)


def _operands(M, N, K, seed):
    rng = np.random.default_rng(seed)
    xq = rng.integers(-127, 128, (M, K), dtype=np.int64).astype(np.int8)
    wq = rng.integers(-127, 128, (N, K), dtype=np.int64).astype(np.int8)
    ws = (rng.random(N, dtype=np.float32) * 1e-3 + 1e-4).astype(np.float32)
    b = rng.normal(0, 0.5, N).astype(np.float32)
    return xq, wq, ws, b


def _exact(xq, wq, a_scale, ws, b):
    acc = xq.astype(np.int64) @ wq.astype(np.int64).T  # exact
    assert np.abs(acc).max() < 2 ** 31
    sc = (ws * np.float32(a_scale)).astype(np.float32)
    # the epilogue's fused multiply-add: acc (as fp32) * sc + b rounded once (the float64
    # product of two fp32 values is exact)
    prod = acc.astype(np.float32).astype(np.float64) * sc.astype(np.float64)
    return (prod + b.astype(np.float64)).astype(np.float32)


@pytest.mark.parametrize("M,N,K", [(8192, 512, 2048), (300, 520, 512), (256, 1024, 256)])
def test_linear_w8a8_fp32_and_residual(M, N, K):
    from cortex.kernels import ops

    xq, wq, ws, b = _operands(M, N, K, seed=M + N)
    a_scale = 0.0123
    want = _exact(xq, wq, a_scale, ws, b)
    res = np.random.default_rng(1).normal(0, 1, (M, N)).astype(np.float32)
    d = {k: torch.from_numpy(v).to(DEV) for k, v in dict(x=xq, w=wq, ws=ws, b=b, r=res).items()}
    y = ops.linear_w8a8(d["x"], a_scale, d["w"], d["ws"], d["b"]).cpu().numpy()
    np.testing.assert_allclose(y, want, rtol=1e-6, atol=1e-6 * np.abs(want).max())
    r = d["r"].clone()
    ops.linear_w8a8(d["x"], a_scale, d["w"], d["ws"], d["b"], residual=r, out=r)  # in place
    np.testing.assert_allclose(r.cpu().numpy(), res + want, rtol=1e-6, atol=1e-6 * np.abs(res + want).max())


@pytest.mark.parametrize("M,N,K", [(8192, 2048, 512), (300, 264, 384)])
def test_linear_w8a8_gelu_int8_out(M, N, K):
    from cortex.kernels import ops

    xq, wq, ws, b = _operands(M, N, K, seed=K)
    a_scale, out_scale = 0.02, 0.05
    y = _exact(xq, wq, a_scale, ws, b)
    want = _q(F.gelu(torch.from_numpy(y).double()).numpy(), out_scale)
    d = {k: torch.from_numpy(v).to(DEV) for k, v in dict(x=xq, w=wq, ws=ws, b=b).items()}
    got = ops.linear_w8a8(d["x"], a_scale, d["w"], d["ws"], d["b"], act="gelu", out_dtype=torch.int8,
                          out_scale=out_scale).cpu().numpy()
    diff = np.abs(got.astype(np.int32) - want.astype(np.int32))
    # the kernel's GELU is within half a bf16 step of erf-GELU: a rounding boundary may fall either way
    assert diff.max() <= 1 and (diff == 0).mean() > 0.999
    got0 = ops.linear_w8a8(d["x"], a_scale, d["w"], d["ws"], d["b"], out_dtype=torch.int8,
                           out_scale=out_scale).cpu().numpy()
    np.testing.assert_array_equal(got0, _q(y, out_scale))  # no activation: the formula exactly


def test_residual_ln_int8_rows():
    from cortex.kernels import ops

    torch.manual_seed(4)
    M, N, K = 4103, 512, 512  # enough rows that the bf16 variant does not split K across workgroups
    a = torch.randn(M, K).bfloat16().to(DEV)
    w = (0.05 * torch.randn(N, K)).bfloat16().to(DEV)
    res = torch.randn(M, N).to(DEV)
    g, be = (1 + 0.1 * torch.randn(N)).to(DEV), (0.1 * torch.randn(N)).to(DEV)
    out_b, xn = ops.linear_residual_ln(a, w, None, None, residual=res, ln=(g, be, 1e-5))
    out_q, xq = ops.linear_residual_ln(a, w, None, None, residual=res, ln=(g, be, 1e-5), xq_scale=0.04)
    assert xq.dtype == torch.int8 and torch.equal(out_b, out_q)
    y = F.layer_norm(out_q.cpu(), (N,), g.cpu(), be.cpu(), 1e-5).numpy()
    diff = np.abs(xq.cpu().numpy().astype(np.int32) - _q(y, 0.04).astype(np.int32))
    assert diff.max() <= 1 and (diff == 0).mean() > 0.999


def test_model_w8a8_within_parity_bar():
    """CORTEX_S, INT8 weights, all 7 self-attention blocks on int8 activations (qkv, out_proj
    and both MLP linears), B = 32 x 512: max-abs against the oracle's fp32 forward (the
    reference arithmetic) within 2e-2; eager equals graph replay."""
    import bench
    from cortex.quantization.w8a8 import disable_w8a8, enable_w8a8
    from cortex.runtime import CapturedForward

    model, scales = bench.build_model(torch.device(DEV), with_scales=True)
    assert enable_w8a8(model, scales) == 7
    from cortex.quantization.w8a8 import w8a8_scales
    assert all(w8a8_scales(b)[2] is not None for b in model.encoder.self_attn_blocks)
    try:
        nid, tb, val, bidx = bench.make_events(32, 512, seed=3)
        ev = [torch.from_numpy(a).to(DEV) for a in (nid, tb, val, bidx)]
        with torch.no_grad():
            got = model(*ev, batch_size=32)["behavior"].cpu()
        sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
        ref = O.forward(sd, O.CORTEX_S_SHAPE, nid, tb, val, bidx, batch_size=32)
        err = float((got - torch.as_tensor(ref)).abs().max())
        assert err <= 2e-2, err
        cap = CapturedForward(model, batch_size=32, n_events=32 * 512)
        assert torch.equal(cap(*ev).cpu(), got)
    finally:
        disable_w8a8(model)


def test_ln_rows_i8():
    from cortex.kernels import ops

    torch.manual_seed(8)
    x = (torch.randn(3001, 512) * 2 + 0.5).to(DEV)
    g, b = (1 + 0.1 * torch.randn(512)).to(DEV), (0.1 * torch.randn(512)).to(DEV)
    q = ops.ln_rows_i8(x, g, b, 1e-5, 0.03).cpu().numpy()
    y = F.layer_norm(x.cpu(), (512,), g.cpu(), b.cpu(), 1e-5).numpy()
    diff = np.abs(q.astype(np.int32) - _q(y, 0.03).astype(np.int32))
    assert diff.max() <= 1 and (diff == 0).mean() > 0.999


def test_linear_residual_ln_w8a8():
    from cortex.kernels import ops

    M, N, K = 8192, 512, 512
    xq, wq, ws, b = _operands(M, N, K, seed=21)
    res = np.random.default_rng(2).normal(0, 1, (M, N)).astype(np.float32)
    a_scale = 0.01
    want = res + _exact(xq, wq, a_scale, ws, b)
    d = {k: torch.from_numpy(v).to(DEV) for k, v in dict(x=xq, w=wq, ws=ws, b=b, r=res).items()}
    g, be = (1 + 0.1 * torch.randn(N)).to(DEV), (0.1 * torch.randn(N)).to(DEV)
    out, xn = ops.linear_residual_ln_w8a8(d["x"], a_scale, d["w"], d["ws"], d["b"], residual=d["r"], ln=(g, be, 1e-5))
    np.testing.assert_allclose(out.cpu().numpy(), want, rtol=1e-6, atol=1e-6 * np.abs(want).max())
    y = F.layer_norm(out.cpu(), (N,), g.cpu(), be.cpu(), 1e-5)
    torch.testing.assert_close(xn.cpu().float(), y.bfloat16().float(), rtol=2 ** -7, atol=1e-5)
    out2, xq2 = ops.linear_residual_ln_w8a8(d["x"], a_scale, d["w"], d["ws"], d["b"], residual=d["r"],
                                            ln=(g, be, 1e-5), xn_dtype=torch.int8, xn_scale=0.05)
    assert torch.equal(out2, out)
    diff = np.abs(xq2.cpu().numpy().astype(np.int32) - _q(y.numpy(), 0.05).astype(np.int32))
    assert diff.max() <= 1 and (diff == 0).mean() > 0.999


def test_qkv_attention_w8a8_vs_float64():
    """int8 projection (exact int32 sums) then bf16 attention, against float64 attention of
    the same dequantised operands (q, k, v rounded to bf16 as the kernel keeps them)."""
    from cortex.kernels import ops

    B, L, D, H = 4, 256, 512, 8
    rng = np.random.default_rng(4)
    xq = rng.integers(-127, 128, (B * L, D)).astype(np.int8)
    wq, ws = O.quantize_int8(rng.normal(0, 0.02, (3 * D, D)).astype(np.float32))
    bias = rng.normal(0, 0.1, 3 * D).astype(np.float32)
    a_scale = 0.02
    d = {k: torch.from_numpy(v).to(DEV) for k, v in dict(x=xq, w=wq, ws=ws, b=bias).items()}
    got = ops.qkv_attention_w8a8(d["x"], a_scale, d["w"], d["ws"], d["b"], B, L, H).cpu().float()
    proj = (xq.astype(np.float64) @ wq.astype(np.float64).T) * (a_scale * ws.astype(np.float64)) + bias
    qkv = torch.from_numpy(proj).bfloat16().double().reshape(B, L, 3, H, D // H).permute(2, 0, 3, 1, 4)
    q, k, v = qkv[0], qkv[1], qkv[2]
    att = torch.softmax(q @ k.transpose(-1, -2) / 8.0, dim=-1) @ v  # (B, H, L, Dh)
    ref = att.permute(0, 2, 1, 3).reshape(B * L, D)
    assert float((got - ref).abs().max()) <= 2e-2 * float(ref.abs().max())
    oq = ops.qkv_attention_w8a8(d["x"], a_scale, d["w"], d["ws"], d["b"], B, L, H, out_dtype=torch.int8,
                                out_scale=0.01).cpu().numpy()
    # the kernel quantises the fp32 attention output; `got` is that output rounded to bf16
    # (0.4 % relative), so about one element in a hundred sits across a rounding boundary
    diff = np.abs(oq.astype(np.int32) - _q(got.numpy(), 0.01).astype(np.int32))
    assert diff.max() <= 1 and (diff == 0).mean() > 0.97


@pytest.mark.parametrize("B", [1, 8])
def test_model_w8a8_small_batches(B):
    """W8A8 blocks at the serving batch sizes where the default path splits K across
    workgroups: still within 2e-2 of the oracle, and the worker's graph path agrees."""
    import bench
    from cortex.models.config import CORTEX_S
    from cortex.quantization.w8a8 import disable_w8a8, enable_w8a8
    from cortex.serve import InferenceWorker

    model, scales = bench.build_model(torch.device(DEV), with_scales=True)
    enable_w8a8(model, scales)
    try:
        nid, tb, val, bidx = bench.make_events(B, 512, seed=30 + B)
        ev = [torch.from_numpy(a).to(DEV) for a in (nid, tb, val, bidx)]
        with torch.no_grad():
            got = model(*ev, batch_size=B)["behavior"].cpu()
        sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
        ref = O.forward(sd, O.CORTEX_S_SHAPE, nid, tb, val, bidx, batch_size=B)
        assert float((got - torch.as_tensor(ref)).abs().max()) <= 2e-2
        w = InferenceWorker(model, CORTEX_S, torch.device(DEV), max_batch_size=B)
        cuts = np.flatnonzero(np.diff(bidx)) + 1
        payloads = [{"request_id": i, "events": {"neuron_id": a, "time_bin": t, "value": v}}
                    for i, (a, t, v) in enumerate(zip(np.split(nid, cuts), np.split(tb, cuts), np.split(val, cuts)))]
        rows = torch.tensor([r["behavior"] for r in w._run_batch_sync(payloads)])
        assert float((rows - got).abs().max()) <= 1e-5
        w.shutdown()
    finally:
        disable_w8a8(model)
