"""Fused norm + linear on the GPU vs the oracle (a5, a6, a7)."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import cortex_oracle as O
from tests._bars import bf16_steps

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel_err(out: torch.Tensor, ref: torch.Tensor) -> float:
    return float((out.double() - ref.double()).abs().max() / ref.double().abs().max().clamp_min(1e-30))


@pytest.mark.parametrize("M,K,N", [(16, 64, 128), (64, 128, 256), (256, 512, 512), (8192, 512, 1536),
                                   (8192, 512, 2048), (33, 70, 97), (1, 512, 2048)])
def test_rms_norm_linear_fp32(M, K, N):
    """fp32: <= 1e-5 relative to the oracle (fp32 MFMA, fp32 accumulation)."""
    from cortex.kernels.fused_rmsnorm import rms_norm_linear

    torch.manual_seed(17)
    x, w = torch.randn(M, K), torch.randn(K, N)
    g = torch.ones(K) + 0.02 * torch.randn(K)
    out = rms_norm_linear(x.to(DEV), g.to(DEV), w.to(DEV))
    ref = O.rms_norm_linear(x.double(), g.double(), w.double()).float()
    assert out.shape == (M, N) and out.dtype == torch.float32
    assert _rel_err(out.cpu(), ref) <= 1e-5
    torch.testing.assert_close(out.cpu(), ref, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("M,K,N", [(8192, 512, 1536), (8192, 512, 2048), (8192, 512, 512), (33, 70, 97)])
def test_rms_norm_linear_bf16(M, K, N):
    from cortex.kernels.fused_rmsnorm import rms_norm_linear

    torch.manual_seed(17)
    x = torch.randn(M, K).bfloat16()
    w = torch.randn(K, N).bfloat16()
    g = (torch.ones(K) + 0.02 * torch.randn(K)).bfloat16()
    out = rms_norm_linear(x.to(DEV), g.to(DEV), w.to(DEV))
    ref = O.rms_norm_linear(x, g, w)  # x_norm rounded to bf16 as in the reference, fp32 matmul
    assert out.dtype == torch.bfloat16
    torch.testing.assert_close(out.float().cpu(), ref, rtol=1e-2, atol=2e-2 * float(ref.abs().max()) / 8)


def test_rms_norm_linear_bias_and_3d():
    from cortex.kernels.fused_rmsnorm import rms_norm_linear

    torch.manual_seed(3)
    x, g, w, b = torch.randn(2, 256, 512), torch.ones(512), torch.randn(512, 1536), torch.randn(1536)
    out = rms_norm_linear(x.to(DEV), g.to(DEV), w.to(DEV), b.to(DEV))
    assert out.shape == (2, 256, 1536)
    ref = O.rms_norm_linear(x.reshape(-1, 512).double(), g.double(), w.double(), b.double()).float()
    assert _rel_err(out.reshape(-1, 1536).cpu(), ref) <= 1e-5


def _config2(N, seed=0):
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.normal(0, 1, (8192, 512)).astype(np.float32)).bfloat16()
    g = torch.from_numpy(rng.normal(1, 0.02, 512).astype(np.float32))
    w = rng.normal(0, 0.02, (N, 512)).astype(np.float32)
    q, s = O.quantize_int8(w)
    return x, g, torch.from_numpy(q), torch.from_numpy(s)


@pytest.mark.parametrize("N", [1536, 2048, 512])
def test_rms_int8_linear_config2(N):
    """Config 2: RMSNorm(eps 1e-6) + INT8 per-channel linear, bf16 in/out."""
    from cortex.kernels.fused_rmsnorm import norm_linear_int8

    x, g, q, s = _config2(N)
    out = norm_linear_int8(x.to(DEV), q.to(DEV), s.to(DEV), norm="rms", gamma=g.to(DEV), eps=1e-6)
    wdq = torch.from_numpy(O.dequantize(q.numpy(), s.numpy()))
    ref = O.rms_norm_linear(x, g, wdq.T.contiguous())  # bf16 x_norm, fp32 contraction
    assert out.dtype == torch.bfloat16
    err = (out.float().cpu() - ref).abs()
    # one bf16 rounding of the output plus accumulation-order noise
    assert float((err / ref.abs().clamp_min(1e-3)).median()) < 4e-3
    assert float(err.max()) <= 2e-2 * float(ref.abs().max())
    steps = bf16_steps(float(err.max()), float(ref.abs().max()))
    print(f"[parity] config 2 N={N}: max err {float(err.max()):.3e} = {steps:.2f} bf16 steps at max|ref|", flush=True)
    assert steps <= 1.0  # observed 0.5-0.65


def test_layernorm_gelu_residual_epilogues_fp32():
    """LayerNorm prologue + GELU epilogue and residual epilogue, fp32 compute vs torch CPU."""
    from cortex.kernels import ops

    torch.manual_seed(5)
    x = torch.randn(300, 512) * 3 + 1
    ln_w, ln_b = 1 + 0.1 * torch.randn(512), 0.1 * torch.randn(512)
    w = torch.randn(2048, 512) * 0.02
    q, s = O.quantize_int8(w.numpy())
    qd, sd = torch.from_numpy(q), torch.from_numpy(s)
    h = ops.norm_linear(x.to(DEV), weight_int8=qd.to(DEV), weight_scale=sd.to(DEV), norm="layer",
                        gamma=ln_w.to(DEV), beta=ln_b.to(DEV), eps=1e-5, act="gelu", out_dtype=torch.float32,
                        compute_dtype=torch.float32)
    wdq = torch.from_numpy(O.dequantize(q, s))
    ref_h = F.gelu(F.linear(F.layer_norm(x, (512,), ln_w, ln_b, 1e-5), wdq))
    assert _rel_err(h.cpu(), ref_h) <= 1e-5
    w2 = torch.randn(512, 2048) * 0.02
    res = torch.randn(300, 512)
    y = ops.norm_linear(h, weight=w2.to(DEV), residual=res.to(DEV), out_dtype=torch.float32,
                        compute_dtype=torch.float32)
    ref_y = res + F.linear(ref_h, w2)
    assert _rel_err(y.cpu(), ref_y) <= 1e-5


def test_broadcast_residual_rows():
    """res_rows broadcasts a batch-invariant residual (the learned latents) over the batch."""
    from cortex.kernels import ops

    torch.manual_seed(9)
    a = torch.randn(4 * 256, 512).bfloat16()
    w = torch.randn(512, 512) * 0.02
    lat = torch.randn(256, 512)
    y = ops.norm_linear(a.to(DEV), weight=w.to(DEV), residual=lat.to(DEV), res_rows=256,
                        out_dtype=torch.float32, compute_dtype=torch.bfloat16)
    ref = lat.repeat(4, 1) + a.float() @ w.bfloat16().float().T
    torch.testing.assert_close(y.cpu(), ref, rtol=1e-4, atol=1e-4)


def test_layer_norm_kernel_and_row_stats():
    from cortex.kernels import ops

    torch.manual_seed(2)
    x = torch.randn(777, 512) * 2 + 0.5
    w, b = torch.randn(512), torch.randn(512)
    y = ops.layer_norm(x.to(DEV), w.to(DEV), b.to(DEV), 1e-5)
    torch.testing.assert_close(y.cpu(), F.layer_norm(x, (512,), w, b, 1e-5), rtol=1e-5, atol=2e-5)
    st = ops.row_stats(x.to(DEV), "rms", 1e-6).cpu()
    torch.testing.assert_close(st[:, 1], torch.sqrt(x.pow(2).mean(-1) + 1e-6), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("K", [256, 512, 768, 1024])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32])
def test_norm_rows_vs_torch(K, xdt):
    """The norm half of the bf16 fused path: RMS/LayerNorm rows rounded once to bf16.

    Against torch fp32 on the CPU: at most one bf16 step apart (the fp32 sums differ
    only in order, so a rounding boundary can fall either way)."""
    from cortex.kernels import ops

    torch.manual_seed(K)
    x = (torch.randn(517, K) * 2 + 0.3).to(xdt)
    g, b = 1 + 0.1 * torch.randn(K), 0.1 * torch.randn(K)
    xf = x.float()
    ref_rms = (xf / torch.sqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)) * g
    ref_ln = F.layer_norm(xf, (K,), g, b, 1e-5)
    for norm, ref, kw in (("rms", ref_rms, {"gamma": g, "eps": 1e-6}),
                          ("layer", ref_ln, {"gamma": g, "beta": b, "eps": 1e-5})):
        kw = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in kw.items()}
        y = ops.norm_rows(x.to(DEV), norm, **kw).cpu()
        assert y.dtype == torch.bfloat16 and y.shape == (517, K)
        step = ref.abs() * 2.0 ** -7 + 1e-5  # one bf16 step, plus fp32 cancellation near 0
        assert bool(((y.float() - ref).abs() <= step).all()), norm
        exact = float((y == ref.bfloat16()).float().mean())
        assert exact > 0.99, (norm, exact)
    # bf16 gamma, strided rows
    xs = torch.randn(64, 2 * K).to(xdt)[:, :K]
    y = ops.norm_rows(xs.to(DEV), "rms", g.bfloat16().to(DEV)).cpu()
    xsf = xs.float()
    ref = (xsf / torch.sqrt(xsf.pow(2).mean(-1, keepdim=True) + 1e-6)) * g.bfloat16().float()
    assert bool(((y.float() - ref).abs() <= ref.abs() * 2.0 ** -7 + 1e-5).all())


@pytest.mark.parametrize("R,C", [(512, 1536), (512, 2048), (70, 97), (1, 5), (64, 64), (129, 1)])
def test_transpose_bf16_exact(R, C):
    from cortex.kernels import ops

    torch.manual_seed(R * 7 + C)
    w = torch.randn(R, C).bfloat16()
    t = ops.transpose_bf16(w.to(DEV)).cpu()
    assert t.shape == (C, R) and t.is_contiguous()
    assert torch.equal(t.view(torch.int16), w.T.contiguous().view(torch.int16))


def _exact_rows(M, K, seed):
    """Rows x = c * s with s in {-1, +1}, c a power of two: with eps = 0 the RMS is |c| and
    x / rms = s exactly.  Gains are powers of two, so the normalised row s * gamma is exact in
    bf16, and so is a weight that carries the gain (w * gamma, the int8 path's widening)."""
    g = torch.Generator().manual_seed(seed)
    s = torch.randint(0, 2, (M, K), generator=g).float() * 2 - 1
    c = 2.0 ** torch.randint(-3, 4, (M, 1), generator=g).float()
    gam = 2.0 ** torch.randint(-2, 3, (K,), generator=g).float()
    return (s * c).bfloat16(), s, gam


@pytest.mark.parametrize("M,N,K,wform", [(8192, 1536, 512, "int8"), (8192, 512, 512, "int8"), (300, 200, 256, "int8"),
                                         (1, 2048, 512, "int8"), (777, 1024, 448, "bf16"), (64, 64, 64, "bf16")])
def test_fused_rms_linear_one_launch_exact_rows(M, N, K, wform):
    """cortex_norm_linear_fused on rows whose normalisation is exact: fp32 output within 1e-5
    of a float64 contraction of gamma * sign rows with the (widened) weight, scale and bias."""
    from cortex.kernels import ops

    x, sgn, gam = _exact_rows(M, K, seed=M + N + K)
    g = torch.Generator().manual_seed(N)
    w = torch.randn(N, K, generator=g) * 0.03
    bias = torch.randn(N, generator=g) * 0.1
    if wform == "int8":
        q, s = O.quantize_int8(w.numpy())
        wd, sd, wref = torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV), torch.from_numpy(O.dequantize(q, s))
    else:
        wd, sd, wref = w.bfloat16().to(DEV), None, w.bfloat16().float()
    out = ops.norm_linear_fused(x.to(DEV), wd, sd, norm="rms", gamma=gam.to(DEV), eps=0.0, bias=bias.to(DEV),
                                out_dtype=torch.float32)
    ref = (sgn.double() * gam.double()) @ wref.double().T + bias.double()
    assert out.shape == (M, N)
    assert _rel_err(out.cpu(), ref) <= 1e-5


@pytest.mark.parametrize("norm", ["rms", "layer"])
@pytest.mark.parametrize("act", [None, "gelu"])
def test_fused_norm_linear_vs_oracle(norm, act):
    """The one-launch path with a gain given to the kernel (rows normalised in the kernel, the
    int8 weight streamed): bf16 output against the normalised rows rounded to bf16 (as the
    reference does) times the dequantised weight in float64; the row statistics differ from
    torch's only in summation order, so a rounding of the normalised row may flip by one bf16
    step: within 2 bf16 steps of the output plus 1e-3 of the largest output everywhere, and
    within one step for 99 % of outputs."""
    from cortex.kernels import ops

    M, N, K = 1000, 768, 512
    g = torch.Generator().manual_seed(11)
    x = (torch.randn(M, K, generator=g) * 2 + 0.4).bfloat16()
    gam = 1 + 0.05 * torch.randn(K, generator=g)
    bet = 0.1 * torch.randn(K, generator=g)
    w = torch.randn(N, K, generator=g) * 0.03
    q, s = O.quantize_int8(w.numpy())
    wdq = torch.from_numpy(O.dequantize(q, s)).double()
    out = ops.norm_linear_fused(x.to(DEV), torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV), norm=norm,
                                gamma=gam.to(DEV), beta=bet.to(DEV), eps=1e-6 if norm == "rms" else 1e-5, act=act)
    xf = x.float()
    if norm == "rms":
        y = (xf / torch.sqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)) * gam
    else:
        y = F.layer_norm(xf, (K,), gam, bet, 1e-5)
    ref = y.bfloat16().double() @ wdq.T
    if act == "gelu":
        ref = F.gelu(ref)
    got = out.double().cpu()
    step = ref.abs() * 2.0 ** -8 + 1e-30
    err = (got - ref).abs()
    assert bool((err <= 2 * step + 1e-3 * float(ref.abs().max())).all()), float(err.max())
    assert float((err <= step + 1e-5 * float(ref.abs().max())).float().mean()) >= 0.99


def test_config2_is_one_launch_and_kn_weights_are_cached():
    """Config 2 through the API: one kernel per call (the fused one).  The RMS gain is folded into
    a cached bf16 copy of the weight once per (weight, gamma) pair -- one cortex_fold_gain,
    rebuilt when either changes in place -- for the int8 and the (K, N) weight alike."""
    from cortex import _native as nat
    from cortex.kernels import ops
    from cortex.kernels.fused_rmsnorm import norm_linear_int8, rms_norm_linear

    x, gam, q, s = _config2(1536)
    xd, gd, qd, sd = x.to(DEV), gam.to(DEV), q.to(DEV), s.to(DEV)
    names = []
    real = nat.call

    def spy(name, *a):
        names.append(name)
        return real(name, *a)
    nat.call = spy
    try:
        norm_linear_int8(xd, qd, sd, norm="rms", gamma=gd, eps=1e-6)
        assert names == ["cortex_fold_gain", "cortex_norm_linear_fused"], names  # the gain folded once
        names.clear()
        norm_linear_int8(xd, qd, sd, norm="rms", gamma=gd, eps=1e-6)
        assert names == ["cortex_norm_linear_fused"], names
        w = (torch.randn(512, 1536) * 0.02).bfloat16().to(DEV)
        names.clear()
        a = rms_norm_linear(xd, gd, w)
        b = rms_norm_linear(xd, gd, w)
        assert names.count("cortex_norm_linear_fused") == 2 and names.count("cortex_fold_gain") == 1, names
        torch.testing.assert_close(a, b, rtol=0, atol=0)
        w.mul_(2)  # in place: the cached rows must follow
        c = rms_norm_linear(xd, gd, w)
        assert names.count("cortex_fold_gain") == 2, names
        torch.testing.assert_close(c.float(), 2 * a.float(), rtol=1e-2, atol=1e-2)
        gd.mul_(0.5)  # so must a change of gamma
        d = rms_norm_linear(xd, gd, w)
        assert names.count("cortex_fold_gain") == 3, names
        torch.testing.assert_close(d.float(), a.float(), rtol=1e-2, atol=1e-2)
    finally:
        nat.call = real


@pytest.mark.parametrize("wdt", [torch.int8, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("kn", [False, True])
@pytest.mark.parametrize("gdt", [torch.float32, torch.bfloat16])
def test_fold_gain_exact(wdt, kn, gdt):
    """cortex_fold_gain: bf16(float(w) * gamma) per element, bit-exact against torch's fp32
    product rounded to bf16 (round to nearest even), for both weight layouts."""
    from cortex.kernels import ops

    g = torch.Generator().manual_seed(5)
    N, K = 200, 448
    if wdt == torch.int8:
        w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    else:
        w = (torch.randn(N, K, generator=g) * 0.05).to(wdt)
    gam = (1 + 0.1 * torch.randn(K, generator=g)).to(gdt)
    src = w.T.contiguous() if kn else w
    out = ops.fold_gain(src.to(DEV), gam.to(DEV), kn=kn).cpu()
    ref = (w.float() * gam.float()).bfloat16()
    assert out.shape == (N, K) and out.dtype == torch.bfloat16
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("M,N,K,wform", [(8192, 1536, 512, "int8"), (300, 200, 256, "bf16"), (1, 64, 448, "int8")])
def test_rms_linear_folded_gain_exact_rows(M, N, K, wform):
    """The API's RMS path: gain folded into the cached weight, 1 / rms on the accumulator.  With
    power-of-two gains the folded weight is exact and with rows c * sign (eps = 0) 1 / rms is
    exact, so the fp32 output is within 1e-5 of a float64 contraction."""
    from cortex.kernels import ops

    x, sgn, gam = _exact_rows(M, K, seed=M + N)
    g = torch.Generator().manual_seed(N + K)
    w = torch.randn(N, K, generator=g) * 0.03
    bias = torch.randn(N, generator=g) * 0.1
    if wform == "int8":
        q, s = O.quantize_int8(w.numpy())
        kw = {"weight_int8": torch.from_numpy(q).to(DEV), "weight_scale": torch.from_numpy(s).to(DEV)}
        wref = torch.from_numpy(O.dequantize(q, s))
    else:
        kw = {"weight": w.bfloat16().to(DEV)}
        wref = w.bfloat16().float()
    out = ops.norm_linear(x.to(DEV), **kw, norm="rms", gamma=gam.to(DEV), eps=0.0, bias=bias.to(DEV),
                          out_dtype=torch.float32, compute_dtype=torch.bfloat16)
    ref = (sgn.double() * gam.double()) @ wref.double().T + bias.double()
    assert out.shape == (M, N)
    assert _rel_err(out.cpu(), ref) <= 1e-5


@pytest.mark.parametrize("M,N,K,act,odt", [(1, 256, 64, None, torch.float32), (300, 200, 64, "gelu", torch.bfloat16),
                                            (257, 520, 128, None, torch.float32), (257, 520, 128, "gelu", torch.float32),
                                            (1000, 2048, 512, "gelu", torch.bfloat16), (7937, 2048, 128, None, torch.bfloat16),
                                            (7937, 1536, 64, "gelu", torch.float32)])
def test_rms_without_gain_row_scaled_gemm(M, N, K, act, odt):
    """RMS without a gain on a bf16 weight (the form the API hands over after folding the gain):
    the tiled GEMM sums the squares of its own A fragments and scales the accumulator by
    1 / rms.  The shapes reach every tile it picks (128 x 128 with and without the K split over
    two wave groups, 256 x 192, 256 x 256), a single K step (K = 64), one step per wave group
    (K = 128), M = 1 and ragged M and N.  Against the float64 value of the same arithmetic,
    act(x W^T / sqrt(mean(x^2) + eps) * scale + bias): fp32 output within 1e-5 of the largest
    output, bf16 output within one bf16 rounding (2^-8 relative) plus 1e-5 of the largest."""
    from cortex.kernels import ops

    g = torch.Generator().manual_seed(M + N + K)
    x = (torch.randn(M, K, generator=g) * (1 + 3 * torch.rand(M, 1, generator=g))).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.05).bfloat16()
    sc = 0.5 + torch.rand(N, generator=g)
    bias = 0.1 * torch.randn(N, generator=g)
    out = ops.norm_linear_fused(x.to(DEV), w.to(DEV), sc.to(DEV), norm="rms", gamma=None, eps=1e-6,
                                bias=bias.to(DEV), act=act, out_dtype=odt)
    xd = x.double()
    rinv = 1.0 / torch.sqrt(xd.pow(2).mean(-1, keepdim=True) + 1e-6)
    ref = (xd @ w.double().T) * rinv * sc.double() + bias.double()
    if act == "gelu":
        ref = F.gelu(ref)
    assert out.shape == (M, N) and out.dtype == odt
    got = out.double().cpu()
    big = float(ref.abs().max())
    if odt == torch.float32:
        assert _rel_err(got, ref) <= 1e-5
    else:
        assert bool(((got - ref).abs() <= ref.abs() * 2.0 ** -8 + 1e-5 * big).all()), float((got - ref).abs().max())


@pytest.mark.parametrize("N", [1536, 512])
def test_config2_widen_mode_streams_int8(N, monkeypatch):
    """CORTEX_INT8_WEIGHTS=widen: norm_linear_int8 hands the int8 weight and the gain to the kernel
    (rows normalised in the kernel, no folded copy) in one launch, and agrees with the default
    (folded) path and the oracle to the config-2 tolerance."""
    from cortex import _native as nat
    from cortex.kernels import ops
    from cortex.kernels.fused_rmsnorm import norm_linear_int8

    x, g, q, s = _config2(N, seed=3)
    xd, gd, qd, sd = x.to(DEV), g.to(DEV), q.to(DEV), s.to(DEV)
    ref = O.rms_norm_linear(x, g, torch.from_numpy(O.dequantize(q.numpy(), s.numpy())).T.contiguous())
    folded = norm_linear_int8(xd, qd, sd, norm="rms", gamma=gd, eps=1e-6).float().cpu()
    monkeypatch.setattr(ops, "INT8_WEIGHTS", "widen")
    names, real = [], nat.call

    def spy(name, *a):
        names.append(name)
        return real(name, *a)
    monkeypatch.setattr(nat, "call", spy)
    streamed = norm_linear_int8(xd, qd, sd, norm="rms", gamma=gd, eps=1e-6).float().cpu()
    assert names == ["cortex_norm_linear_fused"], names
    for out in (folded, streamed):
        err = (out - ref).abs()
        assert float((err / ref.abs().clamp_min(1e-3)).median()) < 4e-3
        assert float(err.max()) <= 2e-2 * float(ref.abs().max())
