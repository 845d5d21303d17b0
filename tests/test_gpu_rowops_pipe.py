"""LayerNorm row kernel, dtype conversion and the tiled bf16-operand GEMMs on the GPU.

The LayerNorm rows (a5's norm half) are checked against torch's CPU LayerNorm in
fp32 (fp32 output <= 2e-5 absolute at unit scale; bf16 output within one bf16
rounding of the fp32 result).  The tiled GEMMs (a6/a7: bf16 rows x int8 or bf16
weight rows, per-channel scale, bias, GELU, fp32 residual, K split over wave groups
or over workgroups) are checked against a float64 contraction of the same bf16/int8
operands, and the int8-widen and bf16-image weight forms are checked to agree with
each other.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import cortex_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 values at |x| (2^(e-7) for |x| in [2^e, 2^(e+1)))."""
    e = torch.floor(torch.log2(x.abs().clamp_min(1e-30)))
    return torch.pow(2.0, e - 7)


@pytest.mark.parametrize("K", [256, 512, 768, 1024])
@pytest.mark.parametrize("M", [1, 7, 8192])
def test_ln_rows_single(M, K):
    from cortex.kernels import ops

    torch.manual_seed(K + M)
    x = torch.randn(M, K) * 2.5 + 0.7
    w, b = 1 + 0.2 * torch.randn(K), 0.2 * torch.randn(K)
    ob, of = ops.ln_rows(x.to(DEV), (w.to(DEV), b.to(DEV), 1e-5), out_bf16=True, out_f32=True)
    ref = F.layer_norm(x, (K,), w, b, 1e-5)
    torch.testing.assert_close(of.cpu(), ref, rtol=0, atol=2e-5 * float(ref.abs().max()))
    # bf16 output is the fp32 value rounded once: within one bf16 spacing of the exact result
    err = (ob.float().cpu() - ref).abs()
    assert bool((err <= _bf16_ulp(ref) + 2e-5 * float(ref.abs().max())).all())


@pytest.mark.parametrize("K", [256, 512])
def test_ln_rows_double(K):
    """final_norm followed by the behaviour head's norm in one pass."""
    from cortex.kernels import ops

    torch.manual_seed(11)
    M = 8192
    x = torch.randn(M, K) * 4 - 1
    w1, b1 = 1 + 0.3 * torch.randn(K), 0.3 * torch.randn(K)
    w2, b2 = 1 + 0.3 * torch.randn(K), 0.3 * torch.randn(K)
    of = ops.ln_rows(x.to(DEV), (w1.to(DEV), b1.to(DEV), 1e-5), (w2.to(DEV), b2.to(DEV), 1e-6),
                     out_bf16=False, out_f32=True)
    ref = F.layer_norm(F.layer_norm(x, (K,), w1, b1, 1e-5), (K,), w2, b2, 1e-6)
    torch.testing.assert_close(of.cpu(), ref, rtol=0, atol=3e-5 * float(ref.abs().max()))


def test_ln_rows_strided_rows():
    """Rows with a leading stride larger than K (a column slice of a wider buffer)."""
    from cortex.kernels import ops

    torch.manual_seed(4)
    big = torch.randn(300, 1024)
    x = big[:, :512]
    w, b = torch.randn(512), torch.randn(512)
    of = ops.ln_rows(x.to(DEV), (w.to(DEV), b.to(DEV), 1e-5), out_bf16=False, out_f32=True)
    torch.testing.assert_close(of.cpu(), F.layer_norm(x, (512,), w, b, 1e-5), rtol=0, atol=1e-4)


@pytest.mark.parametrize("src", [torch.int8, torch.float32, torch.bfloat16])
def test_convert_exact(src):
    from cortex.kernels import ops

    torch.manual_seed(1)
    if src == torch.int8:
        t = torch.randint(-127, 128, (2048, 512), dtype=torch.int8)
    else:
        t = (torch.randn(1001, 37) * 100).to(src)
    for dst in (torch.bfloat16, torch.float32):
        out = ops.convert(t.to(DEV), dst).cpu()
        assert out.dtype == dst
        assert torch.equal(out, t.to(dst)), (src, dst)  # RNE to bf16, exact widening


def _operands(M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(M, K, generator=g).bfloat16()
    w = torch.randn(N, K, generator=g) * 0.05
    q, s = O.quantize_int8(w.numpy())
    return a, torch.from_numpy(q), torch.from_numpy(s)


def _ref(a, q, s, bias=None, act=None, res=None, res_rows=0):
    y = a.double() @ q.double().T * s.double()
    if bias is not None:
        y = y + bias.double()
    if act == "gelu":
        y = F.gelu(y)
    if res is not None:
        r = res.double()
        if res_rows:
            r = r.repeat(a.shape[0] // res_rows, 1)
        y = y + r
    return y


@pytest.mark.parametrize("M,N,K", [(8192, 1536, 512), (8192, 2048, 512), (8192, 512, 2048), (8192, 512, 512),
                                   (16384, 1024, 512), (300, 512, 512), (1, 1024, 512), (130, 200, 64)])
def test_gemm_int8_and_image(M, N, K):
    """int8 weights widened in the kernel and their bf16 image agree, and both match fp64."""
    from cortex.kernels import ops

    a, q, s = _operands(M, N, K, seed=M + N + K)
    ad, qd, sd = a.to(DEV), q.to(DEV), s.to(DEV)
    y8 = ops.norm_linear(ad, weight_int8=qd, weight_scale=sd, out_dtype=torch.float32)
    img = ops.convert(qd, torch.bfloat16)
    yi = ops.norm_linear(ad, weight=img, weight_scale=sd, out_dtype=torch.float32)
    if K % 64 == 0 and N % 8 == 0:  # both on the bf16 GEMM kernel: the same widened operands
        torch.testing.assert_close(yi, y8, rtol=0, atol=0)
    ref = _ref(a, q, s)
    scale = float(ref.abs().max())
    assert float((y8.cpu().double() - ref).abs().max()) <= 1e-5 * scale
    assert float((yi.cpu().double() - ref).abs().max()) <= 1e-5 * scale
    torch.testing.assert_close(yi, y8, rtol=0, atol=2e-6 * scale)


@pytest.mark.parametrize("wform", ["int8", "image"])
def test_gemm_gelu_bf16_out(wform):
    """MLP-up shape: GELU epilogue, bf16 output within bf16 rounding of the fp64 result."""
    from cortex.kernels import ops

    M, N, K = 8192, 2048, 512
    a, q, s = _operands(M, N, K, seed=5)
    ad, qd, sd = a.to(DEV), q.to(DEV), s.to(DEV)
    w = {"weight_int8": qd} if wform == "int8" else {"weight": ops.convert(qd, torch.bfloat16)}
    y = ops.norm_linear(ad, **w, weight_scale=sd, act="gelu", out_dtype=torch.bfloat16).cpu().double()
    ref = _ref(a, q, s, act="gelu")
    err = (y - ref).abs()
    assert bool((err <= _bf16_ulp(ref) + 1e-5 * float(ref.abs().max())).all())


@pytest.mark.parametrize("wform", ["int8", "image"])
def test_gelu_epilogue_dense_grid(wform):
    """The bf16-output GELU epilogue on every bf16 value in [-12, 12] (and +-inf): a
    K=64 GEMM whose rows hold x in column 0 and whose weight rows are e_0 (scale 1)
    returns GELU(x) rounded to bf16.  Bar: within half a bf16 step of the float64
    erf-GELU plus 1e-4 relative (approximation) and 1e-8 absolute (the far
    negative tail, where |GELU| < 6e-9); GELU(+inf) = +inf."""
    from cortex.kernels import ops

    v = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float()
    x = torch.unique(v[torch.isfinite(v) & (v.abs() <= 12)])
    x = torch.cat([x, torch.tensor([float("inf")])])
    M, N, K = x.numel(), 16, 64
    a = torch.zeros(M, K)
    a[:, 0] = x
    q = torch.zeros(N, K, dtype=torch.int8)
    q[:, 0] = 1
    ad, qd, sd = a.to(torch.bfloat16).to(DEV), q.to(DEV), torch.ones(N, device=DEV)
    w = {"weight_int8": qd} if wform == "int8" else {"weight": ops.convert(qd, torch.bfloat16)}
    y = ops.norm_linear(ad, **w, weight_scale=sd, act="gelu", out_dtype=torch.bfloat16).cpu().double()
    xd = x.double()
    ref = 0.5 * xd * (1 + torch.erf(xd / 2 ** 0.5))
    fin = torch.isfinite(xd)
    assert bool((y[~fin] == float("inf")).all())
    err = (y[fin] - ref[fin, None]).abs()
    bound = 0.5 * _bf16_ulp(ref[fin, None]) + 1e-4 * ref[fin, None].abs() + 1e-8
    assert bool((err <= bound).all()), float((err - bound).max())


def test_gemm_bias_and_broadcast_residual():
    """Bias epilogue, and the latents residual broadcast every 256 rows into fp32 output."""
    from cortex.kernels import ops

    M, N, K, L = 32 * 256, 512, 512, 256
    a, q, s = _operands(M, N, K, seed=8)
    bias = torch.randn(N)
    lat = torch.randn(L, N)
    ad, qd, sd = a.to(DEV), q.to(DEV), s.to(DEV)
    img = ops.convert(qd, torch.bfloat16)
    y = ops.norm_linear(ad, weight=img, weight_scale=sd, bias=bias.to(DEV), out_dtype=torch.float32).cpu()
    ref = _ref(a, q, s, bias=bias)
    assert float((y.double() - ref).abs().max()) <= 1e-5 * float(ref.abs().max())
    y2 = ops.norm_linear(ad, weight=img, weight_scale=sd, residual=lat.to(DEV), res_rows=L,
                         out_dtype=torch.float32).cpu()
    ref2 = _ref(a, q, s, res=lat, res_rows=L)
    assert float((y2.double() - ref2).abs().max()) <= 1e-5 * float(ref2.abs().max())


@pytest.mark.parametrize("M,K,form", [(16384, 2048, "int8"), (16384, 2048, "image"), (20000, 512, "image"),
                                      (300, 2048, "image")])
def test_residual_gemm_every_grid(M, K, form):
    """Residual GEMMs into the fp32 stream (MLP-down 2048 -> 512 and the 512 -> 512 shape) at
    one and at several workgroups per CU (B = 64 and larger batches): the K split over two
    wave groups at every grid size, with a ragged last row tile; within 1e-5 of float64
    (computed on the device) relative to the largest output, in place over the residual."""
    from cortex.kernels import ops

    N = 512
    a, q, s = _operands(M, N, K, seed=M + K)
    ad, qd, sd = a.to(DEV), q.to(DEV), s.to(DEV)
    res = torch.randn(M, N, device=DEV)
    w = {"weight_int8": qd} if form == "int8" else {"weight": ops.convert(qd, torch.bfloat16)}
    ref = (ad.double() @ (qd.double() * sd.double()[:, None]).T) + res.double()
    out = res.clone()
    ops.norm_linear(ad, **w, weight_scale=sd, residual=out, out_dtype=torch.float32, out=out)
    err = float((out.double() - ref).abs().max())
    assert err <= 1e-5 * float(ref.abs().max()), err


@pytest.mark.parametrize("M,N,K,res_rows", [(8192, 512, 2048, 0), (8000, 512, 2048, 0), (2900, 512, 2048, 0),
                                            (8192, 256, 1024, 256), (4096, 768, 3072, 0), (2048, 1024, 2048, 0)])
def test_direct_weight_residual_gemm(M, N, K, res_rows):
    """The direct-weight residual GEMM (MLP-down on the fragment-order weight, grids of at most
    one 128 x 128 tile per CU): within 1e-5 of float64, and bit-identical to the K-split
    128 x 128 kernel on the bf16 image, whose per-group MFMA sequence it repeats.  Ragged last
    row tile, broadcast residual rows, in place over the residual."""
    from cortex.kernels import ops

    a, q, s = _operands(M, N, K, seed=M + N + K)
    ad, qd, sd = a.to(DEV), q.to(DEV), s.to(DEV)
    g = torch.Generator().manual_seed(9)
    bias = (0.1 * torch.randn(N, generator=g)).to(DEV)
    res = torch.randn(res_rows or M, N, generator=g).to(DEV)
    dev = torch.device(DEV)
    assert ops.frag_res_ok(M, N, K, dev)
    img = ops.convert(qd, torch.bfloat16)
    out_f = res.clone() if not res_rows else None
    y_f = ops.linear_residual_frag(ad, ops.frag_weight(qd), sd, bias, residual=res if res_rows else out_f,
                                   res_rows=res_rows, out=out_f)
    if out_f is not None:
        assert y_f.data_ptr() == out_f.data_ptr()
    y_i = ops.norm_linear(ad, weight=img, weight_scale=sd, bias=bias, residual=res, res_rows=res_rows,
                          out_dtype=torch.float32)
    r = res.double().repeat(M // res_rows, 1) if res_rows else res.double()
    ref = (ad.double() @ (qd.double() * sd.double()[:, None]).T) + bias.double() + r
    assert float((y_f.double() - ref).abs().max()) <= 1e-5 * float(ref.abs().max())
    if not ops.splitk_splits(M, N, K, dev) and -(-M // 128) * (N // 128) <= 256:
        torch.testing.assert_close(y_f, y_i, rtol=0, atol=0)


def test_gemm_float_weight_image():
    """A float nn.Linear weight rounded to bf16 (no scale), residual into fp32 output."""
    from cortex.kernels import ops

    M, N, K = 4096, 512, 2048
    g = torch.Generator().manual_seed(3)
    a = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    res = torch.randn(M, N, generator=g)
    y = ops.norm_linear(a.to(DEV), weight=w.to(DEV), residual=res.to(DEV), out_dtype=torch.float32).cpu()
    ref = res.double() + a.double() @ w.double().T
    assert float((y.double() - ref).abs().max()) <= 1e-5 * float(ref.abs().max())


@pytest.mark.parametrize("M,N,act,out", [(16384, 1024, None, torch.bfloat16), (32768, 2048, "gelu", torch.bfloat16),
                                         (65179, 1024, None, torch.bfloat16), (8192, 512, None, torch.float32)])
def test_gemm_outputs_repeatable(M, N, act, out):
    """Every output element is written with the value computed for it, on every launch.

    The kernels write their outputs with device-scope write-through stores (single-wave grids)
    or write-back ones, some of them while later K steps run; when these stores were inline
    assembly, a VALU write to a store's data registers too soon after it (a hazard the compiler
    did not see) changed a few rows from launch to launch at these shapes.  Five launches into
    fresh buffers must agree bit for bit and with float64."""
    from cortex.kernels import ops

    K = 512
    g = torch.Generator().manual_seed(M + N)
    a = torch.randn(M, K, generator=g).bfloat16()
    q, s = O.quantize_int8((torch.randn(N, K, generator=g) * 0.05).numpy())
    ad, img, sd = a.to(DEV), ops.convert(torch.from_numpy(q).to(DEV), torch.bfloat16), torch.from_numpy(s).to(DEV)
    first = None
    for _ in range(5):
        y = ops.norm_linear(ad, weight=img, weight_scale=sd, act=act, out_dtype=out)
        if first is None:
            first = y.clone()
        else:
            assert torch.equal(y, first)
    ref = _ref(a, torch.from_numpy(q), torch.from_numpy(s), act=act)
    err = (first.cpu().double() - ref).abs()
    if out == torch.bfloat16:
        assert bool((err <= _bf16_ulp(ref) + 1e-5 * float(ref.abs().max())).all())
    else:
        assert float(err.max()) <= 1e-5 * float(ref.abs().max())


@pytest.mark.parametrize("M,N,act,with_bias,with_scale", [(8192, 2048, "gelu", True, True),
                                                          (16000, 1024, None, True, False),
                                                          (8000, 2048, "gelu", False, True),
                                                          (16384, 1024, None, False, False)])
def test_wide_tile_bf16_epilogue(M, N, act, with_bias, with_scale):
    """bf16-output GEMMs at K = 512 on 256 x 256 tiles filling the chip (the MLP-up and
    kv-projection shapes): bias or none, scale or none, GELU or none, a ragged last row tile.
    Every element within one bf16 rounding of float64, every launch bit-identical."""
    from cortex.kernels import ops

    K = 512
    g = torch.Generator().manual_seed(M + N + 3)
    a = torch.randn(M, K, generator=g).bfloat16()
    q, s = O.quantize_int8((torch.randn(N, K, generator=g) * 0.05).numpy())
    q, s = torch.from_numpy(q), torch.from_numpy(s)
    bias = torch.randn(N, generator=g) if with_bias else None
    img = ops.convert(q.to(DEV), torch.bfloat16)
    if not with_scale:  # the scale folded into a float weight rounded to bf16 (exact in float64 below)
        w = (q.double() * s.double()[:, None]).to(torch.bfloat16)
        img, s_dev, wref = w.to(DEV), None, w.double()
    else:
        s_dev, wref = s.to(DEV), q.double() * s.double()[:, None]
    ad = a.to(DEV)
    ys = [ops.norm_linear(ad, weight=img, weight_scale=s_dev, bias=None if bias is None else bias.to(DEV),
                          act=act, out_dtype=torch.bfloat16) for _ in range(3)]
    assert all(torch.equal(y, ys[0]) for y in ys[1:])
    ref = a.double() @ wref.T
    if bias is not None:
        ref = ref + bias.double()
    if act == "gelu":
        ref = F.gelu(ref)
    err = (ys[0].cpu().double() - ref).abs()
    assert bool((err <= _bf16_ulp(ref) + 1e-5 * float(ref.abs().max())).all()), float(err.max())


@pytest.mark.parametrize("N", [1, 2, 8])
@pytest.mark.parametrize("form", ["bf16x_bf16w", "bf16x_int8w", "f32x_f32w_fp32", "f32x_f32w_bf16"])
def test_narrow_output_rows(N, form):
    """N <= 8 outputs (the behaviour head's 512 -> 1 projection) on the row-dot kernel."""
    from cortex.kernels import ops

    g = torch.Generator().manual_seed(N)
    M, K = 64, 512
    x = torch.randn(M, K, generator=g)
    w = torch.randn(N, K, generator=g) * 0.05
    res = torch.randn(M, N, generator=g)
    if form == "bf16x_bf16w":
        xb, wb = x.bfloat16(), w.bfloat16()
        y = ops.norm_linear(xb.to(DEV), weight=wb.to(DEV), residual=res.to(DEV), out_dtype=torch.float32)
        ref = xb.double() @ wb.double().T + res.double()
    elif form == "bf16x_int8w":
        xb = x.bfloat16()
        q, s = O.quantize_int8(w.numpy())
        q, s = torch.from_numpy(q), torch.from_numpy(s)
        y = ops.norm_linear(xb.to(DEV), weight_int8=q.to(DEV), weight_scale=s.to(DEV), out_dtype=torch.float32)
        ref = xb.double() @ q.double().T * s.double()
    elif form == "f32x_f32w_fp32":
        y = ops.norm_linear(x.to(DEV), weight=w.to(DEV), act="gelu", out_dtype=torch.float32,
                            compute_dtype=torch.float32)
        ref = torch.nn.functional.gelu(x.double() @ w.double().T)
    else:  # fp32 operands under bf16 compute: both rounded to bf16 first
        y = ops.norm_linear(x.to(DEV), weight=w.to(DEV), out_dtype=torch.float32, compute_dtype=torch.bfloat16)
        ref = x.bfloat16().double() @ w.bfloat16().double().T
    assert y.shape == (M, N)
    assert float((y.cpu().double() - ref).abs().max()) <= 1e-5 * float(ref.abs().max())


@pytest.mark.parametrize("M,N,K,res_rows", [(8192, 512, 512, 0), (300, 512, 512, 0), (8192, 512, 512, 256),
                                            (77, 256, 256, 0), (200, 256, 512, 0), (96, 512, 256, 32),
                                            (1024, 256, 2048, 0), (40, 512, 128, 8)])
@pytest.mark.parametrize("inplace", [False, True])
def test_linear_residual_ln(M, N, K, res_rows, inplace):
    """Residual linear + LayerNorm in one kernel (out_proj + norm_mlp): the fp32 residual
    output within 1e-5 of a float64 contraction of the same operands; the bf16 LayerNorm
    of it within one bf16 rounding of the fp32 LayerNorm of the kernel's own output.
    K = 256 / 512 run the direct-weight form (each N), other K the LDS-ring form."""
    from cortex.kernels import ops

    a, q, s = _operands(M, N, K, seed=M + N + K)
    g = torch.Generator().manual_seed(5)
    bias = 0.1 * torch.randn(N, generator=g)
    res = torch.randn(res_rows or M, N, generator=g) * 2.0 + 0.3
    gam, bet = 1 + 0.2 * torch.randn(N, generator=g), 0.2 * torch.randn(N, generator=g)
    w_img = ops.convert(q.to(DEV), torch.bfloat16)
    res_d = res.to(DEV)
    # the int8 weight itself, widened in the kernel: bit-identical to its bf16 image
    x8, xn8 = ops.linear_residual_ln(a.to(DEV), q.to(DEV), s.to(DEV), bias.to(DEV), residual=res_d.clone(),
                                     ln=(gam.to(DEV), bet.to(DEV), 1e-5), res_rows=res_rows)
    out = res_d if (inplace and not res_rows) else None
    x, xn = ops.linear_residual_ln(a.to(DEV), w_img, s.to(DEV), bias.to(DEV), residual=res_d,
                                   ln=(gam.to(DEV), bet.to(DEV), 1e-5), res_rows=res_rows, out=out)
    if out is not None:
        assert x.data_ptr() == res_d.data_ptr()
    ref = _ref(a, q, s, bias=bias, res=res, res_rows=res_rows)
    # (few rows take the K-split kernel with the image, a different fp32 summation order)
    for xo, xno in ((x, xn), (x8, xn8)):
        xc = xo.cpu()
        assert (xc.double() - ref).abs().max() <= 1e-5 * ref.abs().max()
        ln = F.layer_norm(xc, (N,), gam, bet, 1e-5)
        err = (xno.cpu().float() - ln).abs()
        assert (err <= _bf16_ulp(ln) + 1e-5 * float(ln.abs().max())).all(), float(err.max())
    if not ops.splitk_splits(M, N, K, torch.device(DEV)):  # no K split: the same operands in the same order
        torch.testing.assert_close(x8, x, rtol=0, atol=0)
        torch.testing.assert_close(xn8, xn, rtol=0, atol=0)
    if ops.frag_ok(M, N, K, torch.device(DEV)):
        # the weight in fragment order (direct-weight kernel): the same fragments in the same
        # order as the LDS-ring kernel on the bf16 image, so bit-identical to it, bf16 and int8 xn
        wf = ops.frag_weight(q.to(DEV))
        # (the residual from the host copy: the in-place case above overwrote res_d)
        xf, xnf = ops.linear_residual_ln(a.to(DEV), wf, s.to(DEV), bias.to(DEV), residual=res.to(DEV),
                                         ln=(gam.to(DEV), bet.to(DEV), 1e-5), res_rows=res_rows, frag=True)
        torch.testing.assert_close(xf, x8, rtol=0, atol=0)
        torch.testing.assert_close(xnf, xn8, rtol=0, atol=0)
        kw = dict(residual=res.to(DEV), ln=(gam.to(DEV), bet.to(DEV), 1e-5), res_rows=res_rows, xq_scale=0.03)
        xq_n = ops.linear_residual_ln(a.to(DEV), w_img, s.to(DEV), bias.to(DEV), **kw)
        kw["residual"] = res.to(DEV)
        xq_f = ops.linear_residual_ln(a.to(DEV), wf, s.to(DEV), bias.to(DEV), frag=True, **kw)
        torch.testing.assert_close(xq_f[0], xq_n[0], rtol=0, atol=0)
        torch.testing.assert_close(xq_f[1], xq_n[1], rtol=0, atol=0)


@pytest.mark.parametrize("N,K", [(512, 512), (256, 256), (48, 96), (16, 32)])
@pytest.mark.parametrize("src", [torch.int8, torch.bfloat16, torch.float32])
def test_frag_weight_layout(N, K, src):
    """cortex_frag_weight: 1 KiB block (n16, k32) = 64 lanes x 8 values, lane l = row 16 n16 +
    l % 16, K 32 k32 + 8 (l / 16) .. +7, the values of cortex_convert's bf16 image, checked
    against the same permutation of the image taken on the CPU (and a strided source)."""
    from cortex.kernels import ops

    g = torch.Generator().manual_seed(N + K)
    if src == torch.int8:
        full = torch.randint(-127, 128, (N, K + 16), generator=g, dtype=torch.int8)
    else:
        full = (torch.randn(N, K + 16, generator=g) * 3).to(src)
    w_d = full.to(DEV)[:, :K]  # device rows with a stride of K + 16
    assert w_d.stride(0) == K + 16
    w = full[:, :K]
    img = w.to(torch.bfloat16) if src != torch.float32 else ops.convert(w.contiguous().to(DEV), torch.bfloat16).cpu()
    want = img.reshape(N // 16, 16, K // 32, 4, 8).permute(0, 2, 3, 1, 4).reshape(-1)
    got = ops.frag_weight(w_d).cpu().reshape(-1)
    assert torch.equal(got.view(torch.int16), want.contiguous().view(torch.int16))


@pytest.mark.parametrize("M,N,K,splits,res_rows", [(256, 512, 2048, 8, 0), (256, 512, 512, 8, 0), (1, 512, 2048, 4, 0),
                                                  (300, 512, 1024, 2, 0), (512, 256, 512, 4, 256), (2048, 512, 2048, 4, 0)])
@pytest.mark.parametrize("ln", [False, True])
def test_split_k_residual_linears(M, N, K, splits, res_rows, ln):
    """K split across workgroups through the C-ABI at explicit slab counts (ragged M,
    one row, broadcast residual, in place): the fp32 output within 1e-5 of a float64
    contraction; with the LayerNorm, the bf16 rows within one bf16 rounding of the fp32
    LayerNorm of the kernel's own output."""
    from cortex import _native as nat
    from cortex.kernels import ops

    a, q, s = _operands(M, N, K, seed=M + K + splits)
    g = torch.Generator().manual_seed(9)
    bias = 0.1 * torch.randn(N, generator=g)
    res = torch.randn(res_rows or M, N, generator=g) * 2.0 + 0.3
    gam, bet = 1 + 0.2 * torch.randn(N, generator=g), 0.2 * torch.randn(N, generator=g)
    ad, w_img, sd, bd = a.to(DEV), ops.convert(q.to(DEV), torch.bfloat16), s.to(DEV), bias.to(DEV)
    res_d = res.to(DEV)
    out = res_d if not res_rows else torch.empty(M, N, device=DEV)
    ws = torch.empty(nat.load().cortex_splitk_workspace_bytes(M, N, splits), dtype=torch.uint8, device=DEV)
    stream = nat.stream_of(torch.device(DEV))
    if ln:
        gd, bt = gam.to(DEV), bet.to(DEV)
        xn = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
        nat.call("cortex_linear_residual_ln_splitk", M, N, K, nat.ptr(ad), K, nat.ptr(w_img), K, nat.ptr(sd),
                 nat.ptr(bd), nat.ptr(res_d), N, res_rows, nat.ptr(out), N, nat.ptr(gd), nat.ptr(bt), 1e-5,
                 nat.ptr(xn), N, splits, nat.ptr(ws), ws.numel(), stream)
    else:
        nat.call("cortex_linear_residual_splitk", M, N, K, nat.ptr(ad), K, nat.ptr(w_img), K, nat.ptr(sd),
                 nat.ptr(bd), nat.ptr(res_d), N, res_rows, nat.ptr(out), N, splits, nat.ptr(ws), ws.numel(), stream)
    ref = _ref(a, q, s, bias=bias, res=res, res_rows=res_rows)
    xc = out.cpu()
    assert (xc.double() - ref).abs().max() <= 1e-5 * ref.abs().max()
    if ln:
        lnr = F.layer_norm(xc, (N,), gam, bet, 1e-5)
        err = (xn.cpu().float() - lnr).abs()
        assert (err <= _bf16_ulp(lnr) + 1e-5 * float(lnr.abs().max())).all(), float(err.max())



def _rider(sizes, seed=0):
    g = torch.Generator().manual_seed(seed)
    src = [torch.randint(-127, 128, (n,), generator=g, dtype=torch.int8).to(DEV) for n in sizes]
    return src, [torch.full(s.shape, 7.0, dtype=torch.bfloat16, device=DEV) for s in src]


@pytest.mark.parametrize("sizes", [(16,), (32768,), (32768 * 3 + 16, 48, 65536), tuple([4096 + 16 * i for i in range(8)])])
def test_widen_riders_exact_and_rows_unchanged(sizes):
    """int8 -> bf16 widening (exact: every int8 value is a bf16 value) on a launch of its own and
    riding on the LayerNorm row kernel and on the tokenizer + LayerNorm kernel: whole and partial
    workgroup chunks, up to 8 arrays; the host kernels' own rows are bit-identical with and
    without the rider."""
    from cortex.kernels import ops

    src, dst = _rider(sizes)
    ops.widen_int8(list(zip(src, dst)))
    torch.cuda.synchronize()
    for s, d in zip(src, dst):
        assert torch.equal(d, s.to(torch.bfloat16))
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1000, 512, generator=g).to(DEV)
    ln = (torch.randn(512, generator=g).to(DEV), torch.randn(512, generator=g).to(DEV), 1e-5)
    src, dst = _rider(sizes, 2)
    ref = ops.ln_rows(x, ln)
    out = ops.ln_rows(x, ln, widen=list(zip(src, dst)))
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    for s, d in zip(src, dst):
        assert torch.equal(d, s.to(torch.bfloat16))
    tabs = [torch.randn(n, 512, generator=g).mul(0.02).to(DEV) for n in (137, 600, 8)]
    ids = [torch.randint(0, n, (777,), generator=g).to(DEV) for n in (137, 600, 8)]
    src, dst = _rider(sizes, 3)
    ref = ops.tokenize_ln(*tabs, *ids, ln)
    out = ops.tokenize_ln(*tabs, *ids, ln, widen=list(zip(src, dst)))
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    for s, d in zip(src, dst):
        assert torch.equal(d, s.to(torch.bfloat16))


@pytest.mark.parametrize("shapes", [((512, 512),), ((512, 2048), (1536, 512), (512, 512), (2048, 512)),
                                    ((16, 64), (64, 64), (48, 1024))])
def test_widen_rider_fragment_order(shapes):
    """Widening riders that write MFMA fragment order (K given per array): each destination
    equals cortex_frag_weight's layout of the same int8 weight, next to plain arrays in the same
    launch, on a launch of its own and riding on the LayerNorm row kernel."""
    from cortex.kernels import ops

    g = torch.Generator().manual_seed(len(shapes))
    for host in ("alone", "ln_rows"):
        items, want = [], []
        for i, (n, k) in enumerate(shapes):
            q = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).to(DEV)
            d = torch.full((n, k), 7.0, dtype=torch.bfloat16, device=DEV)
            frag = i % 2 == 0
            items.append((q, d, k if frag else 0))
            want.append(ops.frag_weight(q) if frag else q.to(torch.bfloat16))
        if host == "alone":
            ops.widen_int8(items)
        else:
            x = torch.randn(300, 512, generator=g).to(DEV)
            ln = (torch.ones(512, device=DEV), torch.zeros(512, device=DEV), 1e-5)
            assert torch.equal(ops.ln_rows(x, ln, widen=items), ops.ln_rows(x, ln))
        torch.cuda.synchronize()
        for (q, d, k), w in zip(items, want):
            assert torch.equal(d.view(torch.int16), w.view(torch.int16)), (host, tuple(q.shape), k)
