"""Dispatchers on ROCm tensors (reference test group 3: dispatcher and fallback).

GPU tensors always take the HIP kernels: the ``*_reference`` formulations, which the
dispatchers return for tensors on other devices, are replaced by spies that fail the test
if they are ever called.  Also: the derived-weight cache of ``rms_norm_linear`` /
``norm_linear_int8`` when the first call is captured into a HIP graph.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import cortex_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture
def no_reference(monkeypatch):
    """Replace every *_reference formulation with a spy that records calls."""
    import cortex.kernels.fused_rmsnorm as fr
    import cortex.kernels.sparse_xattn as sx
    import cortex.kernels.tokenizer as tk

    calls = []

    def spy(name):
        def f(*a, **k):
            calls.append(name)
            raise AssertionError(f"{name} called on GPU tensors")
        return f

    monkeypatch.setattr(tk, "fused_tokenizer_reference", spy("fused_tokenizer_reference"))
    monkeypatch.setattr(sx, "sparse_cross_attention_reference", spy("sparse_cross_attention_reference"))
    monkeypatch.setattr(fr, "rms_norm_linear_reference", spy("rms_norm_linear_reference"))
    return calls


def test_gpu_tensors_never_take_the_reference(no_reference):
    from cortex import _native
    from cortex.kernels.fused_rmsnorm import rms_norm_linear
    from cortex.kernels.sparse_xattn import sparse_cross_attention
    from cortex.kernels.tokenizer import fused_tokenizer

    assert _native.available()
    g = torch.Generator().manual_seed(42)
    n, t, v = (torch.randn(r, 64, generator=g) * 0.02 for r in (37, 60, 8))
    nid, tb = torch.randint(0, 37, (300,), generator=g), torch.randint(0, 60, (300,), generator=g)
    val = torch.randint(0, 8, (300,), generator=g)
    out = fused_tokenizer(n.to(DEV), t.to(DEV), v.to(DEV), nid.to(DEV), tb.to(DEV), val.to(DEV))
    np.testing.assert_array_equal(out.cpu().numpy(), O.tokenize(n.numpy(), t.numpy(), v.numpy(), nid, tb, val))

    x, gm, w = torch.randn(64, 128, generator=g), 1 + 0.02 * torch.randn(128, generator=g), \
        torch.randn(128, 96, generator=g)
    out = rms_norm_linear(x.to(DEV), gm.to(DEV), w.to(DEV))
    torch.testing.assert_close(out.cpu(), O.rms_norm_linear(x.double(), gm.double(), w.double()).float(),
                               rtol=1e-4, atol=1e-4)

    q, k, vv = (torch.randn(2, 2, s, 64, generator=g) / 8 for s in (128, 192, 192))
    mask = torch.tensor([[True, False, True], [False, True, True]])
    for bm in (None, mask):
        out = sparse_cross_attention(q.to(DEV), k.to(DEV), vv.to(DEV), bm)
        want = O.sparse_cross_attention(q.numpy(), k.numpy(), vv.numpy(), None if bm is None else bm.numpy())
        np.testing.assert_allclose(out.cpu().numpy(), want, rtol=1e-4, atol=1e-4)
    assert no_reference == []


def test_fold_cache_first_call_captured():
    """The first rms_norm_linear call on a fresh (weight, gain) pair is captured into a HIP graph:
    the graph recomputes the folded rows itself, and a later eager call builds its own instead of
    reading rows that capture only recorded.  Eager results equal the graph's on every replay."""
    from cortex.kernels import ops
    from cortex.kernels.fused_rmsnorm import norm_linear_int8

    torch.manual_seed(5)
    M, K, N = 256, 512, 384
    x = torch.randn(M, K, device=DEV).to(torch.bfloat16)
    gm = (1 + 0.02 * torch.randn(K)).to(DEV)
    wq = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=DEV)
    ws = torch.rand(N, device=DEV) * 1e-3 + 1e-4
    before = len(ops._KN_CACHE)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            out_g = norm_linear_int8(x, wq, ws, norm="rms", gamma=gm)
    torch.cuda.current_stream().wait_stream(s)
    assert len(ops._KN_CACHE) == before  # nothing cached from inside the capture
    want = O.rms_norm_linear(x.cpu().float(), gm.cpu(), (wq.cpu().float() * ws.cpu()[:, None]).t())
    for _ in range(3):
        graph.replay()
        eager = norm_linear_int8(x, wq, ws, norm="rms", gamma=gm)  # builds (then hits) its own rows
        torch.cuda.synchronize()
        assert torch.equal(eager, out_g)
        err = float((eager.float().cpu() - want).abs().max() / want.abs().max())
        assert err <= 2e-2 and err <= 4e-3  # the contract bar; observed level about 1e-3
    assert len(ops._KN_CACHE) >= min(before + 1, ops._KN_CACHE_SIZE)
    # a hit under capture pins the entry: flooding the cache afterwards does not evict it
    graph2 = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph2, stream=s):
            out_g2 = norm_linear_int8(x, wq, ws, norm="rms", gamma=gm)
    torch.cuda.current_stream().wait_stream(s)
    for i in range(ops._KN_CACHE_SIZE + 2):
        norm_linear_int8(x[:8], wq, ws, norm="rms", gamma=gm + (i + 1) * 1e-3)
    graph2.replay()
    torch.cuda.synchronize()
    assert torch.equal(out_g2, norm_linear_int8(x, wq, ws, norm="rms", gamma=gm))
