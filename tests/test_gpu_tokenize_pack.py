"""Tokenizer + pack on the GPU vs the oracle: bit-exact (a1, a2)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import cortex_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _tables(N, T, V, D, dtype, seed=42):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(s, D, generator=g).to(dtype) for s in (N, T, V))


def _ids(E, N, T, V, seed=99):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randint(0, s, (E,), generator=g, dtype=torch.int64) for s in (N, T, V))


def _ref_torch(n, t, v, nid, tb, val):
    """Left-to-right add in the table dtype on the CPU (bf16 adds round to nearest even)."""
    return (n[nid] + t[tb]) + v[val]


@pytest.mark.parametrize("E,D,N,T,V", [(1, 64, 32, 64, 8), (127, 64, 32, 64, 8), (128, 64, 256, 512, 8),
                                       (1024, 128, 256, 512, 8), (4096, 256, 512, 1024, 8),
                                       (16384, 512, 512, 1024, 16), (33, 70, 5, 7, 3)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fused_tokenizer_bitexact(E, D, N, T, V, dtype):
    from cortex.kernels.tokenizer import fused_tokenizer

    n, t, v = _tables(N, T, V, D, dtype)
    nid, tb, val = _ids(E, N, T, V)
    out = fused_tokenizer(n.to(DEV), t.to(DEV), v.to(DEV), nid.to(DEV), tb.to(DEV), val.to(DEV))
    assert out.shape == (E, D) and out.dtype == dtype
    if dtype == torch.float32:
        want = O.tokenize(n.numpy(), t.numpy(), v.numpy(), nid.numpy(), tb.numpy(), val.numpy())
        np.testing.assert_array_equal(out.cpu().numpy(), want)
    else:
        assert torch.equal(out.cpu(), _ref_torch(n, t, v, nid, tb, val))


def test_fused_tokenizer_edge_cases():
    from cortex.kernels.tokenizer import fused_tokenizer

    n, t, v = (x.to(DEV) for x in _tables(32, 64, 8, 128, torch.float32))
    empty = torch.zeros(0, dtype=torch.int64, device=DEV)
    assert fused_tokenizer(n, t, v, empty, empty, empty).shape == (0, 128)
    big = torch.randint(0, 32, (128,), device=DEV)
    nid = big[::2]  # strided view
    tb = torch.randint(0, 64, (64,), device=DEV)
    val = torch.randint(0, 8, (64,), device=DEV)
    out = fused_tokenizer(n, t, v, nid, tb, val)
    want = O.tokenize(n.cpu().numpy(), t.cpu().numpy(), v.cpu().numpy(), nid.cpu().numpy(), tb.cpu().numpy(),
                      val.cpu().numpy())
    np.testing.assert_array_equal(out.cpu().numpy(), want)
    with pytest.raises(ValueError):
        fused_tokenizer(n.t(), t, v, nid, tb, val)
    with pytest.raises(ValueError):
        fused_tokenizer(n, t, v, nid, tb[:-1], val)
    # out-of-range index: zero row, no out-of-bounds access, IndexError when checked
    bad = nid.clone()
    bad[5] = 32
    out = fused_tokenizer(n, t, v, bad, tb, val)
    assert (out[5] == 0).all()
    with pytest.raises(IndexError):
        fused_tokenizer(n, t, v, bad, tb, val, check_indices=True)


def _config0_inputs(seed=0, shuffle=False, B=32):
    rng = np.random.default_rng(seed)
    counts = rng.integers(128, 513, B)
    E = int(counts.sum())
    nid = rng.integers(0, 137, E)
    tb = rng.integers(0, 600, E)
    val = np.clip(rng.poisson(1.0, E) + 1, 0, 7)
    bidx = np.repeat(np.arange(B), counts)
    if shuffle:
        p = rng.permutation(E)
        nid, tb, val, bidx = nid[p], tb[p], val[p], bidx[p]
    tabs = [rng.normal(0, 0.02, (s, 512)).astype(np.float32) for s in (137, 600, 8)]
    return tabs, nid, tb, val, bidx


@pytest.mark.parametrize("shuffle", [False, True])
def test_tokenize_and_pack_config0_bitexact(shuffle):
    """Config 0: B=32, E_b ~ U[128,512], tables 137/600/8 x 512 fp32 -> CSR and padded, bit-exact."""
    from cortex.kernels.tokenizer import tokenize_and_pack

    tabs, nid, tb, val, bidx = _config0_inputs(shuffle=shuffle)
    want_tok = O.tokenize(*tabs, nid, tb, val)
    want = O.pack_events(want_tok, bidx)
    args = [torch.from_numpy(a).to(DEV) for a in (*tabs, nid, tb, val, bidx)]
    tok, off = tokenize_and_pack(*args, batch_size=32, layout="csr")
    np.testing.assert_array_equal(off.cpu().numpy(), want.offsets)
    np.testing.assert_array_equal(tok.cpu().numpy(), want.csr)
    pad, mask = tokenize_and_pack(*args, layout="padded")
    np.testing.assert_array_equal(pad.cpu().numpy(), want.padded)
    np.testing.assert_array_equal(mask.cpu().numpy(), want.mask)


@pytest.mark.parametrize("seed", range(4))
def test_pack_plan_stable_rank_random(seed):
    """Unsorted batch indices with many collisions, empty samples, E not a multiple of 64."""
    from cortex.kernels.pack import pack_plan

    rng = np.random.default_rng(seed)
    E = int(rng.integers(1, 5000))
    B = int(rng.integers(1, 300))
    bidx = rng.integers(0, B, E)
    p = O.pack_events(np.zeros((E, 1), np.float32), bidx, batch_size=B)
    off, order, rank = pack_plan(torch.from_numpy(bidx).to(DEV), B)
    np.testing.assert_array_equal(off.cpu().numpy(), p.offsets)
    np.testing.assert_array_equal(order.cpu().numpy(), p.order)
    np.testing.assert_array_equal(rank.cpu().numpy(), p.rank)


def test_pack_plan_large_multi_chunk():
    """E spans several 1024-event chunks (and a chunk size above 1024)."""
    from cortex.kernels.pack import pack_plan

    rng = np.random.default_rng(7)
    for E, B in ((131072, 256), (1_200_000, 64)):
        bidx = np.sort(rng.integers(0, B, E)) if E > 200000 else rng.integers(0, B, E)
        p = O.pack_events(np.zeros((E, 1), np.float32), bidx, batch_size=B)
        off, order, rank = pack_plan(torch.from_numpy(bidx).to(DEV), B)
        np.testing.assert_array_equal(off.cpu().numpy(), p.offsets)
        np.testing.assert_array_equal(order.cpu().numpy(), p.order)


@pytest.mark.parametrize("E,B", [(65536, 1024), (65537, 1024), (5000, 1025), (64, 1), (65536, 3)])
def test_pack_plan_path_boundaries(E, B):
    """Either side of the one-launch plan's limits (B <= 1024, E <= 65536): same results."""
    from cortex.kernels.pack import pack_plan

    rng = np.random.default_rng(E + B)
    bidx = rng.integers(0, B, E)
    p = O.pack_events(np.zeros((E, 1), np.float32), bidx, batch_size=B)
    off, order, rank = pack_plan(torch.from_numpy(bidx).to(DEV), B)
    np.testing.assert_array_equal(off.cpu().numpy(), p.offsets)
    np.testing.assert_array_equal(order.cpu().numpy(), p.order)
    np.testing.assert_array_equal(rank.cpu().numpy(), p.rank)


def test_pack_events_drop_in_matches_oracle():
    from cortex.models.cortex import _pack_events

    rng = np.random.default_rng(11)
    E = 700
    bidx = rng.integers(0, 9, E)
    x = rng.normal(size=(E, 96)).astype(np.float32)
    want = O.pack_events(x, bidx)
    out, mask = _pack_events(torch.from_numpy(x).to(DEV), torch.from_numpy(bidx).to(DEV))
    np.testing.assert_array_equal(out.cpu().numpy(), want.padded)
    np.testing.assert_array_equal(mask.cpu().numpy(), want.mask)
    e_out, e_mask = _pack_events(torch.zeros(0, 96, device=DEV), torch.zeros(0, dtype=torch.int64, device=DEV))
    assert e_out.shape == (1, 0, 96) and e_mask.shape == (1, 0)


def test_invalid_batch_index_sets_flag_and_stays_in_bounds():
    from cortex.kernels import ops

    tabs, nid, tb, val, bidx = _config0_inputs(B=4)
    bidx = bidx.copy()
    bidx[3] = 4  # == B: invalid
    bidx[10] = -1
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    t = [torch.from_numpy(a).to(DEV) for a in (*tabs, nid, tb, val, bidx)]
    off, order, _ = ops.pack_plan(t[6], 4, err=err)
    tok = ops.tokenize(*t[:6], order=order, csr_offsets=off, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) & 2
    valid = (bidx >= 0) & (bidx < 4)
    assert int(off[-1].item()) == int(valid.sum())
    assert (tok[int(valid.sum()):] == 0).all()


def _bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    e = torch.floor(torch.log2(x.abs().clamp_min(1e-30)))
    return torch.pow(2.0, e - 7)


@pytest.mark.parametrize("D", [256, 512])
def test_tokenize_ln_matches_tokens_then_layernorm(D):
    """Tokens (bit-exact oracle sum, CSR order of shuffled events) -> LayerNorm -> bf16, one pass;
    an out-of-range index gives LN(0) = beta and sets the error flag."""
    from cortex.kernels import ops

    B, per = 6, 300
    E = B * per
    n, t, v = _tables(512, 1024, 8, D, torch.float32)
    nid, tb, val = _ids(E, 512, 1024, 8, seed=5)
    nid[17] = 4096  # out of range
    g = torch.Generator().manual_seed(8)
    bidx = torch.repeat_interleave(torch.arange(B), per)[torch.randperm(E, generator=g)]
    w, b = 1 + 0.1 * torch.randn(D, generator=g), 0.1 * torch.randn(D, generator=g)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    offsets, order, _ = ops.pack_plan(bidx.to(DEV), B)
    out = ops.tokenize_ln(n.to(DEV), t.to(DEV), v.to(DEV), nid.to(DEV), tb.to(DEV), val.to(DEV),
                          (w.to(DEV), b.to(DEV), 1e-5), order=order, csr_offsets=offsets, err=err)
    assert out.dtype == torch.bfloat16 and out.shape == (E, D)
    assert int(err.item()) & 1
    ordr = order.cpu().numpy()
    nid_ok = nid.clone()
    bad = nid_ok >= 512
    nid_ok[bad] = 0
    tok = torch.from_numpy(O.tokenize(n.numpy(), t.numpy(), v.numpy(), nid_ok.numpy(), tb.numpy(), val.numpy()))
    tok[bad] = 0.0
    ref = torch.nn.functional.layer_norm(tok[torch.from_numpy(ordr)], (D,), w, b, 1e-5)
    diff = (out.float().cpu() - ref).abs()
    assert bool((diff <= _bf16_ulp(ref) + 1e-5 * float(ref.abs().max())).all())
    r_bad = int(np.nonzero(ordr == 17)[0][0])
    torch.testing.assert_close(out[r_bad].float().cpu(), b.bfloat16().float(), rtol=0, atol=0)


def _sorted_cases():
    rng = np.random.default_rng(5)
    cases = {}
    b = np.sort(rng.integers(3, 40, 5000))  # empty samples 0-2, gaps in the middle, empty tail up to B = 50
    cases["gaps"] = (b, 50)
    b = np.sort(rng.integers(0, 8, 4096))
    b[1023], b[1024] = b[1024], b[1023] - 1 if b[1023] > 0 else 1  # one inversion across the 1024-event boundary
    cases["inversion_at_range_edge"] = (b, 8)
    b = np.sort(rng.integers(0, 16, 3000))
    b[2999] = 16  # sorted but the last index is out of range
    cases["out_of_range_tail"] = (b, 16)
    cases["single_event"] = (np.array([2]), 5)
    cases["one_sample"] = (np.zeros(65536, dtype=np.int64), 1)
    cases["all_distinct_1024"] = (np.arange(1024), 1024)
    # a negative index just before a valid one: the boundary loop must not start below 0
    cases["negative_before_valid"] = (np.array([-2, 0, 0, 1]), 4)
    cases["very_negative_before_valid"] = (np.array([-(1 << 40), 0]), 2)
    b = np.sort(rng.integers(0, 6, 2500))
    b[1024] = -7  # first event of the second range
    cases["negative_at_range_start"] = (b, 6)
    b = np.sort(rng.integers(0, 21, 4000))
    b[2047], b[2048] = b[2048], b[2047] - 1 if b[2047] > 0 else 1
    cases["inversion_4000"] = (b, 21)
    # above 4096 events the check runs wide (a workgroup per 256 events) before the plan kernel
    b = np.sort(rng.integers(0, 21, 20000))
    b[5119], b[5120] = b[5120], b[5119] - 1 if b[5119] > 0 else 1
    cases["inversion_wide"] = (b, 21)
    b = np.sort(rng.integers(0, 33, 20000))
    b[256], b[255] = b[255], b[256] + 1  # an inversion across a 256-event range edge
    cases["inversion_wide_range_edge"] = (b, 34)
    b = np.sort(rng.integers(0, 30, 17000))
    b[16999] = 30
    cases["out_of_range_tail_wide"] = (b, 30)
    cases["sorted_4096"] = (np.sort(rng.integers(0, 33, 4096)), 33)
    cases["sorted_4097"] = (np.sort(rng.integers(0, 33, 4097)), 40)
    cases["sorted_16447"] = (np.sort(rng.integers(0, 33, 16447)), 33)  # partial last wave of the wide check
    # above 65536 events (or above 1024 samples) the general three-launch plan follows the wide
    # check and returns at once when every range was sorted
    cases["sorted_70000"] = (np.sort(rng.integers(0, 200, 70000)), 200)
    b = np.sort(rng.integers(0, 200, 70000))
    b[60000], b[60001] = b[60001], b[60000] - 1 if b[60000] > 0 else 1
    cases["inversion_70000"] = (b, 200)
    b = np.sort(rng.integers(0, 90, 66000))
    b[65999] = 90
    cases["out_of_range_tail_66000"] = (b, 90)
    cases["sorted_b2000"] = (np.sort(rng.integers(0, 2000, 9000)), 2000)
    b = np.sort(rng.integers(0, 2000, 9000))
    b[0] = -3
    cases["negative_first_b2000"] = (b, 2000)
    return cases


@pytest.mark.parametrize("name", list(_sorted_cases()))
def test_pack_plan_sorted_fast_path(name):
    """Sorted batch indices take the identity plan (checked inside the plan kernel up to 4096
    events, by the wide pack_sorted_kernel above, also ahead of the general three-launch plan
    past 65536 events or 1024 samples); anything else found
    there -- an inversion, an index out of range -- falls back to the full plan.  Same
    results as the oracle either way, with and without ranks; with the identity flag, a
    sorted in-range plan sets it (order is then the identity by definition) and any other
    clears it and writes order."""
    from cortex.kernels import ops

    bidx, B = _sorted_cases()[name]
    valid = (bidx >= 0) & (bidx < B)
    p = O.pack_events(np.zeros((int(valid.sum()), 1), np.float32), bidx[valid], batch_size=B)
    t = torch.from_numpy(bidx.astype(np.int64)).to(DEV)
    for with_rank in (False, True):
        err = torch.zeros(1, dtype=torch.int32, device=DEV)
        off, order, rank = ops.pack_plan(t, B, err=err, with_rank=with_rank)
        torch.cuda.synchronize()
        assert bool(int(err.item()) & 2) == (not valid.all())
        np.testing.assert_array_equal(off.cpu().numpy(), p.offsets)
        n = int(p.offsets[-1])
        np.testing.assert_array_equal(order.cpu().numpy()[:n], np.flatnonzero(valid)[p.order])
        if with_rank:
            np.testing.assert_array_equal(rank.cpu().numpy()[valid], p.rank)
    err = torch.full((1,), 0x5C, dtype=torch.int32, device=DEV)  # stale bits: cleared by the plan itself
    off, order, _, ident = ops.pack_plan(t, B, err=err, with_rank=False, identity=True, clear_err=True)
    torch.cuda.synchronize()
    assert int(err.item()) == (0 if valid.all() else 2)
    sorted_ok = bool(valid.all() and (np.diff(bidx) >= 0).all())
    assert int(ident.item()) == int(sorted_ok)
    np.testing.assert_array_equal(off.cpu().numpy(), p.offsets)
    if not sorted_ok:
        n = int(p.offsets[-1])
        np.testing.assert_array_equal(order.cpu().numpy()[:n], np.flatnonzero(valid)[p.order])


@pytest.mark.parametrize("E,B,shuffle,rank", [(0, 4, False, False), (3000, 8, False, False), (3000, 8, True, False),
                                              (16384, 32, False, False), (16384, 32, True, False),
                                              (70000, 2000, False, False), (70000, 2000, True, True)])
def test_pack_plan_widen_rider(E, B, shuffle, rank):
    """cortex_pack_plan_widen on every plan path (one launch up to 4096 events, the wide sorted
    check, the three-launch plan with and without ranks, no events): the plan is exactly the
    one without a rider, and the rider's int8 arrays (ragged sizes, one not a whole workgroup
    chunk) come out widened exactly."""
    from cortex.kernels import ops

    g = torch.Generator().manual_seed(E + B)
    bidx = torch.sort(torch.randint(0, B, (E,), generator=g)).values
    if shuffle:
        bidx = bidx[torch.randperm(E, generator=g)]
    bidx = bidx.to(DEV)
    src = [torch.randint(-127, 128, (n,), generator=g, dtype=torch.int8).to(DEV) for n in (262144, 8192 + 48, 16)]
    dst = [torch.zeros(s.shape, dtype=torch.bfloat16, device=DEV) for s in src]
    want = ops.pack_plan(bidx, B, with_rank=rank, identity=not rank)
    got = ops.pack_plan(bidx, B, with_rank=rank, identity=not rank, widen=list(zip(src, dst)))
    torch.cuda.synchronize()
    if not rank:
        assert int(got[3].item()) == int(want[3].item())
    assert torch.equal(got[0], want[0])
    if rank or not int(want[3].item()):  # order is written unless the identity flag is set
        assert torch.equal(got[1], want[1])
    if rank:
        assert torch.equal(got[2], want[2])
    for s, d in zip(src, dst):
        assert torch.equal(d, s.to(torch.bfloat16))
