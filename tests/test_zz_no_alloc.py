"""cortex_pack_plan_noalloc (the pack plan on the library's static scratch, for callers
that cannot allocate) against cortex_pack_plan with a caller workspace, through the C-ABI.

Two calls in a row, the second with a smaller input, then the reverse order of paths:
the three-launch plan (per-chunk counts in the scratch) and the sorted fast path (status
words in the scratch above 8192 events).  Bit-exact offsets, order, ranks and error flags.  Sizes whose
counts do not fit the scratch are refused on the host with an error, before any launch.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _lib():
    from cortex import _native as nat

    return nat, nat.load()


def _plan(nat, lib, bidx: torch.Tensor, B: int, with_rank: bool, noalloc: bool):
    E = bidx.shape[0]
    offsets = torch.full((B + 1,), -7, dtype=torch.int64, device=DEV)
    order = torch.full((E,), -7, dtype=torch.int64, device=DEV)
    dst = torch.full((E,), -7, dtype=torch.int64, device=DEV)
    rank = torch.full((E,), -7, dtype=torch.int64, device=DEV) if with_rank else None
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    stream = nat.stream_of(torch.device(DEV))
    if noalloc:
        rc = lib.cortex_pack_plan_noalloc(nat.ptr(bidx), 1, E, B, nat.ptr(offsets), nat.ptr(order), nat.ptr(dst),
                                          nat.ptr(rank), nat.ptr(err), stream)
    else:
        ws_bytes = lib.cortex_pack_workspace_bytes(E, B)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
        rc = lib.cortex_pack_plan(nat.ptr(bidx), 1, E, B, nat.ptr(offsets), nat.ptr(order), nat.ptr(dst),
                                  nat.ptr(rank), nat.ptr(ws), ws_bytes, nat.ptr(err), None, 0, stream)
    assert rc == 0, lib.cortex_last_error()
    torch.cuda.synchronize()
    return [t.cpu() for t in (offsets, order, dst, rank, err) if t is not None]


def _case(kind: str, E: int, B: int, seed: int) -> torch.Tensor:
    rng = np.random.default_rng(seed)
    b = np.sort(rng.integers(0, B, E))
    if kind == "shuffled":
        b = b[rng.permutation(E)]
    if kind == "bad":
        b[E // 3] = B + 5
    return torch.from_numpy(b.astype(np.int64)).to(DEV)


@pytest.mark.parametrize("calls", [
    # (kind, E, B, with_rank): large three-launch plan, then a small sorted one
    [("shuffled", 200_000, 300, True), ("sorted", 3000, 40, False)],
    # small sorted (fast path), then a smaller shuffled one with an invalid index
    [("sorted", 60_000, 1000, False), ("bad", 5000, 17, False)],
])
def test_noalloc_pack_plan_equals_workspace_plan(calls):
    nat, lib = _lib()
    for i, (kind, E, B, with_rank) in enumerate(calls):
        print(f"noalloc call {i}: {kind} E={E} B={B} rank={with_rank}", flush=True)
        bidx = _case(kind, E, B, seed=10 + i)
        assert lib.cortex_pack_workspace_bytes(E, B) <= lib.cortex_pack_noalloc_max_workspace_bytes()
        want = _plan(nat, lib, bidx, B, with_rank, noalloc=False)
        got = _plan(nat, lib, bidx, B, with_rank, noalloc=True)
        for g, w in zip(got, want):
            torch.testing.assert_close(g, w, rtol=0, atol=0)
        assert bool(int(got[-1].item()) & 2) == (kind == "bad")


def test_noalloc_refuses_sizes_beyond_its_scratch():
    nat, lib = _lib()
    cap = lib.cortex_pack_noalloc_max_workspace_bytes()
    E, B = 1 << 20, 8192  # 1024 chunks x 8192 samples of counts: 32 MiB
    assert lib.cortex_pack_workspace_bytes(E, B) > cap
    rc = lib.cortex_pack_plan_noalloc(None, 1, E, B, None, None, None, None, None, None)
    assert rc == -4 and b"above its maximum" in lib.cortex_last_error()
