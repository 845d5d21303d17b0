"""Cortex-S INT8 inference forward on one MI355X.

Headline: samples/s of the Cortex-S INT8 forward at B = 32 x 512 synthetic events,
p50/p99 latency at B = 1, the roofline fraction of the dominant kernel and of the
other hot kernels, and the CPU oracle timed on the host cores.

A step is one forward of the fixed workload (CORTEX_S, weights quantised to INT8 per
channel on the GPU, bf16 MFMA with fp32 accumulation and an fp32 residual stream,
B = 32 samples x 512 events) replayed from a HIP graph captured on the resident event
buffers: the inputs are in HBM before the timed region and a step copies nothing.
The first few dozen replays of a fresh process run while the GPU clocks ramp up: they
are reported as ``cold_start``, and the headline's W warmup + K timed replays follow the
eager forward and the per-kernel timings.  ``steady_state`` re-times 200 replays after
every other measurement.

Usage:
  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--quick]
      prints exactly one JSON line on stdout
  python bench.py --kernel NAME [--iters N]
      launches one hot kernel N times on synthetic operands of its forward shape (for
      rocprofv3 --kernel-trace / --pmc runs); NAME in KERNELS, or one of the API
      configurations 0-2 (API_WORKLOADS)
  python bench.py --copy-calibration [--iters N]
      a plain 64 MiB device-to-device copy N times (the reference for PMC byte counters)
"""

from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "cortex-engine_amd"))
sys.path.insert(0, str(ROOT))

import numpy as np  # noqa: E402
import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "Cortex-S INT8 samples/s @B=32,512 ev; p99 latency @B=1; % HBM/MFMA peak"
B_MAIN, PER_MAIN, L, D, H, DH = 32, 512, 256, 512, 8, 64
M_ROWS = B_MAIN * L


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def make_events(batch: int, per_sample, seed: int):
    """Synthetic spike events: nid U[0,137), time bin U[0,600), value = clip(Poisson(1)+1, 0, 7).

    ``per_sample`` is an int (same count for every sample) or a per-sample array."""
    rng = np.random.default_rng(seed)
    counts = np.full(batch, per_sample) if np.isscalar(per_sample) else np.asarray(per_sample)
    E = int(counts.sum())
    return (rng.integers(0, 137, E), rng.integers(0, 600, E), np.clip(rng.poisson(1.0, E) + 1, 0, 7),
            np.repeat(np.arange(batch), counts))


def build_model(dev, with_scales: bool = False):
    """CORTEX_S, seed 0, calibrated on one batch of 8 x 512 synthetic events and converted
    to INT8 weights; with ``with_scales`` also the calibration scales (for the W8A8 mode)."""
    from cortex.models import CortexModel
    from cortex.models.config import CORTEX_S
    from cortex.quantization.calibrate import (attach_calibration_hooks, convert_model, derive_scales,
                                               remove_calibration_hooks)

    torch.manual_seed(0)
    model = CortexModel(CORTEX_S).to(dev).eval()
    calib = [torch.from_numpy(a).to(dev) for a in make_events(8, 512, seed=1)]
    hooks = attach_calibration_hooks(model)
    with torch.no_grad():
        model(*calib, batch_size=8)
    remove_calibration_hooks(hooks)
    scales = derive_scales(model, hooks)
    model = convert_model(model, scales, inplace=True)
    return (model, scales) if with_scales else model


# --------------------------------------------------------------------------- hot kernels


def _int8_image(n: int, k: int, dev, seed: int):
    """An INT8 per-channel weight (as QuantizedLinear holds it) and its bf16 execution image."""
    from cortex.kernels import ops

    g = torch.Generator(device="cpu").manual_seed(seed)
    w = torch.randn(n, k, generator=g) * 0.02
    q, s = ops.quantize_int8(w.to(dev))
    return ops.convert(q, torch.bfloat16), s


def make_kernel(name: str, dev):
    """(launch callable, launches per forward, bound, algorithmic flops, algorithmic bytes, label)
    for one hot kernel at its Cortex-S B=32 x 512-event shape, on synthetic operands."""
    from cortex.kernels import ops

    g = torch.Generator(device="cpu").manual_seed(7)
    bf = torch.bfloat16

    def rnd(*shape, dtype=torch.float32, scale=1.0):
        return (torch.randn(*shape, generator=g) * scale).to(dtype).to(dev)

    def gemm(n, k, act=None, residual=False, seed=1):
        x = rnd(M_ROWS, k, dtype=bf)
        w, s = _int8_image(n, k, dev, seed)
        res = rnd(M_ROWS, n) if residual else None
        out = torch.empty(M_ROWS, n, dtype=torch.float32 if residual else bf, device=dev)
        if residual and ops.frag_res_ok(M_ROWS, n, k, dev):  # the forward's form: the fragment-order weight
            wf = ops.frag_weight(w)
            fn = lambda: ops.linear_residual_frag(x, wf, s, None, residual=res, out=out)  # noqa: E731
        else:
            fn = lambda: ops.norm_linear(x, weight=w, weight_scale=s, act=act, residual=res,  # noqa: E731
                                         out_dtype=out.dtype, compute_dtype=bf, out=out)
        flops = 2.0 * M_ROWS * n * k
        # compulsory bytes: activations, the INT8 weight and its scales, residual, output
        byts = M_ROWS * k * 2 + n * k + 4 * n + (M_ROWS * n * 4 if residual else 0) + M_ROWS * n * out.element_size()
        return fn, flops, byts

    if name == "gemm_mlp2_residual":
        fn, fl, by = gemm(512, 2048, residual=True)
        return fn, 7, "hbm", fl, by, ("MLP down 2048->512 + fp32 residual, M=8192 (gemm_res_dw_kernel, "
                                      "128x128 tiles, K split over two wave groups, each wavefront's weight "
                                      "fragments straight into registers)")
    if name == "gemm_mlp0_gelu":
        fn, fl, by = gemm(2048, 512, act="gelu")
        return fn, 7, "mfma", fl, by, "MLP up 512->2048 + GELU, bf16 out, M=8192 (gemm_bf16_kernel)"
    if name == "qkv_attention":
        xn = rnd(M_ROWS, D, dtype=bf)
        w, sc = _int8_image(3 * D, D, dev, 2)
        out = torch.empty(M_ROWS, D, dtype=bf, device=dev)
        fn = lambda: ops.qkv_attention(xn, w, sc, None, B_MAIN, L, H, out=out)  # noqa: E731
        fl = 2.0 * M_ROWS * 3 * D * D + 4.0 * B_MAIN * H * L * L * DH  # projection + attention
        by = M_ROWS * D * 2 + 3 * D * D + 3 * D * 4 + M_ROWS * D * 2  # xn, int8 weight, scales, output
        return fn, 7, "mfma", fl, by, ("QKV projection 512->1536 + self-attention B=32 H=8 L=256 Dh=64, "
                                      "per (head, sample) (qkv_attention_kernel)")
    if name == "out_residual_ln":
        a = rnd(M_ROWS, D, dtype=bf)
        w, sc = _int8_image(D, D, dev, 3)
        wf = ops.frag_weight(w)  # the forward's layout for this kernel (bf16 images)
        res = rnd(M_ROWS, D)
        g_, b_ = rnd(D), rnd(D)
        fn = lambda: ops.linear_residual_ln(a, wf, sc, None, residual=res, ln=(g_, b_, 1e-5), out=res,  # noqa: E731
                                            frag=True)
        fl = 2.0 * M_ROWS * D * D
        by = M_ROWS * D * 2 + D * D + 4 * D + M_ROWS * D * 4 * 2 + M_ROWS * D * 2 + 2 * D * 4
        return fn, 8, "hbm", fl, by, ("attention out 512->512 + fp32 residual + the next LayerNorm, M=8192 "
                                      "(gemm_rowln_dw_kernel: 32-row full-width tiles, each wavefront's weight "
                                      "rows straight into registers)")
    if name == "attention_cross":
        E = B_MAIN * PER_MAIN
        kv = rnd(E, 2 * D, dtype=bf)
        q = rnd(1, H, L, DH, dtype=bf, scale=0.25)
        off = torch.arange(0, E + 1, PER_MAIN, device=dev)
        o_buf, o = ops.merge_heads_out(B_MAIN, L, H, DH, bf, dev)
        fn = lambda: ops.attention(q, ops.heads_view(kv, 1, E, H, 0, D),  # noqa: E731
                                   ops.heads_view(kv, 1, E, H, D, D), kv_offsets=off, out=o, batch=B_MAIN)
        fl = 4.0 * H * L * DH * E
        by = L * D * 2 + E * 2 * D * 2 + M_ROWS * D * 2
        return fn, 1, "mfma", fl, by, "cross-attention latents x 512 CSR events/sample (attention_fast_kernel)"
    if name == "ln_rows":
        x = rnd(M_ROWS, D)
        w, b = rnd(D), rnd(D)
        out = torch.empty(M_ROWS, D, dtype=bf, device=dev)

        def fn():
            ops.ln_rows(x, (w, b, 1e-5))
        by = M_ROWS * D * 4 + M_ROWS * D * 2 + 2 * D * 4
        del out
        return fn, 6, "hbm", 0.0, by, "LayerNorm rows fp32 -> bf16, M=8192 K=512 (ln_rows_kernel)"
    if name == "tokenize":
        E = B_MAIN * PER_MAIN
        nid, tb, val, bidx = (torch.from_numpy(a).to(dev) for a in make_events(B_MAIN, PER_MAIN, seed=3))
        ne, te, ve = rnd(512, D, scale=0.02), rnd(1024, D, scale=0.02), rnd(8, D, scale=0.02)
        lw, lb = rnd(D), rnd(D)
        offsets, order, _, ident = ops.pack_plan(bidx, B_MAIN, with_rank=False, identity=True)
        fn = lambda: ops.tokenize_ln(ne, te, ve, nid, tb, val, (lw, lb, 1e-5), order=order,  # noqa: E731
                                     csr_offsets=offsets, identity=ident)
        # compulsory: 3 indices per event (the sorted plan is the identity), bf16 row out, the
        # touched table rows (137 neuron, 600 time, 8 value) and the LayerNorm parameters
        by = E * (D * 2 + 3 * 8) + (137 + 600 + 8) * D * 4 + 2 * D * 4 + (B_MAIN + 1) * 8
        return fn, 1, "hbm", 0.0, by, ("fused tokenizer + norm_kv LayerNorm into bf16 CSR rows, E=16384 D=512 "
                                      "(tokenize_ln_kernel)")
    if name.startswith("api_"):
        return make_api_workload(name, dev)
    raise ValueError(f"unknown kernel {name}")


def _api_events(dev, seed: int = 0):
    """B = 32 ragged samples, E_b ~ U{128..512}, and fp32 tables 137/600/8 x 512 ~ N(0, 0.02)."""
    rng = np.random.default_rng(seed)
    B, D = 32, 512
    counts = rng.integers(128, 513, B)
    E = int(counts.sum())
    ev = [torch.from_numpy(a).to(dev) for a in (rng.integers(0, 137, E), rng.integers(0, 600, E),
                                                 np.clip(rng.poisson(1.0, E) + 1, 0, 7), np.repeat(np.arange(B), counts))]
    tables = [torch.from_numpy(rng.normal(0, 0.02, (n, D)).astype(np.float32)).to(dev) for n in (137, 600, 8)]
    return rng, B, D, counts, E, ev, tables


def make_api_workload(name: str, dev):
    """The kernel-level configurations through the public API, as make_kernel's tuple (the whole
    call is the unit: every kernel it launches is in the trace):

    * api_tokenize_pack: config 0, fused_tokenizer + pack to CSR rows, fp32;
    * api_sparse_xattn: config 1, sparse_cross_attention bf16 with per-sample lengths;
    * api_norm_linear_int8_n{1536,2048,512}: config 2, RMSNorm (eps 1e-6) + INT8 linear,
      M = 8192, K = 512, bf16 in / out."""
    from cortex.kernels.fused_rmsnorm import norm_linear_int8
    from cortex.kernels import ops
    from cortex.kernels.sparse_xattn import sparse_cross_attention
    from cortex.kernels.tokenizer import tokenize_and_pack

    if name == "api_tokenize_pack":
        rng, B, D, counts, E, ev, tables = _api_events(dev)
        by = E * (D * 4 + 4 * 8) + (137 + 600 + 8) * D * 4 + (B + 1) * 8
        return (lambda: tokenize_and_pack(*tables, *ev, batch_size=B)), 1, "hbm", 0.0, by, \
            f"config 0: fused tokenizer + pack, CSR rows, fp32, B=32 E={E} D=512"
    if name == "api_sparse_xattn":
        rng, B, D, counts, E, ev, tables = _api_events(dev)
        H, L, Dh, Ek = 8, 256, 64, 512
        g = torch.Generator(device="cpu").manual_seed(1)
        q, k, v = ((torch.randn(B, H, n, Dh, generator=g) / 8).bfloat16().to(dev) for n in (L, Ek, Ek))
        lens = torch.from_numpy(rng.integers(128, 513, B)).to(dev)
        fl = 4.0 * H * L * Dh * float(lens.sum())
        by = 2 * (2 * B * H * L * Dh) + 2 * 2 * H * Dh * float(lens.sum())
        return (lambda: sparse_cross_attention(q, k, v, kv_lengths=lens)), 1, "mfma", fl, by, \
            "config 1: sparse cross-attention bf16, q (32,8,256,64), k/v (32,8,512,64), lengths U{128..512}"
    m = re.fullmatch(r"api_norm_linear_int8_n(\d+)", name)
    if m:
        n, M, K = int(m.group(1)), 8192, 512
        g = torch.Generator(device="cpu").manual_seed(2)
        x = torch.randn(M, K, generator=g).bfloat16().to(dev)
        gam = (1 + 0.02 * torch.randn(K, generator=g)).to(dev)
        q, sc = ops.quantize_int8((0.02 * torch.randn(n, K, generator=g)).to(dev))
        fl = 2.0 * M * n * K
        by = M * K * 2 + n * K + n * 4 + M * n * 2
        return (lambda: norm_linear_int8(x, q, sc, norm="rms", gamma=gam, eps=1e-6, out_dtype=torch.bfloat16)), \
            1, ("hbm" if n <= 512 else "mfma"), fl, by, f"config 2: RMSNorm + INT8 linear, M=8192 K=512 N={n}, bf16"
    raise ValueError(f"unknown API workload {name}")


KERNELS = ("gemm_mlp2_residual", "gemm_mlp0_gelu", "qkv_attention", "out_residual_ln", "attention_cross", "ln_rows",
           "tokenize")
API_WORKLOADS = ("api_tokenize_pack", "api_sparse_xattn", "api_norm_linear_int8_n1536", "api_norm_linear_int8_n2048",
                 "api_norm_linear_int8_n512")


def time_launches(fn, iters: int = 20, reps: int = 5) -> float:
    """Average seconds per launch: `iters` launches captured in a HIP graph (so host launch
    cost does not enter), replayed `reps` times between HIP events on the current stream."""
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(iters):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(reps):
        graph.replay()
    t1.record(stream)
    t1.synchronize()
    return t0.elapsed_time(t1) / 1e3 / (iters * reps)


def traffic_from_profiles(name: str):
    """HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (scaled by the
    counters' reading for a plain copy of known size), as recorded in profiles/<name>_pmc.txt."""
    p = ROOT / "profiles" / f"{name}_pmc.txt"
    if not p.exists():
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", p.read_text(), re.M)
    return float(m.group(1)) if m else None


def kernel_rooflines(dev):
    rows = {}
    for name in KERNELS:
        fn, per_fwd, bound, flops, byts, label = make_kernel(name, dev)
        sec = time_launches(fn)
        r = {"kernel": label, "avg_us": round(sec * 1e6, 2), "launches_per_forward": per_fwd, "bound": bound,
             "hbm_gbs": round(byts / sec / 1e9, 1), "hbm_frac": round(byts / sec / 1e9 / HBM_PEAK_GBS, 4),
             "bytes_per_launch": int(byts)}
        if flops:
            r["tflops"] = round(flops / sec / 1e12, 2)
            r["mfma_frac"] = round(flops / sec / 1e12 / BF16_PEAK_TFLOPS, 4)
            r["flops_per_launch"] = flops
        rows[name] = r
        del fn
    torch.cuda.empty_cache()
    return rows


def roofline_of(name: str, r: dict) -> dict:
    if r["bound"] == "hbm":
        out = {"bound": "hbm", "achieved": r["hbm_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
               "frac": r["hbm_frac"]}
    else:
        out = {"bound": "mfma", "achieved": r["tflops"], "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
               "frac": r["mfma_frac"]}
    out["traffic"] = traffic_from_profiles(name)
    out.update({"name": name, "kernel": r["kernel"], "avg_us": r["avg_us"],
                "algorithmic_bytes": r["bytes_per_launch"]})
    if "flops_per_launch" in r:
        out["algorithmic_flops"] = r["flops_per_launch"]
    return out


# --------------------------------------------------------------------------- forward-level


def section_breakdown(model, inputs, dev, step_ms: float):
    """Per-section GPU time (ms) of the graph-replayed forward, in the reference profiler's sections
    (scripts/profile_inference.py:137-211).  Each section is the forward's own code on the forward's
    intermediate tensors (``CortexModel._token_rows``, ``_cross_rows``, ``_encode``, the head),
    captured in a HIP graph and replayed like the step, so that pack_plan + tokenizer + cross_attn
    + self_attn_all + behavior_head add up to the step (``sum_ms`` beside ``step_ms``).
    The tokenizer section includes ``norm_kv`` (fused into the gather); cross_attn includes the
    first block's ``norm_attn`` (fused into its out-projection).  ``mlp_only`` is one block's
    ``x + mlp(norm_mlp(x))`` (the LayerNorm row kernel, MLP-up + GELU, MLP-down + residual);
    ``self_attn_single`` is block 0."""
    from cortex.kernels import ops
    from cortex.models._layers import apply_linear, exec_weights, normalize_bf16

    nid, tb, val, bidx = inputs
    B, cfg = B_MAIN, model.config
    enc = model.encoder
    comp = cfg.compute_dtype
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    blk = enc.self_attn_blocks[0]
    with torch.no_grad():
        offsets, order, _, ident = ops.pack_plan(bidx, B, err=err, with_rank=False, identity=True)
        tokens = model._token_rows(nid, tb, val, offsets, order, err, ident)
        x0, xn0 = model._cross_rows(tokens, offsets, B)
        lat = model._encode(x0.clone(), B, xn0)
        x_all, x_one, x_mlp = x0.clone(), x0.clone(), x0.clone()

        def mlp_only():
            hn = normalize_bf16(x_mlp, blk.norm_mlp)
            h = ops.norm_linear(hn, **exec_weights(blk.mlp[0], comp), act="gelu", out_dtype=comp, compute_dtype=comp)
            return apply_linear(blk.mlp[2], h, residual=x_mlp, out_dtype=torch.float32, compute=comp, out=x_mlp)

        parts = {
            "pack_plan": lambda: ops.pack_plan(bidx, B, err=err, with_rank=False, identity=True),
            "tokenizer": lambda: model._token_rows(nid, tb, val, offsets, order, err, ident),
            "cross_attn": lambda: model._cross_rows(tokens, offsets, B),
            "self_attn_all": lambda: model._encode(x_all, B, xn0),
            "self_attn_single": lambda: blk.forward_rows(x_one, B, L, inplace=True, xn=xn0),
            "mlp_only": mlp_only,
            "behavior_head": lambda: model.behavior_head.forward_rows(lat, B, pre_norm=enc.final_norm),
        }
        times = {k: round(time_launches(fn, iters=10, reps=5) * 1e3, 4) for k, fn in parts.items()}
    total = sum(times[k] for k in ("pack_plan", "tokenizer", "cross_attn", "self_attn_all", "behavior_head"))
    return {**times, "sum_ms": round(total, 4), "step_ms": round(step_ms, 4),
            "how": "each section graph-replayed alone on the forward's own intermediate tensors"}


def latency_b1(model, dev, n_requests: int, per_sample: int = 512):
    """p50/p99 wall latency of B=1 requests: pinned H2D of the events, graph replay, D2H of (1, 2)."""
    from cortex.runtime import CapturedForward

    cap = CapturedForward(model, batch_size=1, n_events=per_sample)
    host = [torch.from_numpy(a).pin_memory() for a in make_events(1, per_sample, seed=7)]
    dev_in = (cap.neuron_ids, cap.time_bins, cap.values, cap.batch_indices)  # the graph's input buffers
    out_host = torch.empty((1, 2), dtype=torch.float32).pin_memory()
    lat = []
    for i in range(n_requests + 20):
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        for d, h in zip(dev_in, host):
            d.copy_(h, non_blocking=True)  # pinned H2D straight into the graph's inputs
        out = cap()
        out_host.copy_(out, non_blocking=True)
        torch.cuda.synchronize(dev)
        if i >= 20:
            lat.append((time.perf_counter() - t0) * 1e3)
    lat.sort()
    return {"p50_ms": round(lat[len(lat) // 2], 4), "p99_ms": round(lat[int(len(lat) * 0.99) - 1], 4),
            "requests": n_requests, "events_per_request": per_sample, "path": "hip graph replay"}


def worker_latency(model, dev, n_requests: int, per_sample: int = 512):
    """The serving worker end to end, one B=1 request at a time (reference payload contract:
    a list of event dicts), and a B=256 batch of columnar payloads: host packing, one pinned
    H2D, graph replay, D2H of the behaviour, wall clock -- one batch at a time, and pipelined
    (``submit_batch`` / ``collect``, two batches in flight)."""
    from cortex.models.config import CORTEX_S
    from cortex.serve import InferenceWorker

    w = InferenceWorker(model, CORTEX_S, dev, max_batch_size=256)
    nid, tb, val, _ = make_events(1, per_sample, seed=8)
    one = [{"request_id": "r0", "events": [{"neuron_id": int(a), "time_bin": int(b), "value": int(c)}
                                           for a, b, c in zip(nid, tb, val)]}]
    lat = []
    for i in range(n_requests + 20):
        t0 = time.perf_counter()
        w._run_batch_sync(one)
        if i >= 20:
            lat.append((time.perf_counter() - t0) * 1e3)
    lat.sort()
    rng = np.random.default_rng(12)
    counts = np.clip(rng.poisson(512, 256), 64, 2048)
    nid, tb, val, _ = make_events(256, counts, seed=13)
    cuts = np.cumsum(counts)[:-1]
    batch = [{"request_id": f"r{i}", "events": {"neuron_id": a, "time_bin": b, "value": c}}
             for i, (a, b, c) in enumerate(zip(np.split(nid, cuts), np.split(tb, cuts), np.split(val, cuts)))]
    for _ in range(3):
        w._run_batch_sync(batch)
    reps = 10
    t0 = time.perf_counter()
    for _ in range(reps):
        w._run_batch_sync(batch)
    sec = (time.perf_counter() - t0) / reps
    # pipelined: the next batch is packed and submitted while the current one runs;
    # steady state timed between batch completions
    pending, done = None, []
    for _ in range(reps + 3):
        nxt = w.submit_batch(batch)
        if pending is not None:
            w.collect(pending)
            done.append(time.perf_counter())
        pending = nxt
    w.collect(pending)
    done.append(time.perf_counter())
    psec = (done[-1] - done[2]) / (len(done) - 3)
    w.shutdown()
    return {"b1_p50_ms": round(lat[len(lat) // 2], 4), "b1_p99_ms": round(lat[int(len(lat) * 0.99) - 1], 4),
            "b1_requests": n_requests, "b1_events": per_sample, "b1_payload": "list of event dicts",
            "b256_ms_per_batch": round(sec * 1e3, 3), "b256_samples_per_s": round(256 / sec, 1),
            "b256_pipelined_ms_per_batch": round(psec * 1e3, 3), "b256_pipelined_samples_per_s": round(256 / psec, 1),
            "b256_events": int(counts.sum()), "b256_payload": "columnar arrays"}


def streaming_windows(model, dev, sessions: int = 256, steps: int = 12, b1_requests: int = 200):
    """Streaming decode with the device event-page cache: every step each session sends one
    new 50-bin stride of events (one columnar host -> device page write for all sessions;
    timed from the arrived host arrays, the binning of raw spikes is upstream), then one
    batch of 600-bin windows is assembled on the device and decoded; pages that left every
    window age out by LRU.  Poisson spike counts over 137 neurons at ~512 events per window.

    ``ms_per_step``: the pipelined loop (the next stride is written and the next batch
    submitted while the GPU runs the current one), timed between batch completions;
    ``sync_ms_per_step``: one step at a time, each ending in its result copy.  p50/p99 for
    a single session (B=1)."""
    from cortex.cache import EventWindowCache
    from cortex.models.config import CORTEX_S
    from cortex.serve import InferenceWorker

    stride, window = 50, 600
    n_strides = window // stride - 1 + 2 * (steps + 3)
    rate = 512 / (window * 137)
    rng = np.random.default_rng(21)
    w = InferenceWorker(model, CORTEX_S, dev, max_batch_size=sessions)
    cache = EventWindowCache(num_pages=sessions * 16 + 64, page_events=512, bins_per_page=stride, device=dev)
    names = [f"s{i}" for i in range(sessions)]
    counts = rng.poisson(rate, (sessions, n_strides * stride, 137)).astype(np.int8)

    def stride_columns(b0):  # upstream binning: page counts, then (neuron, absolute bin, value)
        s_, t, n = np.nonzero(counts[:, b0:b0 + stride])
        return (np.full(sessions, b0), np.bincount(s_, minlength=sessions), n.astype(np.int64),
                t.astype(np.int64) + b0, np.clip(counts[s_, t + b0, n], 1, 7).astype(np.int64))

    def requests(b0):
        return [{"request_id": s, "session_id": s, "window_start": b0 + stride - window} for s in names]

    for b0 in range(0, window - stride, stride):
        cache.write_columns(names, *stride_columns(b0))
    first = window - stride
    cols = [stride_columns(first + k * stride) for k in range(2 * (steps + 3))]
    pending, done = None, []
    for k in range(steps + 3):
        cache.write_columns(names, *cols[k])
        nxt = w.submit_windows(requests(first + k * stride), cache, window)
        if pending is not None:
            w.collect(pending)
            done.append(time.perf_counter())
        pending = nxt
    w.collect(pending)
    done.append(time.perf_counter())
    sec = (done[-1] - done[2]) / (len(done) - 3)  # steady state: between batch completions
    times = []
    for k in range(steps + 3, 2 * (steps + 3)):
        t0 = time.perf_counter()
        cache.write_columns(names, *cols[k])
        w.run_windows_sync(requests(first + k * stride), cache, window)
        if k >= steps + 6:
            times.append(time.perf_counter() - t0)
    sync_sec = float(np.median(times))  # a step that captures a graph for a new event bucket is an outlier
    one = rng.poisson(rate, (window + (b1_requests + 10) * stride, 137))

    def page(b0):
        t, n = np.nonzero(one[b0:b0 + stride])
        return n.astype(np.int64), t.astype(np.int64) + b0, np.clip(one[t + b0, n], 1, 7).astype(np.int64)

    for b0 in range(0, window - stride, stride):
        cache.write("solo", b0, *page(b0))
    lat = []
    for i in range(b1_requests + 10):
        b0 = window - stride + i * stride
        new = page(b0)
        t0 = time.perf_counter()
        cache.write("solo", b0, *new)
        w.run_windows_sync([{"request_id": "solo", "session_id": "solo", "window_start": b0 + stride - window}],
                           cache, window)
        if i >= 10:
            lat.append((time.perf_counter() - t0) * 1e3)
    lat.sort()
    w.shutdown()
    return {"sessions": sessions, "ms_per_step": round(sec * 1e3, 3), "samples_per_s": round(sessions / sec, 1),
            "sync_ms_per_step": round(sync_sec * 1e3, 3), "sync_samples_per_s": round(sessions / sync_sec, 1),
            "b1_p50_ms": round(lat[len(lat) // 2], 4), "b1_p99_ms": round(lat[int(len(lat) * 0.99) - 1], 4),
            "b1_requests": b1_requests, "hit_rate": round(cache.hit_rate, 4)}


def serving_sweep(model, dev, batches=(1, 8, 32, 128, 256), reps: int = 20):
    """Serving-shaped forward: E_b = clip(Poisson(512), 64, 2048) per sample, one graph per batch."""
    from cortex.runtime import CapturedForward

    rng = np.random.default_rng(11)
    out = []
    for B in batches:
        counts = np.clip(rng.poisson(512, B), 64, 2048)
        inputs = [torch.from_numpy(a).to(dev) for a in make_events(B, counts, seed=100 + B)]
        cap = CapturedForward(model, batch_size=B, n_events=int(counts.sum()), inputs=tuple(inputs))
        for _ in range(3):
            cap()
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        for _ in range(reps):
            cap()
        torch.cuda.synchronize(dev)
        sec = (time.perf_counter() - t0) / reps
        out.append({"batch": B, "events": int(counts.sum()), "ms_per_forward": round(sec * 1e3, 4),
                    "samples_per_s": round(B / sec, 1)})
        del cap, inputs
        torch.cuda.empty_cache()
    return out


def norm_linear_api(dev, M: int = 8192, K: int = 512, widths=(1536, 2048, 512)) -> dict:
    """Standalone RMSNorm (eps 1e-6) + linear through the public API, bf16 rows (M, K): the
    ``(K, N)`` bf16 weight of ``rms_norm_linear`` and the INT8 per-channel weight of
    ``norm_linear_int8``; microseconds per call, graph-replayed."""
    from cortex.kernels import ops
    from cortex.kernels.fused_rmsnorm import norm_linear_int8, rms_norm_linear

    g = torch.Generator(device="cpu").manual_seed(2)
    x = torch.randn(M, K, generator=g).bfloat16().to(dev)
    gam = (1 + 0.02 * torch.randn(K, generator=g)).to(dev)
    out = {}
    for n in widths:
        w = (0.02 * torch.randn(n, K, generator=g)).to(dev)
        q, sc = ops.quantize_int8(w)
        wkn = w.t().contiguous().bfloat16()
        t_kn = time_launches(lambda: rms_norm_linear(x, gam, wkn))
        t_i8 = time_launches(lambda: norm_linear_int8(x, q, sc, norm="rms", gamma=gam, eps=1e-6,
                                                      out_dtype=torch.bfloat16))
        prev = ops.INT8_WEIGHTS
        ops.INT8_WEIGHTS = "widen"  # the int8 weight streamed, rows normalised in the kernel
        try:
            t_w = time_launches(lambda: norm_linear_int8(x, q, sc, norm="rms", gamma=gam, eps=1e-6,
                                                         out_dtype=torch.bfloat16))
        finally:
            ops.INT8_WEIGHTS = prev
        fl = 2 * M * n * K
        act_bytes = M * K * 2 + n * 4 + M * n * 2  # rows in, scales, bf16 out
        out[f"N{n}"] = {
            "rms_norm_linear_kn_bf16_us": round(t_kn * 1e6, 2),
            # the default: the gain folded once into cached bf16 rows of the int8 weight
            "int8_image_us": round(t_i8 * 1e6, 2),
            "int8_image_tflops": round(fl / t_i8 / 1e12, 1),
            "int8_image_mfma_frac": round(fl / t_i8 / 1e12 / BF16_PEAK_TFLOPS, 4),
            "int8_image_hbm_frac": round((act_bytes + 2 * n * K) / t_i8 / 1e9 / HBM_PEAK_GBS, 4),
            # the int8 weight itself read by the kernel (rows normalised in the kernel)
            "int8_streamed_us": round(t_w * 1e6, 2),
            "int8_streamed_tflops": round(fl / t_w / 1e12, 1),
            "int8_streamed_mfma_frac": round(fl / t_w / 1e12 / BF16_PEAK_TFLOPS, 4),
            "int8_streamed_hbm_frac": round((act_bytes + n * K) / t_w / 1e9 / HBM_PEAK_GBS, 4)}
    return {"M": M, "K": K,
            "note": "int8_image: the RMS gain folded once into a cached bf16 copy of the int8 weight (2 N K bytes "
                    "read, 1/rms applied to the accumulator); int8_streamed: CORTEX_INT8_WEIGHTS=widen, the int8 "
                    "weight itself read (N K bytes), rows normalised in the kernel; each hbm_frac counts the bytes "
                    "its own kernel reads",
            "derived_weight_bytes": ops.derived_weight_bytes(), **out}


def api_configs(dev) -> dict:
    """The kernel-level workloads through the public API (graph-replayed, microseconds per
    call), each with the roofline fraction of its algorithmic work:

    * tokenize + pack, fp32 tables 137/600/8 x 512, B = 32 with E_b ~ U{128..512}: bytes =
      E (D 4 + 4 x 8) + tables + (B + 1) 8 (token rows written, four int64 indices read);
      CSR rows and the padded (B, E_max, D) + mask layout;
    * sparse cross-attention, bf16, q (32, 8, 256, 64), k / v (32, 8, 512, 64) ~ N(0,1)/8,
      true lengths U{128..512} per sample: FLOPs = 4 H L Dh sum(E_b) (the padding is skipped);
      bytes = 2 (2 B H L Dh) + 2 2 H Dh sum(E_b) (q and o, then k and v over the true lengths),
      both fractions reported."""
    from cortex.kernels.sparse_xattn import sparse_cross_attention
    from cortex.kernels.tokenizer import tokenize_and_pack

    rng = np.random.default_rng(0)
    B, D = 32, 512
    counts = rng.integers(128, 513, B)
    E = int(counts.sum())
    ev = [torch.from_numpy(a).to(dev) for a in (rng.integers(0, 137, E), rng.integers(0, 600, E),
                                                 np.clip(rng.poisson(1.0, E) + 1, 0, 7), np.repeat(np.arange(B), counts))]
    tables = [torch.from_numpy(rng.normal(0, 0.02, (n, D)).astype(np.float32)).to(dev) for n in (137, 600, 8)]
    t_csr = time_launches(lambda: tokenize_and_pack(*tables, *ev, batch_size=B))
    t_pad = time_launches(lambda: tokenize_and_pack(*tables, *ev, batch_size=B, layout="padded",
                                                    max_events=int(counts.max())))
    bytes0 = E * (D * 4 + 4 * 8) + (137 + 600 + 8) * D * 4 + (B + 1) * 8
    H, L, Dh, Ek = 8, 256, 64, 512
    g = torch.Generator(device="cpu").manual_seed(1)
    q, k, v = ((torch.randn(B, H, n, Dh, generator=g) / 8).bfloat16().to(dev) for n in (L, Ek, Ek))
    lens = torch.from_numpy(rng.integers(128, 513, B)).to(dev)
    t_x = time_launches(lambda: sparse_cross_attention(q, k, v, kv_lengths=lens))
    fl = 4.0 * H * L * Dh * float(lens.sum())
    # q read and o written (bf16), k and v read over the true lengths only
    by1 = 2 * (2 * B * H * L * Dh) + 2 * 2 * H * Dh * float(lens.sum())
    return {
        "tokenize_pack_fp32": {"events": E, "csr_us": round(t_csr * 1e6, 2), "padded_us": round(t_pad * 1e6, 2),
                               "algorithmic_bytes": bytes0, "csr_GBps": round(bytes0 / t_csr / 1e9, 1),
                               "csr_hbm_frac": round(bytes0 / t_csr / 1e9 / HBM_PEAK_GBS, 4)},
        "sparse_cross_attention_bf16": {"us": round(t_x * 1e6, 2), "flops": fl, "tflops": round(fl / t_x / 1e12, 1),
                                        "mfma_frac": round(fl / t_x / 1e12 / BF16_PEAK_TFLOPS, 4),
                                        "algorithmic_bytes": int(by1), "GBps": round(by1 / t_x / 1e9, 1),
                                        "hbm_frac": round(by1 / t_x / 1e9 / HBM_PEAK_GBS, 4),
                                        "binding": "hbm (arithmetic intensity %.0f FLOP/B, below the bf16 ridge of "
                                                   "312)" % (fl / by1)},
    }


def w8a8_kernels(dev) -> dict:
    """The int8 kernels of the W8A8 blocks alone at the B = 32 x 512 shapes (graph-replayed):
    microseconds and the fraction of the 5.0 POP/s dense int8 MFMA peak (2 M N K per GEMM)."""
    from cortex.kernels import ops

    g = torch.Generator(device="cpu").manual_seed(3)

    def i8(*shape):
        return torch.randint(-127, 128, shape, generator=g, dtype=torch.int8).to(dev)

    M = M_ROWS
    s = {n: (torch.rand(n, generator=g) * 1e-3 + 1e-4).to(dev) for n in (D, 3 * D, 4 * D)}
    x, h, o = i8(M, D), i8(M, 4 * D), i8(M, D)
    w_up, w_down, w_qkv, w_out = i8(4 * D, D), i8(D, 4 * D), i8(3 * D, D), i8(D, D)
    res = torch.randn(M, D, generator=g).to(dev)
    ln = (torch.ones(D, device=dev), torch.zeros(D, device=dev), 1e-5)
    cases = {
        "mlp_up_gelu_int8": (lambda: ops.linear_w8a8(x, 0.02, w_up, s[4 * D], act="gelu", out_dtype=torch.int8,
                                                     out_scale=0.05), 2.0 * M * 4 * D * D),
        "mlp_down_residual": (lambda: ops.linear_w8a8(h, 0.02, w_down, s[D], residual=res, out=res),
                              2.0 * M * D * 4 * D),
        "qkv_attention": (lambda: ops.qkv_attention_w8a8(x, 0.02, w_qkv, s[3 * D], None, B_MAIN, L, H,
                                                         out_dtype=torch.int8, out_scale=0.01),
                          2.0 * M * 3 * D * D),
        "out_residual_ln": (lambda: ops.linear_residual_ln_w8a8(o, 0.02, w_out, s[D], residual=res, ln=ln, out=res,
                                                                xn_dtype=torch.int8, xn_scale=0.05),
                            2.0 * M * D * D),
    }
    out = {}
    for name, (fn, ops_) in cases.items():
        sec = time_launches(fn)
        out[name] = {"us": round(sec * 1e6, 2), "int8_tops": round(ops_ / sec / 1e12, 1),
                     "int8_frac": round(ops_ / sec / 1e12 / 5000.0, 4)}
    out["note"] = "qkv_attention counts the projection only (its bf16 attention part is not int8 work)"
    return out


def w8a8_forward(model, scales, dev, inputs, reference: torch.Tensor, reps: int = 50) -> dict:
    """The opt-in W8A8 blocks (cortex.quantization.w8a8) on the same B = 32 x 512 forward:
    samples/s (graph replay) and the largest difference to the default path's behaviour."""
    from cortex.quantization.w8a8 import disable_w8a8, enable_w8a8
    from cortex.runtime import CapturedForward

    n = enable_w8a8(model, scales)
    try:
        cap = CapturedForward(model, batch_size=B_MAIN, n_events=B_MAIN * PER_MAIN, inputs=tuple(inputs))
        out = cap().clone()
        for _ in range(5):
            cap()
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        for _ in range(reps):
            cap()
        torch.cuda.synchronize(dev)
        sec = (time.perf_counter() - t0) / reps
        del cap
    finally:
        disable_w8a8(model)
    kern = w8a8_kernels(dev)
    return {"blocks": n, "ms_per_forward": round(sec * 1e3, 4), "samples_per_s": round(B_MAIN / sec, 1),
            "max_abs_diff_vs_default": float((out - reference).abs().max()), "kernels": kern,
            "note": "int8 activations in the self-attention blocks (qkv, out_proj, both MLP linears; calibrated "
                    "act_scale); not the reference's arithmetic, opt-in"}


def _time_captured(model, dev, inputs, reps: int = 50) -> tuple[float, torch.Tensor]:
    """Seconds per B = 32 x 512 forward replayed from a HIP graph, and its output."""
    from cortex.runtime import CapturedForward

    cap = CapturedForward(model, batch_size=B_MAIN, n_events=B_MAIN * PER_MAIN, inputs=tuple(inputs))
    out = cap().clone()
    for _ in range(5):
        cap()
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for _ in range(reps):
        cap()
    torch.cuda.synchronize(dev)
    sec = (time.perf_counter() - t0) / reps
    del cap
    return sec, out


def weights_and_modes(model, dev, inputs, reference: torch.Tensor) -> dict:
    """Resident weight bytes of the default forward (INT8 weights + their bf16 execution images),
    of the widen mode (INT8 weights streamed and widened on chip, no images) and of the window
    mode (INT8 weights + two bf16 windows filled by riders of the row kernels), with each mode's
    time; and the float32-compute forward (the reference's own arithmetic: fp32
    activations, INT8 weights dequantised) on the same weights and events."""
    from cortex.models import CortexModel, _layers
    from cortex.models.config import CORTEX_S, CortexConfig

    wb = _layers.resident_weight_bytes(model)
    prev = _layers.INT8_WEIGHTS
    try:  # every mode timed the same way, the default first
        _layers.INT8_WEIGHTS = "image"
        sec_i, _ = _time_captured(model, dev, inputs)
        _layers.INT8_WEIGHTS = "widen"
        sec_w, out_w = _time_captured(model, dev, inputs)
        _layers.INT8_WEIGHTS = "window"
        sec_v, out_v = _time_captured(model, dev, inputs)
    finally:
        _layers.INT8_WEIGHTS = prev
    win_bytes = _layers.resident_weight_bytes(model)["bf16_windows"]
    res = {"resident_weight_bytes": wb["total"], "int8_weight_bytes": wb["int8_weights"],
           "bf16_image_bytes": wb["bf16_images"], "ms_per_forward": round(sec_i * 1e3, 4),
           "widen": {"resident_weight_bytes": wb["parameters_and_buffers"], "ms_per_forward": round(sec_w * 1e3, 4),
                     "samples_per_s": round(B_MAIN / sec_w, 1),
                     "max_abs_diff_vs_default": float((out_w - reference).abs().max()),
                     "note": "CORTEX_INT8_WEIGHTS=widen: every kernel reads the int8 weights and widens them "
                             "on chip; the default keeps bf16 images because they were measured faster"},
           "window": {"resident_weight_bytes": wb["parameters_and_buffers"] + win_bytes, "bf16_window_bytes": win_bytes,
                      "ms_per_forward": round(sec_v * 1e3, 4), "samples_per_s": round(B_MAIN / sec_v, 1),
                      "max_abs_diff_vs_default": float((out_v - reference).abs().max()),
                      "note": "CORTEX_INT8_WEIGHTS=window: int8 weights resident; each weight group widened into "
                              "a shared bf16 window by extra workgroups of the row kernel launched just before "
                              "it (tokenizer + LayerNorm, then each block's LayerNorm rows)"},
           "reference_int8_bytes_note": "the reference's INT8 model holds 27.8 MB (benchmarks/quantization/"
                                        "results.md:15-18)"}
    torch.manual_seed(0)
    f32 = CortexModel(CortexConfig(**{**CORTEX_S.model_dump(), "dtype": "float32"})).to(dev).eval()
    f32.load_state_dict({k: v for k, v in model.state_dict().items()}, strict=False)
    from cortex.quantization.calibrate import QuantizedLinear

    for name, mod in list(model.named_modules()):  # the same INT8 linears in the fp32-compute model
        if isinstance(mod, QuantizedLinear):
            parent_name, _, leaf = name.rpartition(".")
            parent = f32.get_submodule(parent_name) if parent_name else f32
            setattr(parent, leaf, mod)
    sec_f, out_f = _time_captured(f32, dev, inputs, reps=20)
    res["fp32_compute"] = {"ms_per_forward": round(sec_f * 1e3, 4), "samples_per_s": round(B_MAIN / sec_f, 1),
                           "max_abs_diff_vs_default": float((out_f - reference).abs().max()),
                           "note": "fp32 activations and fp32 MFMA with the INT8 weights dequantised in the "
                                   "kernel: the reference QuantizedLinear arithmetic (1e-5 parity bar)"}
    del f32
    torch.cuda.empty_cache()
    return res


def cpu_baseline(model, budget_s: float = 12.0, b1_budget_s: float = 18.0):
    """The CPU oracle (fp32 activations, INT8 weights dequantised as the reference's QuantizedLinear)
    on the host cores, with the reference's protocol (profile_inference.py: 5 warmup + up to 30 timed
    B=32 x 512-event forwards, mean), bounded by ``budget_s``; the per-section split of one forward;
    and p50/p99 over up to 1000 B=1 requests within ``b1_budget_s``."""
    from oracle import cortex_oracle as O

    torch.set_num_threads(os.cpu_count() or 1)
    sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    arrs = make_events(B_MAIN, PER_MAIN, seed=0)
    for _ in range(5):
        O.forward(sd, O.CORTEX_S_SHAPE, *arrs)
    n, t0, each = 0, time.perf_counter(), []
    while True:
        t = time.perf_counter()
        O.forward(sd, O.CORTEX_S_SHAPE, *arrs)
        each.append(time.perf_counter() - t)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 30:
            break
    each.sort()
    sections: dict = {}
    O.forward(sd, O.CORTEX_S_SHAPE, *arrs, sections=sections)
    one = make_events(1, PER_MAIN, seed=7)
    for _ in range(5):
        O.forward(sd, O.CORTEX_S_SHAPE, *one)
    lat, t1 = [], time.perf_counter()
    while len(lat) < 1000 and time.perf_counter() - t1 < b1_budget_s:
        t = time.perf_counter()
        O.forward(sd, O.CORTEX_S_SHAPE, *one)
        lat.append((time.perf_counter() - t) * 1e3)
    lat.sort()
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(B_MAIN * n / el, 2), "unit": "samples/s", "cores": torch.get_num_threads(),
            "kind": "port", "sample": f"{n} forwards of B=32 x 512 events (CORTEX_S, INT8 dequantised to fp32, "
                                      f"oracle restatement) in {el:.1f} s after 5 warmup",
            "cpu": cpu, "median_forward_ms": round(each[len(each) // 2] * 1e3, 2),
            "sections_ms": {k: round(v * 1e3, 2) for k, v in sections.items()},
            "api_median_of_100_ms": cpu_api_medians(),
            "b1_p50_ms": round(lat[len(lat) // 2], 3), "b1_p99_ms": round(lat[max(int(len(lat) * 0.99) - 1, 0)], 3),
            "b1_requests": len(lat)}


def _median_ms(fn, iters: int = 100, warmup: int = 5, budget_s: float = 4.0) -> tuple[float, int]:
    """Median wall time of ``fn`` over up to ``iters`` calls within ``budget_s`` (the reference's
    kernel-benchmark protocol, cortex/kernels/bench_tokenizer.py:93-110, on the host)."""
    for _ in range(warmup):
        fn()
    times, t0 = [], time.perf_counter()
    while len(times) < iters and time.perf_counter() - t0 < budget_s:
        t = time.perf_counter()
        fn()
        times.append((time.perf_counter() - t) * 1e3)
    times.sort()
    return round(times[len(times) // 2], 3), len(times)


def cpu_api_medians() -> dict:
    """Configs 0-2 on the host cores, median of up to 100 calls each: the oracle's tokenize + pack
    (fp32, B = 32, E_b ~ U{128..512}), the masked attention of config 1 in fp32 (torch's SDPA with
    the key-padding mask, the library routine the oracle is pinned against) and the oracle's
    RMSNorm + linear at M = 8192, K = 512 on the dequantised INT8 weight (fp32)."""
    from oracle import cortex_oracle as O

    rng = np.random.default_rng(0)
    B, D = 32, 512
    counts = rng.integers(128, 513, B)
    E = int(counts.sum())
    nid, tb, val = rng.integers(0, 137, E), rng.integers(0, 600, E), np.clip(rng.poisson(1.0, E) + 1, 0, 7)
    bidx = np.repeat(np.arange(B), counts)
    tabs = [rng.normal(0, 0.02, (n, D)).astype(np.float32) for n in (137, 600, 8)]
    out = {}
    ms, n = _median_ms(lambda: O.pack_events(O.tokenize(*tabs, nid, tb, val), bidx))
    out["tokenize_pack_fp32"] = {"ms": ms, "calls": n, "events": E}
    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(B, 8, m, 64, generator=g) / 8 for m in (256, 512, 512))
    lens = torch.from_numpy(rng.integers(128, 513, B))
    keep = (torch.arange(512)[None, :] < lens[:, None])[:, None, None, :]
    ms, n = _median_ms(lambda: torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=keep))
    out["sparse_cross_attention_fp32"] = {"ms": ms, "calls": n}
    x = torch.randn(8192, 512, generator=g).bfloat16()
    gam = 1 + 0.02 * torch.randn(512, generator=g)
    for width in (1536, 2048, 512):
        qw, sc = O.quantize_int8((0.02 * torch.randn(width, 512, generator=g)).numpy())
        w_kn = torch.from_numpy(O.dequantize(qw, sc)).t().contiguous()
        ms, n = _median_ms(lambda: O.rms_norm_linear(x, gam, w_kn))
        out[f"norm_linear_int8_n{width}"] = {"ms": ms, "calls": n}
    return out


# --------------------------------------------------------------------------- modes


def run_kernel_only(name: str, iters: int) -> int:
    dev = torch.device("cuda:0")
    fn, _, _, _, _, label = make_kernel(name, dev)
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    sec = time_launches(fn, iters, reps=3)
    print(f"{name}: {label}: {sec * 1e6:.2f} us/launch over {3 * iters} graph-replayed launches", flush=True)
    return 0


def run_copy_calibration(iters: int) -> int:
    dev = torch.device("cuda:0")
    n = 64 << 20
    a = torch.ones(n, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    for _ in range(iters):
        b.copy_(a)
    torch.cuda.synchronize()
    print(f"copy: {iters} x {n} bytes read + {n} bytes written", flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--latency-requests", type=int, default=1000)
    ap.add_argument("--quick", action="store_true", help="skip latency, sweep, breakdown and CPU baseline")
    ap.add_argument("--kernel", choices=KERNELS + API_WORKLOADS,
                    help="launch one hot kernel (or one API workload) only, for profiling")
    ap.add_argument("--copy-calibration", action="store_true", help="64 MiB copies only (PMC calibration)")
    ap.add_argument("--iters", type=int, default=20)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: the Cortex forward is measured per GPU (got --gpus {args.gpus}); "
              "multi-GPU sharding is by batch and is not run here", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    if args.kernel:
        return run_kernel_only(args.kernel, args.iters)
    if args.copy_calibration:
        return run_copy_calibration(args.iters)
    dev = torch.device("cuda:0")
    from cortex.runtime import CapturedForward

    log("bench: building CORTEX_S INT8 model")
    model, scales = build_model(dev, with_scales=True)
    B, per = B_MAIN, PER_MAIN
    inputs = [torch.from_numpy(a).to(dev) for a in make_events(B, per, seed=0)]
    # the graph reads the resident event buffers in place (no staging copies in a step)
    cap = CapturedForward(model, batch_size=B, n_events=B * per, inputs=tuple(inputs))
    log("bench: graph captured; warmup")

    def timed_steps() -> float:  # W untimed replays, then K timed ones: seconds for the K
        for _ in range(args.warmup):
            cap()
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        for _ in range(args.steps):
            cap()
        torch.cuda.synchronize(dev)
        return time.perf_counter() - t0

    # The first few dozen replays of a fresh process run while the GPU clocks are still
    # ramping up (a short run is up to 4 % slower there).  They are timed and reported as
    # `cold_start`; the headline is timed after the eager forward and the kernel timings below
    # have brought the clocks up, with the same W + K protocol.
    cold_ms = timed_steps() / args.steps * 1e3
    log(f"bench: cold start {cold_ms:.4f} ms/step")

    with torch.no_grad():  # eager (no graph) forward, for reference
        for _ in range(3):
            model(*inputs, batch_size=B)
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        for _ in range(10):
            model(*inputs, batch_size=B)
        torch.cuda.synchronize(dev)
    eager_ms = (time.perf_counter() - t0) / 10 * 1e3

    kern = kernel_rooflines(dev)
    dominant = max(kern, key=lambda k: kern[k]["avg_us"] * kern[k]["launches_per_forward"])
    roof = roofline_of(dominant, kern[dominant])
    log(f"bench: dominant kernel {dominant}: {roof['avg_us']} us, {roof['achieved']} {roof['unit']}")

    elapsed = timed_steps()
    ms_step = elapsed / args.steps * 1e3
    value = B * args.steps / elapsed
    log(f"bench: {ms_step:.4f} ms/step, {value:.1f} samples/s")
    extra = {}
    if not args.quick:
        with torch.no_grad():
            extra["sections_ms"] = section_breakdown(model, inputs, dev, ms_step)
        log(f"bench: sections {extra['sections_ms']}")
        extra["latency_b1"] = latency_b1(model, dev, args.latency_requests)
        log(f"bench: latency {extra['latency_b1']}")
        extra["serving_sweep"] = serving_sweep(model, dev)
        log(f"bench: serving {extra['serving_sweep']}")
        extra["serve_worker"] = worker_latency(model, dev, args.latency_requests)
        log(f"bench: serve worker {extra['serve_worker']}")
        extra["streaming"] = streaming_windows(model, dev)
        log(f"bench: streaming {extra['streaming']}")
        extra["norm_linear_api"] = norm_linear_api(dev)
        log(f"bench: norm + linear API {extra['norm_linear_api']}")
        extra["api_configs"] = api_configs(dev)
        log(f"bench: API configurations {extra['api_configs']}")
        extra["w8a8"] = w8a8_forward(model, scales, dev, inputs, cap(*inputs).clone())
        log(f"bench: w8a8 {extra['w8a8']}")
        try:
            extra["weights"] = weights_and_modes(model, dev, inputs, cap(*inputs).clone())
        except Exception as e:  # a secondary line: never lose the headline for it
            extra["weights"] = {"error": f"{type(e).__name__}: {e}"}
        log(f"bench: weights and modes {extra['weights']}")
    # the same replay once the clocks have settled (after every other GPU measurement)
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for _ in range(200):
        cap()
    torch.cuda.synchronize(dev)
    steady_ms = (time.perf_counter() - t0) / 200 * 1e3
    log(f"bench: steady state {steady_ms:.4f} ms/step")
    cpu = None
    if not (args.no_cpu_baseline or args.quick):
        log("bench: CPU baseline")
        cpu = cpu_baseline(model)
    from oracle.cortex_oracle import CORTEX_S_SHAPE, flops_per_sample

    fwd_flops = B * flops_per_sample(CORTEX_S_SHAPE, per)
    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "samples/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "cortex_s_int8_forward_b32x512", "model": "CORTEX_S (random init, seed 0, INT8 "
                   "per-channel)", "batch": B, "events_per_sample": per,
                   "compute": "bf16 MFMA, fp32 accumulate, fp32 residual", "graph": "hip graph replay"},
        # algorithmic rate: the reference forward's FLOPs (including the batch-invariant latent
        # q projection and the behaviour kv projection, which this forward folds away) per step
        "forward_tflops_algorithmic": round(fwd_flops / (ms_step * 1e-3) / 1e12, 2),
        "forward_mfma_frac_algorithmic": round(fwd_flops / (ms_step * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
        "eager_ms_per_forward": round(eager_ms, 4),
        "cold_start": {"ms_per_step": round(cold_ms, 4), "samples_per_s": round(B / cold_ms * 1e3, 2),
                       "when": "W warmup + K timed replays right after the graph capture, while the GPU "
                               "clocks ramp up; value above repeats W + K after the kernel timings"},
        "steady_state": {"ms_per_step": round(steady_ms, 4), "samples_per_s": round(B / steady_ms * 1e3, 2),
                         "steps": 200, "when": "200 replays after every other GPU measurement of this run"},
        "roofline": roof, "kernels": kern, "cpu_baseline": cpu, **extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
