"""Cortex-S INT8 inference forward on one MI355X: samples/s at B=32 x 512 events,
p50/p99 latency at B=1, the dominant kernel's roofline fraction, and the CPU
oracle timed on the host cores.

A step is one forward of the fixed workload (CORTEX_S, weights quantised to INT8
per channel on the GPU, bf16 MFMA with fp32 accumulation, B = 32 samples x 512
synthetic events) replayed from a HIP graph; its inputs are already resident in
HBM and are copied into the graph's input buffers inside the step.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
Prints exactly one JSON line on stdout.
"""

from __future__ import annotations

import argparse
import json
import os
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


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def make_events(batch: int, per_sample: int, seed: int):
    """Synthetic spike events: nid U[0,137), time bin U[0,600), value = clip(Poisson(1)+1, 0, 7)."""
    rng = np.random.default_rng(seed)
    E = batch * per_sample
    return (rng.integers(0, 137, E), rng.integers(0, 600, E), np.clip(rng.poisson(1.0, E) + 1, 0, 7),
            np.repeat(np.arange(batch), per_sample))


def build_model(dev):
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
    return convert_model(model, derive_scales(model, hooks), inplace=True)


def time_dominant_kernel(model, dev, iters: int = 50):
    """Average duration of the MLP-up GEMM as the forward runs it (bf16 LayerNorm rows x the
    int8 weight's bf16 image, 2048x512, per-channel scale + GELU epilogue, bf16 out) at
    M = 32*256 rows, timed with HIP events on the stream it is launched on."""
    from cortex.kernels import ops
    from cortex.models._layers import exec_weights

    blk = model.encoder.self_attn_blocks[0]
    M, K, N = 32 * 256, 512, 2048
    x = torch.randn(M, K, device=dev).bfloat16()
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    w = exec_weights(blk.mlp[0], torch.bfloat16)

    def launch():
        ops.norm_linear(x, **w, act="gelu", out_dtype=torch.bfloat16, compute_dtype=torch.bfloat16, out=out)

    for _ in range(5):
        launch()
    stream = torch.cuda.current_stream(dev)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(dev)
    t0.record(stream)
    for _ in range(iters):
        launch()
    t1.record(stream)
    t1.synchronize()
    sec = t0.elapsed_time(t1) / 1e3 / iters
    flops = 2.0 * M * N * K
    achieved = flops / sec / 1e12
    return {"bound": "mfma", "achieved": round(achieved, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / BF16_PEAK_TFLOPS, 4), "traffic": None,
            "kernel": "gemm_pipe_kernel (bf16 x bf16-image of int8 W, scale + GELU -> bf16), M=8192 K=512 N=2048",
            "avg_us": round(sec * 1e6, 2), "flops_per_launch": flops}


def section_breakdown(model, inputs, dev, iters: int = 20):
    """Per-section GPU time (ms) of one eager forward, mirroring the reference profiler's sections."""
    from cortex.kernels import ops
    from cortex.models._layers import apply_linear

    nid, tb, val, bidx = inputs
    B, cfg = 32, model.config
    enc, xa, tok = model.encoder, model.encoder.cross_attn, model.tokenizer
    D, L, H = cfg.latent_dim, cfg.num_latents, xa.num_heads
    comp = cfg.compute_dtype
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    times: dict[str, float] = {}

    def timed(name, fn):
        fn()
        a, b = ev(), ev()
        a.record()
        for _ in range(iters):
            r = fn()
        b.record()
        b.synchronize()
        times[name] = round(a.elapsed_time(b) / iters, 4)
        return r

    offsets, order, _ = timed("pack_plan", lambda: ops.pack_plan(bidx, B))
    tokens = timed("tokenizer", lambda: ops.tokenize(tok.neuron_emb.weight, tok.time_emb.weight,
                                                     tok.value_emb.weight, nid, tb, val, order=order,
                                                     csr_offsets=offsets))
    E = tokens.shape[0]

    def cross():
        kv = apply_linear(xa.kv_proj, tokens, norm=xa.norm_kv, out_dtype=comp, compute=comp)
        q = xa.project_queries(enc.latents, comp)
        o_buf, o = ops.merge_heads_out(B, L, H, D // H, comp, dev)
        ops.attention(ops.heads_view(q, 1, L, H), ops.heads_view(kv, 1, E, H, 0, D),
                      ops.heads_view(kv, 1, E, H, D, D), kv_offsets=offsets, out=o, batch=B)
        return apply_linear(xa.out_proj, o_buf, residual=enc.latents, res_rows=L, out_dtype=torch.float32,
                            compute=comp)

    x = timed("cross_attn", cross)
    lat = timed("self_attn_all", lambda: enc.encode_rows(x, B))
    timed("self_attn_single", lambda: enc.self_attn_blocks[0].forward_rows(x, B, L))
    timed("behavior_head", lambda: model.behavior_head.forward_rows(lat, B))
    return times


def latency_b1(model, dev, n_requests: int, per_sample: int = 512):
    """p50/p99 wall latency of B=1 requests: pinned H2D of the events, graph replay, D2H of (1, 2)."""
    from cortex.runtime import CapturedForward

    cap = CapturedForward(model, batch_size=1, n_events=per_sample)
    host = [torch.from_numpy(a).pin_memory() for a in make_events(1, per_sample, seed=7)]
    dev_in = [torch.empty_like(h, device=dev) for h in host]
    out_host = torch.empty((1, 2), dtype=torch.float32).pin_memory()
    lat = []
    for i in range(n_requests + 20):
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        for d, h in zip(dev_in, host):
            d.copy_(h, non_blocking=True)
        out = cap(*dev_in)
        out_host.copy_(out, non_blocking=True)
        torch.cuda.synchronize(dev)
        if i >= 20:
            lat.append((time.perf_counter() - t0) * 1e3)
    lat.sort()
    return {"p50_ms": round(lat[len(lat) // 2], 4), "p99_ms": round(lat[int(len(lat) * 0.99) - 1], 4),
            "requests": n_requests, "events_per_request": per_sample}


def cpu_baseline(model, budget_s: float = 20.0):
    """The CPU oracle (fp32 activations, INT8 weights dequantised as the reference's QuantizedLinear)
    on the host cores: B=32 x 512-event forwards until the time budget is spent."""
    from oracle import cortex_oracle as O

    torch.set_num_threads(os.cpu_count() or 1)
    sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    arrs = make_events(32, 512, seed=0)
    O.forward(sd, O.CORTEX_S_SHAPE, *arrs)  # warm-up
    n, t0 = 0, time.perf_counter()
    while True:
        O.forward(sd, O.CORTEX_S_SHAPE, *arrs)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 30:
            break
    return {"value": round(32 * n / el, 2), "unit": "samples/s", "cores": torch.get_num_threads(),
            "kind": "port", "sample": f"{n} forwards of B=32 x 512 events (CORTEX_S INT8-dequant, fp32) "
                                      f"in {el:.1f} s"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--latency-requests", type=int, default=1000)
    ap.add_argument("--quick", action="store_true", help="skip latency, breakdown and CPU baseline")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: the Cortex forward is measured per GPU (got --gpus {args.gpus}); "
              "multi-GPU sharding is by batch and is not run here", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    from cortex.runtime import CapturedForward

    log("bench: building CORTEX_S INT8 model")
    model = build_model(dev)
    B, per = 32, 512
    inputs = [torch.from_numpy(a).to(dev) for a in make_events(B, per, seed=0)]
    cap = CapturedForward(model, batch_size=B, n_events=B * per)
    log("bench: graph captured; warmup")
    for _ in range(args.warmup):
        cap(*inputs)
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        cap(*inputs)
    torch.cuda.synchronize(dev)
    elapsed = time.perf_counter() - t0
    ms_step = elapsed / args.steps * 1e3
    value = B * args.steps / elapsed
    log(f"bench: {ms_step:.4f} ms/step, {value:.1f} samples/s")

    # eager (no graph) forward time, for reference
    with torch.no_grad():
        for _ in range(3):
            model(*inputs, batch_size=B)
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        for _ in range(10):
            model(*inputs, batch_size=B)
        torch.cuda.synchronize(dev)
    eager_ms = (time.perf_counter() - t0) / 10 * 1e3

    roof = time_dominant_kernel(model, dev)
    log(f"bench: dominant kernel {roof['avg_us']} us, {roof['achieved']} TFLOP/s")
    extra = {}
    if not args.quick:
        with torch.no_grad():
            extra["sections_ms"] = section_breakdown(model, inputs, dev)
        log(f"bench: sections {extra['sections_ms']}")
        extra["latency_b1"] = latency_b1(model, dev, args.latency_requests)
        log(f"bench: latency {extra['latency_b1']}")
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
        "config": {"workload": "cortex_s_int8_forward", "model": "CORTEX_S (random init, seed 0, INT8 per-channel)",
                   "batch": B, "events_per_sample": per, "compute": "bf16 MFMA, fp32 accumulate, fp32 residual",
                   "graph": "hip graph replay"},
        "forward_tflops": round(fwd_flops / (ms_step * 1e-3) / 1e12, 2),
        "eager_ms_per_forward": round(eager_ms, 4),
        "roofline": roof, "cpu_baseline": cpu, **extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
