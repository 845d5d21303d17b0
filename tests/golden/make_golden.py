"""Write the model-level golden vectors under tests/golden/.

This script is the ONLY place that imports the upstream reference package, and it
runs only in the build container where the reference checkout exists (default
``/root/reference``, override with ``CORTEX_REFERENCE_ROOT``).  It pins the three
things that no closed form can pin:

1. the RNG consumption order of ``CortexModel.__init__`` under ``torch.manual_seed``
   (reference cortex/models/cortex.py:82-88, tokenizer.py:42-54,
   perceiver.py:38-52,88-105,132-143, cortex.py:18-27) -- stored as per-tensor
   checksums of the seeded state_dict;
2. the end-to-end composition of ``CortexModel.forward`` in fp32
   (reference cortex/models/cortex.py:90-122) -- stored as ``behavior`` outputs;
3. the INT8 model produced by attach_calibration_hooks -> derive_scales ->
   convert_model (reference cortex/quantization/calibrate.py:99-279) and its
   forward with fp32 activations -- stored as per-layer int8/scale checksums and
   ``behavior`` outputs;
4. the ``return_aux`` output ``masked_spike_logits`` (reference cortex/models/cortex.py:
   56-69,119-120) of both models, whose ``masked_spike_head.proj`` stays float because
   calibration forwards never call that head.

Outputs are data only (inputs and expected outputs); no reference source is copied.
"""

from __future__ import annotations

import json
import os
import sys
from pathlib import Path

import numpy as np
import torch

REF_ROOT = Path(os.environ.get("CORTEX_REFERENCE_ROOT", "/root/reference"))
OUT = Path(__file__).resolve().parent


def _checksum(t: torch.Tensor) -> dict:
    a = t.detach().cpu()
    if a.dtype.is_floating_point:
        a64 = a.double()
        return {
            "shape": list(a.shape),
            "dtype": str(a.dtype),
            "sum": float(a64.sum()),
            "abs_sum": float(a64.abs().sum()),
            "sq_sum": float((a64 * a64).sum()),
            "head": [float(x) for x in a.flatten()[:8].tolist()],
        }
    a64 = a.long()
    return {
        "shape": list(a.shape),
        "dtype": str(a.dtype),
        "sum": int(a64.sum()),
        "abs_sum": int(a64.abs().sum()),
        "sq_sum": int((a64 * a64).sum()),
        "head": [int(x) for x in a.flatten()[:8].tolist()],
    }


def make_inputs(rng: np.random.Generator, counts: list[int], shuffle: bool) -> dict:
    n = int(sum(counts))
    nid = rng.integers(0, 137, size=n, dtype=np.int64)
    tb = rng.integers(0, 600, size=n, dtype=np.int64)
    val = np.clip(rng.poisson(1.0, size=n) + 1, 0, 7).astype(np.int64)
    bidx = np.concatenate([np.full(c, b, dtype=np.int64) for b, c in enumerate(counts)])
    if shuffle:
        perm = rng.permutation(n)
        nid, tb, val, bidx = nid[perm], tb[perm], val[perm], bidx[perm]
    return {"neuron_ids": nid, "time_bins": tb, "values": val, "batch_indices": bidx}


def main() -> None:
    sys.path.insert(0, str(REF_ROOT))
    torch.set_num_threads(1)
    from cortex.models.config import CORTEX_S, CORTEX_XS  # noqa: E402
    from cortex.models.cortex import CortexModel  # noqa: E402
    from cortex.quantization.calibrate import (  # noqa: E402
        attach_calibration_hooks,
        convert_model,
        derive_scales,
        remove_calibration_hooks,
    )

    meta: dict = {"torch": torch.__version__, "cases": {}}
    arrays: dict[str, np.ndarray] = {}
    rng = np.random.default_rng(20261201)

    for cfg_name, cfg, seed in (("xs", CORTEX_XS, 0), ("s", CORTEX_S, 0)):
        torch.manual_seed(seed)
        model = CortexModel(cfg).eval()
        sd_sums = {k: _checksum(v) for k, v in model.state_dict().items()}

        input_sets = {
            "sorted": make_inputs(rng, [40, 17, 64], shuffle=False),
            "shuffled": make_inputs(rng, [23, 1, 50, 31], shuffle=True),
        }
        case: dict = {"seed": seed, "state_dict": sd_sums, "inputs": {}}

        for iname, inp in input_sets.items():
            t = {k: torch.from_numpy(v) for k, v in inp.items()}
            with torch.no_grad():
                out = model(t["neuron_ids"], t["time_bins"], t["values"], t["batch_indices"], return_aux=True)
            for k, v in inp.items():
                arrays[f"{cfg_name}_{iname}_{k}"] = v
            arrays[f"{cfg_name}_{iname}_behavior_fp32"] = out["behavior"].numpy().astype(np.float32)
            arrays[f"{cfg_name}_{iname}_aux_fp32"] = out["masked_spike_logits"].numpy().astype(np.float32)
            case["inputs"][iname] = {"n_events": int(inp["neuron_ids"].shape[0])}

        # INT8: one calibration forward on the "sorted" inputs, then convert.
        hooks = attach_calibration_hooks(model)
        t = {k: torch.from_numpy(v) for k, v in input_sets["sorted"].items()}
        with torch.no_grad():
            model(t["neuron_ids"], t["time_bins"], t["values"], t["batch_indices"])
        remove_calibration_hooks(hooks)
        scales = derive_scales(model, hooks)
        qmodel = convert_model(model, scales, inplace=False).eval()
        qsd = qmodel.state_dict()
        case["int8_state_dict"] = {
            k: _checksum(v) for k, v in qsd.items() if k.endswith(("weight_int8", "weight_scale"))
        }
        case["n_quantized"] = len(scales)
        for iname, inp in input_sets.items():
            t = {k: torch.from_numpy(v) for k, v in inp.items()}
            with torch.no_grad():
                out = qmodel(t["neuron_ids"], t["time_bins"], t["values"], t["batch_indices"], return_aux=True)
            arrays[f"{cfg_name}_{iname}_behavior_int8"] = out["behavior"].numpy().astype(np.float32)
            arrays[f"{cfg_name}_{iname}_aux_int8"] = out["masked_spike_logits"].numpy().astype(np.float32)

        # Exact int8 rows of a few layers (small slices) so a one-off rounding slip shows.
        for key in (
            "encoder.cross_attn.q_proj.weight_int8",
            "encoder.self_attn_blocks.0.mlp.2.weight_int8",
            "behavior_head.out_proj.weight_int8",
        ):
            arrays[f"{cfg_name}_slice_{key}"] = qsd[key][:2].numpy().copy()
        for key in (
            "encoder.cross_attn.q_proj.weight_scale",
            "behavior_head.out_proj.weight_scale",
        ):
            arrays[f"{cfg_name}_slice_{key}"] = qsd[key][:16].numpy().copy()

        meta["cases"][cfg_name] = case

    np.savez_compressed(OUT / "model_golden.npz", **arrays)
    (OUT / "model_golden.json").write_text(json.dumps(meta, indent=1, sort_keys=True))
    print("wrote", OUT / "model_golden.npz", OUT / "model_golden.json")


if __name__ == "__main__":
    main()
