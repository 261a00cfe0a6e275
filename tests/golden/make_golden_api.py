"""Write the golden fixtures for the module-level API: quantize_module,
quantize_module_gpu, QuantLinear.from_linear, quantize_tensor_adaptive, and
quantize_tensor on NaN-bearing weights.

Run ONLY in the build container, where the reference source tree is mounted
at /root/reference (it does not exist on the GPU box); it loads the
reference's codec/modules/gpu_quantize the same way make_golden.py does.

Each scenario runs the reference on recipes.tiny_model() (CPU, fp16) and
records the returned stats dict (per-layer bits, rel_error, escalated, byte
counts, force_fp32_compute) and SHA-256 digests of every replaced layer's
state_dict buffers. quantize_module_gpu runs with device="cpu", where the
reference quantizes through its CPU codec (uniform grid, no double quant, the
CPU top-k order), which is what tensorshrink_amd's GPU codec reproduces.

Output: tests/golden/api_fixtures.json (digests and small arrays only).

Usage:  python tests/golden/make_golden_api.py
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import recipes  # noqa: E402
from make_golden import load_reference  # noqa: E402

SCENARIOS = {
    "qm_default_fp32down": dict(fn="quantize_module", kw=dict(force_fp32_patterns=("down",))),
    "qm_adaptive": dict(fn="quantize_module", kw=dict(adaptive=True, error_threshold=0.09)),
    "qm_adaptive_030": dict(fn="quantize_module", kw=dict(adaptive=True, error_threshold=0.3)),
    "qm_budget": dict(fn="quantize_module", kw=dict(vram_budget_mb=0.45)),
    "qm_u8_nodq": dict(fn="quantize_module", kw=dict(bits=8, double_quant=False, nf_quant=False,
                                                     skip_name_patterns=("embed", "lm_head"))),
    "qmgpu_default": dict(fn="quantize_module_gpu", kw=dict(device="cpu")),
    "qmgpu_adaptive": dict(fn="quantize_module_gpu", kw=dict(device="cpu", adaptive=True, error_threshold=0.09)),
    "qmgpu_budget": dict(fn="quantize_module_gpu", kw=dict(device="cpu", vram_budget_mb=0.5)),
}


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def module_digests(model) -> dict:
    out = {}
    for name, mod in model.named_modules():
        if type(mod).__name__ != "QuantLinear":
            continue
        sd = {}
        for k, v in mod.state_dict().items():
            if v is None:
                continue
            arr = v.detach().cpu()
            raw = arr.view(torch.int16) if arr.dtype in (torch.float16, torch.bfloat16) else arr
            sd[k] = dict(dtype=str(arr.dtype).replace("torch.", ""), shape=list(arr.shape), sha=sha(raw.numpy()))
        out[name] = sd
    return out


def clean_stats(stats: dict) -> dict:
    s = {k: v for k, v in stats.items() if k not in ("cache",)}
    s["layers"] = [dict(l) for l in stats["layers"]]
    return json.loads(json.dumps(s, default=float))


def main():
    codec, modules = load_reference()
    import importlib
    gpu_quantize = importlib.import_module("_tsref.gpu_quantize")
    out = {"_versions": dict(torch=torch.__version__, numpy=np.__version__)}
    for name, sc in SCENARIOS.items():
        model = recipes.tiny_model()
        fn = getattr(modules if sc["fn"] == "quantize_module" else gpu_quantize, sc["fn"])
        stats = fn(model, verbose=False, **sc["kw"])
        out[name] = dict(fn=sc["fn"], kw={k: (list(v) if isinstance(v, tuple) else v) for k, v in sc["kw"].items()},
                         stats=clean_stats(stats), buffers=module_digests(model))
        print(name, [(l["name"], l["bits"], round(l["rel_error"], 5), l["escalated"]) for l in stats["layers"]],
              flush=True)

    # QuantLinear.from_linear on a layer with a bias (defaults: NF4 + double quant)
    model = recipes.tiny_model()
    lin = model.layers[0].up_proj
    ql, err, esc = modules.QuantLinear.from_linear(lin)
    out["from_linear_up0"] = dict(err=err, escalated=esc, bits=ql.bits,
                                  buffers=module_digests(torch.nn.ModuleDict({"ql": ql}))["ql"])

    # quantize_tensor_adaptive with its own defaults (chain 2, 4, 6, 8; no DQ / NF)
    adaptive = {}
    for label, w in (("gauss", recipes.gaussian_weight(256, 512, 41)),
                     ("student", recipes.student_t_weight(256, 512, 42)),
                     ("levels", recipes.tie_heavy_weight(256, 512, 43, levels=2))):
        for thr in (0.05, 0.1, 0.3):
            qt, e, s = codec.quantize_tensor_adaptive(w, error_threshold=thr)
            adaptive[f"{label}_{thr}"] = dict(bits=qt.bits, err=e, escalated=s, packed=sha(qt.packed),
                                              outlier_idx=sha(qt.outlier_idx))
    out["quantize_tensor_adaptive"] = adaptive

    # NaN weights: the outlier threshold (min of the top-k values) is NaN and
    # the clamp turns the whole tensor into NaN, so codes/scale/gmin are what
    # the reference's arithmetic makes of NaN. Small arrays, stored in full.
    nan = {}
    for label, kw in (("u4", dict(bits=4)), ("nf4_dq", dict(bits=4, double_quant=True, nf_quant=True)),
                      ("u8", dict(bits=8)), ("nofrac_u4", dict(bits=4, outlier_frac=0.0))):
        w = recipes.gaussian_weight(16, 256, 44)
        w.view(-1)[[3, 1000, 2047]] = float("nan")
        qt = codec.quantize_tensor(w, group_size=64, **kw)
        rec = {"kw": kw}
        for f in ("packed", "scale", "gmin", "outlier_idx", "outlier_val", "dq_scale_codes", "dq_scale_meta",
                  "dq_gmin_codes", "dq_gmin_meta"):
            v = getattr(qt, f)
            if v is None:
                continue
            v = np.ascontiguousarray(v)
            bits = v.view(np.uint16) if v.dtype == np.float16 else v
            rec[f] = dict(dtype=str(v.dtype), shape=list(v.shape), values=bits.reshape(-1).tolist())
        nan[label] = rec
    out["nan_weights"] = nan

    with open(os.path.join(HERE, "api_fixtures.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
