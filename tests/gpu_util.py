"""Shared helpers for the GPU tests."""
from __future__ import annotations

import hashlib
import sys

import numpy as np
import torch

import recipes


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def weight_for(spec):
    kind = spec["kind"]
    dt = getattr(torch, spec.get("dtype", "float16"))
    if kind == "gauss":
        return recipes.gaussian_weight(spec["rows"], spec["cols"], spec["seed"], sigma=spec.get("sigma", 0.02),
                                       outlier_frac=spec.get("hot", 0.001), dtype=dt)
    if kind == "student":
        return recipes.student_t_weight(spec["rows"], spec["cols"], spec["seed"], dtype=dt)
    if kind == "ties":
        return recipes.tie_heavy_weight(spec["rows"], spec["cols"], spec["seed"], dtype=dt)
    raise ValueError(kind)


def qt_from_golden(d, res):
    """The reference's QuantizedTensor, rebuilt from a golden fixture."""
    import tensorshrink_amd as ts
    m = res["meta"]
    f = {k[3:]: d[k] for k in d.files if k.startswith("qt_")}
    return ts.QuantizedTensor(orig_shape=(m["rows"], m["cols"]), orig_dtype=m["orig_dtype"], bits=m["bits"],
                              group_size=m["group_size"], rows=m["rows"], cols=m["cols"],
                              padded_cols=m["padded_cols"], n_groups=m["n_groups"], packed=f["packed"],
                              scale=f["scale"], gmin=f["gmin"], outlier_idx=f["outlier_idx"],
                              outlier_val=f["outlier_val"], dq_scale_codes=f.get("dq_scale_codes"),
                              dq_scale_meta=f.get("dq_scale_meta"), dq_gmin_codes=f.get("dq_gmin_codes"),
                              dq_gmin_meta=f.get("dq_gmin_meta"), codebook=f.get("codebook"),
                              stage2_packed=f.get("stage2_packed"), stage2_scale=f.get("stage2_scale"),
                              stage2_gmin=f.get("stage2_gmin"))


def max_rel_err(y, y_ref) -> float:
    """max |y - y_ref| / max |y_ref| (the path's GEMM tolerance metric)."""
    y = y.double()
    y_ref = y_ref.double()
    return float((y - y_ref).abs().max() / y_ref.abs().max().clamp_min(1e-30))
