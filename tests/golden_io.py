"""Loading helpers for the committed golden fixtures (tests only)."""
from __future__ import annotations

import json
import os

import numpy as np
import torch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES_DIR = os.path.join(GOLDEN, "cases")


def case_names():
    idx = json.load(open(os.path.join(CASES_DIR, "index.json")))
    return sorted(k for k in idx if not k.startswith("_"))


def load_case(name):
    idx = json.load(open(os.path.join(CASES_DIR, "index.json")))
    res = idx[name]
    d = np.load(os.path.join(CASES_DIR, name + ".npz"))
    spec = res["spec"]
    dt = spec.get("dtype", "float16")
    raw = d[[k for k in d.files if k.startswith("w_")][0]]
    w = torch.from_numpy(raw).view(getattr(torch, dt))
    return spec, res, d, w


def qopts(spec):
    return dict(bits=spec["bits"], group_size=spec["gs"], outlier_frac=spec["frac"],
                double_quant=spec.get("dq", False), nf_quant=spec.get("nf", False),
                companded=spec.get("lm", False))


def digests():
    return json.load(open(os.path.join(GOLDEN, "digests.json")))


QT_FIELDS = ("packed", "scale", "gmin", "outlier_idx", "outlier_val", "dq_scale_codes", "dq_scale_meta",
             "dq_gmin_codes", "dq_gmin_meta", "codebook", "stage2_packed", "stage2_scale", "stage2_gmin")
