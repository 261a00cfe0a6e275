"""Write the golden fixtures for the GOAP quantized-linear path.

Run ONLY in the build container, where the reference source tree is mounted
at /root/reference (it does not exist on the GPU box). The reference package's
own ``__init__`` pulls in ``zstandard`` (absent here), so the four modules on
the path (codec, triton_kernels, modules) are loaded under a synthetic parent
package whose ``__path__`` points at the reference directory.

Outputs (all small, committed under tests/golden/):
  * ``nf_codebooks.npz``   - the NF 2/4/8-bit codebooks as the reference builds them
                             (codec.py:273-317).
  * ``cases/<name>.npz``   - full arrays for small shapes: inputs, every
                             ``QuantizedTensor`` field (codec.py:453-675), the
                             fp32 and native-dtype ``dequantize_tensor`` outputs
                             (codec.py:761-807), the ``QuantLinear`` buffers built
                             from them (modules.py:294-471) and its CPU forward
                             (modules.py:752-804, 924-940) for bf16 activations.
  * ``digests.json``       - SHA-256 digests and samples of the same arrays at
                             config shapes (2, 4 and 5), where
                             storing full arrays would be too large.

Usage:  python tests/golden/make_golden.py [--small] [--large]
"""
from __future__ import annotations

import argparse
import hashlib
import importlib
import json
import os
import sys
import time
import types

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import recipes  # noqa: E402

REF_DIR = "/root/reference"


def load_reference():
    pkg = types.ModuleType("_tsref")
    pkg.__path__ = [REF_DIR]
    sys.modules["_tsref"] = pkg
    codec = importlib.import_module("_tsref.codec")
    modules = importlib.import_module("_tsref.modules")
    return codec, modules


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def qt_arrays(qt) -> dict:
    out = {}
    for f in ("packed", "scale", "gmin", "outlier_idx", "outlier_val",
              "dq_scale_codes", "dq_scale_meta", "dq_gmin_codes", "dq_gmin_meta",
              "codebook", "stage2_packed", "stage2_scale", "stage2_gmin"):
        v = getattr(qt, f)
        if v is not None:
            out[f] = np.ascontiguousarray(v)
    return out


def qt_meta(qt) -> dict:
    return dict(bits=qt.bits, group_size=qt.group_size, rows=qt.rows, cols=qt.cols,
                padded_cols=qt.padded_cols, n_groups=qt.n_groups, orig_dtype=qt.orig_dtype)


def make_weight(spec: dict) -> torch.Tensor:
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


def qopts(spec: dict) -> dict:
    return dict(bits=spec["bits"], group_size=spec["gs"], outlier_frac=spec["frac"],
                double_quant=spec.get("dq", False), nf_quant=spec.get("nf", False),
                companded=spec.get("lm", False))


# Small cases: full arrays are stored. Shapes cover the partial_sort and the
# nth_element top-k regimes, ties at the threshold, group padding, every
# bit-width, DQ on/off, NF/Lloyd-Max/uniform grids and three input dtypes.
SMALL_CASES = [
    dict(name="u4_g128", kind="gauss", rows=64, cols=512, seed=11, bits=4, gs=128, frac=0.002),
    dict(name="nf4_dq_g128", kind="gauss", rows=96, cols=1024, seed=12, bits=4, gs=128, frac=0.001, dq=True, nf=True),
    dict(name="nf4_dq_g64", kind="gauss", rows=80, cols=384, seed=13, bits=4, gs=64, frac=0.004, dq=True, nf=True),
    dict(name="u2_g64", kind="gauss", rows=64, cols=256, seed=14, bits=2, gs=64, frac=0.01),
    dict(name="nf2_dq_g64", kind="gauss", rows=64, cols=512, seed=15, bits=2, gs=64, frac=0.001, dq=True, nf=True),
    dict(name="lm2_dq_g64", kind="student", rows=96, cols=512, seed=16, bits=2, gs=64, frac=0.001, dq=True, lm=True,
         manual_seed=4242),
    dict(name="lm2_big_g64", kind="student", rows=640, cols=512, seed=17, bits=2, gs=64, frac=0.001, dq=True, lm=True,
         manual_seed=777),
    dict(name="lm4_g128", kind="gauss", rows=64, cols=512, seed=18, bits=4, gs=128, frac=0.001, lm=True,
         manual_seed=99),
    dict(name="u8_g128", kind="gauss", rows=48, cols=512, seed=19, bits=8, gs=128, frac=0.001),
    dict(name="nf8_dq_g128", kind="gauss", rows=64, cols=768, seed=20, bits=8, gs=128, frac=0.001, dq=True, nf=True),
    dict(name="rvq6_dq_g128", kind="gauss", rows=64, cols=512, seed=21, bits=6, gs=128, frac=0.002, dq=True),
    dict(name="rvq6_g64", kind="gauss", rows=32, cols=256, seed=22, bits=6, gs=64, frac=0.002),
    dict(name="ties_u4_g64", kind="ties", rows=128, cols=256, seed=23, bits=4, gs=64, frac=0.003),
    dict(name="ties_nth_u4", kind="ties", rows=64, cols=128, seed=24, bits=4, gs=64, frac=0.05),
    dict(name="nth_nf4_dq", kind="gauss", rows=32, cols=256, seed=25, bits=4, gs=128, frac=0.03, dq=True, nf=True),
    dict(name="pad_u4_g64", kind="gauss", rows=24, cols=200, seed=26, bits=4, gs=64, frac=0.005),
    dict(name="pad_nf4_dq_g128", kind="gauss", rows=40, cols=300, seed=27, bits=4, gs=128, frac=0.005, dq=True, nf=True),
    dict(name="pad_u2_g32", kind="gauss", rows=16, cols=100, seed=28, bits=2, gs=32, frac=0.01),
    dict(name="bf16_nf4_dq", kind="gauss", rows=64, cols=512, seed=29, bits=4, gs=128, frac=0.002, dq=True, nf=True,
         dtype="bfloat16"),
    dict(name="fp32_u4", kind="gauss", rows=32, cols=256, seed=30, bits=4, gs=64, frac=0.002, dtype="float32"),
    dict(name="nofrac_nf4", kind="gauss", rows=32, cols=256, seed=31, bits=4, gs=128, frac=0.0, nf=True),
    dict(name="u4_dq_g128_bias", kind="gauss", rows=64, cols=256, seed=32, bits=4, gs=128, frac=0.002, dq=True,
         bias=True),
]

# Config-scale cases: digests and samples only.
LARGE_CASES = [
    dict(name="cfg1_nf4_dq_4096x4096", kind="gauss", rows=4096, cols=4096, seed=1000, bits=4, gs=128, frac=0.001,
         dq=True, nf=True),
    dict(name="cfg2_lm2_dq_11008x4096", kind="student", rows=11008, cols=4096, seed=2000, bits=2, gs=64,
         frac=0.001, dq=True, lm=True, manual_seed=2024),
    dict(name="cfg4_nf8_dq_14336x4096", kind="gauss", rows=14336, cols=4096, seed=1004, bits=8, gs=128, frac=0.001,
         dq=True, nf=True),
    dict(name="cfg4_rvq6_dq_14336x4096", kind="gauss", rows=14336, cols=4096, seed=1005, bits=6, gs=128,
         frac=0.001, dq=True),
    dict(name="cfg5_u4_28672x8192", kind="gauss", rows=28672, cols=8192, seed=5004, sigma=0.015, bits=4, gs=128,
         frac=0.001),
    dict(name="cfg5_nf4_dq_28672x8192", kind="gauss", rows=28672, cols=8192, seed=5004, sigma=0.015, bits=4,
         gs=128, frac=0.001, dq=True, nf=True),
    dict(name="cfg2_lm2_g64_11008x4096", kind="student", rows=11008, cols=4096, seed=2000, bits=2, gs=64,
         frac=0.001, lm=True, manual_seed=2024),
]
# Every other layer the config-scale forward tests use, so that each one's
# reference weight (dequantize_tensor) is pinned by a digest.
_NF4 = dict(bits=4, gs=128, frac=0.001, dq=True, nf=True)
_NF8 = dict(bits=8, gs=128, frac=0.001, dq=True, nf=True)
_RVQ6 = dict(bits=6, gs=128, frac=0.001, dq=True)
_LLAMA8B = dict(q=(4096, 4096), k=(1024, 4096), v=(1024, 4096), o=(4096, 4096), gate=(14336, 4096),
                up=(14336, 4096), down=(4096, 14336))
_LLAMA70B = dict(q=(8192, 8192), k=(1024, 8192), v=(1024, 8192), o=(8192, 8192), gate=(28672, 8192),
                 up=(28672, 8192), down=(8192, 28672))
# BASELINE config 5's bit-width mix: attention 8-bit, MLP 4-bit, down 2-bit companded
_CFG5 = dict(q=_NF8, k=_NF8, v=_NF8, o=_NF8, gate=_NF4, up=_NF4,
             down=dict(bits=2, gs=64, frac=0.001, dq=True, lm=True, manual_seed=7))
for _i, (_n, (_r, _c)) in enumerate(_LLAMA8B.items()):
    if _i > 0:  # layer 0 (q, seed 1000) is cfg1 above
        LARGE_CASES.append(dict(name=f"cfg3_{_n}_nf4_dq_{_r}x{_c}", kind="gauss", rows=_r, cols=_c, seed=1000 + _i,
                                **_NF4))
for _i, _n in ((4, "gate"), (5, "up"), (6, "down")):
    _r, _c = _LLAMA8B[_n]
    if _i != 4:
        LARGE_CASES.append(dict(name=f"cfg4_{_n}_nf8_dq_{_r}x{_c}", kind="gauss", rows=_r, cols=_c, seed=1000 + _i,
                                **_NF8))
    if _i != 5:
        LARGE_CASES.append(dict(name=f"cfg4_{_n}_rvq6_dq_{_r}x{_c}", kind="gauss", rows=_r, cols=_c,
                                seed=1000 + _i, **_RVQ6))
for _i, (_n, (_r, _c)) in enumerate(_LLAMA70B.items()):
    LARGE_CASES.append(dict(name=f"cfg5_{_n}_{_r}x{_c}", kind="gauss", rows=_r, cols=_c, seed=5100 + _i,
                            sigma=0.015, **_CFG5[_n]))


def run_case(codec, modules, spec: dict, full: bool):
    w = make_weight(spec)
    if spec.get("lm"):
        torch.manual_seed(spec["manual_seed"])
    t0 = time.time()
    qt = codec.quantize_tensor(w, **qopts(spec))
    t_q = time.time() - t0
    arrays = qt_arrays(qt)
    meta = qt_meta(qt)
    deq32 = codec.dequantize_tensor(qt, dtype=torch.float32).numpy()
    deq_native = codec.dequantize_tensor(qt)
    rel = codec.relative_error(w, qt)
    res = dict(meta=meta, spec=spec, rel_error=rel, quantize_seconds=t_q)
    ql = None
    if qt.bits in (2, 4, 8):
        bias = None
        if spec.get("bias"):
            g = torch.Generator().manual_seed(spec["seed"] + 500)
            bias = (torch.randn(qt.rows, generator=g) * 0.1).to(w.dtype)
        ql = modules.QuantLinear(qt, bias, use_triton=False)
    if full:
        out = {f"w_{spec.get('dtype', 'float16')}": w.view(torch.int16 if w.element_size() == 2 else torch.int32).numpy()}
        out.update({f"qt_{k}": v for k, v in arrays.items()})
        out["deq_f32"] = deq32
        out["deq_native"] = deq_native.view(torch.int16 if deq_native.element_size() == 2 else torch.int32).numpy()
        if ql is not None:
            out["ql_outlier_row"] = ql.outlier_row.numpy()
            out["ql_outlier_col"] = ql.outlier_col.numpy()
            out["ql_outlier_delta"] = ql.outlier_delta.numpy()
            sc, gm = ql._get_scale_gmin()
            out["ql_scale_f32"] = sc.numpy()
            out["ql_gmin_f32"] = gm.numpy()
            if ql.bias is not None:
                out["ql_bias"] = ql.bias.view(torch.int16).numpy()
            for m in (1, 3, 17):
                x = recipes.activations(m, qt.cols, seed=7 + m)
                with torch.no_grad():
                    y = ql(x)
                out[f"x_m{m}"] = x.view(torch.int16).numpy()
                out[f"y_cpu_m{m}"] = y.view(torch.int16).numpy()
        return res, out
    # digest mode
    dig = {k: sha(v) for k, v in arrays.items()}
    dig["deq_f32"] = sha(deq32)
    dig["deq_native"] = sha(deq_native.view(torch.int16).numpy())
    res["digests"] = dig
    res["outlier_idx_head"] = arrays["outlier_idx"][:64].tolist()
    res["outlier_idx_tail"] = arrays["outlier_idx"][-64:].tolist()
    res["outlier_val_head_bits"] = arrays["outlier_val"][:64].view(np.uint16).tolist()
    res["n_outliers"] = int(arrays["outlier_idx"].shape[0])
    res["packed_row0_head"] = arrays["packed"][0, :32].tolist()
    res["packed_rowlast_tail"] = arrays["packed"][-1, -32:].tolist()
    if "codebook" in arrays:
        res["codebook_bits"] = arrays["codebook"].view(np.uint16 if arrays["codebook"].dtype == np.float16
                                                       else np.uint32).tolist()
    if ql is not None:
        res["ql_digests"] = dict(outlier_row=sha(ql.outlier_row.numpy()), outlier_col=sha(ql.outlier_col.numpy()),
                                 outlier_delta=sha(ql.outlier_delta.numpy()))
    return res, None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--small", action="store_true")
    ap.add_argument("--large", action="store_true")
    ap.add_argument("--only", default=None, help="comma-separated case names")
    ap.add_argument("--missing", action="store_true", help="large cases without a digest yet")
    args = ap.parse_args()
    if not (args.small or args.large):
        args.small = True
    codec, modules = load_reference()
    versions = dict(torch=torch.__version__, numpy=np.__version__)
    try:
        import scipy
        versions["scipy"] = scipy.__version__
    except Exception:
        pass
    if args.small:
        cb = {f"nf{b}": codec._get_nf_codebook(b) for b in (2, 4, 8)}
        np.savez(os.path.join(HERE, "nf_codebooks.npz"), **cb)
        os.makedirs(os.path.join(HERE, "cases"), exist_ok=True)
        index = {}
        for spec in SMALL_CASES:
            if args.only and spec["name"] != args.only:
                continue
            res, out = run_case(codec, modules, spec, full=True)
            np.savez_compressed(os.path.join(HERE, "cases", spec["name"] + ".npz"), **out)
            index[spec["name"]] = res
            print("small", spec["name"], res["meta"], f"rel={res['rel_error']:.4f}", flush=True)
        index_path = os.path.join(HERE, "cases", "index.json")
        old = json.load(open(index_path)) if (args.only and os.path.exists(index_path)) else {}
        old.update(index)
        json.dump(dict(old, _versions=versions), open(index_path, "w"), indent=1, sort_keys=True)
    if args.large:
        path = os.path.join(HERE, "digests.json")
        dig = json.load(open(path)) if os.path.exists(path) else {}
        only = set(args.only.split(",")) if args.only else None
        for spec in LARGE_CASES:
            if only and spec["name"] not in only:
                continue
            if args.missing and spec["name"] in dig:
                continue
            t0 = time.time()
            res, _ = run_case(codec, modules, spec, full=False)
            dig[spec["name"]] = res
            dig["_versions"] = versions
            json.dump(dig, open(path, "w"), indent=1, sort_keys=True)
            print("large", spec["name"], f"{time.time() - t0:.1f}s", f"rel={res['rel_error']:.4f}", flush=True)


if __name__ == "__main__":
    main()
