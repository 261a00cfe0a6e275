"""GPU GOAP quantize / dequantize / QuantLinear construction: bit-exact against
the reference's golden vectors (small shapes) and digests (config shapes)."""
import numpy as np
import pytest
import torch

from golden_io import QT_FIELDS, case_names, digests, load_case, qopts
from gpu_util import qt_from_golden, say, sha, weight_for

pytestmark = pytest.mark.gpu


def _ts():
    import tensorshrink_amd as ts
    return ts


def _quantize(spec, w):
    ts = _ts()
    if spec.get("lm"):
        torch.manual_seed(spec["manual_seed"])
    return ts.quantize_tensor(w, **qopts(spec))


def _assert_fields(qt, d):
    for f in QT_FIELDS:
        key = "qt_" + f
        v = getattr(qt, f)
        if key in d.files:
            assert v is not None, f
            assert v.dtype.itemsize == d[key].dtype.itemsize, f
            assert v.shape == d[key].shape, (f, v.shape, d[key].shape)
            np.testing.assert_array_equal(v.view(np.uint8), d[key].view(np.uint8), err_msg=f)
        else:
            assert v is None, f


@pytest.mark.parametrize("name", case_names())
def test_quantize_matches_golden(name):
    spec, res, d, w = load_case(name)
    say("quantize", name)
    qt = _quantize(spec, w)
    _assert_fields(qt, d)
    m = res["meta"]
    assert (qt.rows, qt.cols, qt.padded_cols, qt.n_groups, qt.bits, qt.orig_dtype) == \
        (m["rows"], m["cols"], m["padded_cols"], m["n_groups"], m["bits"], m["orig_dtype"])


@pytest.mark.parametrize("name", [n for n in case_names()])
def test_quantize_device_input_matches_golden(name):
    spec, res, d, w = load_case(name)
    if spec.get("lm"):
        pytest.skip("Lloyd-Max draws its sample from the input device's RNG, as the reference does")
    qt = _ts().quantize_tensor(w.cuda(), **qopts(spec))
    _assert_fields(qt, d)


@pytest.mark.parametrize("name", case_names())
def test_dequantize_matches_golden(name):
    spec, res, d, w = load_case(name)
    ts = _ts()
    qt = qt_from_golden(d, res)
    deq32 = ts.dequantize_tensor(qt, dtype=torch.float32)
    np.testing.assert_array_equal(deq32.numpy().view(np.uint32), d["deq_f32"].view(np.uint32))
    nat = ts.dequantize_tensor(qt)
    raw = nat.view(torch.int16 if nat.element_size() == 2 else torch.int32).numpy()
    np.testing.assert_array_equal(raw, d["deq_native"])
    assert abs(ts.relative_error(w, qt) - res["rel_error"]) < 1e-5


@pytest.mark.parametrize("name", [n for n in case_names()])
def test_quantlinear_buffers_match_golden(name):
    spec, res, d, w = load_case(name)
    if spec["bits"] == 6:
        pytest.skip("the reference QuantLinear has no 6-bit buffers")
    ts = _ts()
    bias = torch.from_numpy(d["ql_bias"]).view(w.dtype) if "ql_bias" in d.files else None
    ql = ts.QuantLinear(qt_from_golden(d, res), bias)
    for f in ("outlier_row", "outlier_col", "outlier_delta"):
        np.testing.assert_array_equal(getattr(ql, f).cpu().numpy().view(np.uint8), d["ql_" + f].view(np.uint8),
                                      err_msg=f)
    sd = ql.state_dict()
    assert "outlier_row_ptr" not in sd
    assert sd["packed"].dtype == torch.uint8 and sd["outlier_delta"].dtype == torch.float16
    if spec.get("dq"):
        assert "scale" not in sd and sd["dq_scale_meta"].dtype == torch.float16
    else:
        assert sd["scale"].dtype == torch.float16
    # to_quantized_tensor round trip keeps codes and metadata
    q2 = ql.to_quantized_tensor()
    np.testing.assert_array_equal(q2.packed, d["qt_packed"])


@pytest.mark.slow
@pytest.mark.parametrize("name", sorted(k for k in digests() if not k.startswith("_")))
def test_config_scale_digests(name):
    dig = digests()[name]
    spec = dig["spec"]
    say("config digest", name)
    w = weight_for(spec)
    torch.cuda.synchronize()
    qt = _quantize(spec, w)
    assert qt.n_outliers() == dig["n_outliers"]
    assert qt.outlier_idx[:64].tolist() == dig["outlier_idx_head"]
    assert qt.outlier_idx[-64:].tolist() == dig["outlier_idx_tail"]
    for f, h in dig["digests"].items():
        if f in ("deq_f32", "deq_native"):
            continue
        assert sha(getattr(qt, f)) == h, f
    ts = _ts()
    deq = ts.dequantize_tensor(qt, dtype=torch.float32)
    assert sha(deq.numpy()) == dig["digests"]["deq_f32"]
    if "ql_digests" in dig:
        ql = ts.QuantLinear(qt)
        for f, h in dig["ql_digests"].items():
            assert sha(getattr(ql, f).cpu().numpy()) == h, f


@pytest.mark.parametrize("dtype,k", [(torch.float16, 2000), (torch.float32, 2000), (torch.float16, 2)])
def test_topk_outliers_with_nan(dtype, k):
    """NaN weights rank above every number in torch.topk; the device candidate
    filter keeps them and the host replay puts them where torch does."""
    from oracle import codec_ref as O
    from tensorshrink_amd import codec
    g = torch.Generator().manual_seed(k)
    w = torch.randn(512, 4096, generator=g).to(dtype)
    w.view(-1)[[5, 70000, 1500000, 2000000]] = float("nan")
    say("topk nan", dtype, k)
    oi, ov = codec._topk_outliers(w.cuda(), k)
    ov_ref, oi_ref = O.topk_abs(w.float().reshape(-1).numpy(), k)
    np.testing.assert_array_equal(oi, oi_ref)
    np.testing.assert_array_equal(ov, ov_ref)
