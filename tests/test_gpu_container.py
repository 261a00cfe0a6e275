"""The .tsk container with the GPU codec: save_container and
stream_quantize_safetensors_dir write what quantize_tensor_adaptive (pinned to
the reference by the API fixtures) returns for each eligible tensor, and a
quantized model survives save_quant_module -> load_quantized_module with the
same buffers and the same forward output."""
import json

import numpy as np
import pytest
import torch

import recipes
from gpu_util import say

pytestmark = pytest.mark.gpu

SKIP = ("norm", "bias", "position", "shared", "relative_attention_bias")


def _sorted_outliers(qt):
    order = np.argsort(qt.outlier_idx.astype(np.int64) // qt.cols, kind="stable")
    return qt.outlier_idx[order], qt.outlier_val[order]


def _same_qt(a, b):
    assert (a.bits, a.group_size, a.rows, a.cols, a.padded_cols) == (b.bits, b.group_size, b.rows, b.cols,
                                                                     b.padded_cols)
    for f in ("packed", "scale", "gmin", "codebook"):
        x, y = getattr(a, f), getattr(b, f)
        assert (x is None) == (y is None), f
        if x is not None:
            np.testing.assert_array_equal(x.view(np.uint8), y.view(np.uint8), err_msg=f)
    ia, va = _sorted_outliers(a)
    ib, vb = _sorted_outliers(b)
    np.testing.assert_array_equal(ia, ib)
    np.testing.assert_array_equal(va.view(np.uint16), vb.view(np.uint16))


def test_save_container_matches_codec(tmp_path):
    import tensorshrink_amd as ts
    sd = recipes.tiny_model().state_dict()
    say("save_container tiny_model")
    stats = ts.save_container(sd, tmp_path / "m.tsk", error_threshold=0.09)
    bits = {s["name"]: s["bits"] for s in stats["tensors"]}
    with ts.ContainerReader(tmp_path / "m.tsk") as r:
        assert r.names() == list(sd)
        for name, t in sd.items():
            elig = t.dim() >= 2 and t.numel() >= 16384 and not any(p in name.lower() for p in SKIP)
            assert r.kind(name) == ("quant" if elig else "raw"), name
            if not elig:
                assert torch.equal(r.get(name), t)
                continue
            qt, err, esc = ts.quantize_tensor_adaptive(t, error_threshold=0.09, allowed_bits=(2, 4, 8))
            _same_qt(r.get_quantized(name), qt)
            e = r.manifest["tensors"][name]
            assert e["rel_error"] == pytest.approx(err, abs=1e-7) and e["escalated"] == esc
            # the container view dequantizes like the tensor it stores
            ref = ts.dequantize_tensor(qt)
            assert torch.equal(r.get(name).to(ref.dtype), ref)
            assert bits[name] == qt.bits
    assert stats["file_bytes"] < stats["orig_bytes"]


@pytest.mark.parametrize("dq", [False, True])
def test_save_load_quant_module(tmp_path, dq):
    import tensorshrink_amd as ts
    model = recipes.tiny_model()
    ts.quantize_module(model, verbose=False, double_quant=dq, nf_quant=dq, force_fp32_patterns=("down",))
    model = model.cuda()
    say("save_quant_module dq", dq)
    info = ts.save_quant_module(model, tmp_path / "q.tsk", verbose=False)
    fresh = recipes.tiny_model(seed=5).cuda()
    with ts.ContainerReader(tmp_path / "q.tsk") as r:
        got = ts.load_quantized_module(fresh, r, verbose=False)
        man = r.manifest["tensors"]
    qs = {n: m for n, m in model.named_modules() if isinstance(m, ts.QuantLinear)}
    assert info["n_quant"] == len(qs) + sum(m.bias is not None for m in qs.values())
    assert got["n_quant_replaced"] == len(qs)
    for n, q in qs.items():
        l = dict(fresh.named_modules())[n]
        assert isinstance(l, ts.QuantLinear) and l.bits == q.bits
        assert l.force_fp32_compute == ("down" in n) == man[n + ".weight"]["force_fp32_compute"]
        assert torch.equal(l.packed, q.packed)
        if not dq:
            assert torch.equal(l.scale, q.scale) and torch.equal(l.gmin, q.gmin)
            assert torch.equal(l.outlier_row, q.outlier_row) and torch.equal(l.outlier_col, q.outlier_col)
        if q.bias is not None:
            assert torch.equal(l.bias, q.bias)
        x = recipes.activations(7, q.in_features).cuda()
        y0, y1 = q(x).float(), l(x).float()
        w0, w1 = q.dequantize_weight(torch.float32), l.dequantize_weight(torch.float32)
        # DQ layers reload with f16 scale/gmin (the container stores no DQ
        # codes), otherwise the weights are equal up to the outlier deltas'
        # f16 re-rounding
        tol = 2e-2 if dq else 1e-3
        assert float((w0 - w1).abs().max()) <= tol * float(w0.abs().max()), n
        assert float((y0 - y1).abs().max()) <= tol * float(y0.abs().max()), n
    # raw entries (norms, embed, lm_head, small layer) restored exactly
    for n in ("layers.0.input_norm.weight", "lm_head.weight", "embed_tokens.weight", "tiny.weight", "tiny.bias"):
        assert torch.equal(fresh.state_dict()[n].cpu(), model.state_dict()[n].cpu()), n


def _write_checkpoint(d, sd, sharded):
    from safetensors.torch import save_file
    d.mkdir()
    sd = {k: v.contiguous() for k, v in sd.items()}
    if not sharded:
        save_file(sd, str(d / "model.safetensors"))
        return
    keys = list(sd)
    a, b = keys[: len(keys) // 2], keys[len(keys) // 2:]
    save_file({k: sd[k] for k in a}, str(d / "model-00001-of-00002.safetensors"))
    save_file({k: sd[k] for k in b}, str(d / "model-00002-of-00002.safetensors"))
    wm = {k: "model-00001-of-00002.safetensors" for k in a}
    wm.update({k: "model-00002-of-00002.safetensors" for k in b})
    (d / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": wm}))


@pytest.mark.parametrize("sharded,parallel", [(False, True), (True, True), (True, False)])
def test_stream_quantize_safetensors_dir(tmp_path, sharded, parallel):
    import tensorshrink_amd as ts
    sd = recipes.tiny_model().state_dict()
    _write_checkpoint(tmp_path / "ckpt", sd, sharded)
    say("stream_quantize sharded", sharded, "parallel", parallel)
    st = ts.stream_quantize_safetensors_dir(tmp_path / "ckpt", tmp_path / "s.tsk", progress=False,
                                            parallel=parallel, n_workers=2)
    assert st["n_tensors"] == len(sd)
    with ts.ContainerReader(tmp_path / "s.tsk") as r:
        assert sorted(r.names()) == sorted(sd)
        for name, t in sd.items():
            if r.kind(name) == "raw":
                assert torch.equal(r.get(name), t)
                continue
            qt, err, esc = ts.quantize_tensor_adaptive(t, group_size=128, outlier_frac=0.003, error_threshold=0.06,
                                                       allowed_bits=(2, 4, 8))
            _same_qt(r.get_quantized(name), qt)
            assert r.manifest["tensors"][name]["escalated"] == esc


def test_stream_quantize_budget_plan(tmp_path):
    import tensorshrink_amd as ts
    sd = recipes.tiny_model().state_dict()
    _write_checkpoint(tmp_path / "ckpt", sd, False)
    st = ts.stream_quantize_safetensors_dir(tmp_path / "ckpt", tmp_path / "b.tsk", progress=False,
                                            vram_budget_mb=0.5)
    elig = {s["name"]: s["bits"] for s in st["tensors"] if s["bits"] is not None}
    assert elig and set(elig.values()) <= {4, 8}
    with ts.ContainerReader(tmp_path / "b.tsk") as r:
        for name, bits in elig.items():
            qt = ts.quantize_tensor(sd[name], bits=bits, group_size=128, outlier_frac=0.003)
            _same_qt(r.get_quantized(name), qt)
            assert r.manifest["tensors"][name]["escalated"] == (bits == 8)


@pytest.mark.parametrize("opts", [dict(bits=6, group_size=64, outlier_frac=0.002),
                                  dict(bits=2, group_size=64, outlier_frac=0.001, companded=True),
                                  dict(bits=8, group_size=128, outlier_frac=0.0, double_quant=True, nf_quant=True)])
def test_save_load_formats(tmp_path, opts):
    """6-bit RVQ (stage-2 parts stored), companded 2-bit (codebook part) and a
    layer without outliers through save_quant_module -> load_quantized_module:
    the reloaded layer's weights and forward equal the original's."""
    import tensorshrink_amd as ts
    w = recipes.student_t_weight(384, 512, 61)
    lin = torch.nn.Linear(512, 384, bias=True, dtype=torch.float16)
    lin.weight.data = w.half()
    lin.bias.data = (torch.randn(384, generator=torch.Generator().manual_seed(2)) * 0.1).half()
    model = torch.nn.Sequential(lin)
    qt = ts.quantize_tensor(lin.weight.data, **opts)
    model[0] = ts.QuantLinear(qt, lin.bias.data)
    ts.save_quant_module(model, tmp_path / "f.tsk", verbose=False)
    fresh = torch.nn.Sequential(torch.nn.Linear(512, 384, bias=True, dtype=torch.float16))
    with ts.ContainerReader(tmp_path / "f.tsk") as r:
        ts.load_quantized_module(fresh, r, verbose=False)
        e = r.manifest["tensors"]["0.weight"]
        # any codebook part (NF or Lloyd-Max) marks the entry "companded" (container.py:203-206)
        has_cb = bool(opts.get("companded") or opts.get("nf_quant"))
        assert e["bits"] == opts["bits"] and e.get("companded", False) == has_cb
        if opts["bits"] == 6:
            assert "stage2_packed" in e["segments_v2"]["parts"]
    q0, q1 = model[0], fresh[0]
    assert isinstance(q1, ts.QuantLinear) and q1.bits == q0.bits
    w0, w1 = q0.dequantize_weight(torch.float32), q1.dequantize_weight(torch.float32)
    assert float((w0 - w1).abs().max()) <= 1e-3 * float(w0.abs().max())
    # a double-quant layer reloads with the f16 scale/gmin (no DQ codes in the
    # container): outputs within a bf16 ulp or two
    tol = 1e-2 if opts.get("double_quant") else 1e-3
    for M in (1, 20):
        x = recipes.activations(M, 512, seed=M).cuda()
        y0, y1 = q0(x).float(), q1(x).float()
        assert float((y0 - y1).abs().max()) <= tol * float(y0.abs().max()), M
