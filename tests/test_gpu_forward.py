"""QuantLinear forward on the decode (M <= 16) and prefill (M > 16) kernels:
max |y - y_ref| / max |y_ref| <= 1e-2 against the reference's
dequantize-then-matmul in float32/float64."""
import ctypes

import numpy as np
import pytest
import torch

import recipes
from golden_io import case_names, load_case, qopts
from gpu_util import max_rel_err, qt_from_golden, say, weight_for

pytestmark = pytest.mark.gpu

TOL = 1e-2  # max relative error, fp32 accumulation


def _ts():
    import tensorshrink_amd as ts
    return ts


@pytest.mark.parametrize("name", case_names())
@pytest.mark.parametrize("M", [1, 3, 16, 17, 64, 300])
def test_forward_small_cases(name, M):
    spec, res, d, w = load_case(name)
    ts = _ts()
    say("forward", name, M)
    bias = torch.from_numpy(d["ql_bias"]).view(w.dtype) if "ql_bias" in d.files else None
    ql = ts.QuantLinear(qt_from_golden(d, res), bias)
    x = recipes.activations(M, res["meta"]["cols"], seed=100 + M)
    y = ql(x.cuda())
    assert y.dtype == torch.bfloat16 and y.shape == (M, res["meta"]["rows"])
    W = torch.from_numpy(d["deq_f32"]).double()
    y_ref = x.double() @ W.T
    if bias is not None:
        y_ref += bias.double()
    err = max_rel_err(y.cpu(), y_ref)
    assert err <= TOL, err
    if M > 16:  # the fused MFMA kernel, which runs without a workspace
        if bias is not None:
            ql.bias = bias.cuda()
        err = max_rel_err(_forward_no_workspace(ql, x.cuda()).cpu(), y_ref)
        assert err <= TOL, ("fused", err)


@pytest.mark.parametrize("M", [1, 5, 16, 40])
def test_forward_fp16_activations(M):
    spec, res, d, w = load_case("nf4_dq_g128")
    ql = _ts().QuantLinear(qt_from_golden(d, res))
    x = recipes.activations(M, res["meta"]["cols"], seed=5, dtype=torch.float16)
    y = ql(x.cuda())
    assert y.dtype == torch.float16
    y_ref = x.double() @ torch.from_numpy(d["deq_f32"]).double().T
    assert max_rel_err(y.cpu(), y_ref) <= TOL


def test_forward_fp32_and_3d_input():
    spec, res, d, w = load_case("u4_dq_g128_bias")
    bias = torch.from_numpy(d["ql_bias"]).view(w.dtype)
    ql = _ts().QuantLinear(qt_from_golden(d, res), bias)
    x = recipes.activations(6, res["meta"]["cols"], seed=9).float().reshape(2, 3, -1)
    y = ql(x.cuda())
    assert y.shape == (2, 3, res["meta"]["rows"]) and y.dtype == torch.float32
    y_ref = x.double().reshape(6, -1) @ torch.from_numpy(d["deq_f32"]).double().T + bias.double()
    assert max_rel_err(y.cpu().reshape(6, -1), y_ref) <= TOL


def _oracle_opts(opts):
    return dict(bits=opts["bits"], group_size=opts["group_size"], outlier_frac=opts["outlier_frac"],
                double_quant=opts.get("double_quant", False), nf_quant=opts.get("nf_quant", False))


def _layer(rows, cols, seed, opts, sigma=0.02):
    """QuantLinear for a seeded layer and its reference weight: the oracle's
    dequantize_tensor of the oracle's quantize, after checking that the GPU
    codec's arrays equal the oracle's bit for bit."""
    ts = _ts()
    from oracle import codec_ref as O
    w = recipes.gaussian_weight(rows, cols, seed, sigma=sigma)
    qt = ts.quantize_tensor(w, **opts)
    q_ref = O.quantize(w, **_oracle_opts(opts))
    for f in ("packed", "outlier_idx", "outlier_val", "scale", "gmin", "dq_scale_codes", "stage2_packed"):
        if f in q_ref:
            np.testing.assert_array_equal(getattr(qt, f).view(np.uint8), q_ref[f].view(np.uint8), err_msg=f)
    W = torch.from_numpy(O.dequantize(q_ref, "f32")).cuda()
    return ts.QuantLinear(qt), W


def _pinned(name):
    """QuantLinear for a config-scale digest case and its reference weight:
    the GPU codec's arrays and float32 dequantize_tensor output, each checked
    against the reference's SHA-256 digest before use."""
    from golden_io import digests, qopts
    from gpu_util import sha
    ts = _ts()
    dig = digests()[name]
    spec = dig["spec"]
    w = weight_for(spec)
    if spec.get("lm"):
        torch.manual_seed(spec["manual_seed"])
    qt = ts.quantize_tensor(w, **qopts(spec))
    del w
    for f, h in dig["digests"].items():
        if f not in ("deq_f32", "deq_native"):
            assert sha(getattr(qt, f)) == h, (name, f)
    W = ts.dequantize_tensor(qt, device="cuda", dtype=torch.float32)
    assert sha(W.cpu().numpy()) == dig["digests"]["deq_f32"], name
    return ts.QuantLinear(qt), W


NF4 = dict(bits=4, group_size=128, outlier_frac=0.001, double_quant=True, nf_quant=True)
CFG3_NAMES = ["cfg1_nf4_dq_4096x4096"] + [f"cfg3_{n}_nf4_dq_{r}x{c}" for n, r, c in recipes.LLAMA3_8B_LINEARS[1:]]
CFG4_NAMES = {8: ["cfg4_nf8_dq_14336x4096", "cfg4_up_nf8_dq_14336x4096", "cfg4_down_nf8_dq_4096x14336"],
              6: ["cfg4_gate_rvq6_dq_14336x4096", "cfg4_rvq6_dq_14336x4096", "cfg4_down_rvq6_dq_4096x14336"]}
CFG5_NAMES = [f"cfg5_{n}_{r}x{c}" for n, r, c in recipes.LLAMA3_70B_LINEARS]


@pytest.mark.slow
@pytest.mark.parametrize("M", [1, 16])
def test_cfg1_4096_nf4(M):
    ql, W = _pinned("cfg1_nf4_dq_4096x4096")
    x = recipes.activations(M, 4096).cuda()
    err = max_rel_err(ql(x).float(), x.float() @ W.T)
    say("cfg1 M", M, "err", err)
    assert err <= TOL


@pytest.mark.slow
@pytest.mark.parametrize("name", ["cfg2_lm2_dq_11008x4096", "cfg2_lm2_g64_11008x4096"])
def test_cfg2_11008_lm2(name):
    """2-bit Lloyd-Max, group 64, with and without double quant."""
    ql, W = _pinned(name)
    for M in (1, 4, 8):
        x = recipes.activations(M, 4096).cuda()
        err = max_rel_err(ql(x).float(), x.float() @ W.T)
        say("cfg2", name, M, err)
        assert err <= TOL, (M, err)


@pytest.mark.slow
def test_cfg3_llama8b_layer():
    for name, (lname, n, k) in zip(CFG3_NAMES, recipes.LLAMA3_8B_LINEARS):
        ql, W = _pinned(name)
        for M in (1, 4, 16):
            x = recipes.activations(M, k).cuda()
            err = max_rel_err(ql(x).float(), x.float() @ W.T)
            say("cfg3", lname, M, err)
            assert err <= TOL, (lname, M, err)
        del ql, W
        torch.cuda.empty_cache()


@pytest.mark.parametrize("bits,frac", [(4, 0.05), (8, 0.03), (6, 0.02)])
def test_forward_dense_outliers(bits, frac):
    """Rows with many outliers (about 100 per row at 5 %, several in one
    64-column k-step of a row): the decode kernel's tile slots and the
    prefill kernel's per-row walk, through QuantLinear and the C-ABI without
    a workspace."""
    opts = dict(bits=bits, group_size=128, outlier_frac=frac, double_quant=True, nf_quant=bits != 6)
    ql, W = _layer(256, 2048, 31 + bits, opts)
    for M in (1, 16, 64, 300):
        x = recipes.activations(M, 2048, seed=M).cuda()
        err = max_rel_err(ql(x).float(), x.float() @ W.T)
        say("dense outliers", bits, frac, M, err)
        assert err <= TOL, (M, err)
        if M > 16:
            err = max_rel_err(_forward_no_workspace(ql, x).float(), x.float() @ W.T)
            assert err <= TOL, ("fused", M, err)


def test_forward_outliers_in_one_row():
    """Every outlier of the layer in one row (the decode tile slots of one
    tile and the prefill walk of one thread take them all), at decode and
    prefill sizes."""
    ts = _ts()
    from oracle import codec_ref as O
    w = recipes.gaussian_weight(512, 1024, 55, outlier_frac=0.0)
    w[300, ::2] = (torch.arange(512, dtype=torch.float32) % 7 + 3).to(w.dtype)  # 512 large values in row 300
    opts = dict(bits=4, group_size=128, outlier_frac=512 / (512 * 1024), double_quant=True, nf_quant=True)
    qt = ts.quantize_tensor(w, **opts)
    q_ref = O.quantize(w, **_oracle_opts(opts))
    np.testing.assert_array_equal(qt.outlier_idx, q_ref["outlier_idx"])
    assert (qt.outlier_idx // 1024 == 300).all()
    ql = ts.QuantLinear(qt)
    W = torch.from_numpy(O.dequantize(q_ref, "f32")).cuda()
    for M in (1, 7, 16, 33, 260):
        x = recipes.activations(M, 1024, seed=M).cuda()
        err = max_rel_err(ql(x).float(), x.float() @ W.T)
        say("one-row outliers", M, err)
        assert err <= TOL, (M, err)


@pytest.mark.slow
@pytest.mark.parametrize("bits", [8, 6])
@pytest.mark.parametrize("layer", [0, 1, 2])
def test_cfg4_prefill_2048(bits, layer):
    """the fused dequant-into-LDS MFMA kernel (QuantLinear's
    path above 16 rows) on the Llama-3-8B gate/up/down at M = 2048, 8-bit NF8
    + double quant and 6-bit RVQ, against x @ W^T with the digest-pinned W.
    Also the dequantize + library GEMM path (a workspace passed through the
    C-ABI) on the same layer."""
    name = CFG4_NAMES[bits][layer]
    ql, W = _pinned(name)
    x = recipes.activations(2048, ql.in_features).cuda()
    ref = x.float() @ W.T
    y = ql(x)
    err = max_rel_err(y.float(), ref)
    say("cfg4", bits, name, "fused", err)
    assert err <= TOL, err
    err_g = max_rel_err(_forward_gemm(ql, x).float(), ref)
    say("cfg4", bits, name, "dequant+gemm", err_g)
    assert err_g <= TOL, err_g


@pytest.mark.slow
def test_cfg5_llama70b_layer_decode():
    """BASELINE config 5's layer (8-bit attention, 4-bit MLP, 2-bit companded
    down) at decode sizes against the digest-pinned weights."""
    for name, (lname, n, k) in zip(CFG5_NAMES, recipes.LLAMA3_70B_LINEARS):
        ql, W = _pinned(name)
        for M in (1, 4, 16):
            x = recipes.activations(M, k, seed=M).cuda()
            err = max_rel_err(ql(x).float(), x.float() @ W.T)
            say("cfg5", lname, M, err)
            assert err <= TOL, (lname, M, err)
        del ql, W
        torch.cuda.empty_cache()


@pytest.mark.parametrize("shape", [(520, 1024), (4096, 4096), (1024, 8192)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("fmt", ["nf4_dq", "lloyd2"])
def test_decode_device_codebook_matches_launch_args(fmt, dtype, shape):
    """The kernel-level API passes the codebook as a device tensor, so the
    decode kernel stages it and centres / rounds the table entries on the
    GPU; QuantLinear passes a host copy, whose entries are centred and rounded
    on the host and go in as launch arguments. Both must give the same tables:
    identical outputs at decode sizes, for bf16 and f16 activations. At M = 1
    the 4-bit layers take 4-wave workgroups (520 x 1024, packed table),
    8-wave ones (4096 x 4096) and 16-wave ones (1024 x 8192); the last two
    use 256-byte table rows and stage the device codebook in the partials
    buffer."""
    ts = _ts()
    rows, cols = shape
    opts = NF4 if fmt == "nf4_dq" else dict(bits=2, group_size=64, outlier_frac=0.001, companded=True)
    ql = ts.QuantLinear(ts.quantize_tensor(recipes.student_t_weight(rows, cols, 31), **opts))
    assert ql.codebook is not None
    dq = bool(opts.get("double_quant"))
    for M in (1, 5, 16):
        x = recipes.activations(M, cols, seed=M, dtype=dtype).cuda()
        kw = dict(codebook=ql.codebook, outlier_row=ql.outlier_row, outlier_col=ql.outlier_col,
                  outlier_delta=ql.outlier_delta, n_groups=ql.n_groups)
        if dq:
            kw.update(dq_scale_codes=ql.dq_scale_codes, dq_scale_meta=ql.dq_scale_meta,
                      dq_gmin_codes=ql.dq_gmin_codes, dq_gmin_meta=ql.dq_gmin_meta, dq_group_size=ql.dq_group_size)
        y_dev = ts.fused_quantized_linear(x, ql.packed, None if dq else ql.scale, None if dq else ql.gmin, None,
                                          opts["bits"], opts["group_size"], ql.cols, ql.out_features, dtype, **kw)
        y_arg = ql(x)
        torch.cuda.synchronize()
        say("device codebook", fmt, dtype, shape, M)
        assert y_dev is not None and y_dev.dtype == dtype
        assert torch.equal(y_dev, y_arg), (fmt, dtype, shape, M)


def test_kernel_api_functions():
    ts = _ts()
    spec, res, d, w = load_case("u4_dq_g128_bias")
    ql = ts.QuantLinear(qt_from_golden(d, res))
    x = recipes.activations(5, res["meta"]["cols"], seed=3).cuda()
    y = ts.fused_quantized_linear(x, ql.packed, None, None, None, 4, 128, ql.cols, ql.out_features, torch.bfloat16,
                                  return_fp32=True, outlier_row=ql.outlier_row, outlier_col=ql.outlier_col,
                                  outlier_delta=ql.outlier_delta, dq_scale_codes=ql.dq_scale_codes,
                                  dq_scale_meta=ql.dq_scale_meta, dq_gmin_codes=ql.dq_gmin_codes,
                                  dq_gmin_meta=ql.dq_gmin_meta, dq_group_size=ql.dq_group_size,
                                  n_groups=ql.n_groups)
    W = torch.from_numpy(d["deq_f32"]).cuda()
    assert y.dtype == torch.float32
    assert max_rel_err(y, x.float() @ W.T) <= TOL
    # uncorrected GEMM + standalone outlier pass == corrected GEMM
    y0 = ts.fused_quantized_linear(x, ql.packed, None, None, None, 4, 128, ql.cols, ql.out_features, torch.bfloat16,
                                   return_fp32=True, dq_scale_codes=ql.dq_scale_codes, dq_scale_meta=ql.dq_scale_meta,
                                   dq_gmin_codes=ql.dq_gmin_codes, dq_gmin_meta=ql.dq_gmin_meta,
                                   dq_group_size=ql.dq_group_size, n_groups=ql.n_groups)
    y1 = ts.apply_outlier_correction(y0.clone(), x, ql.outlier_row, ql.outlier_col, ql.outlier_delta)
    assert torch.allclose(y1, y, rtol=1e-5, atol=1e-5)
    # dense dequant of the QuantLinear view equals the codec view off the outliers
    Wq = ql.dequantize_weight(torch.float32)
    mask = torch.ones(W.numel(), dtype=torch.bool, device="cuda")
    mask[torch.from_numpy(d["qt_outlier_idx"].astype(np.int64)).cuda()] = False
    assert torch.equal(Wq.reshape(-1)[mask], W.reshape(-1)[mask])


@pytest.mark.parametrize("opts", [NF4, dict(bits=8, group_size=128, outlier_frac=0.001, double_quant=True,
                                            nf_quant=True),
                                  dict(bits=6, group_size=64, outlier_frac=0.002, double_quant=False)])
def test_forward_group_matches_single(opts):
    """QuantLinear.forward_group (one launch for layers sharing x) against the
    per-layer forward and the float32 reference."""
    ts = _ts()
    shapes = [(512, 1024), (128, 1024), (136, 1024)]
    made = [_layer(n, k, 70 + i, opts) for i, (n, k) in enumerate(shapes)]
    qls = [m[0] for m in made]
    torch.manual_seed(0)
    qls[1].bias = torch.randn(qls[1].out_features, dtype=torch.bfloat16).cuda()
    for M in (1, 5, 16, 24, 32):
        x = recipes.activations(M, 1024, seed=M).cuda()
        ys = ts.QuantLinear.forward_group(qls, x)
        for q, (ql, W), y in zip(qls, made, ys):
            y1 = ql(x)
            assert y.shape == y1.shape and y.dtype == y1.dtype
            # the same decode kernel up to 16 rows; above, an 8-bit layer alone
            # runs the prefill kernel, which rounds W to bf16 per element
            assert max_rel_err(y.float(), y1.float()) <= (1e-3 if M <= 16 else TOL)
            ref = x.float() @ W.T + (ql.bias.float() if ql.bias is not None else 0)
            assert max_rel_err(y.float(), ref) <= TOL


@pytest.mark.parametrize("opts", [dict(bits=2, group_size=64, outlier_frac=0.001, companded=True),
                                  dict(bits=4, group_size=128, outlier_frac=0.001, companded=True, double_quant=True),
                                  dict(bits=8, group_size=128, outlier_frac=0.001, companded=True)])
def test_forward_group_per_layer_codebooks(opts):
    """Lloyd-Max codebooks are fitted per tensor: a grouped launch builds each
    workgroup's code table from its own layer's codebook (launch arguments up
    to 16 entries, device memory beyond), so it must equal the per-layer
    forwards."""
    ts = _ts()
    qls = []
    for i, n in enumerate((384, 128, 200)):
        torch.manual_seed(40 + i)  # Lloyd-Max samples from the global RNG
        w = recipes.student_t_weight(n, 1024, 90 + i) if i != 1 else recipes.gaussian_weight(n, 1024, 90 + i)
        qls.append(ts.QuantLinear(ts.quantize_tensor(w, **opts)))
    cbs = [q.codebook.cpu() for q in qls]
    assert not torch.equal(cbs[0], cbs[1]) and not torch.equal(cbs[1], cbs[2])
    for M in (1, 4, 16, 32):
        x = recipes.activations(M, 1024, seed=M).cuda()
        ys = ts.QuantLinear.forward_group(qls, x)
        for q, y in zip(qls, ys):
            # (8-bit layers alone run the prefill kernel above 16 rows)
            assert max_rel_err(y.float(), q(x).float()) <= (1e-3 if M <= 16 else TOL), (M, q.out_features)


@pytest.mark.parametrize("opts", [dict(bits=8, group_size=128, outlier_frac=0.002, double_quant=True, nf_quant=True),
                                  dict(bits=2, group_size=64, outlier_frac=0.002, double_quant=True),
                                  dict(bits=6, group_size=128, outlier_frac=0.002, double_quant=True),
                                  dict(bits=4, group_size=32, outlier_frac=0.002, double_quant=False)])
def test_forward_ragged_cols(opts):
    """Columns a multiple of 8 but not of the group size (the last group is
    partial and padded): decode (x chunks past the last column read as zero,
    also in the per-group x sums at M = 1) and the prefill kernel."""
    ql, W = _layer(200, 1000, 97, opts)
    for M in (1, 3, 16, 40):
        x = recipes.activations(M, 1000, seed=M).cuda()
        ref = x.float() @ W.T
        assert max_rel_err(ql(x).float(), ref) <= TOL, M
        if M > 16:
            assert max_rel_err(_forward_no_workspace(ql, x).float(), ref) <= TOL, ("fused", M)


@pytest.mark.parametrize("opts", [NF4, dict(bits=8, group_size=128, outlier_frac=0.002, double_quant=True, nf_quant=True),
                                  dict(bits=2, group_size=64, outlier_frac=0.002, double_quant=True),
                                  dict(bits=6, group_size=128, outlier_frac=0.002, double_quant=True)])
def test_forward_mid_m(opts):
    """17 to 128 rows of x on a layer of few row tiles: the decode kernel's
    blocks of 16 tokens up to 32 rows (codes of at most 6 bits), the prefill
    kernel above (K split through QuantLinear's workspace, unsplit through
    the C-ABI without one), with a float32 output of row stride past N."""
    from tensorshrink_amd import _lib as L
    ql, W = _layer(256, 1024, 98, opts)
    ql.bias = (torch.randn(256, generator=torch.Generator().manual_seed(4)) * 0.1).to(torch.bfloat16).cuda()
    for M in (17, 32, 33, 48, 64, 65, 100, 128):
        x = recipes.activations(M, 1024, seed=M).cuda()
        ref = x.float() @ W.T + ql.bias.float()
        assert max_rel_err(ql(x).float(), ref) <= TOL, M
        ldy = 300
        y = torch.full((M, ldy), 7.0, dtype=torch.float32, device="cuda")
        L.check(L.load().ts_qlinear_forward(ctypes.byref(ql._layer), x.data_ptr(), M, 1024, L.TS_BF16, y.data_ptr(),
                                            ldy, L.TS_F32, ql.bias.data_ptr(), None, 0, L.stream_ptr()), "fwd")
        assert max_rel_err(y[:, :256], ref) <= TOL, ("f32", M)
        assert bool((y[:, 256:] == 7.0).all()), M  # the stride's tail is untouched


def test_forward_mid_m_many_tiles():
    """Small M on 520 + 128 row tiles in one grouped launch (M = 20, 32: the
    multi-block decode launch with 4-wave workgroups, each wave streaming
    several batches, outputs looped over the workgroup's threads), and the
    520-tile layer alone on the prefill kernel's 128-row tiles (M = 20, 33,
    100, 200)."""
    ts = _ts()
    ql, W = _layer(8320, 256, 99, NF4)
    ql2, W2 = _layer(2048, 256, 100, NF4)
    for M in (20, 32):
        x = recipes.activations(M, 256, seed=M).cuda()
        y, y2 = ts.QuantLinear.forward_group([ql, ql2], x)
        assert max_rel_err(y.float(), x.float() @ W.T) <= TOL, M
        assert max_rel_err(y2.float(), x.float() @ W2.T) <= TOL, M
    for M in (20, 33, 100, 200):
        x = recipes.activations(M, 256, seed=M).cuda()
        assert max_rel_err(ql(x).float(), x.float() @ W.T) <= TOL, M


@pytest.mark.parametrize("opts", [dict(bits=4, group_size=32, outlier_frac=0.002, double_quant=True),
                                  dict(bits=8, group_size=32, outlier_frac=0.002, double_quant=False)])
def test_forward_decode_passes(opts):
    """Layers the prefill kernel does not take (992 columns of group size 32:
    K not a multiple of its 64-column k-step) run the decode kernel's token
    blocks at any M, in passes of 64 rows, before the one-thread-per-output
    kernel."""
    ql, W = _layer(520, 992, 96, opts)
    for M in (17, 33, 64, 65, 130):
        x = recipes.activations(M, 992, seed=M).cuda()
        assert max_rel_err(ql(x).float(), x.float() @ W.T) <= TOL, M


def test_forward_random_shapes():
    """A seeded sweep over formats, shapes and batch sizes, so every dispatch
    boundary (decode, its token blocks and passes, the prefill tile shapes,
    ragged columns, the generic kernel) meets the dequantized weight's
    float32 product."""
    ts = _ts()
    rng = np.random.default_rng(1234)
    fmts = [dict(bits=4, group_size=128, double_quant=True, nf_quant=True), dict(bits=4, group_size=64),
            dict(bits=4, group_size=32, double_quant=True), dict(bits=8, group_size=128, nf_quant=True),
            dict(bits=8, group_size=64, double_quant=True), dict(bits=2, group_size=64, double_quant=True),
            dict(bits=2, group_size=128), dict(bits=6, group_size=128, double_quant=True), dict(bits=6, group_size=64)]
    for case in range(36):
        opts = dict(fmts[case % len(fmts)])
        opts["outlier_frac"] = float(rng.choice([0.0, 0.001, 0.01]))
        rows = int(rng.integers(16, 5200))
        cols = int(rng.choice([8 * int(rng.integers(8, 400)), int(rng.integers(64, 3000))]))
        M = int(rng.choice([1, 2, 7, 16, 17, 31, 33, 64, 65, 100, 129, 200, 257, 600]))
        w = recipes.gaussian_weight(rows, cols, 500 + case)
        ql = ts.QuantLinear(ts.quantize_tensor(w, **opts))
        x = recipes.activations(M, cols, seed=case).cuda()
        W = ql.dequantize_weight(torch.float32)
        err = max_rel_err(ql(x).float(), x.float() @ W.T)
        say("random", case, opts, rows, cols, M, err)
        assert err <= TOL, (case, opts, rows, cols, M, err)


def _dense_row_weight(rows, cols, seed):
    """Gaussian weight with two rows of large values (row 5 on every column,
    row 77 on every third), so the top-k outliers crowd those rows and every
    other row holds dozens: K splits then start past 16 of a row's entries."""
    w = recipes.gaussian_weight(rows, cols, seed)
    w[5, :] *= 50
    w[77, ::3] *= 50
    return w


@pytest.mark.parametrize("fmt,rows,cols,M,xdt,bias", [
    (dict(bits=4, group_size=128, double_quant=True, nf_quant=True), 1024, 4096, 200, torch.bfloat16, True),
    (dict(bits=8, group_size=128, double_quant=True, nf_quant=True), 4096, 2048, 300, torch.bfloat16, False),
    (dict(bits=6, group_size=128, double_quant=True), 512, 8192, 160, torch.bfloat16, True),
    (dict(bits=2, group_size=64, double_quant=True), 1002, 2048, 140, torch.float16, True),
    (dict(bits=4, group_size=64), 1024, 4096, 2048, torch.float16, False),
    (dict(bits=8, group_size=128, double_quant=True, nf_quant=True), 3072, 4096, 1024, torch.bfloat16, True),
    (dict(bits=6, group_size=128, double_quant=True), 3072, 4096, 1024, torch.float16, False),
])
def test_forward_split_k(fmt, rows, cols, M, xdt, bias):
    """Shapes whose launch plan splits K (128 x 128, 256 x 128 and, at
    3072 x 4096 with M = 1024, 256 x 256 tiles on 8 waves): QuantLinear
    hands the fused kernel a workspace for the partial sums; the split result
    (with dense outlier rows, bias, fp16 / bf16) meets the float64 product
    and agrees with the unsplit kernel."""
    ts = _ts()
    from tensorshrink_amd import _lib as L
    w = _dense_row_weight(rows, cols, 900 + rows)
    b = (torch.randn(rows, generator=torch.Generator().manual_seed(7)) * 0.5).to(xdt) if bias else None
    ql = ts.QuantLinear(ts.quantize_tensor(w, outlier_frac=0.01, **fmt), b)
    lay = ctypes.byref(ql._layer)
    nws = L.load().ts_forward_partials_bytes(lay, M)
    assert nws > 0 and nws % (4 * M * rows) == 0 and nws < L.load().ts_forward_workspace_bytes(lay, M)
    x = recipes.activations(M, cols, seed=M, dtype=xdt).cuda()
    W = ql.dequantize_weight(torch.float32).double()
    y_ref = x.double() @ W.T
    if b is not None:
        y_ref += b.double().cuda()
    y = ql(x)
    y0 = _forward_no_workspace(ql, x)
    say("split-k", fmt, rows, cols, M, nws // (4 * M * rows), max_rel_err(y, y_ref), max_rel_err(y, y0))
    assert y.dtype == xdt
    assert max_rel_err(y, y_ref) <= TOL
    assert max_rel_err(y0, y_ref) <= TOL
    assert max_rel_err(y, y0) <= 4e-3


def test_forward_split_k_f32_strided():
    """The K-split path through the C-ABI: fp32 output with a row stride past
    the layer's rows (the stride tail stays untouched), two calls in a row
    sharing one workspace, the second with fewer rows and a bias (added in the
    reduction pass)."""
    ts = _ts()
    from tensorshrink_amd import _lib as L
    rows, cols, ldy = 1024, 4096, 1100
    ql = ts.QuantLinear(ts.quantize_tensor(_dense_row_weight(rows, cols, 31), **dict(NF4, outlier_frac=0.01)))
    W = ql.dequantize_weight(torch.float32).double()
    lib, lay = L.load(), ctypes.byref(ql._layer)
    ws = torch.empty(lib.ts_forward_partials_bytes(lay, 300), dtype=torch.uint8, device="cuda")
    bias = (torch.randn(rows, generator=torch.Generator().manual_seed(9)) * 0.5).to(torch.bfloat16).cuda()
    for M, b in ((300, None), (150, bias)):
        need = lib.ts_forward_partials_bytes(lay, M)
        assert 0 < need <= ws.numel()
        x = recipes.activations(M, cols, seed=M).cuda()
        y = torch.full((M, ldy), 7.0, dtype=torch.float32, device="cuda")
        L.check(lib.ts_qlinear_forward(lay, x.data_ptr(), M, cols, L.dtype_code(x.dtype), y.data_ptr(), ldy,
                                       L.dtype_code(torch.float32), L.ptr(b), ws.data_ptr(), ws.numel(),
                                       L.stream_ptr()), "split fwd")
        y_ref = x.double() @ W.T + (b.double() if b is not None else 0)
        assert max_rel_err(y[:, :rows], y_ref) <= TOL
        assert bool((y[:, rows:] == 7.0).all())


@pytest.mark.parametrize("split", [False, True])
def test_forward_prefill_ragged_rows_strided(split):
    """The prefill epilogue's 16-byte row chunks on an output whose rows are
    aligned (row stride a multiple of 16 bytes) but whose width is not a
    multiple of the chunk (1018 columns): the last chunk of each row is
    stored element by element and the stride tail stays untouched; bf16 and
    fp32 outputs, with and without the K-split workspace."""
    from tensorshrink_amd import _lib as L
    ql, W = _layer(1018, 2048, 95, NF4)
    lib, lay = L.load(), ctypes.byref(ql._layer)
    M = 300
    x = recipes.activations(M, 2048, seed=5).cuda()
    ref = x.float() @ W.T
    nws = lib.ts_forward_partials_bytes(lay, M) if split else 0
    assert (nws > 0) == split
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device="cuda")
    for ydt, ldy in ((torch.bfloat16, 1024), (torch.float32, 1020)):
        y = torch.full((M, ldy), 7.0, dtype=ydt, device="cuda")
        L.check(lib.ts_qlinear_forward(lay, x.data_ptr(), M, 2048, L.TS_BF16, y.data_ptr(), ldy, L.dtype_code(ydt),
                                       None, ws.data_ptr() if split else None, nws, L.stream_ptr()), "fwd")
        assert max_rel_err(y[:, :1018].float(), ref) <= TOL, ydt
        assert bool((y[:, 1018:] == 7.0).all()), ydt


@pytest.mark.parametrize("opts", [NF4, dict(bits=2, group_size=64, outlier_frac=0.002, double_quant=True)])
def test_forward_decode_x_from_l2(opts):
    """Decode at 9-16 rows with x too large for LDS on layers whose rows fit
    two batches per wave of 8: the 8-wave straight-line launches that read x
    from L2, with one batch per wave (2048 x 4096) and two (4112 x 8192, 257
    row tiles), against the dequantized weight's float32 product."""
    ts = _ts()
    for rows, cols in ((2048, 4096), (4112, 8192)):
        ql = ts.QuantLinear(ts.quantize_tensor(recipes.gaussian_weight(rows, cols, 94), **opts))
        W = ql.dequantize_weight(torch.float32)
        for M in (9, 12, 16):
            x = recipes.activations(M, cols, seed=M).cuda()
            assert max_rel_err(ql(x).float(), x.float() @ W.T) <= TOL, (rows, M)
        del ql, W


def test_forward_group_fallbacks():
    """Mixed formats, M > 32, and 17-32 rows on layers of more than 12288
    rows in all run one forward per layer."""
    ts = _ts()
    a, Wa = _layer(256, 512, 81, NF4)
    b, Wb = _layer(256, 512, 82, dict(bits=8, group_size=128, outlier_frac=0.0, double_quant=False))
    for M in (3, 40):
        x = recipes.activations(M, 512, seed=M).cuda()
        ya, yb = ts.QuantLinear.forward_group([a, b], x)
        assert max_rel_err(ya.float(), x.float() @ Wa.T) <= TOL
        assert max_rel_err(yb.float(), x.float() @ Wb.T) <= TOL
    c, Wc = _layer(6400, 256, 83, NF4)
    d, Wd = _layer(6400, 256, 84, NF4)
    for M in (16, 24):
        x = recipes.activations(M, 256, seed=M).cuda()
        yc, yd = ts.QuantLinear.forward_group([c, d], x)
        assert max_rel_err(yc.float(), c(x).float()) <= 1e-3
        assert max_rel_err(yd.float(), x.float() @ Wd.T) <= TOL


def _forward_gemm(ql, x):
    """ts_qlinear_forward with a workspace: dequantize + one library GEMM."""
    from tensorshrink_amd import _lib as L
    y = torch.empty(x.shape[0], ql.out_features, dtype=x.dtype, device=x.device)
    b = None if ql.bias is None else ql.bias.to(x.dtype).contiguous()
    lib = L.load()
    n = lib.ts_forward_workspace_bytes(ctypes.byref(ql._layer), x.shape[0])
    ws = torch.empty(n, dtype=torch.uint8, device=x.device)
    dt = L.dtype_code(x.dtype)
    L.check(lib.ts_qlinear_forward(ctypes.byref(ql._layer), x.data_ptr(), x.shape[0], ql.in_features, dt,
                                   y.data_ptr(), ql.out_features, dt, L.ptr(b), ws.data_ptr(), n, L.stream_ptr()),
            "fwd gemm")
    return y


def _forward_no_workspace(ql, x):
    """ts_qlinear_forward without a workspace: the fused MFMA prefill kernel."""
    import ctypes
    from tensorshrink_amd import _lib as L
    y = torch.empty(x.shape[0], ql.out_features, dtype=x.dtype, device=x.device)
    b = None if ql.bias is None else ql.bias.to(x.dtype).contiguous()
    dt = L.dtype_code(x.dtype)
    L.check(L.load().ts_qlinear_forward(ctypes.byref(ql._layer), x.data_ptr(), x.shape[0], ql.in_features, dt,
                                        y.data_ptr(), ql.out_features, dt, L.ptr(b), None, 0, L.stream_ptr()), "fwd")
    return y


@pytest.mark.parametrize("opts", [NF4, dict(bits=8, group_size=128, outlier_frac=0.001, double_quant=True,
                                            nf_quant=True),
                                  dict(bits=6, group_size=64, outlier_frac=0.002, double_quant=False),
                                  dict(bits=2, group_size=64, outlier_frac=0.05, double_quant=True),
                                  dict(bits=4, group_size=32, outlier_frac=0.05, double_quant=False)])
def test_dequantize_weight_vector_pass_matches_scalar(opts):
    """QuantLinear view (outlier = base + delta (+ stage 2), modules.py:786-802):
    the vectorised pass (8-column chunks) against the per-element pass (chosen
    by a row stride that breaks 16-byte alignment), bit for bit in every
    output dtype, outliers included. 1032 columns: 129 chunks of 8 per row, so
    waves straddle rows and the last wave is partial; the 5 % cases put
    several outliers in one 8-column chunk."""
    ts = _ts()
    from tensorshrink_amd import _lib as L
    ql, _ = _layer(200, 1032, 91, opts)
    assert ql.outlier_row.numel() > 0
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        fused = ql.dequantize_weight(dt)
        wide = torch.empty(ql.rows, ql.cols + 1, dtype=dt, device="cuda")
        L.check(L.lib().ts_dequantize(ctypes.byref(ql._layer), L.TS_DEQ_QLINEAR, None, None, 0, wide.data_ptr(),
                                      ql.cols + 1, L.dtype_code(dt), L.stream_ptr(wide.device)), "dequantize")
        ref = wide[:, :ql.cols].contiguous()
        iv = torch.int32 if dt == torch.float32 else torch.int16
        assert torch.equal(fused.view(iv), ref.view(iv)), dt


@pytest.mark.parametrize("M", [1, 5, 300])
def test_forward_graph_replay(M):
    """QuantLinear.forward captured in a HIP graph and replayed four times, with
    eager work and synchronisation between replays: every replay equals the
    eager call (decode kernel for M <= 16, the fused prefill kernel above)."""
    ts = _ts()
    ql, W = _layer(1024, 2048, 77, NF4)
    ql.bias = torch.randn(ql.out_features, dtype=torch.bfloat16).cuda()
    x = recipes.activations(M, 2048).cuda()
    y_eager = ql(x)
    torch.cuda.synchronize()
    static_x = x.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ql(static_x)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_y = ql(static_x)
    ref = x.float() @ W.T + ql.bias.float()
    for i in range(4):
        other = ql(x[: max(1, M // 2)])  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        assert max_rel_err(static_y.float(), y_eager.float()) <= 1e-3, i
        assert max_rel_err(static_y.float(), ref) <= TOL, i
        del other


@pytest.mark.parametrize("M,dtype,bias", [(17, torch.bfloat16, False), (300, torch.bfloat16, True),
                                          (520, torch.float16, True)])
def test_forward_gemm_path(M, dtype, bias):
    """M > 16 with a workspace: dequantize into it + one library GEMM (bias in
    the epilogue), against the fused kernel and the float32 reference."""
    ts = _ts()
    from tensorshrink_amd import _lib as L
    ql, W = _layer(768, 1536, 90 + M, NF4)
    if bias:
        torch.manual_seed(M)
        ql.bias = (torch.randn(768) * 0.1).to(dtype).cuda()
    assert L.load().ts_forward_workspace_bytes(__import__("ctypes").byref(ql._layer), M) >= 768 * 1536 * 2
    assert L.load().ts_forward_workspace_bytes(__import__("ctypes").byref(ql._layer), 16) == 0
    x = recipes.activations(M, 1536, seed=M, dtype=dtype).cuda()
    y = _forward_gemm(ql, x)
    y_fused = ql(x)
    ref = x.float() @ W.T + (ql.bias.float() if bias else 0)
    say("gemm path", M, dtype, bias, max_rel_err(y.float(), ref), max_rel_err(y_fused.float(), ref))
    assert y.dtype == dtype
    assert max_rel_err(y.float(), ref) <= TOL
    assert max_rel_err(y_fused.float(), ref) <= TOL
    assert max_rel_err(y.float(), y_fused.float()) <= TOL


@pytest.mark.parametrize("M", [9, 16])
def test_forward_group_two_row_tiles(M):
    """M > 8 at K = 4096 (x read from global memory) with more tiles than one
    resident round: two 16-row tiles per workgroup share each x fragment.
    8200-row layers: an odd tile count (a workgroup with one live tile) and a
    partial last tile."""
    ts = _ts()
    made = [_layer(8200, 4096, 300 + i, NF4) for i in range(2)]
    qls = [m[0] for m in made]
    torch.manual_seed(M)
    qls[1].bias = (torch.randn(8200) * 0.1).to(torch.bfloat16).cuda()
    x = recipes.activations(M, 4096, seed=M).cuda()
    ys = ts.QuantLinear.forward_group(qls, x)
    for ql, (_, W), y in zip(qls, made, ys):
        ref = x.float() @ W.T + (ql.bias.float() if ql.bias is not None else 0)
        err = max_rel_err(y.float(), ref)
        say("two row tiles", M, err)
        assert err <= TOL, err


@pytest.mark.parametrize("bits,gs,dq", [(4, 32, True), (4, 32, False), (2, 64, True)])
def test_forward_quarter_group_codes(bits, gs, dq):
    """Layers whose lanes hold 4 code bytes per group (4-bit group 32, 2-bit
    group 64): one 16-byte load per lane and a transpose across the wave's
    16-lane rows, at every x path (DPP at M = 1, LDS, global)."""
    opts = dict(bits=bits, group_size=gs, outlier_frac=0.002, double_quant=dq, nf_quant=bits == 4)
    ql, W = _layer(520, 3072, 40 + bits + gs, opts)
    for M in (1, 5, 16):
        x = recipes.activations(M, 3072, seed=M).cuda()
        err = max_rel_err(ql(x).float(), x.float() @ W.T)
        say("quarter groups", bits, gs, dq, M, err)
        assert err <= TOL, (M, err)


@pytest.mark.slow
def test_forward_group_persistent_schedule():
    """Launches beyond one resident round of waves run the persistent decode
    schedule (workgroups loop over tiles, refilling their batches across tile
    boundaries): config 3's gate/up as one grouped launch (2 x 896 tiles x 4
    waves) with a bias on one layer, against the digest-pinned weights, at
    M = 1 (persistent) and 4 (the other schedule)."""
    ts = _ts()
    (gq, Wg), (uq, Wu) = _pinned(CFG3_NAMES[4]), _pinned(CFG3_NAMES[5])
    torch.manual_seed(1)
    uq.bias = (torch.randn(uq.out_features) * 0.1).to(torch.bfloat16).cuda()
    for M in (1, 4):
        x = recipes.activations(M, 4096, seed=40 + M).cuda()
        yg, yu = ts.QuantLinear.forward_group([gq, uq], x)
        for y, W, b, q in ((yg, Wg, None, gq), (yu, Wu, uq.bias, uq)):
            ref = x.float() @ W.T + (b.float() if b is not None else 0)
            err = max_rel_err(y.float(), ref)
            say("persistent group", M, err)
            assert err <= TOL, (M, err)
            assert max_rel_err(y.float(), q(x).float()) <= 1e-3


def test_gemm_path_m_buckets():
    """The dequantize + library GEMM path (a workspace passed through the
    C-ABI) over many prompt lengths: one timing sweep per power-of-two M
    bucket, its winner reused at every M of the bucket, and more distinct
    shapes than the plan cache keeps (the oldest are evicted), each result
    against x @ W^T."""
    ql, W = _layer(512, 1024, 93, NF4)
    Ms = list(range(65, 140)) + [200, 256, 257, 1000]
    for M in Ms:
        x = recipes.activations(M, 1024, seed=M).cuda()
        err = max_rel_err(_forward_gemm(ql, x).float(), x.float() @ W.T)
        assert err <= TOL, (M, err)
    # a shape evicted earlier is planned again and still right
    x = recipes.activations(65, 1024, seed=65).cuda()
    assert max_rel_err(_forward_gemm(ql, x).float(), x.float() @ W.T) <= TOL
