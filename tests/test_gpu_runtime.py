"""Runtime around the kernels: CUDAGraphQuantModel (HIP graph capture and
replay), fused_quantized_linear captured on its first call, StreamingQuantModel
(host-resident weights streamed in per layer), and the bounded per-tile
outlier slot table."""
import numpy as np
import pytest
import torch
import torch.nn as nn

import recipes
from gpu_util import say

pytestmark = pytest.mark.gpu

K = 512
FORMATS = [dict(bits=4, double_quant=True, nf_quant=True), dict(bits=8), dict(bits=2, companded=True),
           dict(bits=6), dict(bits=4, group_size=64), dict(bits=8, double_quant=True, nf_quant=True)]


class Stack(nn.Module):
    def __init__(self, layers):
        super().__init__()
        self.layers = nn.ModuleList(layers)

    def forward(self, x):
        for l in self.layers:
            x = torch.nn.functional.silu(l(x)) * 0.5
        return x


def _stack(n=len(FORMATS), bias=True):
    import tensorshrink_amd as ts
    layers = []
    for i in range(n):
        opts = dict(FORMATS[i % len(FORMATS)])
        opts.setdefault("outlier_frac", 0.002)
        w = recipes.student_t_weight(K, K, 200 + i) if i % 2 else recipes.gaussian_weight(K, K, 200 + i)
        b = (torch.randn(K, generator=torch.Generator().manual_seed(i)) * 0.05).half() if bias and i % 3 == 0 \
            else None
        layers.append(ts.QuantLinear(ts.quantize_tensor(w, **opts), b))
    return Stack(layers).cuda()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_graph_replay_matches_eager(dtype):
    import tensorshrink_amd as ts
    model = _stack()
    g = ts.CUDAGraphQuantModel(model, warmup_runs=2)
    with torch.no_grad():
        for M in (1, 4, 33):
            for step in range(4):
                x = recipes.activations(M, K, seed=100 * M + step, dtype=dtype).cuda()
                y = g(x)
                torch.cuda.synchronize()
                ref = model(x)  # eager, between replays
                torch.cuda.synchronize()
                say("graph", dtype, M, step)
                assert y.dtype == dtype and torch.equal(y, ref), (M, step)
        assert len(g._graphs) == 3
        # a captured shape in the other dtype is a new graph
        g(recipes.activations(1, K, dtype=torch.float16 if dtype == torch.bfloat16 else torch.bfloat16).cuda())
        assert len(g._graphs) == 4
    g.release()
    assert not g._graphs


def test_graph_structured_output():
    import tensorshrink_amd as ts
    model = _stack(3)

    class Two(nn.Module):
        def __init__(self):
            super().__init__()
            self.m = model

        def forward(self, x, scale=None):
            y = self.m(x)
            return {"y": y, "pair": (y * scale, x + 1)}

    g = ts.CUDAGraphQuantModel(Two())
    with torch.no_grad():
        for s in range(3):
            x = recipes.activations(2, K, seed=s).cuda()
            sc = torch.full((1,), float(s + 1), device="cuda", dtype=torch.bfloat16)
            out = g(x, scale=sc)
            y = model(x)
            assert torch.equal(out["y"], y) and torch.equal(out["pair"][0], y * sc)
            assert torch.equal(out["pair"][1], x + 1)


def test_fused_quantized_linear_first_call_under_capture():
    """The derived outlier tables of never-seen buffers are built inside the
    graph; every replay matches the eager call."""
    import tensorshrink_amd as ts
    w = recipes.gaussian_weight(256, K, 77)
    ql = ts.QuantLinear(ts.quantize_tensor(w, bits=4, outlier_frac=0.01))
    orow, ocol, odel = ql.outlier_row.clone(), ql.outlier_col.clone(), ql.outlier_delta.clone()
    for M in (3, 40):
        x = recipes.activations(M, K, seed=M).cuda()
        xs = x.clone()
        kw = dict(bits=4, group_size=128, cols=K, out_features=256, compute_dtype=torch.bfloat16,
                  outlier_row=orow, outlier_col=ocol, outlier_delta=odel)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            yg = ts.fused_quantized_linear(xs, ql.packed, ql.scale, ql.gmin, None, **kw)
        for r in range(3):
            xs.copy_(recipes.activations(M, K, seed=10 * r + M).cuda())
            graph.replay()
            torch.cuda.synchronize()
            ref = ts.fused_quantized_linear(xs, ql.packed, ql.scale, ql.gmin, None, **kw)
            torch.cuda.synchronize()
            say("fql capture", M, r)
            assert torch.equal(ref, ql(xs)), (M, r)
            if M > 16:  # the same MFMA kernel inside and outside the graph
                assert torch.equal(yg, ref), (M, r)
            else:  # no tile slots under capture: the generic kernel
                err = float((yg.float() - ref.float()).abs().max() / ref.float().abs().max())
                assert err <= 1e-2, (M, r, err)
        orow, ocol, odel = orow.clone(), ocol.clone(), odel.clone()  # new storage: not cached


@pytest.mark.parametrize("depth", [1, 2])
def test_streaming_matches_resident(depth):
    import tensorshrink_amd as ts
    model = _stack(8)
    xs = [recipes.activations(M, K, seed=M).cuda() for M in (1, 16, 40)]
    with torch.no_grad():
        ref = [model(x) for x in xs]
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    st = ts.stream_offload_module(model, prefetch_depth=depth, verbose=False)
    torch.cuda.synchronize()
    resident_seen = []
    # runs after the streamer's own pre-hook: this layer and its prefetches
    hooks = [l.register_forward_pre_hook(lambda m, i: resident_seen.append(st.stats()["layers_currently_on_gpu"]))
             for l in model.layers]
    assert st.stats()["layers_currently_on_gpu"] == 0
    assert torch.cuda.memory_allocated() < before
    assert all(not l.packed.is_cuda and l.packed.is_pinned() for l in model.layers)
    with torch.no_grad():
        for x, r in zip(xs, ref):
            y = model(x)
            torch.cuda.synchronize()
            say("streaming depth", depth, x.shape[0])
            assert torch.equal(y, r)
    assert max(resident_seen) == depth + 1
    assert st.stats()["layers_currently_on_gpu"] == 0
    for h in hooks:
        h.remove()
    st.disable()
    with pytest.raises(RuntimeError):
        model(xs[0])  # host-resident without the hooks
    model.cuda()
    with torch.no_grad():
        assert torch.equal(model(xs[1]), ref[1])


def test_slot_table_bound():
    """Outliers crowded into one 16-row tile of a 16384-row layer would pad
    every tile to about 4000 slots; the table is not built and the decode
    kernel (M <= 16) reads each tile's outliers through the CSR row offsets,
    with the same result."""
    import tensorshrink_amd as ts
    from oracle import codec_ref as O
    w = recipes.gaussian_weight(16384, 256, 91, outlier_frac=0.0)
    w[:16] *= 200
    qt = ts.quantize_tensor(w, bits=4, outlier_frac=0.001)
    assert (qt.outlier_idx // 256 < 16).sum() > 3900  # all but the near-zero entries of rows 0-15
    ql = ts.QuantLinear(qt)
    assert ql.tile_outlier_cap == 0 and ql.tile_outliers.numel() == 0
    q_ref = O.quantize(w, bits=4, outlier_frac=0.001)
    np.testing.assert_array_equal(qt.outlier_idx, q_ref["outlier_idx"])
    W = torch.from_numpy(O.dequantize(q_ref, "f32")).cuda()
    for M in (1, 8, 16, 20):
        x = recipes.activations(M, 256, seed=M).cuda()
        ref = x.float() @ W.T
        err = float((ql(x).float() - ref).abs().max() / ref.abs().max())
        say("slot bound", M, err)
        assert err <= 1e-2, (M, err)


def _csr_view(q):
    """A copy of the layer's kernel view without the per-tile slot table."""
    from tensorshrink_amd import _lib as L
    v = L.QLayer.from_buffer_copy(q._layer)
    v.tile_outliers = None
    v.tile_outlier_cap = 0
    return v


@pytest.mark.parametrize("fmt", [dict(bits=4, double_quant=True, nf_quant=True), dict(bits=8, nf_quant=True),
                                 dict(bits=2, companded=True, group_size=64)])
def test_decode_csr_outliers_match_slots(fmt):
    """Without the per-tile slot table the decode kernel reads each tile's
    outliers through the CSR row offsets: the same outputs as with the slots,
    in one launch per layer (x through the wave slots at M = 1, staged in LDS
    at M = 4 / 16) and in a grouped launch, which reports "not covered"
    (status 1) unless the decode kernel takes every layer."""
    import ctypes
    import tensorshrink_amd as ts
    from tensorshrink_amd import _lib as L
    qls = [ts.QuantLinear(ts.quantize_tensor(recipes.gaussian_weight(n, K, 60 + i), outlier_frac=0.01, **fmt))
           for i, n in enumerate((300, 200))]
    views = [_csr_view(q) for q in qls]
    lib = L.load()
    for M in (1, 4, 16):
        x = recipes.activations(M, K, seed=M).cuda()
        dt = L.dtype_code(x.dtype)
        refs = [q(x) for q in qls]  # slot table
        ys = []
        for q, v, r in zip(qls, views, refs):
            y = torch.empty(M, q.out_features, dtype=x.dtype, device="cuda")
            rc = lib.ts_qlinear_forward(ctypes.byref(v), x.data_ptr(), M, K, dt, y.data_ptr(), q.out_features, dt,
                                        None, None, 0, L.stream_ptr())
            assert rc == L.TS_OK
            ys.append(y)
        yg = [torch.empty(M, q.out_features, dtype=x.dtype, device="cuda") for q in qls]
        rc = lib.ts_qlinear_forward_group((ctypes.POINTER(L.QLayer) * 2)(*[ctypes.pointer(v) for v in views]), 2,
                                          x.data_ptr(), M, K, dt, (ctypes.c_void_p * 2)(*[y.data_ptr() for y in yg]),
                                          (ctypes.c_int64 * 2)(*[q.out_features for q in qls]), dt,
                                          (ctypes.c_void_p * 2)(None, None), L.stream_ptr())
        assert rc == L.TS_OK, rc
        for r, y, g in zip(refs, ys, yg):
            scale = r.float().abs().max()
            assert float((y.float() - r.float()).abs().max() / scale) <= 2e-3
            assert float((g.float() - r.float()).abs().max() / scale) <= 2e-3


def test_decode_csr_outliers_two_tiles_per_workgroup():
    """The CSR outliers in the two-tile workgroups of large M = 16 launches
    (4-bit, x read from L2)."""
    import ctypes
    import tensorshrink_amd as ts
    from tensorshrink_amd import _lib as L
    q = ts.QuantLinear(ts.quantize_tensor(recipes.gaussian_weight(8192, 4096, 66), bits=4, outlier_frac=0.002))
    v = _csr_view(q)
    x = recipes.activations(16, 4096, seed=5).cuda()
    r = q(x)
    y = torch.empty_like(r)
    dt = L.dtype_code(x.dtype)
    assert L.load().ts_qlinear_forward(ctypes.byref(v), x.data_ptr(), 16, 4096, dt, y.data_ptr(), 8192, dt, None,
                                       None, 0, L.stream_ptr()) == L.TS_OK
    assert float((y.float() - r.float()).abs().max() / r.float().abs().max()) <= 2e-3


def test_reassigned_tensors_rebuild_the_view():
    """A loader that re-creates module tensors by setattr (as transformers
    does for non-persistent buffers after loading) must not leave the kernel
    view on freed memory: QuantLinear has no non-persistent buffers, its
    derived tables are plain attributes, and reassigning any tensor the
    kernels read rebuilds the view."""
    import tensorshrink_amd as ts
    w = recipes.gaussian_weight(256, K, 78)
    ql = ts.QuantLinear(ts.quantize_tensor(w, bits=4, outlier_frac=0.01))
    assert not ql._non_persistent_buffers_set
    assert all(n not in ql._buffers for n in ("outlier_row_ptr", "tile_outliers", "outlier_colsorted"))
    xs = [recipes.activations(M, K, seed=M).cuda() for M in (2, 40)]
    ref = [ql(x) for x in xs]
    for name in ("packed", "scale", "gmin", "outlier_row", "outlier_col", "outlier_delta", "outlier_row_ptr",
                 "tile_outliers", "outlier_colsorted"):
        old = getattr(ql, name)
        setattr(ql, name, old.clone())
        assert getattr(ql, name).data_ptr() != old.data_ptr()
        del old
        torch.cuda.empty_cache()
        for x, r in zip(xs, ref):
            assert torch.equal(ql(x), r), name
    # moved and cast with the module
    ql.half()
    assert ql.outlier_row_ptr.dtype == torch.int32 and ql.tile_outliers.dtype == torch.int64
    for x, r in zip(xs, ref):
        assert torch.equal(ql(x), r)


def test_streaming_and_graphs_bf16_model():
    """A model cast to bf16 (QuantLinear keeps its metadata dtypes) streamed
    from host memory, then captured: outputs equal the resident model's."""
    import tensorshrink_amd as ts
    model = _stack(4).to(torch.bfloat16)
    x = recipes.activations(3, K, seed=9).cuda()
    with torch.no_grad():
        ref = model(x)
        st = ts.stream_offload_module(model, verbose=False)
        assert torch.equal(model(x), ref)
        st.disable()
        model.cuda()
        g = ts.CUDAGraphQuantModel(model)
        for _ in range(3):
            assert torch.equal(g(x), ref)
