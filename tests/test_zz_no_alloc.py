"""ts_build_outlier_tables_noalloc (the entry point that allocates nothing)
against ts_build_outlier_tables with a caller workspace: identical row-sorted
tables, deltas and row offsets, bit for bit, on two calls in a row (the
second with fewer outliers, so stale scratch from the first must not leak
into it), with no change in the device's free memory."""
import ctypes

import numpy as np
import pytest
import torch

import recipes
from gpu_util import say

pytestmark = pytest.mark.gpu


def _layer_and_outliers(rows, cols, seed, frac):
    import tensorshrink_amd as ts
    w = recipes.gaussian_weight(rows, cols, seed, outlier_frac=frac)
    qt = ts.quantize_tensor(w, bits=4, group_size=128, outlier_frac=frac, double_quant=True, nf_quant=True)
    return qt


def _tables(qt, noalloc):
    from tensorshrink_amd import _lib as L
    import tensorshrink_amd as ts
    dev = torch.device("cuda")
    lib = L.lib()
    n = qt.n_outliers()
    # a QuantLinear only to get a kernel view of the layer's code buffers
    ql = ts.QuantLinear(qt)
    view = ql._make_layer(with_outliers=False)
    idx = torch.from_numpy(np.ascontiguousarray(qt.outlier_idx, dtype=np.int32)).to(dev)
    val = torch.from_numpy(np.ascontiguousarray(qt.outlier_val, dtype=np.float16)).to(dev)
    out = dict(row=torch.full((n,), -1, dtype=torch.int32, device=dev),
               col=torch.full((n,), -1, dtype=torch.int32, device=dev),
               delta=torch.zeros(n, dtype=torch.float16, device=dev),
               rp=torch.full((qt.rows + 1,), -1, dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    if noalloc:
        free0 = torch.cuda.mem_get_info()[0]
        rc = lib.ts_build_outlier_tables_noalloc(ctypes.byref(view), idx.data_ptr(), val.data_ptr(), n,
                                                 out["row"].data_ptr(), out["col"].data_ptr(),
                                                 out["delta"].data_ptr(), out["rp"].data_ptr(), L.stream_ptr(dev))
        torch.cuda.synchronize()
        free1 = torch.cuda.mem_get_info()[0]
    else:
        ws_n = lib.ts_outlier_tables_workspace_bytes(n, qt.rows)
        ws = torch.empty(max(1, ws_n), dtype=torch.uint8, device=dev)
        rc = lib.ts_build_outlier_tables(ctypes.byref(view), idx.data_ptr(), val.data_ptr(), n,
                                         out["row"].data_ptr(), out["col"].data_ptr(), out["delta"].data_ptr(),
                                         out["rp"].data_ptr(), ws.data_ptr(), ws.numel(), L.stream_ptr(dev))
        torch.cuda.synchronize()
        free0 = free1 = 0
    L.check(rc, "outlier tables")
    return {k: v.cpu().numpy() for k, v in out.items()}, free0 - free1, ql


def test_noalloc_outlier_tables_match_workspace_version():
    cases = [(1024, 2048, 901, 0.02), (256, 1024, 902, 0.005)]  # second call: fewer outliers
    for i, (rows, cols, seed, frac) in enumerate(cases):
        qt = _layer_and_outliers(rows, cols, seed, frac)
        say("noalloc tables", rows, cols, qt.n_outliers())
        ref, _, ql = _tables(qt, noalloc=False)
        got, grew, _ = _tables(qt, noalloc=True)
        for k in ("row", "col", "delta", "rp"):
            np.testing.assert_array_equal(got[k].view(np.uint8), ref[k].view(np.uint8), err_msg=f"call {i}: {k}")
        # the QuantLinear built through the usual path holds the same tables
        np.testing.assert_array_equal(got["row"], ql.outlier_row.cpu().numpy())
        np.testing.assert_array_equal(got["delta"].view(np.uint16), ql.outlier_delta.cpu().numpy().view(np.uint16))
        if i > 0:
            assert grew == 0, f"device free memory dropped by {grew} bytes"


def test_noalloc_outlier_tables_rejects_oversize():
    from tensorshrink_amd import _lib as L
    qt = _layer_and_outliers(64, 256, 903, 0.01)
    import tensorshrink_amd as ts
    view = ts.QuantLinear(qt)._make_layer(with_outliers=False)
    n = 262145
    buf = torch.zeros(n, dtype=torch.int32, device="cuda")
    rc = L.lib().ts_build_outlier_tables_noalloc(ctypes.byref(view), buf.data_ptr(), buf.data_ptr(), n,
                                                 buf.data_ptr(), buf.data_ptr(), buf.data_ptr(), None,
                                                 L.stream_ptr())
    assert rc == L.TS_BAD_ARG
