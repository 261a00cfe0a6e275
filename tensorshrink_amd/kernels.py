"""Kernel-level API of the reference's triton_kernels.py, on libtensorshrink_hip.

Same names, signatures and "None means not covered" contract as
``fused_quantized_linear`` (triton_kernels.py:714-945),
``apply_outlier_correction`` (:948-991) and ``dequantize_weight``
(:1114-1186), for callers that drive the kernels with QuantLinear-style
buffers directly. ``QuantLinear.forward`` does not go through this module: it
keeps a prebuilt kernel view of its buffers and launches once per call.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib as L

KERNELS_AVAILABLE = True
SUPPORTED_BITS = (2, 4, 6, 8)
SUPPORTED_GROUP_SIZE = 128
_SUPPORTED_GROUP_SIZES = {32, 64, 128, 256}


def _row_ptr(outlier_row: torch.Tensor, rows: int) -> torch.Tensor:
    rp = torch.empty(rows + 1, dtype=torch.int32, device=outlier_row.device)
    L.check(L.lib().ts_outlier_row_ptr(outlier_row.data_ptr(), outlier_row.numel(), rows, rp.data_ptr(),
                                       L.stream_ptr(outlier_row.device)), "outlier row offsets")
    return rp


def tile_outlier_slots(row_ptr: torch.Tensor, outlier_row: torch.Tensor, outlier_col: torch.Tensor,
                       outlier_delta: torch.Tensor, rows: int):
    """Per-16-row-tile outlier slots for the decode kernel (ts_build_tile_outliers):
    returns (slots u64 as int64 [n_tiles * cap], cap). cap is the largest
    per-tile count rounded up to a multiple of 8; reading it back syncs the
    stream, so QuantLinear builds the table once at construction.

    Every tile is padded to the fullest tile's count, so outliers crowded
    into a few tiles would inflate the table: past max(4 x (n + 8 x tiles),
    2^20) slots (8 MiB) no table is built and (empty, 0) is returned; the
    decode kernel then reports the layer as not covered and the forward takes
    the generic kernel."""
    dev = row_ptr.device
    lib = L.lib()
    mx = torch.empty(1, dtype=torch.int32, device=dev)
    L.check(lib.ts_tile_outlier_max(row_ptr.data_ptr(), rows, mx.data_ptr(), L.stream_ptr(dev)), "tile outlier count")
    cap = max(8, (int(mx.item()) + 7) // 8 * 8)
    n_tiles = (rows + 15) // 16
    if n_tiles * cap > max(4 * (outlier_row.numel() + 8 * n_tiles), 1 << 20):
        return torch.zeros(0, dtype=torch.int64, device=dev), 0
    slots = torch.empty(n_tiles * cap, dtype=torch.int64, device=dev)
    L.check(lib.ts_build_tile_outliers(row_ptr.data_ptr(), outlier_row.data_ptr(), outlier_col.data_ptr(),
                                       outlier_delta.data_ptr(), rows, cap, slots.data_ptr(), L.stream_ptr(dev)),
            "tile outlier slots")
    return slots, cap


# Derived outlier tables per set of outlier buffers, so that repeated calls
# with the same QuantLinear-style buffers neither rebuild them nor sync the
# host (the first call builds them; later calls, including ones under graph
# capture, reuse them). Keyed on the buffers' storage and version. A first
# call made under graph capture builds the row offsets and column-sorted
# copy inside the graph (they are then rebuilt on every replay, and not
# cached: their contents exist only once the graph runs) and no tile slots,
# which need a host read; the launch then takes the MFMA or generic kernel.
_DERIVED: dict = {}
_DERIVED_MAX = 256


def _derived_outliers(outlier_row, outlier_col, outlier_delta, rows: int, need_slots: bool):
    key = (outlier_row.device.index, outlier_row.data_ptr(), outlier_row.numel(), outlier_row._version,
           outlier_col.data_ptr(), outlier_col._version, outlier_delta.data_ptr(), outlier_delta._version, rows)
    ent = _DERIVED.get(key)
    capturing = torch.cuda.is_current_stream_capturing()
    if ent is None:
        if len(_DERIVED) >= _DERIVED_MAX and not capturing:
            _DERIVED.pop(next(iter(_DERIVED)))
        dev = outlier_row.device
        rp = _row_ptr(outlier_row, rows)
        ocs = torch.empty(outlier_row.numel(), dtype=torch.int32, device=dev)
        L.check(L.lib().ts_build_colsorted_outliers(rp.data_ptr(), outlier_col.data_ptr(), outlier_delta.data_ptr(),
                                                    rows, ocs.data_ptr(), L.stream_ptr(dev)), "column-sorted outliers")
        ent = {"rp": rp, "ocs": ocs, "slots": None, "cap": 0,
               "keep": (outlier_row, outlier_col, outlier_delta)}
        if capturing:
            return ent
        _DERIVED[key] = ent
    if need_slots and ent["slots"] is None and not capturing:
        ent["slots"], ent["cap"] = tile_outlier_slots(ent["rp"], outlier_row, outlier_col, outlier_delta, rows)
    return ent


def fused_quantized_linear(
    x: torch.Tensor, packed: torch.Tensor, scale: Optional[torch.Tensor], gmin: Optional[torch.Tensor],
    bias: Optional[torch.Tensor], bits: int, group_size: int, cols: int, out_features: int,
    compute_dtype: torch.dtype, return_fp32: bool = False, out: Optional[torch.Tensor] = None,
    outlier_row: Optional[torch.Tensor] = None, outlier_col: Optional[torch.Tensor] = None,
    outlier_delta: Optional[torch.Tensor] = None, outliers_sorted: bool = True, use_buffer_pool: bool = True,
    codebook: Optional[torch.Tensor] = None, dq_scale_codes: Optional[torch.Tensor] = None,
    dq_scale_meta: Optional[torch.Tensor] = None, dq_gmin_codes: Optional[torch.Tensor] = None,
    dq_gmin_meta: Optional[torch.Tensor] = None, dq_group_size: int = 0, n_groups: Optional[int] = None,
    stage2_packed: Optional[torch.Tensor] = None, stage2_scale: Optional[torch.Tensor] = None,
    stage2_gmin: Optional[torch.Tensor] = None,
) -> Optional[torch.Tensor]:
    """y = x W^T + outliers (+ bias) with fp32 accumulation; None when not covered."""
    if not x.is_cuda or bits not in SUPPORTED_BITS or compute_dtype not in (torch.float16, torch.bfloat16):
        return None
    if n_groups is None:
        if scale is None:
            return None
        n_groups = scale.shape[1]
    if outlier_row is not None and outlier_row.numel() > 0 and not outliers_sorted:
        return None
    lib = L.lib()
    x2d = x.reshape(-1, x.shape[-1]).to(compute_dtype).contiguous()
    M = x2d.shape[0]
    s = L.QLayer()
    s.bits, s.group_size = bits, group_size
    s.rows, s.cols, s.n_groups = out_features, cols, n_groups
    s.padded_cols = n_groups * group_size
    s.packed, s.packed_stride = packed.data_ptr(), packed.shape[1]
    if dq_scale_codes is not None:
        s.dq_scale_codes, s.dq_scale_meta = dq_scale_codes.data_ptr(), dq_scale_meta.data_ptr()
        s.dq_gmin_codes, s.dq_gmin_meta = dq_gmin_codes.data_ptr(), dq_gmin_meta.data_ptr()
        s.dq_group_size = dq_group_size
    else:
        sc16 = scale.to(torch.float16).contiguous()
        gm16 = gmin.to(torch.float16).contiguous()
        s.scale, s.gmin = sc16.data_ptr(), gm16.data_ptr()
    cb = codebook.to(torch.float32).contiguous() if codebook is not None else None
    s.codebook = L.ptr(cb)
    if stage2_packed is not None:
        s.stage2_packed, s.stage2_stride = stage2_packed.data_ptr(), stage2_packed.shape[1]
        s.stage2_scale, s.stage2_gmin = stage2_scale.data_ptr(), stage2_gmin.data_ptr()
    if outlier_row is not None and outlier_row.numel() > 0:
        ent = _derived_outliers(outlier_row, outlier_col, outlier_delta, out_features, need_slots=M <= 128)
        s.outlier_row, s.outlier_col = outlier_row.data_ptr(), outlier_col.data_ptr()
        s.outlier_delta, s.n_outliers = outlier_delta.data_ptr(), outlier_row.numel()
        s.outlier_row_ptr = ent["rp"].data_ptr()
        if s.padded_cols < 65535:
            s.outlier_colsorted = ent["ocs"].data_ptr()
        if ent["slots"] is not None and ent["cap"] > 0:  # the decode kernel reads outliers per tile
            s.tile_outliers, s.tile_outlier_cap = ent["slots"].data_ptr(), ent["cap"]
    ydt = torch.float32 if return_fp32 else compute_dtype
    if out is None or out.shape != (M, out_features) or out.dtype != ydt or not out.is_contiguous():
        out = torch.empty(M, out_features, dtype=ydt, device=x.device)
    b = bias.to(compute_dtype).contiguous() if bias is not None else None
    # the prefill kernel's K-split partial sums, where the shape uses them
    nws = lib.ts_forward_partials_bytes(ctypes.byref(s), M) if M > 16 else 0
    ws = torch.empty(nws, dtype=torch.uint8, device=x.device) if nws else None
    rc = lib.ts_qlinear_forward(ctypes.byref(s), x2d.data_ptr(), M, x2d.shape[1], L.dtype_code(compute_dtype),
                                out.data_ptr(), out_features, L.dtype_code(ydt), L.ptr(b), L.ptr(ws), nws,
                                L.stream_ptr(x.device))
    if rc == L.TS_NOT_COVERED:
        return None
    L.check(rc, "fused_quantized_linear")
    return out.reshape(*x.shape[:-1], out_features)


def apply_outlier_correction(out: torch.Tensor, x2d: torch.Tensor, outlier_row: torch.Tensor,
                             outlier_col: torch.Tensor, outlier_delta: torch.Tensor) -> Optional[torch.Tensor]:
    """out[m, row[k]] += x[m, col[k]] * delta[k] on an fp32 result; tables sorted by row."""
    if not out.is_cuda or out.dtype != torch.float32:
        return None
    n = outlier_row.numel()
    if n == 0:
        return out
    out2d = out.reshape(-1, out.shape[-1])
    rows = out2d.shape[1]
    rp = _derived_outliers(outlier_row, outlier_col, outlier_delta, rows, need_slots=False)["rp"]
    x2d = x2d.contiguous()
    L.check(L.lib().ts_apply_outlier_correction(out2d.data_ptr(), out2d.shape[0], out2d.stride(0), x2d.data_ptr(),
                                                x2d.stride(0), L.dtype_code(x2d.dtype), rp.data_ptr(),
                                                outlier_col.data_ptr(), outlier_delta.data_ptr(), rows,
                                                L.stream_ptr(out.device)), "apply_outlier_correction")
    return out


def dequantize_weight(packed: torch.Tensor, scale: torch.Tensor, gmin: torch.Tensor, bits: int, rows: int,
                      cols: int, padded_cols: int, n_groups: int, group_size: int = SUPPORTED_GROUP_SIZE,
                      compute_dtype: torch.dtype = torch.float16,
                      codebook: Optional[torch.Tensor] = None) -> Optional[torch.Tensor]:
    """Dense W [rows, cols] in compute_dtype, no outliers (the caller folds
    them in, as modules.py:912-919 does). scale/gmin are taken at f16."""
    if not packed.is_cuda or bits not in (2, 4, 8):
        return None
    s = L.QLayer()
    s.bits, s.group_size, s.rows, s.cols, s.padded_cols, s.n_groups = bits, group_size, rows, cols, padded_cols, n_groups
    s.packed, s.packed_stride = packed.data_ptr(), packed.shape[1]
    sc16 = scale.to(torch.float16).contiguous()
    gm16 = gmin.to(torch.float16).contiguous()
    s.scale, s.gmin = sc16.data_ptr(), gm16.data_ptr()
    cb = codebook.to(torch.float32).contiguous() if codebook is not None else None
    s.codebook = L.ptr(cb)
    out = torch.empty(rows, cols, dtype=compute_dtype, device=packed.device)
    L.check(L.lib().ts_dequantize(ctypes.byref(s), L.TS_DEQ_QLINEAR, None, None, 0, out.data_ptr(), cols,
                                  L.dtype_code(compute_dtype), L.stream_ptr(packed.device)), "dequantize_weight")
    return out
