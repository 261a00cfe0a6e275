"""ctypes binding of libtensorshrink_hip.so (include/tensorshrink_hip.h).

The library is the only compute path of this package: there is no CPU or
PyTorch fallback. Loading fails loudly when the shared library has not been
built (``python -m tensorshrink_amd.build``) and every entry point raises when
no ROCm GPU is visible.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libtensorshrink_hip.so")

TS_OK, TS_NOT_COVERED, TS_BAD_ARG, TS_HIP_ERROR, TS_WORKSPACE = 0, 1, 2, 3, 4
TS_F16, TS_BF16, TS_F32 = 0, 1, 2
TS_DEQ_CODEC, TS_DEQ_QLINEAR = 0, 1

_DTYPE_CODE = {torch.float16: TS_F16, torch.bfloat16: TS_BF16, torch.float32: TS_F32}

c_i32, c_i64, c_f32, c_vp, c_sz = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t


class QLayer(ctypes.Structure):
    """Mirror of ts_qlayer."""
    _fields_ = [
        ("bits", c_i32), ("group_size", c_i32),
        ("rows", c_i64), ("cols", c_i64), ("padded_cols", c_i64), ("n_groups", c_i64),
        ("packed", c_vp), ("packed_stride", c_i64),
        ("scale", c_vp), ("gmin", c_vp),
        ("dq_scale_codes", c_vp), ("dq_scale_meta", c_vp), ("dq_gmin_codes", c_vp), ("dq_gmin_meta", c_vp),
        ("dq_group_size", c_i64),
        ("codebook", c_vp),
        ("outlier_row", c_vp), ("outlier_col", c_vp), ("outlier_delta", c_vp), ("n_outliers", c_i64),
        ("outlier_row_ptr", c_vp),
        ("stage2_packed", c_vp), ("stage2_stride", c_i64), ("stage2_scale", c_vp), ("stage2_gmin", c_vp),
        ("tile_outliers", c_vp), ("tile_outlier_cap", c_i64), ("codebook_host", c_vp),
        ("outlier_colsorted", c_vp),
    ]


class QInput(ctypes.Structure):
    """Mirror of ts_qinput."""
    _fields_ = [("w", c_vp), ("w_dtype", ctypes.c_int), ("rows", c_i64), ("cols", c_i64)]


class GroupOpts(ctypes.Structure):
    """Mirror of ts_group_opts."""
    _fields_ = [("bits", c_i32), ("group_size", c_i32), ("threshold", c_f32), ("clamp", c_i32),
                ("codebook", c_vp), ("codebook_len", c_i32)]


# name -> (restype, argtypes); the declarations of include/tensorshrink_hip.h
PROTOTYPES = {
    "ts_status_str": (ctypes.c_char_p, [ctypes.c_int]),
    "ts_version": (ctypes.c_char_p, []),
    "ts_forward_workspace_bytes": (c_sz, [ctypes.POINTER(QLayer), c_i64]),
    "ts_forward_partials_bytes": (c_sz, [ctypes.POINTER(QLayer), c_i64]),
    "ts_qlinear_forward": (ctypes.c_int, [ctypes.POINTER(QLayer), c_vp, c_i64, c_i64, ctypes.c_int, c_vp, c_i64,
                                          ctypes.c_int, c_vp, c_vp, c_sz, c_vp]),
    "ts_qlinear_forward_group": (ctypes.c_int, [ctypes.POINTER(ctypes.POINTER(QLayer)), ctypes.c_int, c_vp, c_i64,
                                                c_i64, ctypes.c_int, ctypes.POINTER(c_vp), ctypes.POINTER(c_i64),
                                                ctypes.c_int, ctypes.POINTER(c_vp), c_vp]),
    "ts_apply_outlier_correction": (ctypes.c_int, [c_vp, c_i64, c_i64, c_vp, c_i64, ctypes.c_int, c_vp, c_vp, c_vp,
                                                   c_i64, c_vp]),
    "ts_dequantize": (ctypes.c_int, [ctypes.POINTER(QLayer), ctypes.c_int, c_vp, c_vp, c_i64, c_vp, c_i64,
                                     ctypes.c_int, c_vp]),
    "ts_outlier_row_ptr": (ctypes.c_int, [c_vp, c_i64, c_i64, c_vp, c_vp]),
    "ts_outlier_tables_workspace_bytes": (c_sz, [c_i64, c_i64]),
    "ts_tile_outlier_max": (ctypes.c_int, [c_vp, c_i64, c_vp, c_vp]),
    "ts_build_tile_outliers": (ctypes.c_int, [c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_vp, c_vp]),
    "ts_build_colsorted_outliers": (ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_vp, c_vp]),
    "ts_build_outlier_tables_noalloc": (ctypes.c_int, [ctypes.POINTER(QLayer), c_vp, c_vp, c_i64, c_vp, c_vp, c_vp,
                                                       c_vp, c_vp]),
    "ts_build_outlier_tables": (ctypes.c_int, [ctypes.POINTER(QLayer), c_vp, c_vp, c_i64, c_vp, c_vp, c_vp, c_vp,
                                               c_vp, c_sz, c_vp]),
    "ts_topk_workspace_bytes": (c_sz, [c_i64, c_i64]),
    "ts_topk_candidates_count": (ctypes.c_int, [ctypes.POINTER(QInput), c_i64, c_vp, c_sz, ctypes.POINTER(c_i64),
                                                c_vp]),
    "ts_topk_candidates_write": (ctypes.c_int, [ctypes.POINTER(QInput), c_i64, c_vp, c_vp, c_vp, c_vp]),
    "ts_topk_select": (ctypes.c_int, [c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp]),
    "ts_quantize_groups": (ctypes.c_int, [ctypes.POINTER(QInput), ctypes.POINTER(GroupOpts), c_vp, c_i64, c_vp,
                                          c_vp, c_vp, c_vp, c_vp]),
    "ts_lm_sample": (ctypes.c_int, [ctypes.POINTER(QInput), ctypes.POINTER(GroupOpts), c_vp, c_vp, c_vp, c_i64,
                                    c_vp, c_vp]),
    "ts_lloyd_max_fit_host": (ctypes.c_int, [c_vp, c_i64, c_vp, c_i32, c_i32, c_vp]),
    "ts_gather_f16": (ctypes.c_int, [c_vp, ctypes.c_int, c_vp, c_i64, c_vp, c_vp]),
    "ts_double_quantize": (ctypes.c_int, [c_vp, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp]),
    "ts_rvq_residual": (ctypes.c_int, [ctypes.POINTER(QInput), ctypes.POINTER(QLayer), c_vp, c_vp, c_i64, c_vp,
                                       c_vp]),
    "ts_sq_error_sums": (ctypes.c_int, [ctypes.POINTER(QInput), c_vp, ctypes.c_int, c_vp, c_vp]),
}

_lib: Optional[ctypes.CDLL] = None


class KernelError(RuntimeError):
    """A libtensorshrink_hip entry point returned an error status."""


class NotCovered(KernelError):
    """TS_NOT_COVERED: a shape or format outside what the kernels cover."""


def load() -> ctypes.CDLL:
    """Load and type the shared library (no GPU needed)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built: run `python -m tensorshrink_amd.build` (hipcc, gfx950). "
                "tensorshrink_amd has no CPU fallback.")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def lib() -> ctypes.CDLL:
    """The library, after checking that a GPU is visible."""
    if not torch.cuda.is_available():
        raise RuntimeError("tensorshrink_amd needs a ROCm GPU (MI355X / gfx950); none is visible and there is "
                           "no CPU fallback")
    return load()


def check(rc: int, what: str) -> None:
    if rc == TS_OK:
        return
    msg = load().ts_status_str(rc).decode()
    if rc == TS_NOT_COVERED:
        raise NotCovered(f"{what}: {msg}")
    raise KernelError(f"{what}: {msg} (status {rc})")


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def stream_ptr(device: Optional[torch.device] = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}; expected float16, bfloat16 or float32") from None
