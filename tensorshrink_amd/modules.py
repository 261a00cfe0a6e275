"""QuantLinear and quantize_module on the MI355X kernels.

Drop-in for modules.py of GDNickk/tensorshrink v0.4.0: ``QuantLinear``
(modules.py:282-1026) registers the same buffers with the same names, dtypes
and contents (packed, scale/gmin or dq_*, codebook, outlier_row/col sorted by
row, outlier_delta, bias), and ``quantize_module`` (modules.py:1258-1455) takes
the same arguments. The forward runs one libtensorshrink_hip launch per call
(decode kernel for M <= 16 and small M on short layers, MFMA prefill kernel
above), with the outlier
correction and bias fused; there is no CPU or PyTorch fallback path.

Additions over the reference:
  * derived tensors, built from the outlier buffers at construction and kept
    as plain attributes (not buffers: absent from state_dict, and left alone
    by loaders that re-create non-persistent buffers), which ``_apply`` moves
    with the module:
    ``outlier_row_ptr`` - int32 [rows + 1] CSR offsets into the row-sorted
    outlier tables;
    ``tile_outliers`` - per-16-row-tile outlier slots (u64: col, row in tile,
    f16 delta; ``tile_outlier_cap`` slots per tile) that the decode kernel
    reads at a fixed address;
    ``outlier_colsorted`` - per-row column-sorted outliers (u32: col | f16
    delta << 16) that the prefill kernel walks while it dequantizes a row;
  * the kernel view (raw addresses of every tensor the kernels read) is
    rebuilt whenever one of those tensors is reassigned or the module is
    moved or cast;
  * 6-bit RVQ layers register ``stage2_packed``, ``stage2_scale`` and
    ``stage2_gmin`` (the reference QuantLinear cannot serve bits=6).
``WeightCache`` (a dense-weight cache) is not part of this path: passing
``cache=`` raises.
"""
from __future__ import annotations

import ctypes
from typing import Iterable, List, Optional, Sequence, Tuple, Union

import numpy as np
import torch
import torch.nn as nn

from . import _lib as L
from .codec import (
    DEFAULT_DQ_GROUP_SIZE,
    LayerBitStats,
    QuantizedTensor,
    TopkPrefetch,
    budget_allocate_bits,
    estimate_resident_nbytes as _estimate_resident_nbytes,
    quantize_tensor,
    quantize_tensor_adaptive,
    relative_error,
)

DEFAULT_SKIP_PATTERNS = ("norm", "ln_", "embed", "lm_head", "shared", "position")
DEFAULT_MIN_NUMEL = 16384
DEFAULT_MAX_DEQUANT_ROWS = 4096
T5_EXTRA_SKIP_PATTERNS = (".wo",)


class QuantLinear(nn.Module):
    """nn.Linear replacement backed by packed 2/4/6/8-bit GOAP weights."""

    def __init__(self, qt: QuantizedTensor, bias: Optional[torch.Tensor] = None,
                 max_dequant_rows: Union[int, str] = DEFAULT_MAX_DEQUANT_ROWS, force_fp32_compute: bool = False,
                 cache=None, fast_dequant: bool = True, use_triton: bool = True,
                 device: Optional[torch.device] = None):
        super().__init__()
        if len(qt.orig_shape) != 2:
            raise ValueError("QuantLinear requires a 2D weight (out_features, in_features)")
        if cache is not None:
            raise NotImplementedError("WeightCache is not part of the tensorshrink_amd path")
        if qt.smooth_scale is not None:
            raise NotImplementedError("smooth-scaled tensors are not covered by tensorshrink_amd")
        self.out_features, self.in_features = qt.orig_shape
        self.bits = qt.bits
        self.group_size = qt.group_size
        self.rows, self.cols = qt.rows, qt.cols
        self.padded_cols = qt.padded_cols
        self.n_groups = qt.n_groups
        self.orig_dtype_str = qt.orig_dtype
        self.max_dequant_rows = DEFAULT_MAX_DEQUANT_ROWS if max_dequant_rows == "auto" else max(1, int(max_dequant_rows))
        self.cache = None
        self.fast_dequant = fast_dequant
        self.use_triton = use_triton
        self.force_fp32_compute = force_fp32_compute
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device()) \
            if torch.cuda.is_available() else None
        if dev is None or dev.type != "cuda":
            L.lib()  # raises: no GPU
        lib = L.lib()

        def t(a, dtype=None):
            x = torch.from_numpy(np.ascontiguousarray(a))
            return (x.to(dtype) if dtype is not None else x).to(dev)

        self.register_buffer("packed", t(qt.packed))
        self.double_quant = qt.dq_scale_codes is not None
        if self.double_quant:
            self.dq_group_size = int(qt.dq_scale_codes.shape[0] // qt.dq_scale_meta.shape[0])
            self.register_buffer("dq_scale_codes", t(qt.dq_scale_codes))
            self.register_buffer("dq_scale_meta", t(qt.dq_scale_meta))
            self.register_buffer("dq_gmin_codes", t(qt.dq_gmin_codes))
            self.register_buffer("dq_gmin_meta", t(qt.dq_gmin_meta))
            self.scale = None
            self.gmin = None
        else:
            self.dq_group_size = 0
            self.register_buffer("scale", t(qt.scale))
            self.register_buffer("gmin", t(qt.gmin))
        self.companded = qt.codebook is not None
        if self.companded:
            self.register_buffer("codebook", t(qt.codebook, torch.float32))
        else:
            self.codebook = None
        if qt.bits == 6:
            self.register_buffer("stage2_packed", t(qt.stage2_packed))
            self.register_buffer("stage2_scale", t(qt.stage2_scale))
            self.register_buffer("stage2_gmin", t(qt.stage2_gmin))

        # Outlier tables (modules.py:414-448) built on the GPU: stable row
        # sort, delta = f16(val - base) with QuantLinear's float32 scale/gmin.
        n = qt.n_outliers()
        orow = torch.empty(n, dtype=torch.int32, device=dev)
        ocol = torch.empty(n, dtype=torch.int32, device=dev)
        odelta = torch.empty(n, dtype=torch.float16, device=dev)
        rptr = torch.empty(self.rows + 1, dtype=torch.int32, device=dev)
        idx = t(np.ascontiguousarray(qt.outlier_idx, dtype=np.int32))
        val = t(np.ascontiguousarray(qt.outlier_val, dtype=np.float16))
        layer = self._make_layer(with_outliers=False)
        ws_n = lib.ts_outlier_tables_workspace_bytes(n, self.rows)
        ws = torch.empty(max(1, ws_n), dtype=torch.uint8, device=dev)
        with torch.cuda.device(dev):
            L.check(lib.ts_build_outlier_tables(ctypes.byref(layer), idx.data_ptr(), val.data_ptr(), n,
                                                orow.data_ptr(), ocol.data_ptr(), odelta.data_ptr(),
                                                rptr.data_ptr(), ws.data_ptr(), ws.numel(), L.stream_ptr(dev)),
                    "outlier tables")
        self.register_buffer("outlier_row", orow)
        self.register_buffer("outlier_col", ocol)
        self.register_buffer("outlier_delta", odelta)
        self.outlier_row_ptr = rptr
        # derived per-tile slots for the decode kernel (fixed-address loads)
        if n > 0:
            from .kernels import tile_outlier_slots
            with torch.cuda.device(dev):
                slots, self.tile_outlier_cap = tile_outlier_slots(rptr, orow, ocol, odelta, self.rows)
        else:
            slots, self.tile_outlier_cap = torch.zeros(0, dtype=torch.int64, device=dev), 0
        self.tile_outliers = slots
        # derived column-sorted copy per row for the prefill kernel
        ocs = torch.empty(n, dtype=torch.int32, device=dev)
        if n > 0:
            with torch.cuda.device(dev):
                L.check(lib.ts_build_colsorted_outliers(rptr.data_ptr(), ocol.data_ptr(), odelta.data_ptr(),
                                                        self.rows, ocs.data_ptr(), L.stream_ptr(dev)),
                        "column-sorted outliers")
        self.outlier_colsorted = ocs
        if bias is not None:
            self.register_buffer("bias", bias.detach().clone().to(dev))
        else:
            self.bias = None
        self._layer = None
        self._bias_cache = {}
        self._rebuild_cache()
        self._view_tracking = True

    # -- kernel view -----------------------------------------------------
    def _make_layer(self, with_outliers: bool = True) -> L.QLayer:
        s = L.QLayer()
        s.bits, s.group_size = self.bits, self.group_size
        s.rows, s.cols, s.padded_cols, s.n_groups = self.rows, self.cols, self.padded_cols, self.n_groups
        s.packed = self.packed.data_ptr()
        s.packed_stride = self.packed.shape[1]
        if self.double_quant:
            s.dq_scale_codes = self.dq_scale_codes.data_ptr()
            s.dq_scale_meta = self.dq_scale_meta.data_ptr()
            s.dq_gmin_codes = self.dq_gmin_codes.data_ptr()
            s.dq_gmin_meta = self.dq_gmin_meta.data_ptr()
            s.dq_group_size = self.dq_group_size
        else:
            s.scale = self.scale.data_ptr()
            s.gmin = self.gmin.data_ptr()
        if self.companded:
            s.codebook = self.codebook.data_ptr()
            # host copy kept alive with the view (decode takes <= 16 entries as
            # launch arguments); read back only when the codebook changed
            key = (id(self.codebook), self.codebook.data_ptr(), self.codebook._version)
            if getattr(self, "_codebook_key", None) != key:
                self._codebook_host = np.ascontiguousarray(self.codebook.detach().cpu().numpy(), dtype=np.float32)
                self._codebook_key = key
            s.codebook_host = self._codebook_host.ctypes.data
        if self.bits == 6:
            s.stage2_packed = self.stage2_packed.data_ptr()
            s.stage2_stride = self.stage2_packed.shape[1]
            s.stage2_scale = self.stage2_scale.data_ptr()
            s.stage2_gmin = self.stage2_gmin.data_ptr()
        if with_outliers and self.outlier_row.numel() > 0:
            s.outlier_row = self.outlier_row.data_ptr()
            s.outlier_col = self.outlier_col.data_ptr()
            s.outlier_delta = self.outlier_delta.data_ptr()
            s.n_outliers = self.outlier_row.numel()
            s.outlier_row_ptr = self.outlier_row_ptr.data_ptr()
            if self.tile_outlier_cap > 0:
                s.tile_outliers = self.tile_outliers.data_ptr()
                s.tile_outlier_cap = self.tile_outlier_cap
            if self.padded_cols < 65535:
                s.outlier_colsorted = self.outlier_colsorted.data_ptr()
        return s

    def _rebuild_cache(self) -> None:
        self._layer = self._make_layer() if self.packed.is_cuda else None
        self._bias_cache = {}

    # Tensors whose addresses the kernel view holds, and the derived ones
    # among them (plain attributes, moved by _apply).
    _KERNEL_TENSORS = frozenset((
        "packed", "scale", "gmin", "dq_scale_codes", "dq_scale_meta", "dq_gmin_codes", "dq_gmin_meta", "codebook",
        "stage2_packed", "stage2_scale", "stage2_gmin", "outlier_row", "outlier_col", "outlier_delta", "bias",
        "outlier_row_ptr", "tile_outliers", "outlier_colsorted"))
    _DERIVED = ("outlier_row_ptr", "tile_outliers", "outlier_colsorted")

    def __setattr__(self, name, value):
        super().__setattr__(name, value)
        # a reassigned tensor (e.g. a loader setting a buffer) gets a view on
        # its new address; in-place updates keep their address
        if name in QuantLinear._KERNEL_TENSORS and self.__dict__.get("_view_tracking", False):
            self._rebuild_cache()

    def _set_tensors(self, tensors: dict) -> None:
        """Reassign several kernel tensors (buffers or derived) at once and
        rebuild the view once."""
        for n, v in tensors.items():
            if n in self._buffers:
                self._buffers[n] = v
            else:
                self.__dict__[n] = v
        self._rebuild_cache()

    def _kernel_tensor(self, name: str) -> Optional[torch.Tensor]:
        return self._buffers[name] if name in self._buffers else self.__dict__.get(name)

    # Buffers the kernels read with a fixed element type. Module-wide casts
    # (`.half()`, `.to(torch.bfloat16)`) convert every floating buffer; these
    # are cast back so the kernel view keeps reading them as it expects (the
    # reference casts its metadata to float32 where it uses it, so the same
    # flow works there).
    _FIXED_DTYPES = {
        "scale": torch.float16, "gmin": torch.float16, "dq_scale_meta": torch.float16,
        "dq_gmin_meta": torch.float16, "codebook": torch.float32, "outlier_delta": torch.float16,
        "stage2_scale": torch.float16, "stage2_gmin": torch.float16,
    }

    def _apply(self, fn, recurse=True):
        result = super()._apply(fn, recurse=recurse)
        for name in self._DERIVED:
            t = self.__dict__.get(name)
            if t is not None:
                self.__dict__[name] = fn(t)
        for name, dt in self._FIXED_DTYPES.items():
            b = self._buffers.get(name)
            if b is not None and b.dtype != dt:
                self._buffers[name] = b.to(dt)
        self._rebuild_cache()
        return result

    # -- introspection (modules.py:527-593) ------------------------------
    @property
    def weight(self) -> torch.Tensor:
        return torch.empty(self.out_features, self.in_features, dtype=torch.int8, device="meta")

    def packed_nbytes(self) -> int:
        n = self.packed.numel() * self.packed.element_size()
        if self.double_quant:
            for b in (self.dq_scale_codes, self.dq_scale_meta, self.dq_gmin_codes, self.dq_gmin_meta):
                n += b.numel() * b.element_size()
        else:
            n += self.scale.numel() * self.scale.element_size() + self.gmin.numel() * self.gmin.element_size()
        if self.bits == 6:
            for b in (self.stage2_packed, self.stage2_scale, self.stage2_gmin):
                n += b.numel() * b.element_size()
        for b in (self.outlier_row, self.outlier_col, self.outlier_delta):
            n += b.numel() * b.element_size()
        return n

    @staticmethod
    def estimate_resident_nbytes(qt: QuantizedTensor) -> int:
        return _estimate_resident_nbytes(qt)

    def dense_equiv_nbytes(self, itemsize: int = 2) -> int:
        return self.out_features * self.in_features * itemsize

    def dequantize_weight(self, dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """Dense W [out, in] as this layer computes with it (outliers = base + delta)."""
        w = torch.empty(self.rows, self.cols, dtype=dtype, device=self.packed.device)
        L.check(L.lib().ts_dequantize(ctypes.byref(self._layer), L.TS_DEQ_QLINEAR, None, None, 0, w.data_ptr(),
                                      self.cols, L.dtype_code(dtype), L.stream_ptr(self.packed.device)),
                "dequantize")
        return w

    def to_quantized_tensor(self) -> QuantizedTensor:
        """Rebuild a QuantizedTensor (modules.py:595-645); outlier_val = f16(base + delta)."""
        row = self.outlier_row.cpu().numpy().astype(np.int64)
        col = self.outlier_col.cpu().numpy().astype(np.int64)
        idx = (row * self.cols + col).astype(np.int32)
        if self.bits == 6:
            # RVQ: the delta is relative to stage 1 (the stage-2 residual is
            # added everywhere, outliers included), so the stored value is
            # f16(stage-1 base + delta)
            s1 = self._make_layer(with_outliers=False)
            s1.bits, s1.stage2_packed, s1.stage2_scale, s1.stage2_gmin, s1.stage2_stride = 4, None, None, None, 0
            base = torch.empty(self.rows, self.cols, dtype=torch.float32, device=self.packed.device)
            L.check(L.lib().ts_dequantize(ctypes.byref(s1), L.TS_DEQ_QLINEAR, None, None, 0, base.data_ptr(),
                                          self.cols, L.dtype_code(torch.float32), L.stream_ptr(self.packed.device)),
                    "dequantize")
            w = base.reshape(-1)[torch.from_numpy(idx.astype(np.int64)).to(base.device)] + \
                self.outlier_delta.to(torch.float32)
        else:
            w = self.dequantize_weight(torch.float32).reshape(-1)[
                torch.from_numpy(idx.astype(np.int64)).to(self.packed.device)]
        oval = w.to(torch.float16).cpu().numpy() if idx.size else np.zeros(0, np.float16)
        kw = dict(orig_shape=(self.out_features, self.in_features), orig_dtype=self.orig_dtype_str, bits=self.bits,
                  group_size=self.group_size, rows=self.rows, cols=self.cols, padded_cols=self.padded_cols,
                  n_groups=self.n_groups, packed=self.packed.cpu().numpy(), outlier_idx=idx, outlier_val=oval)
        if self.double_quant:
            kw.update(dq_scale_codes=self.dq_scale_codes.cpu().numpy(), dq_scale_meta=self.dq_scale_meta.cpu().numpy(),
                      dq_gmin_codes=self.dq_gmin_codes.cpu().numpy(), dq_gmin_meta=self.dq_gmin_meta.cpu().numpy())
            sc = self.dq_scale_codes.cpu().numpy().astype(np.float32).reshape(self.dq_scale_meta.shape[0], -1)
            gc = self.dq_gmin_codes.cpu().numpy().astype(np.float32).reshape(self.dq_gmin_meta.shape[0], -1)
            sm = self.dq_scale_meta.cpu().numpy().astype(np.float32)
            gm = self.dq_gmin_meta.cpu().numpy().astype(np.float32)
            n = self.rows * self.n_groups
            kw["scale"] = (sc * sm[:, :1] + sm[:, 1:]).ravel()[:n].reshape(self.rows, self.n_groups).astype(np.float16)
            kw["gmin"] = (gc * gm[:, :1] + gm[:, 1:]).ravel()[:n].reshape(self.rows, self.n_groups).astype(np.float16)
        else:
            kw.update(scale=self.scale.cpu().numpy(), gmin=self.gmin.cpu().numpy())
        if self.companded:
            kw["codebook"] = self.codebook.cpu().numpy()
        if self.bits == 6:
            kw.update(stage2_packed=self.stage2_packed.cpu().numpy(), stage2_scale=self.stage2_scale.cpu().numpy(),
                      stage2_gmin=self.stage2_gmin.cpu().numpy())
        return QuantizedTensor(**kw)

    # -- forward (modules.py:819-940) -------------------------------------
    def _bias_as(self, dtype: torch.dtype) -> Optional[torch.Tensor]:
        if self.bias is None:
            return None
        # keyed on the bias tensor and its version: a reassigned or updated
        # bias is converted again
        key = (dtype, id(self.bias), self.bias._version)
        b = self._bias_cache.get(key)
        if b is None:
            self._bias_cache = {k: v for k, v in self._bias_cache.items() if k[1:] == key[1:]}
            b = self.bias.to(dtype).contiguous()
            self._bias_cache[key] = b
        return b

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self._layer is None or not x.is_cuda:
            raise RuntimeError("QuantLinear.forward runs on the GPU kernels only: move the module and the input "
                               "to a ROCm device")
        in_dtype = x.dtype
        M = 1
        for d in x.shape[:-1]:
            M *= d
        lead = x.shape[:-1]
        x2d = x.reshape(M, self.in_features)
        if self.force_fp32_compute or in_dtype == torch.float32:
            # fp32 compute: GPU dequant (QuantLinear view) + a plain library GEMM.
            w = self.dequantize_weight(torch.float32)
            b = self._bias_as(torch.float32)
            y = torch.nn.functional.linear(x2d.to(torch.float32), w, b)
            return y.to(in_dtype).reshape(*lead, self.out_features)
        if in_dtype not in (torch.float16, torch.bfloat16):
            raise TypeError(f"unsupported activation dtype {in_dtype}")
        if not x2d.is_contiguous():
            x2d = x2d.contiguous()
        y = torch.empty(M, self.out_features, dtype=in_dtype, device=x.device)
        b = self._bias_as(in_dtype)
        dt = L.dtype_code(in_dtype)
        lib = L.load()
        # the decode kernel (M <= 16, and blocks of 16 tokens up to 24-32 rows
        # on layers of at most 4096 rows and 6-bit codes), else the fused
        # dequant-into-LDS MFMA kernel;
        # its fp32 K-split partial sums, where the shape uses them, in a
        # workspace from torch's caching allocator (never the GEMM library
        # path's size)
        nws = lib.ts_forward_partials_bytes(ctypes.byref(self._layer), M) if M > 16 else 0
        ws = torch.empty(nws, dtype=torch.uint8, device=x.device) if nws else None
        with torch.cuda.device(x.device):
            L.check(lib.ts_qlinear_forward(ctypes.byref(self._layer), x2d.data_ptr(), M, self.in_features, dt,
                                           y.data_ptr(), self.out_features, dt, L.ptr(b),
                                           L.ptr(ws), nws, L.stream_ptr(x.device)), "qlinear forward")
        return y.reshape(*lead, self.out_features)

    @staticmethod
    def forward_group(layers: Sequence["QuantLinear"], x: torch.Tensor) -> List[torch.Tensor]:
        """[layer(x) for layer in layers] in one kernel launch when the layers
        share a format and the input has at most 16 rows, or at most 32 with
        at most 12288 weight rows in all (q/k/v or gate/up at decode; q/k/v
        at short prefills); otherwise, or when the launch is not covered, one
        forward per layer. No counterpart in the reference, whose model code
        calls each QuantLinear in turn (modules.py:896-905)."""
        layers = list(layers)
        in_dtype = x.dtype
        M = 1
        for d in x.shape[:-1]:
            M *= d
        ok = (1 <= len(layers) <= 4 and M <= 32 and x.is_cuda and in_dtype in (torch.float16, torch.bfloat16)
              and all(q._layer is not None and not q.force_fp32_compute and q.in_features == layers[0].in_features
                      for q in layers))
        if ok:
            lead = x.shape[:-1]
            x2d = x.reshape(M, layers[0].in_features)
            if not x2d.is_contiguous():
                x2d = x2d.contiguous()
            ys = [torch.empty(M, q.out_features, dtype=in_dtype, device=x.device) for q in layers]
            bs = [q._bias_as(in_dtype) for q in layers]
            n = len(layers)
            qls = (ctypes.POINTER(L.QLayer) * n)(*[ctypes.pointer(q._layer) for q in layers])
            yp = (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys])
            ld = (ctypes.c_int64 * n)(*[q.out_features for q in layers])
            bp = (ctypes.c_void_p * n)(*[L.ptr(b) for b in bs])
            dt = L.dtype_code(in_dtype)
            with torch.cuda.device(x.device):
                rc = L.load().ts_qlinear_forward_group(qls, n, x2d.data_ptr(), M, layers[0].in_features, dt, yp, ld,
                                                       dt, bp, L.stream_ptr(x.device))
            if rc != L.TS_NOT_COVERED:
                L.check(rc, "qlinear group forward")
                return [y.reshape(*lead, q.out_features) for y, q in zip(ys, layers)]
        return [q(x) for q in layers]

    @classmethod
    def from_linear(cls, linear: nn.Linear, bits: int = 4, group_size: int = 128, outlier_frac: float = 0.001,
                    adaptive: bool = False, error_threshold: float = 0.10,
                    max_dequant_rows: Union[int, str] = DEFAULT_MAX_DEQUANT_ROWS, force_fp32_compute: bool = False,
                    cache=None, fast_dequant: bool = True, use_triton: bool = True, companded: bool = False,
                    double_quant: bool = True, dq_group_size: int = DEFAULT_DQ_GROUP_SIZE,
                    nf_quant: bool = True, _topk=None) -> Tuple["QuantLinear", float, bool]:
        """modules.py:942-1003. (`_topk`, not part of the reference's
        signature: the weight's codec.topk_of() result, computed ahead.)"""
        w = linear.weight.data
        if adaptive:
            qt, err, escalated = quantize_tensor_adaptive(
                w, group_size=group_size, outlier_frac=outlier_frac, error_threshold=error_threshold,
                allowed_bits=(2, 4, 8), companded=companded, double_quant=double_quant,
                dq_group_size=dq_group_size, nf_quant=nf_quant, _topk=_topk)
        else:
            qt = quantize_tensor(w, bits=bits, group_size=group_size, outlier_frac=outlier_frac, companded=companded,
                                 double_quant=double_quant, dq_group_size=dq_group_size, nf_quant=nf_quant,
                                 _topk=_topk)
            err = relative_error(w, qt)
            escalated = False
        bias = linear.bias.data if linear.bias is not None else None
        dev = linear.weight.device if linear.weight.is_cuda else None
        qlin = cls(qt, bias, max_dequant_rows=max_dequant_rows, force_fp32_compute=force_fp32_compute, cache=cache,
                   fast_dequant=fast_dequant, use_triton=use_triton, device=dev)
        return qlin, err, escalated

    @classmethod
    def from_quantized_tensor(cls, qt: QuantizedTensor, bias: Optional[torch.Tensor] = None,
                              max_dequant_rows: Union[int, str] = DEFAULT_MAX_DEQUANT_ROWS,
                              force_fp32_compute: bool = False, cache=None, fast_dequant: bool = True,
                              use_triton: bool = True) -> "QuantLinear":
        return cls(qt, bias, max_dequant_rows=max_dequant_rows, force_fp32_compute=force_fp32_compute, cache=cache,
                   fast_dequant=fast_dequant, use_triton=use_triton)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, bits={self.bits}, "
                f"group_size={self.group_size}, packed_kB={self.packed_nbytes() / 1024:.1f}, "
                f"dense_fp16_kB={self.dense_equiv_nbytes() / 1024:.1f}")


# ---------------------------------------------------------------------------
# whole-model helpers (modules.py:1033-1455)
# ---------------------------------------------------------------------------

def _set_module_by_name(root: nn.Module, dotted: str, new: nn.Module) -> None:
    parts = dotted.split(".")
    obj = root
    for p in parts[:-1]:
        obj = getattr(obj, p)
    setattr(obj, parts[-1], new)


def _iter_target_linears(model: nn.Module, min_numel: int, skip_name_patterns: Iterable[str]):
    pats = tuple(p.lower() for p in skip_name_patterns)
    for name, module in model.named_modules():
        if isinstance(module, nn.Linear) and not isinstance(module, QuantLinear):
            if module.weight.numel() < min_numel:
                continue
            if any(p in name.lower() for p in pats):
                continue
            yield name, module


def model_weight_bytes(model: nn.Module) -> int:
    return sum(p.numel() * p.element_size() for p in model.parameters()) + \
        sum(b.numel() * b.element_size() for b in model.buffers())


def quantize_module(
    model: nn.Module,
    bits: int = 4,
    group_size: int = 128,
    outlier_frac: float = 0.001,
    adaptive: bool = False,
    error_threshold: float = 0.10,
    min_numel: int = DEFAULT_MIN_NUMEL,
    skip_name_patterns: Iterable[str] = DEFAULT_SKIP_PATTERNS,
    max_dequant_rows: Union[int, str] = DEFAULT_MAX_DEQUANT_ROWS,
    force_fp32_patterns: Iterable[str] = (),
    cache_budget_mb: float = 0.0,
    host_cache_budget_mb: float = 0.0,
    fast_dequant: bool = True,
    use_triton: bool = True,
    vram_budget_mb: Optional[float] = None,
    quantize_workers: Optional[int] = 4,
    verbose: bool = True,
    companded: bool = False,
    double_quant: bool = True,
    dq_group_size: int = DEFAULT_DQ_GROUP_SIZE,
    nf_quant: bool = True,
) -> dict:
    """Replace every eligible nn.Linear with a QuantLinear, in place
    (modules.py:1258-1455). Layers are quantized on the GPU one after another,
    in order; the host side of each layer's top-k outlier selection (a
    sequential heap replay that fixes torch.topk's order) runs ahead of the
    loop on `quantize_workers` threads, one layer per thread, and is shared by
    every bit width a layer is quantized at."""
    if cache_budget_mb > 0 or host_cache_budget_mb > 0:
        raise NotImplementedError("WeightCache is not part of the tensorshrink_amd path")
    targets = list(_iter_target_linears(model, min_numel, skip_name_patterns))
    fp32_pats = tuple(p.lower() for p in force_fp32_patterns)
    stats = {"n_replaced": 0, "orig_bytes": 0, "packed_bytes": 0, "layers": [], "cache": None}

    def record(name, qlin, err, escalated, force_fp32, itemsize):
        ob = qlin.dense_equiv_nbytes(itemsize=itemsize)
        pb = qlin.packed_nbytes()
        stats["n_replaced"] += 1
        stats["orig_bytes"] += ob
        stats["packed_bytes"] += pb
        stats["layers"].append(dict(name=name, bits=qlin.bits, rel_error=err, escalated=escalated, orig_bytes=ob,
                                    packed_bytes=pb, force_fp32_compute=force_fp32))
        if verbose:
            print(f"  [{qlin.bits}b{'*' if escalated else ' '}{' fp32' if force_fp32 else ''}] {name:60s} "
                  f"err={err:.4f} {ob / 1e6:8.3f}MB -> {pb / 1e6:8.3f}MB")

    if vram_budget_mb is not None:
        if companded:
            raise ValueError("companded=True is not yet supported with vram_budget_mb (budget-aware path)")
        computed, lstats = {}, []
        pre = TopkPrefetch([lin.weight.data for _, lin in targets], outlier_frac, int(quantize_workers or 1))
        for i, (name, lin) in enumerate(targets):
            w = lin.weight.data
            tk = pre.get(i)
            q4 = quantize_tensor(w, bits=4, group_size=group_size, outlier_frac=outlier_frac, _topk=tk)
            q8 = quantize_tensor(w, bits=8, group_size=group_size, outlier_frac=outlier_frac, _topk=tk)
            e4, e8 = relative_error(w, q4), relative_error(w, q8)
            lstats.append(LayerBitStats(name, _estimate_resident_nbytes(q4), _estimate_resident_nbytes(q8), e4, e8))
            computed[name] = {4: (q4, e4), 8: (q8, e8)}
        plan = budget_allocate_bits(lstats, vram_budget_mb * 1024 * 1024)
        for name, lin in targets:
            qt, err = computed[name][plan[name]]
            f32 = any(p in name.lower() for p in fp32_pats)
            bias = lin.bias.data if lin.bias is not None else None
            qlin = QuantLinear(qt, bias, max_dequant_rows=max_dequant_rows, force_fp32_compute=f32,
                               device=lin.weight.device if lin.weight.is_cuda else None)
            _set_module_by_name(model, name, qlin)
            record(name, qlin, err, plan[name] == 8, f32, lin.weight.element_size())
        stats["ratio"] = stats["orig_bytes"] / max(1, stats["packed_bytes"]) if stats["orig_bytes"] else 1.0
        stats["vram_budget_mb"] = vram_budget_mb
        stats["budget_bytes_used"] = stats["packed_bytes"]
        return stats

    pre = TopkPrefetch([lin.weight.data for _, lin in targets], outlier_frac, int(quantize_workers or 1))
    for i, (name, lin) in enumerate(targets):
        f32 = any(p in name.lower() for p in fp32_pats)
        qlin, err, esc = QuantLinear.from_linear(
            lin, bits=bits, group_size=group_size, outlier_frac=outlier_frac, adaptive=adaptive,
            error_threshold=error_threshold, max_dequant_rows=max_dequant_rows, force_fp32_compute=f32,
            fast_dequant=fast_dequant, use_triton=use_triton, companded=companded, double_quant=double_quant,
            dq_group_size=dq_group_size, nf_quant=nf_quant, _topk=pre.get(i))
        _set_module_by_name(model, name, qlin)
        targets[i] = None
        record(name, qlin, err, esc, f32, lin.weight.element_size())
    stats["ratio"] = stats["orig_bytes"] / max(1, stats["packed_bytes"]) if stats["orig_bytes"] > 0 else 1.0
    return stats


# ---------------------------------------------------------------------------
# container save / load (modules.py:1458-1562)
# ---------------------------------------------------------------------------

def save_quant_module(model: nn.Module, path, verbose: bool = True) -> dict:
    """Write a quantized model to a .tsk container (modules.py:1458-1496):
    each QuantLinear's weight as a quantized entry straight from its packed
    buffers (scale/gmin as f16, outlier values as f16(base + delta), as
    QuantLinear.to_quantized_tensor rebuilds them), its bias raw, and every
    other state_dict entry raw; a QuantLinear's own buffers are not repeated."""
    from .container import ContainerWriter
    written, prefixes = set(), []
    with ContainerWriter(path) as w:
        for name, mod in model.named_modules():
            if not isinstance(mod, QuantLinear):
                continue
            w.add_quantized(f"{name}.weight", mod.to_quantized_tensor(), force_fp32_compute=mod.force_fp32_compute)
            written.add(f"{name}.weight")
            prefixes.append(f"{name}.")
            if mod.bias is not None:
                w.add_raw(f"{name}.bias", mod.bias)
                written.add(f"{name}.bias")
        n_raw = 0
        for key, t in model.state_dict().items():
            if key in written or any(key.startswith(p) for p in prefixes):
                continue
            w.add_raw(key, t)
            n_raw += 1
    if verbose:
        print(f"  saved {len(written)} quantized tensors + {n_raw} raw tensors -> {path}")
    return {"n_quant": len(written), "n_raw": n_raw}


def load_quantized_module(model: nn.Module, reader, max_dequant_rows: Union[int, str] = DEFAULT_MAX_DEQUANT_ROWS,
                          cache_budget_mb: float = 0.0, host_cache_budget_mb: float = 0.0,
                          fast_dequant: bool = True, use_triton: bool = True, parallel: bool = True,
                          verbose: bool = True) -> dict:
    """Populate a freshly built model from a container (modules.py:1499-1562):
    every nn.Linear whose "<name>.weight" is a quantized entry becomes a
    QuantLinear built from the packed data on the current GPU (frames
    decompressed in parallel threads with `parallel`), with the entry's
    force_fp32_compute flag; the raw entries the model's state_dict names are
    loaded with load_state_dict(strict=False)."""
    if cache_budget_mb > 0 or host_cache_budget_mb > 0:
        raise NotImplementedError("WeightCache is not part of the tensorshrink_amd path")
    names = set(reader.names())
    targets = []
    for name, mod in list(model.named_modules()):
        if isinstance(mod, nn.Linear) and not isinstance(mod, QuantLinear):
            wkey, bkey = f"{name}.weight", f"{name}.bias"
            if wkey in names and reader.kind(wkey) == "quant":
                f32 = bool(reader.manifest["tensors"][wkey].get("force_fp32_compute", False))
                targets.append((name, wkey, bkey if bkey in names else None, f32))
    keys = [t[1] for t in targets]
    qts = reader.get_quantized_many(keys) if parallel and len(keys) > 1 else {k: reader.get_quantized(k)
                                                                              for k in keys}
    for name, wkey, bkey, f32 in targets:
        bias = reader.get(bkey) if bkey is not None else None
        q = QuantLinear.from_quantized_tensor(qts[wkey], bias, max_dequant_rows=max_dequant_rows,
                                              force_fp32_compute=f32, fast_dequant=fast_dequant,
                                              use_triton=use_triton)
        _set_module_by_name(model, name, q)
        if verbose:
            print(f"  loaded quantized: {name}")
    keys_now = set(model.state_dict().keys())
    raw = {n: reader.get(n) for n in names if n in keys_now and reader.kind(n) == "raw"}
    model.load_state_dict(raw, strict=False)
    if verbose:
        print(f"  loaded {len(raw)} raw tensors, replaced {len(targets)} Linear layers")
    return {"n_quant_replaced": len(targets), "n_raw_loaded": len(raw), "cache": None}
