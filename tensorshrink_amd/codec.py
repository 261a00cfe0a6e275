"""GOAP codec on the GPU: the drop-in counterpart of the reference codec.

Mirrors the public surface of codec.py in GDNickk/tensorshrink v0.4.0
(``QuantizedTensor`` codec.py:102-188, ``quantize_tensor`` :453-675,
``dequantize_tensor`` :761-807, ``relative_error`` :850-857,
``quantize_tensor_adaptive`` :863-931, ``estimate_resident_nbytes`` :934-979,
``budget_allocate_bits`` :997-1033) with the same argument meaning, defaults
and error behaviour, and returns the same ``QuantizedTensor`` of host numpy
arrays. The heavy work runs in libtensorshrink_hip on the GPU:

  * top-k outlier extraction: GPU candidate filter + exact replay of the CPU
    top-k selection order (ties included) on the host;
  * clamp, per-group min/max, scale, code assignment and bit packing in one
    GPU pass; double quantization in a second;
  * Lloyd-Max fit: the sample is drawn with torch.randperm from the input
    device's generator (as the reference does) and normalized on the GPU; the
    12-round fit keeps the reference's sequential float32 sums on the host.

Outputs are bit-identical to the reference CPU codec for CPU inputs.
``smooth=True`` is not covered (it depends on ``pow``, which is not correctly
rounded and differs between CPU and GPU libraries) and raises.
"""
from __future__ import annotations

import ctypes
import dataclasses
import math
import threading
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _lib as L

DEFAULT_GROUP_SIZE = 128
DEFAULT_OUTLIER_FRAC = 0.001
DEFAULT_ERROR_THRESHOLD = 0.10
DEFAULT_DQ_GROUP_SIZE = 256
DEFAULT_SMOOTH_ALPHA = 0.5
DEFAULT_COMPAND_ITERS = 12
DEFAULT_COMPAND_SAMPLE_CAP = 300_000
DEFAULT_ADAPTIVE_BIT_CHAIN: Tuple[int, ...] = (2, 4, 6, 8)
_EPS = 1e-8


@dataclasses.dataclass
class QuantizedTensor:
    """One compressed weight tensor (field list and dtypes as codec.py:102-151)."""

    orig_shape: Tuple[int, ...]
    orig_dtype: str
    bits: int
    group_size: int
    rows: int
    cols: int
    padded_cols: int
    n_groups: int
    packed: np.ndarray
    scale: np.ndarray
    gmin: np.ndarray
    outlier_idx: np.ndarray
    outlier_val: np.ndarray
    dq_scale_codes: Optional[np.ndarray] = None
    dq_scale_meta: Optional[np.ndarray] = None
    dq_gmin_codes: Optional[np.ndarray] = None
    dq_gmin_meta: Optional[np.ndarray] = None
    smooth_scale: Optional[np.ndarray] = None
    stage2_packed: Optional[np.ndarray] = None
    stage2_scale: Optional[np.ndarray] = None
    stage2_gmin: Optional[np.ndarray] = None
    codebook: Optional[np.ndarray] = None

    def n_outliers(self) -> int:
        return int(self.outlier_idx.shape[0])

    def compressed_nbytes(self) -> int:
        total = self.packed.nbytes + self.outlier_idx.nbytes + self.outlier_val.nbytes
        if self.dq_scale_codes is not None:
            total += (self.dq_scale_codes.nbytes + self.dq_scale_meta.nbytes + self.dq_gmin_codes.nbytes
                      + self.dq_gmin_meta.nbytes)
        else:
            total += self.scale.nbytes + self.gmin.nbytes
        if self.smooth_scale is not None:
            total += self.smooth_scale.nbytes
        if self.stage2_packed is not None:
            total += self.stage2_packed.nbytes + self.stage2_scale.nbytes + self.stage2_gmin.nbytes
        if self.codebook is not None:
            total += self.codebook.nbytes
        return total

    def orig_nbytes(self) -> int:
        itemsize = {"float16": 2, "bfloat16": 2, "float32": 4}.get(self.orig_dtype, 2)
        return int(np.prod(self.orig_shape)) * itemsize


# ---------------------------------------------------------------------------
# NF codebooks (codec.py:273-317)
# ---------------------------------------------------------------------------
_NF_CODEBOOKS: Dict[int, np.ndarray] = {}


def _compute_nf_codebook(n_levels: int) -> np.ndarray:
    """Centroid of each equal-probability bin of N(0, 1), rescaled to
    [0, n_levels - 1] in float32 (codec.py:273-292)."""
    from scipy.stats import norm
    b = np.linspace(0, 1, n_levels + 1)
    cb = np.zeros(n_levels, dtype=np.float32)
    for i in range(n_levels):
        qa = norm.ppf(max(b[i], 1e-10))
        qb = norm.ppf(min(b[i + 1], 1 - 1e-10))
        cb[i] = (norm.pdf(qa) - norm.pdf(qb)) / max(b[i + 1] - b[i], 1e-10)
    lo, hi = cb.min(), cb.max()
    if hi > lo:
        cb = (cb - lo) / (hi - lo) * (n_levels - 1)
    return cb.astype(np.float32)


def _get_nf_codebook(bits: int) -> np.ndarray:
    """codec.py:297-317, including its scipy-less erfinv fallback."""
    if bits not in _NF_CODEBOOKS:
        n = 1 << bits
        try:
            _NF_CODEBOOKS[bits] = _compute_nf_codebook(n)
        except ImportError:
            cb = np.zeros(n, dtype=np.float32)
            for i in range(n):
                p = (i + 0.5) / n
                cb[i] = math.sqrt(2) * torch.erfinv(torch.tensor(2 * p - 1)).item()
            lo, hi = cb.min(), cb.max()
            if hi > lo:
                cb = (cb - lo) / (hi - lo) * (n - 1)
            _NF_CODEBOOKS[bits] = cb
    return _NF_CODEBOOKS[bits]


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------

def _device() -> torch.device:
    L.lib()
    return torch.device("cuda", torch.cuda.current_device())


def _to_2d(w: torch.Tensor) -> Tuple[torch.Tensor, Tuple[int, ...]]:
    shape = tuple(w.shape)
    if w.dim() == 1:
        raise ValueError("quantize_tensor expects a tensor with ndim >= 2")
    cols = 1
    for d in shape[1:]:
        cols *= d
    return w.reshape(shape[0], cols), shape


def _packed_cols(bits: int, padded_cols: int) -> int:
    if bits == 2:
        return (padded_cols + 3) // 4
    if bits == 4:
        return (padded_cols + 1) // 2
    return padded_cols


def _alloc_packed(rows: int, pcols: int, dev) -> torch.Tensor:
    # 4 spare bytes: the generic packing path ORs whole 32-bit words.
    flat = torch.empty(rows * pcols + 4, dtype=torch.uint8, device=dev)
    return flat[: rows * pcols].view(rows, pcols)


def _qinput(w: torch.Tensor) -> L.QInput:
    return L.QInput(w.data_ptr(), L.dtype_code(w.dtype), w.shape[0], w.shape[1])


def _gpu_weight(w2d: torch.Tensor, dev) -> torch.Tensor:
    t = w2d.detach()
    if t.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        t = t.to(torch.float32)
    return t.to(dev).contiguous()


def _to_host(t: torch.Tensor) -> np.ndarray:
    """Device tensor -> numpy through page-locked memory from torch's caching
    host allocator (a DMA at full link rate instead of a staged pageable copy).
    The array keeps the page-locked block alive; freed blocks are reused."""
    h = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
    h.copy_(t)
    return h.numpy()


def _topk_candidates(wg: torch.Tensor, k: int) -> Tuple[np.ndarray, np.ndarray]:
    """Host (indices, |w|) of the elements the top-k selection can touch, in
    index order: the GPU candidate filter, or every element when k > n / 64."""
    lib = L.lib()
    n = wg.numel()
    st = L.stream_ptr()
    qi = _qinput(wg)
    if k * 64 <= n:
        ws = torch.empty(max(1, lib.ts_topk_workspace_bytes(n, k)), dtype=torch.uint8, device=wg.device)
        cnt = ctypes.c_int64(0)
        L.check(lib.ts_topk_candidates_count(ctypes.byref(qi), k, ws.data_ptr(), ws.numel(), ctypes.byref(cnt), st),
                "topk candidates")
        nc = int(cnt.value)
        cidx = torch.empty(nc, dtype=torch.int64, device=wg.device)
        cval = torch.empty(nc, dtype=torch.float32, device=wg.device)
        L.check(lib.ts_topk_candidates_write(ctypes.byref(qi), k, ws.data_ptr(), cidx.data_ptr(), cval.data_ptr(),
                                             st), "topk candidates")
        return _to_host(cidx), _to_host(cval)
    # nth_element regime (k > n / 64): the selection needs every element.
    return np.arange(n, dtype=np.int64), wg.reshape(-1).to(torch.float32).abs().cpu().numpy()


def _topk_select(ci: np.ndarray, cv: np.ndarray, n: int, k: int) -> Tuple[np.ndarray, np.ndarray]:
    """(indices, |w| values) of torch.topk(|w|, k) in CPU order (codec.py:533-535)
    from the candidate stream (host only; ctypes releases the GIL)."""
    out_i = np.empty(k, np.int64)
    out_v = np.empty(k, np.float32)
    L.check(L.lib().ts_topk_select(ci.ctypes.data, cv.ctypes.data, cv.shape[0], n, k, out_i.ctypes.data,
                                   out_v.ctypes.data), "topk select")
    return out_i, out_v


def _topk_outliers(wg: torch.Tensor, k: int) -> Tuple[np.ndarray, np.ndarray]:
    """(indices, |w| values) of torch.topk(|w|, k) in CPU order (codec.py:533-535)."""
    ci, cv = _topk_candidates(wg, k)
    return _topk_select(ci, cv, wg.numel(), k)


class _Replay(threading.Thread):
    """The top-k heap replay on a host thread, so that the group encode and
    the result copies (which need only the clamp threshold) run meanwhile."""

    def __init__(self, ci: np.ndarray, cv: np.ndarray, n: int, k: int):
        super().__init__(name="ts-topk-replay", daemon=True)
        self.args = (ci, cv, n, k)
        self.result = None
        self.error = None
        self.start()

    def run(self):
        try:
            self.result = _topk_select(*self.args)
        except BaseException as e:  # re-raised by get()
            self.error = e

    def get(self) -> Tuple[np.ndarray, np.ndarray]:
        self.join()
        if self.error is not None:
            raise self.error
        return self.result


def _linspace(lo: float, hi: float, n: int, device) -> np.ndarray:
    """torch.linspace as codec.py:338 calls it (on the input's device)."""
    return torch.linspace(lo, hi, n, device=device).cpu().numpy().astype(np.float32)


class _Done:
    """An already-computed top-k, with the interface of _Replay."""

    def __init__(self, result):
        self.result = result

    def get(self):
        return self.result


def _k_of(n: int, outlier_frac: float) -> int:
    return max(1, int(n * outlier_frac)) if outlier_frac > 0 else 0


def topk_of(w: torch.Tensor, outlier_frac: float) -> Optional[Tuple[np.ndarray, np.ndarray]]:
    """torch.topk(|w|, k) of a weight (indices, |w| values; k from
    outlier_frac as quantize_tensor takes it), or None without outliers: the
    part of a quantize that depends on the weight and outlier_frac only, so
    the quantizes of one tensor at several bit widths can share it. Thread
    safe; the host heap replay releases the GIL."""
    w2d, _ = _to_2d(w)
    n = w2d.shape[0] * w2d.shape[1]
    k = _k_of(n, outlier_frac)
    if not 0 < k < n:
        return None
    wg = _gpu_weight(w2d, _device())
    ci, cv = _topk_candidates(wg, k)
    del wg  # the replay needs only the host candidates
    return _topk_select(ci, cv, n, k)


class TopkPrefetch:
    """topk_of() for a sequence of weights, computed ahead on a thread pool
    of `workers` threads, at most 2 x workers weights ahead of the consumer.
    Each weight's heap replay is sequential, but the replays of different
    weights run in parallel (the replay releases the GIL). get(i) waits for
    weight i's result; the pool holds a weight only until its top-k is done,
    and shuts down after the last one (a consumer that stops early leaves at
    most the window's bounded jobs to finish). With workers <= 1, get(i)
    computes in the calling thread."""

    def __init__(self, weights, outlier_frac: float, workers: int):
        from concurrent.futures import ThreadPoolExecutor
        self.ws = list(weights)
        self.frac = outlier_frac
        self.ex = ThreadPoolExecutor(max_workers=workers) if workers > 1 and len(self.ws) > 1 else None
        self.window = 2 * max(1, workers)
        self.fut = {}
        self.next = 0
        self._fill(0)

    def _fill(self, i: int) -> None:
        if self.ex is None:
            return
        while self.next < len(self.ws) and self.next < i + self.window:
            self.fut[self.next] = self.ex.submit(topk_of, self.ws[self.next], self.frac)
            self.ws[self.next] = None
            self.next += 1

    def get(self, i: int):
        if self.ex is None:
            w, self.ws[i] = self.ws[i], None
            return topk_of(w, self.frac)
        self._fill(i)
        r = self.fut.pop(i).result()
        self._fill(i + 1)
        if not self.fut and self.next >= len(self.ws):
            self.close()  # the last weight: release the pool's threads
        return r

    def close(self) -> None:
        if self.ex is not None:
            for f in self.fut.values():
                f.cancel()
            self.ex.shutdown(wait=True)
            self.ex = None


def _quantize_2d(wg: torch.Tensor, rows: int, cols: int, bits: int, group_size: int, k: int,
                 nf_quant: bool, companded: bool, double_quant: bool, dq_group_size: int,
                 rng_device, topk=None) -> dict:
    """GPU GOAP quantize of a [rows, cols] device tensor; returns numpy fields.
    `topk`: this weight's top-k from topk_of(), computed once for several
    quantizes of it."""
    lib = L.lib()
    dev = wg.device
    st = L.stream_ptr()
    n = rows * cols
    replay = None
    if 0 < k < n and topk is not None:
        if topk[0].shape[0] != k:
            raise ValueError("precomputed top-k does not match outlier_frac")
        replay = _Done(topk)
        nan = bool(np.isnan(topk[1]).any())
        t = float(topk[1].min())  # the k-th largest |w| (NaN when a NaN is ranked in)
        clamp = 1
    elif 0 < k < n:
        ci, cv = _topk_candidates(wg, k)
        replay = _Replay(ci, cv, n, k)
        # The clamp threshold min(topk values) is the k-th largest |w|: every
        # element above it is a candidate, so the candidates' k-th largest is
        # the same float. With NaN (ranked first, and min() propagates it) it
        # waits for the replay.
        nan = bool(np.isnan(cv).any())
        t = float(replay.get()[1].min()) if nan else float(np.partition(cv, cv.shape[0] - k)[cv.shape[0] - k])
        clamp = 1
    else:
        t, clamp = 0.0, 0
    pad = (-cols) % group_size
    padded_cols = cols + pad
    n_groups = padded_cols // group_size
    pcols = _packed_cols(bits, padded_cols)
    packed = _alloc_packed(rows, pcols, dev)
    s16 = torch.empty(rows, n_groups, dtype=torch.float16, device=dev)
    g16 = torch.empty_like(s16)
    qi = _qinput(wg)
    codebook_np = None
    cb_dev = None
    if nf_quant and not companded:
        codebook_np = _get_nf_codebook(bits)
        cb_dev = torch.from_numpy(codebook_np).to(dev)
    elif companded:
        # Pass 1 gives the float32 group scale/gmin; the fit sample is then
        # normalized exactly as the encode pass does (codec.py:579-596).
        s32 = torch.empty(rows, n_groups, dtype=torch.float32, device=dev)
        g32 = torch.empty_like(s32)
        opts = L.GroupOpts(bits, group_size, t, clamp, None, 0)
        L.check(lib.ts_quantize_groups(ctypes.byref(qi), ctypes.byref(opts), packed.data_ptr(), pcols,
                                       s16.data_ptr(), g16.data_ptr(), s32.data_ptr(), g32.data_ptr(), st),
                "group stats")
        nv = rows * padded_cols
        n_levels = 1 << bits
        if nv > DEFAULT_COMPAND_SAMPLE_CAP:
            sidx = torch.randperm(nv, device=rng_device)[:DEFAULT_COMPAND_SAMPLE_CAP].to(dev)
        else:
            sidx = torch.arange(nv, device=dev)
        m = sidx.numel()
        samp = torch.empty(m, dtype=torch.float32, device=dev)
        L.check(lib.ts_lm_sample(ctypes.byref(qi), ctypes.byref(opts), s32.data_ptr(), g32.data_ptr(),
                                 sidx.data_ptr(), m, samp.data_ptr(), st), "Lloyd-Max sample")
        sh = samp.cpu().numpy()
        n_levels = max(1, min(n_levels, m))
        init = _linspace(float(sh.min()), float(sh.max()), n_levels, rng_device)
        cent = np.empty(n_levels, np.float32)
        L.check(lib.ts_lloyd_max_fit_host(sh.ctypes.data, m, init.ctypes.data, n_levels, DEFAULT_COMPAND_ITERS,
                                          cent.ctypes.data), "Lloyd-Max fit")
        cb_dev = torch.from_numpy(cent).to(dev)
        codebook_np = cent.astype(np.float16)
    opts = L.GroupOpts(bits, group_size, t, clamp, L.ptr(cb_dev), 0 if cb_dev is None else cb_dev.numel())
    L.check(lib.ts_quantize_groups(ctypes.byref(qi), ctypes.byref(opts), packed.data_ptr(), pcols, s16.data_ptr(),
                                   g16.data_ptr(), None, None, st), "group encode")
    res = dict(rows=rows, cols=cols, padded_cols=padded_cols, n_groups=n_groups, codebook=codebook_np)
    if double_quant:
        nsg = rows * n_groups
        n_super = (nsg + dq_group_size - 1) // dq_group_size
        for name, v in (("scale", s16), ("gmin", g16)):
            codes = torch.empty(n_super * dq_group_size, dtype=torch.uint8, device=dev)
            meta = torch.empty(n_super, 2, dtype=torch.float16, device=dev)
            recon = torch.empty_like(v)
            L.check(lib.ts_double_quantize(v.data_ptr(), nsg, dq_group_size, codes.data_ptr(), meta.data_ptr(),
                                           recon.data_ptr(), st), "double quant")
            res[f"dq_{name}_codes"] = _to_host(codes)
            res[f"dq_{name}_meta"] = _to_host(meta)
            res[name] = _to_host(recon)
    else:
        res["scale"] = _to_host(s16)
        res["gmin"] = _to_host(g16)
    res["packed"] = _to_host(packed)
    if replay is not None:
        oi, ov = replay.get()
        if not nan and float(ov.min()) != t:
            raise RuntimeError("tensorshrink_amd: top-k threshold disagrees with the replay")
        idx_dev = torch.from_numpy(oi).to(dev)
        oval = torch.empty(k, dtype=torch.float16, device=dev)
        L.check(lib.ts_gather_f16(wg.data_ptr(), L.dtype_code(wg.dtype), idx_dev.data_ptr(), k, oval.data_ptr(), st),
                "outlier values")
        res["outlier_idx"] = oi.astype(np.int32)
        res["outlier_val"] = _to_host(oval)
    else:
        res["outlier_idx"] = np.zeros(0, np.int32)
        res["outlier_val"] = np.zeros(0, np.float16)
    return res


# ---------------------------------------------------------------------------
# public API
# ---------------------------------------------------------------------------

def quantize_tensor(
    w: torch.Tensor,
    bits: int = 4,
    group_size: int = DEFAULT_GROUP_SIZE,
    outlier_frac: float = DEFAULT_OUTLIER_FRAC,
    double_quant: bool = False,
    dq_group_size: int = DEFAULT_DQ_GROUP_SIZE,
    smooth: bool = False,
    smooth_alpha: float = DEFAULT_SMOOTH_ALPHA,
    companded: bool = False,
    nf_quant: bool = False,
    _topk=None,
) -> QuantizedTensor:
    """GOAP quantize of a weight tensor (ndim >= 2) on the GPU (codec.py:453-675).

    Same arguments, defaults and errors as the reference. The input may live
    on the CPU or the GPU; the result holds host numpy arrays. (`_topk`, not
    part of the reference's signature: this weight's topk_of() result.)
    """
    if bits not in (2, 4, 6, 8):
        raise ValueError("bits must be 2, 4, 6, or 8")
    if bits == 6:
        if companded:
            raise ValueError("companded=True is not supported with bits=6 (RVQ)")
        return _quantize_rvq(w, group_size=group_size, outlier_frac=outlier_frac, double_quant=double_quant,
                             dq_group_size=dq_group_size, smooth=smooth, smooth_alpha=smooth_alpha, _topk=_topk)
    if smooth:
        raise NotImplementedError("smooth=True is not covered by tensorshrink_amd")
    orig_dtype = str(w.dtype).replace("torch.", "")
    w2d, orig_shape = _to_2d(w)
    rows, cols = w2d.shape
    dev = _device()
    wg = _gpu_weight(w2d, dev)
    n = rows * cols
    k = _k_of(n, outlier_frac)
    f = _quantize_2d(wg, rows, cols, bits, group_size, k, nf_quant, companded, double_quant, dq_group_size,
                     w.device, topk=_topk)
    return QuantizedTensor(
        orig_shape=orig_shape, orig_dtype=orig_dtype, bits=bits, group_size=group_size, rows=rows, cols=cols,
        padded_cols=f["padded_cols"], n_groups=f["n_groups"], packed=f["packed"], scale=f["scale"],
        gmin=f["gmin"], outlier_idx=f["outlier_idx"], outlier_val=f["outlier_val"],
        dq_scale_codes=f.get("dq_scale_codes"), dq_scale_meta=f.get("dq_scale_meta"),
        dq_gmin_codes=f.get("dq_gmin_codes"), dq_gmin_meta=f.get("dq_gmin_meta"), codebook=f["codebook"])


def _quantize_rvq(w, group_size=DEFAULT_GROUP_SIZE, outlier_frac=DEFAULT_OUTLIER_FRAC, double_quant=False,
                  dq_group_size=DEFAULT_DQ_GROUP_SIZE, smooth=False, smooth_alpha=DEFAULT_SMOOTH_ALPHA, _topk=None):
    """6-bit RVQ (codec.py:678-737): 4-bit uniform stage 1 (outliers, DQ),
    2-bit uniform residual stage 2 (no outliers, no DQ)."""
    if smooth:
        raise NotImplementedError("smooth=True is not covered by tensorshrink_amd")
    lib = L.lib()
    qt4 = quantize_tensor(w, bits=4, group_size=group_size, outlier_frac=outlier_frac, double_quant=double_quant,
                          dq_group_size=dq_group_size, _topk=_topk)
    dev = _device()
    w2d, _ = _to_2d(w)
    wg = _gpu_weight(w2d, dev)
    bufs = _layer_buffers(qt4, dev)
    layer = _layer_struct(qt4, bufs)
    res = torch.empty(qt4.rows, qt4.cols, dtype=torch.float32, device=dev)
    oidx = torch.from_numpy(qt4.outlier_idx).to(dev)
    oval = torch.from_numpy(qt4.outlier_val).to(dev)
    st = L.stream_ptr()
    L.check(lib.ts_rvq_residual(ctypes.byref(_qinput(wg)), ctypes.byref(layer), oidx.data_ptr(), oval.data_ptr(),
                                qt4.n_outliers(), res.data_ptr(), st), "RVQ residual")
    f2 = _quantize_2d(res, qt4.rows, qt4.cols, 2, group_size, 0, False, False, False, dq_group_size, w.device)
    return dataclasses.replace(qt4, bits=6, stage2_packed=f2["packed"], stage2_scale=f2["scale"],
                               stage2_gmin=f2["gmin"])


def _layer_buffers(qt: QuantizedTensor, dev) -> dict:
    """Device copies of the fields a ts_qlayer points at (codec view)."""
    def t(a):
        return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    b = dict(packed=t(qt.packed))
    if qt.dq_scale_codes is not None:
        b.update(dq_scale_codes=t(qt.dq_scale_codes), dq_scale_meta=t(qt.dq_scale_meta),
                 dq_gmin_codes=t(qt.dq_gmin_codes), dq_gmin_meta=t(qt.dq_gmin_meta))
    else:
        b.update(scale=t(qt.scale), gmin=t(qt.gmin))
    if qt.codebook is not None and qt.bits != 6:
        b["codebook"] = t(np.asarray(qt.codebook, dtype=np.float32))
    if qt.bits == 6:
        b.update(stage2_packed=t(qt.stage2_packed), stage2_scale=t(qt.stage2_scale), stage2_gmin=t(qt.stage2_gmin))
    return b


def _layer_struct(qt: QuantizedTensor, b: dict, outliers: Optional[dict] = None) -> L.QLayer:
    s = L.QLayer()
    s.bits = 4 if (qt.bits == 6 and "stage2_packed" not in b) else qt.bits
    s.group_size = qt.group_size
    s.rows, s.cols, s.padded_cols, s.n_groups = qt.rows, qt.cols, qt.padded_cols, qt.n_groups
    s.packed = b["packed"].data_ptr()
    s.packed_stride = b["packed"].shape[1]
    s.scale = L.ptr(b.get("scale"))
    s.gmin = L.ptr(b.get("gmin"))
    if b.get("dq_scale_codes") is not None:
        s.dq_scale_codes = L.ptr(b["dq_scale_codes"])
        s.dq_scale_meta = L.ptr(b["dq_scale_meta"])
        s.dq_gmin_codes = L.ptr(b["dq_gmin_codes"])
        s.dq_gmin_meta = L.ptr(b["dq_gmin_meta"])
        s.dq_group_size = b["dq_scale_codes"].numel() // b["dq_scale_meta"].shape[0]
    s.codebook = L.ptr(b.get("codebook"))
    if outliers is not None and outliers["row"].numel() > 0:
        s.outlier_row = outliers["row"].data_ptr()
        s.outlier_col = outliers["col"].data_ptr()
        s.outlier_delta = outliers["delta"].data_ptr()
        s.n_outliers = outliers["row"].numel()
        s.outlier_row_ptr = outliers["row_ptr"].data_ptr()
    if b.get("stage2_packed") is not None:
        s.stage2_packed = b["stage2_packed"].data_ptr()
        s.stage2_stride = b["stage2_packed"].shape[1]
        s.stage2_scale = b["stage2_scale"].data_ptr()
        s.stage2_gmin = b["stage2_gmin"].data_ptr()
    return s


def _dequantize_device(qt: QuantizedTensor, dtype: torch.dtype) -> torch.Tensor:
    lib = L.lib()
    dev = _device()
    b = _layer_buffers(qt, dev)
    layer = _layer_struct(qt, b)
    out = torch.empty(qt.rows, qt.cols, dtype=dtype, device=dev)
    oidx = torch.from_numpy(np.ascontiguousarray(qt.outlier_idx, dtype=np.int32)).to(dev)
    oval = torch.from_numpy(np.ascontiguousarray(qt.outlier_val, dtype=np.float16)).to(dev)
    L.check(lib.ts_dequantize(ctypes.byref(layer), L.TS_DEQ_CODEC, oidx.data_ptr(), oval.data_ptr(),
                              qt.n_outliers(), out.data_ptr(), qt.cols, L.dtype_code(dtype), L.stream_ptr()),
            "dequantize")
    return out


def dequantize_tensor(qt: QuantizedTensor, device=None, dtype=None) -> torch.Tensor:
    """Dense reconstruction (codec.py:761-807), computed on the GPU and
    returned on `device` (default "cpu", as the reference)."""
    device = device or "cpu"
    out_dtype = dtype or getattr(torch, qt.orig_dtype, torch.float16)
    if qt.smooth_scale is not None:
        raise NotImplementedError("smooth-scaled tensors are not covered by tensorshrink_amd")
    if out_dtype not in (torch.float16, torch.bfloat16, torch.float32):
        d = _dequantize_device(qt, torch.float32).to(out_dtype)
    else:
        d = _dequantize_device(qt, out_dtype)
    return d.reshape(qt.orig_shape).to(device)


def relative_error(w: torch.Tensor, qt: QuantizedTensor) -> float:
    """||w - dequant|| / ||w|| (codec.py:850-857), float64 sums on the GPU."""
    lib = L.lib()
    dev = _device()
    w2d, _ = _to_2d(w)
    wg = _gpu_weight(w2d, dev)
    d = _dequantize_device(qt, torch.float32)
    sums = torch.zeros(2, dtype=torch.float64, device=dev)
    L.check(lib.ts_sq_error_sums(ctypes.byref(_qinput(wg)), d.data_ptr(), L.TS_F32, sums.data_ptr(),
                                 L.stream_ptr()), "relative error")
    num, den = sums.cpu().tolist()
    return float(math.sqrt(num) / max(math.sqrt(den), _EPS))


def quantize_tensor_adaptive(
    w: torch.Tensor,
    group_size: int = DEFAULT_GROUP_SIZE,
    outlier_frac: float = DEFAULT_OUTLIER_FRAC,
    error_threshold: float = DEFAULT_ERROR_THRESHOLD,
    force_bits: Optional[int] = None,
    double_quant: bool = False,
    dq_group_size: int = DEFAULT_DQ_GROUP_SIZE,
    smooth: bool = False,
    smooth_alpha: float = DEFAULT_SMOOTH_ALPHA,
    allowed_bits: Sequence[int] = DEFAULT_ADAPTIVE_BIT_CHAIN,
    companded: bool = False,
    nf_quant: bool = False,
    _topk=None,
) -> Tuple[QuantizedTensor, float, bool]:
    """Escalating bit-width quantize (codec.py:863-931). The top-k outlier
    selection depends on the weight and outlier_frac only: it runs once
    (or comes in as `_topk`, this weight's topk_of()) for the whole chain."""
    if companded and (force_bits == 6 or 6 in allowed_bits):
        raise ValueError("companded=True is not supported with bits=6 (RVQ)")
    if smooth:
        raise NotImplementedError("smooth=True is not covered by tensorshrink_amd")
    kw = dict(group_size=group_size, outlier_frac=outlier_frac, double_quant=double_quant,
              dq_group_size=dq_group_size, smooth=smooth, smooth_alpha=smooth_alpha, companded=companded,
              nf_quant=nf_quant, _topk=_topk)
    if force_bits is not None:
        qt = quantize_tensor(w, bits=force_bits, **kw)
        return qt, relative_error(w, qt), False
    chain = sorted(set(allowed_bits))
    if not chain or any(b not in (2, 4, 6, 8) for b in chain):
        raise ValueError(f"allowed_bits must be a non-empty subset of (2, 4, 6, 8), got {allowed_bits!r}")
    if _topk is None and len(chain) > 1:
        kw["_topk"] = topk_of(w, outlier_frac)
    for i, bits in enumerate(chain):
        qt = quantize_tensor(w, bits=bits, **kw)
        err = relative_error(w, qt)
        if err <= error_threshold or i == len(chain) - 1:
            return qt, err, i > 0
    raise AssertionError("unreachable")


def estimate_resident_nbytes(qt: QuantizedTensor) -> int:
    """Bytes resident as a QuantLinear (codec.py:934-979)."""
    n = qt.n_outliers()
    total = qt.packed.nbytes + n * 4 + n * 4 + n * 2
    if qt.dq_scale_codes is not None:
        total += qt.dq_scale_codes.nbytes + qt.dq_scale_meta.nbytes + qt.dq_gmin_codes.nbytes + qt.dq_gmin_meta.nbytes
    else:
        total += qt.scale.nbytes + qt.gmin.nbytes
    if qt.smooth_scale is not None:
        total += qt.smooth_scale.nbytes
    if qt.stage2_packed is not None:
        total += qt.stage2_packed.nbytes + qt.stage2_scale.nbytes + qt.stage2_gmin.nbytes
    return total


@dataclasses.dataclass
class LayerBitStats:
    """Per-layer 4/8-bit cost and error (codec.py:982-994)."""
    name: str
    bytes4: int
    bytes8: int
    err4: float
    err8: float


def budget_allocate_bits(stats: Sequence[LayerBitStats], budget_bytes: float) -> Dict[str, int]:
    """Greedy 4 -> 8 bit upgrades by error reduction per byte (codec.py:997-1033)."""
    bits = {s.name: 4 for s in stats}
    remaining = budget_bytes - sum(s.bytes4 for s in stats)
    cands: List[Tuple[float, str, int]] = []
    for s in stats:
        extra = s.bytes8 - s.bytes4
        gain = s.err4 - s.err8
        if extra <= 0 or gain <= 0:
            continue
        cands.append((gain / extra, s.name, extra))
    cands.sort(key=lambda c: c[0], reverse=True)
    for _, name, extra in cands:
        if extra <= remaining:
            bits[name] = 8
            remaining -= extra
    return bits
