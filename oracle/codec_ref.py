"""CPU restatement of the reference GOAP codec (TEST INFRASTRUCTURE ONLY).

This module is the checker for the HIP product path. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and only to compute expected values or to time the CPU baseline. The
product (``tensorshrink_amd``) never imports it.

Each function names the reference lines it restates (``codec.py``,
``modules.py`` in GDNickk/tensorshrink v0.4.0). Arithmetic is float32 numpy with
the reference's operation order (separate multiply and add, IEEE division,
round-half-even, float32 comparisons), so results are bit-identical.

Parity pinning (see tests/test_oracle.py for each check):
  * nf_codebook            - golden vectors + independent numeric integration of
                             the bin centroids (scipy.integrate) + symmetry.
  * topk_abs               - torch.topk on CPU (the library routine the reference
                             calls) + golden vectors incl. ties at the threshold.
  * quantize / dequantize  - golden vectors (22 small cases, 6 config-scale
                             digests) + invariants (code range, |err| <= scale/2
                             for uniform grids, pack/unpack round trip,
                             outlier count int(n*frac), DQ reconstruction bound).
  * lloyd_max_fit          - golden vectors (three seeded cases) + invariants
                             (sorted, each centroid the mean of its cell).
  * quantlinear_buffers    - golden vectors (row sort stability, delta bits).
  * quantlinear_forward_cpu- golden CPU forward outputs (bf16).
"""
from __future__ import annotations

import ctypes
import math
import os
from typing import Dict, Optional

import numpy as np

_EPS32 = np.float32(1e-8)
DQ_GROUP_SIZE = 256
COMPAND_ITERS = 12
COMPAND_SAMPLE_CAP = 300_000

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "libts_oracle.so")
        if not os.path.exists(path):
            raise RuntimeError("oracle helper not built: run `make -C oracle`")
        lib = ctypes.CDLL(path)
        lib.ts_oracle_topk.restype = ctypes.c_int
        lib.ts_oracle_topk.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                       ctypes.c_void_p, ctypes.c_void_p]
        lib.ts_oracle_index_add_f32.restype = None
        lib.ts_oracle_index_add_f32.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        _LIB = lib
    return _LIB


# ---------------------------------------------------------------------------
# float helpers
# ---------------------------------------------------------------------------

def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16 bit pattern (uint16)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = np.isnan(a)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b).view(np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------------------
# packing (codec.py:195-240)
# ---------------------------------------------------------------------------

def pack_nibbles(codes: np.ndarray) -> np.ndarray:
    """codec.py:195-202: byte j = code[2j] | code[2j+1] << 4."""
    assert codes.shape[-1] % 2 == 0
    return (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)


def unpack_nibbles(packed: np.ndarray, n: int) -> np.ndarray:
    """codec.py:205-212."""
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), np.uint8)
    out[..., 0::2] = packed & 0x0F
    out[..., 1::2] = (packed >> 4) & 0x0F
    return out[..., :n]


def pack_crumbs(codes: np.ndarray) -> np.ndarray:
    """codec.py:215-226: cols 4j..4j+3 at bits 0-1, 2-3, 4-5, 6-7."""
    assert codes.shape[-1] % 4 == 0
    return (codes[..., 0::4] | (codes[..., 1::4] << 2) | (codes[..., 2::4] << 4)
            | (codes[..., 3::4] << 6)).astype(np.uint8)


def unpack_crumbs(packed: np.ndarray, n: int) -> np.ndarray:
    """codec.py:229-240."""
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 4,), np.uint8)
    for j in range(4):
        out[..., j::4] = (packed >> (2 * j)) & 0x03
    return out[..., :n]


# ---------------------------------------------------------------------------
# codebooks (codec.py:273-361)
# ---------------------------------------------------------------------------

def nf_codebook(bits: int) -> np.ndarray:
    """codec.py:273-292 (scipy path): centroid of each equal-probability bin of
    N(0,1), E[X | a < Phi(X) < b] = (phi(q_a) - phi(q_b)) / (b - a), computed in
    float64 and stored into float32, then min-max rescaled to [0, 2^b - 1] in
    float32."""
    from scipy.stats import norm
    n = 1 << bits
    bounds = np.linspace(0, 1, n + 1)
    cb = np.zeros(n, dtype=np.float32)
    for i in range(n):
        a, b = bounds[i], bounds[i + 1]
        qa = norm.ppf(max(a, 1e-10))
        qb = norm.ppf(min(b, 1 - 1e-10))
        cb[i] = (norm.pdf(qa) - norm.pdf(qb)) / max(b - a, 1e-10)
    lo, hi = cb.min(), cb.max()
    if hi > lo:
        cb = (cb - lo) / (hi - lo) * (n - 1)
    return cb.astype(np.float32)


def searchsorted_mids(values: np.ndarray, codebook: np.ndarray) -> np.ndarray:
    """codec.py:364-373: nearest entry by float32 midpoints, a value equal to a
    midpoint takes the lower code (searchsorted side='left')."""
    k = codebook.shape[0]
    if k <= 1:
        return np.zeros(values.shape, np.int64)
    mids = ((codebook[:-1] + codebook[1:]) / np.float32(2)).astype(np.float32)
    codes = np.searchsorted(mids, values.reshape(-1), side="left")
    return np.clip(codes, 0, k - 1).reshape(values.shape)


def torch_linspace_f32(lo: float, hi: float, steps: int) -> np.ndarray:
    """torch.linspace(lo, hi, steps) in float32 on CPU (codec.py:338).
    Calls the library routine the reference calls."""
    import torch
    return torch.linspace(lo, hi, steps).numpy()


def lloyd_max_fit(values: np.ndarray, n_levels: int, sample_idx: Optional[np.ndarray],
                  iters: int = COMPAND_ITERS) -> np.ndarray:
    """codec.py:320-361. `sample_idx` is torch.randperm(n)[:cap] drawn from the
    global torch RNG by the caller when n > cap (codec.py:329-331), else None."""
    flat = values.reshape(-1).astype(np.float32)
    fit = flat[sample_idx] if sample_idx is not None else flat
    fit = np.ascontiguousarray(fit, dtype=np.float32)
    m = fit.shape[0]
    n_levels = max(1, min(n_levels, m))
    cent = torch_linspace_f32(float(fit.min()), float(fit.max()), n_levels)
    lib = _lib()
    ones = np.ones(m, np.float32)
    for _ in range(iters):
        order = np.argsort(cent, kind="stable")
        cs = cent[order]
        if n_levels > 1:
            mids = ((cs[:-1] + cs[1:]) / np.float32(2)).astype(np.float32)
            assign_sorted = np.searchsorted(mids, fit, side="left")
        else:
            assign_sorted = np.zeros(m, np.int64)
        assign = np.ascontiguousarray(order[assign_sorted].astype(np.int64))
        newc = np.zeros(n_levels, np.float32)
        cnt = np.zeros(n_levels, np.float32)
        lib.ts_oracle_index_add_f32(newc.ctypes.data, assign.ctypes.data, fit.ctypes.data, m)
        lib.ts_oracle_index_add_f32(cnt.ctypes.data, assign.ctypes.data, ones.ctypes.data, m)
        empty = cnt == 0
        cnt = np.maximum(cnt, np.float32(1.0))
        newc = (newc / cnt).astype(np.float32)
        newc[empty] = cent[empty]
        cent = newc
    return np.sort(cent).astype(np.float32)


# ---------------------------------------------------------------------------
# top-k outlier extraction (codec.py:527-550)
# ---------------------------------------------------------------------------

def topk_abs(flat_f32: np.ndarray, k: int):
    """(values, indices) of torch.topk(|flat|, k) on CPU, in its order."""
    a = np.ascontiguousarray(np.abs(flat_f32), dtype=np.float32)
    vals = np.empty(k, np.float32)
    idx = np.empty(k, np.int64)
    rc = _lib().ts_oracle_topk(a.ctypes.data, a.shape[0], k, vals.ctypes.data, idx.ctypes.data)
    if rc != 0:
        raise ValueError("bad top-k arguments")
    return vals, idx


# ---------------------------------------------------------------------------
# double quantization (codec.py:380-435)
# ---------------------------------------------------------------------------

def double_quantize(values_f16: np.ndarray, dq_group_size: int = DQ_GROUP_SIZE):
    """codec.py:380-401 (numpy float32 semantics, NEP 50 scalars)."""
    flat = values_f16.astype(np.float32).ravel()
    n = flat.shape[0]
    pad = (-n) % dq_group_size
    if pad:
        flat = np.concatenate([flat, np.full(pad, flat[-1], np.float32)])
    g = flat.reshape(-1, dq_group_size)
    mn = g.min(axis=1)
    mx = g.max(axis=1)
    ms = ((mx - mn) / np.float32(255.0)).astype(np.float32)
    ms = np.maximum(ms, _EPS32)
    codes = np.rint((g - mn[:, None]) / ms[:, None]).clip(0, 255).astype(np.uint8)
    meta = np.stack([ms, mn], axis=1).astype(np.float16)
    return codes.ravel(), meta


def double_dequantize_f16(codes: np.ndarray, meta: np.ndarray, shape) -> np.ndarray:
    """codec.py:404-417: float32 codes*ms + mm, then float16."""
    n_super = meta.shape[0]
    c = codes.astype(np.float32).reshape(n_super, -1)
    r = c * meta[:, 0].astype(np.float32)[:, None] + meta[:, 1].astype(np.float32)[:, None]
    n = int(np.prod(shape))
    return r.ravel()[:n].reshape(shape).astype(np.float16)


def double_dequantize_f32(codes: np.ndarray, meta: np.ndarray, shape) -> np.ndarray:
    """codec.py:420-435 and modules.py:573-579: float32 codes*ms + mm."""
    n_super = meta.shape[0]
    c = codes.astype(np.float32).reshape(n_super, -1)
    r = c * meta[:, 0].astype(np.float32)[:, None] + meta[:, 1].astype(np.float32)[:, None]
    n = int(np.prod(shape))
    return r.ravel()[:n].reshape(shape).astype(np.float32)


# ---------------------------------------------------------------------------
# quantize (codec.py:453-737)
# ---------------------------------------------------------------------------

def _as_f32(w) -> np.ndarray:
    if hasattr(w, "detach"):
        return w.detach().to(dtype=__import__("torch").float32).numpy().copy()
    return np.asarray(w, dtype=np.float32).copy()


def quantize(w, bits: int = 4, group_size: int = 128, outlier_frac: float = 0.001,
             double_quant: bool = False, dq_group_size: int = DQ_GROUP_SIZE,
             nf_quant: bool = False, companded: bool = False, orig_dtype: str = "float16",
             lm_sample_idx: Optional[np.ndarray] = None, randperm=None) -> Dict[str, np.ndarray]:
    """codec.py:453-675 (smooth=False). `w` is a torch CPU tensor or a numpy
    array. For companded grids with more than COMPAND_SAMPLE_CAP values, the
    caller either passes `lm_sample_idx` or a `randperm(n)` callable that draws
    from the same RNG the reference would use (torch.randperm)."""
    if bits == 6:
        return quantize_rvq(w, group_size, outlier_frac, double_quant, dq_group_size, orig_dtype)
    if hasattr(w, "dtype") and hasattr(w, "detach"):
        orig_dtype = str(w.dtype).replace("torch.", "")
    work = _as_f32(w)
    rows = work.shape[0]
    cols = int(np.prod(work.shape[1:]))
    work = work.reshape(rows, cols)
    flat = work.reshape(-1)
    n = flat.shape[0]
    k = max(1, int(n * outlier_frac)) if outlier_frac > 0 else 0
    if 0 < k < n:
        tv, ti = topk_abs(flat, k)
        t = tv.min()
        out_idx = ti
        out_val = flat[ti].copy()
        np.clip(flat, -t, t, out=flat)
    else:
        out_idx = np.zeros(0, np.int64)
        out_val = np.zeros(0, np.float32)
    pad = (-cols) % group_size
    padded = np.concatenate([work, np.repeat(work[:, -1:], pad, axis=1)], axis=1) if pad else work
    padded_cols = cols + pad
    n_groups = padded_cols // group_size
    g = padded.reshape(rows, n_groups, group_size)
    gmin = g.min(axis=-1)
    gmax = g.max(axis=-1)
    levels = (1 << bits) - 1
    scale = ((gmax - gmin) / np.float32(levels)).astype(np.float32)
    scale = np.maximum(scale, _EPS32)
    v = ((g - gmin[..., None]) / scale[..., None]).astype(np.float32)
    codebook = None
    if nf_quant and not companded:
        cb = nf_codebook(bits)
        codes = searchsorted_mids(v, cb).astype(np.uint8)
        codebook = cb
    elif companded:
        nv = v.size
        if lm_sample_idx is None and nv > COMPAND_SAMPLE_CAP:
            if randperm is None:
                raise ValueError("companded fit over > cap values needs lm_sample_idx or randperm")
            lm_sample_idx = np.asarray(randperm(nv))[:COMPAND_SAMPLE_CAP]
        cbf = lloyd_max_fit(v, 1 << bits, lm_sample_idx if nv > COMPAND_SAMPLE_CAP else None)
        codes = searchsorted_mids(v, cbf).astype(np.uint8)
        codebook = cbf.astype(np.float16)
    else:
        codes = np.clip(np.rint(v), 0, levels).astype(np.uint8)
    codes = codes.reshape(rows, padded_cols)
    if bits == 2:
        extra = (-padded_cols) % 4
        pin = np.concatenate([codes, np.repeat(codes[:, -1:], extra, axis=1)], axis=1) if extra else codes
        packed = pack_crumbs(pin)
    elif bits == 4:
        pin = codes if padded_cols % 2 == 0 else np.concatenate([codes, codes[:, -1:]], axis=1)
        packed = pack_nibbles(pin)
    else:
        packed = np.ascontiguousarray(codes)
    scale16 = scale.astype(np.float16)
    gmin16 = gmin.astype(np.float16)
    res = dict(packed=packed, outlier_idx=out_idx.astype(np.int32), outlier_val=out_val.astype(np.float16),
               _meta=dict(bits=bits, group_size=group_size, rows=rows, cols=cols, padded_cols=padded_cols,
                          n_groups=n_groups, orig_dtype=orig_dtype))
    if double_quant:
        sc_codes, sc_meta = double_quantize(scale16, dq_group_size)
        gm_codes, gm_meta = double_quantize(gmin16, dq_group_size)
        res.update(dq_scale_codes=sc_codes, dq_scale_meta=sc_meta, dq_gmin_codes=gm_codes, dq_gmin_meta=gm_meta)
        scale16 = double_dequantize_f16(sc_codes, sc_meta, scale16.shape)
        gmin16 = double_dequantize_f16(gm_codes, gm_meta, gmin16.shape)
    res["scale"] = scale16
    res["gmin"] = gmin16
    if codebook is not None:
        res["codebook"] = codebook
    return res


def quantize_rvq(w, group_size=128, outlier_frac=0.001, double_quant=False, dq_group_size=DQ_GROUP_SIZE,
                 orig_dtype="float16") -> Dict[str, np.ndarray]:
    """codec.py:678-737: 4-bit uniform stage 1 (outliers, DQ) + 2-bit uniform
    residual stage 2 (no outliers, no DQ)."""
    q1 = quantize(w, 4, group_size, outlier_frac, double_quant, dq_group_size, orig_dtype=orig_dtype)
    w32 = _as_f32(w).reshape(q1["_meta"]["rows"], q1["_meta"]["cols"])
    residual = (w32 - dequantize(q1, out="f32")).astype(np.float32)
    q2 = quantize(residual, 2, group_size, 0.0, False)
    res = dict(q1)
    res["_meta"] = dict(q1["_meta"], bits=6)
    res["stage2_packed"] = q2["packed"]
    res["stage2_scale"] = q2["scale"]
    res["stage2_gmin"] = q2["gmin"]
    return res


# ---------------------------------------------------------------------------
# dequantize (codec.py:740-847)
# ---------------------------------------------------------------------------

def resolve_scale_gmin(q: Dict) -> tuple:
    """codec.py:740-758: float32 scale/gmin, DQ-reconstructed when present."""
    shape = q["scale"].shape
    if q.get("dq_scale_codes") is not None:
        sc = double_dequantize_f32(q["dq_scale_codes"], q["dq_scale_meta"], shape)
    else:
        sc = q["scale"].astype(np.float32)
    if q.get("dq_gmin_codes") is not None:
        gm = double_dequantize_f32(q["dq_gmin_codes"], q["dq_gmin_meta"], shape)
    else:
        gm = q["gmin"].astype(np.float32)
    return sc, gm


def _codes_of(packed: np.ndarray, bits: int, padded_cols: int) -> np.ndarray:
    if bits == 2:
        return unpack_crumbs(packed, padded_cols)
    if bits == 4:
        return unpack_nibbles(packed, padded_cols)
    return packed


def cast_out(a32: np.ndarray, dtype: str) -> np.ndarray:
    """float32 -> orig dtype; bf16 is returned as uint16 bit patterns."""
    if dtype == "float16":
        return a32.astype(np.float16)
    if dtype == "bfloat16":
        return f32_to_bf16_bits(a32)
    return a32.astype(np.float32)


def dequantize(q: Dict, out: str = "f32") -> np.ndarray:
    """codec.py:761-807 (`out='f32'` = dtype=torch.float32, `out='native'` =
    the tensor's original dtype; bf16 as uint16 bits)."""
    meta = q["_meta"]
    if meta["bits"] == 6:
        return dequantize_rvq(q, out)
    rows, cols, pc, ng, gs = meta["rows"], meta["cols"], meta["padded_cols"], meta["n_groups"], meta["group_size"]
    sc, gm = resolve_scale_gmin(q)
    codes = _codes_of(q["packed"], meta["bits"], pc)
    cb = q.get("codebook")
    if cb is not None:
        cv = cb.astype(np.float32)[codes.reshape(-1).astype(np.int64)].reshape(rows, ng, gs)
    else:
        cv = codes.reshape(rows, ng, gs).astype(np.float32)
    deq = (cv * sc[..., None] + gm[..., None]).astype(np.float32)
    flat = deq.reshape(rows, pc)[:, :cols].reshape(-1).copy()
    if q["outlier_idx"].shape[0] > 0:
        flat[q["outlier_idx"].astype(np.int64)] = q["outlier_val"].astype(np.float32)
    res = flat.reshape(rows, cols)
    return res if out == "f32" else cast_out(res, meta["orig_dtype"])


def dequantize_rvq(q: Dict, out: str = "f32") -> np.ndarray:
    """codec.py:810-847."""
    meta = q["_meta"]
    rows, cols, pc, ng, gs = meta["rows"], meta["cols"], meta["padded_cols"], meta["n_groups"], meta["group_size"]
    sc, gm = resolve_scale_gmin(q)
    c1 = unpack_nibbles(q["packed"], pc).reshape(rows, ng, gs).astype(np.float32)
    d1 = (c1 * sc[..., None] + gm[..., None]).astype(np.float32).reshape(rows, pc)[:, :cols]
    flat = d1.reshape(-1).copy()
    if q["outlier_idx"].shape[0] > 0:
        flat[q["outlier_idx"].astype(np.int64)] = q["outlier_val"].astype(np.float32)
    r1 = flat.reshape(rows, cols)
    c2 = unpack_crumbs(q["stage2_packed"], pc).reshape(rows, ng, gs).astype(np.float32)
    s2 = q["stage2_scale"].astype(np.float32)
    g2 = q["stage2_gmin"].astype(np.float32)
    d2 = (c2 * s2[..., None] + g2[..., None]).astype(np.float32).reshape(rows, pc)[:, :cols]
    res = (r1 + d2).astype(np.float32)
    return res if out == "f32" else cast_out(res, meta["orig_dtype"])


def relative_error(w, q: Dict) -> float:
    """codec.py:850-857 (float64 norms here; the reference's float32 norm
    differs in the last bits, so tests compare this with a tolerance)."""
    w32 = _as_f32(w).reshape(q["_meta"]["rows"], q["_meta"]["cols"]).astype(np.float64)
    d = dequantize(q, "f32").astype(np.float64)
    return float(np.linalg.norm((w32 - d).ravel()) / max(np.linalg.norm(w32.ravel()), 1e-8))


# ---------------------------------------------------------------------------
# QuantLinear buffers and CPU forward (modules.py:294-471, 649-715, 752-804)
# ---------------------------------------------------------------------------

def quantlinear_scale_gmin(q: Dict) -> tuple:
    """modules.py:558-583: float32 [rows, n_groups] scale/gmin."""
    return resolve_scale_gmin(q)


def quantlinear_buffers(q: Dict) -> Dict[str, np.ndarray]:
    """modules.py:414-448: outliers stable-sorted by row, and
    delta = fp16(fp32(val) - base), base = cv * sc + gm (modules.py:649-715)."""
    meta = q["_meta"]
    cols, gs, bits = meta["cols"], meta["group_size"], meta["bits"]
    idx = q["outlier_idx"].astype(np.int64)
    if idx.size:
        row = idx // cols
        col = idx % cols
        perm = np.argsort(row, kind="stable")
        row = row[perm].astype(np.int32)
        col = col[perm].astype(np.int32)
        val = q["outlier_val"][perm]
    else:
        row = np.zeros(0, np.int32)
        col = np.zeros(0, np.int32)
        val = q["outlier_val"]
    res = dict(outlier_row=row, outlier_col=col)
    if row.size == 0:
        res["outlier_delta"] = np.zeros(0, np.float16)
        return res
    sc, gm = quantlinear_scale_gmin(q)
    r64 = row.astype(np.int64)
    group = (col // gs).astype(np.int64)
    within = (col % gs).astype(np.int64)
    packed = q["packed"]
    pos = group * gs + within
    if bits == 2:
        b = packed[r64, pos // 4]
        code = ((b >> (2 * (within % 4))) & 0x03).astype(np.float32)
    elif bits == 4:
        b = packed[r64, pos // 2]
        code = np.where(within % 2 == 1, (b >> 4) & 0x0F, b & 0x0F).astype(np.float32)
    else:
        code = packed[r64, pos].astype(np.float32)
    if q.get("codebook") is not None:
        code = q["codebook"].astype(np.float32)[code.astype(np.int64)]
    base = (code * sc[r64, group] + gm[r64, group]).astype(np.float32)
    res["outlier_delta"] = (val.astype(np.float32) - base).astype(np.float16)
    return res


def quantlinear_forward_cpu(q: Dict, bufs: Dict, x, bias=None, max_dequant_rows: int = 4096):
    """modules.py:752-804, 924-940: the reference's CPU fallback forward for a
    bf16/fp16 input (fast_dequant: reconstruction in the input dtype), built
    from torch CPU ops in the reference's order. Used as the timed CPU baseline
    and checked against the golden CPU outputs."""
    import torch
    import torch.nn.functional as F
    meta = q["_meta"]
    rows, cols, pc, ng, gs, bits = (meta["rows"], meta["cols"], meta["padded_cols"], meta["n_groups"],
                                    meta["group_size"], meta["bits"])
    cdt = x.dtype
    sc32, gm32 = quantlinear_scale_gmin(q)
    sc_full = torch.from_numpy(sc32)
    gm_full = torch.from_numpy(gm32)
    packed = torch.from_numpy(q["packed"])
    orow = torch.from_numpy(bufs["outlier_row"])
    ocol = torch.from_numpy(bufs["outlier_col"])
    odelta = torch.from_numpy(bufs["outlier_delta"])
    cb = torch.from_numpy(q["codebook"].astype(np.float32)) if q.get("codebook") is not None else None
    b = bias.to(cdt) if bias is not None else None
    orow_np = bufs["outlier_row"]

    def deq_rows(r0, r1):
        n = r1 - r0
        sc = sc_full[r0:r1].to(cdt)
        gm = gm_full[r0:r1].to(cdt)
        pk = packed[r0:r1]
        if bits == 2:
            c = pk.unsqueeze(-1) >> torch.tensor([0, 2, 4, 6], dtype=torch.uint8)
            codes = (c & 0x03).reshape(n, -1)[:, :pc]
        elif bits == 4:
            codes = torch.stack([pk & 0x0F, (pk >> 4) & 0x0F], dim=-1).reshape(n, -1)[:, :pc]
        else:
            codes = pk
        if cb is not None:
            cv = cb.to(cdt)[codes.reshape(-1).to(torch.long)].reshape(n, ng, gs)
        else:
            cv = codes.reshape(n, ng, gs).to(cdt)
        deq = cv * sc.unsqueeze(-1) + gm.unsqueeze(-1)
        flat = deq.reshape(n, pc)[:, :cols].reshape(-1)
        lo = int(np.searchsorted(orow_np, r0, side="left"))
        hi = int(np.searchsorted(orow_np, r1, side="left"))
        if hi > lo:
            li = (orow[lo:hi] - r0).to(torch.int64) * cols + ocol[lo:hi].to(torch.int64)
            base = flat[li].to(torch.float32)
            flat[li] = (base + odelta[lo:hi].to(torch.float32)).to(cdt)
        return flat.reshape(n, cols).to(cdt)

    if rows <= max_dequant_rows:
        return F.linear(x, deq_rows(0, rows), b)
    outs = []
    for s in range(0, rows, max_dequant_rows):
        e = min(s + max_dequant_rows, rows)
        outs.append(F.linear(x, deq_rows(s, e), b[s:e] if b is not None else None))
    return torch.cat(outs, dim=-1)
