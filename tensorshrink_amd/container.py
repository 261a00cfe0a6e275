"""The .tsk container: a whole quantized state_dict in one append-only file.

Same on-disk layout as the reference's container.py (GDNickk/tensorshrink
v0.4.0), so either implementation reads the other's files:

    [zstd frame of tensor 1] ... [zstd frame of tensor N]
    [manifest JSON, utf-8]
    [u64 little-endian: manifest length] [b"TSHRNK01"]

(container.py:18-30, 59, 288-293). The manifest is
{"format": "tensorshrink-v1", "format_version": 2, "tensors": {name: entry}}.
A quantized entry (container.py:156-220) carries the QuantizedTensor's shape
fields, "n_outliers", "rel_error", "escalated", "force_fp32_compute",
"outlier_encoding": "delta_row_v1" and "segments_v2" = {"blob": {offset,
length} in the file, "parts": {name: {offset, length, np_dtype, shape}} in the
decompressed blob}, with parts packed, scale, gmin, outlier_row_delta,
outlier_col (u16, or u32 when a row delta or a column does not fit),
outlier_val and, for codebook grids, codebook ("companded": true). Outliers
are stable-sorted by row and the row stored as the difference to the
previous outlier's row (container.py:98-141). scale/gmin are the
QuantizedTensor's f16 values (double-quant reconstructed); the double-quant
codes are not stored, as in the reference. A raw entry (container.py:223-242)
holds one array ("segments": {"data": {...}}); bf16 is stored as float32 and
"orig_torch_dtype" restores it. Readers also accept format-1 entries
("segments" with one frame per array).

Addition over the reference: a 6-bit (RVQ) tensor also stores its second
stage as parts stage2_packed / stage2_scale / stage2_gmin, which the
reference drops (its reader ignores parts it does not know).

Compression goes through the system libzstd (tensorshrink_amd._zstd); the
reference's `zstandard` package is not in this image. The frame bytes can
differ from the reference's (zstd version, threading); the decompressed
blobs and the manifest are the format.
"""
from __future__ import annotations

import io
import json
import mmap
import os
import struct
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path
from typing import Dict, Iterable, List, Optional, Tuple

import numpy as np
import torch

from . import _zstd
from .codec import (
    LayerBitStats,
    QuantizedTensor,
    budget_allocate_bits,
    dequantize_tensor,
    estimate_resident_nbytes,
    quantize_tensor,
    quantize_tensor_adaptive,
    relative_error,
)

MAGIC = b"TSHRNK01"
FORMAT = "tensorshrink-v1"
CONTAINER_FORMAT_VERSION = 2
ZSTD_LEVEL = 12
ZSTD_LEVEL_MAX = 19
DEFAULT_CONTAINER_SKIP = ("norm", "bias", "position", "shared", "relative_attention_bias")


# ---------------------------------------------------------------------------
# entries
# ---------------------------------------------------------------------------

def encode_outliers(outlier_idx: np.ndarray, outlier_val: np.ndarray, cols: int):
    """Flat outlier indices -> (row_delta, col, val, dtype name), stable-sorted
    by row; u16 when every row delta and column fits, else u32
    (container.py:98-141)."""
    n = int(outlier_idx.shape[0])
    if n == 0:
        return np.zeros(0, np.uint16), np.zeros(0, np.uint16), np.asarray(outlier_val), "uint16"
    flat = outlier_idx.astype(np.int64)
    order = np.argsort(flat // cols, kind="stable")
    rows = (flat // cols)[order]
    col = (flat % cols)[order]
    delta = np.diff(rows, prepend=0)
    wide = int(delta.max()) >= 65536 or cols - 1 >= 65536
    dt = np.uint32 if wide else np.uint16
    return delta.astype(dt), col.astype(dt), np.asarray(outlier_val)[order], np.dtype(dt).name


def decode_outliers(row_delta: np.ndarray, col: np.ndarray, cols: int) -> np.ndarray:
    """(row_delta, col) -> flat int32 outlier indices (container.py:144-153)."""
    if row_delta.shape[0] == 0:
        return np.zeros(0, np.int32)
    return (np.cumsum(row_delta.astype(np.int64)) * cols + col.astype(np.int64)).astype(np.int32)


def _blob(arrays: List[Tuple[str, np.ndarray]]) -> Tuple[dict, bytes]:
    parts, chunks, off = {}, [], 0
    for name, a in arrays:
        a = np.ascontiguousarray(a)
        b = a.tobytes()
        parts[name] = {"offset": off, "length": len(b), "np_dtype": str(a.dtype), "shape": list(a.shape)}
        chunks.append(b)
        off += len(b)
    return parts, b"".join(chunks)


def quantized_entry(qt: QuantizedTensor, rel_error: Optional[float] = None, escalated: Optional[bool] = None,
                    force_fp32_compute: bool = False) -> Tuple[dict, bytes]:
    """Manifest entry (without file offsets) and uncompressed blob of one
    QuantizedTensor (container.py:156-220)."""
    if qt.smooth_scale is not None:
        raise NotImplementedError("smooth-scaled tensors are not covered by tensorshrink_amd")
    delta, col, val, _ = encode_outliers(qt.outlier_idx, qt.outlier_val, qt.cols)
    arrays = [("packed", qt.packed), ("scale", qt.scale), ("gmin", qt.gmin), ("outlier_row_delta", delta),
              ("outlier_col", col), ("outlier_val", val)]
    entry = {"kind": "quant", "orig_shape": list(qt.orig_shape), "orig_dtype": qt.orig_dtype, "bits": qt.bits,
             "group_size": qt.group_size, "rows": qt.rows, "cols": qt.cols, "padded_cols": qt.padded_cols,
             "n_groups": qt.n_groups, "n_outliers": qt.n_outliers(), "rel_error": rel_error,
             "escalated": None if escalated is None else bool(escalated),
             "force_fp32_compute": bool(force_fp32_compute), "outlier_encoding": "delta_row_v1"}
    if qt.codebook is not None:
        arrays.append(("codebook", qt.codebook))
        entry["companded"] = True
    if qt.bits == 6:
        arrays += [("stage2_packed", qt.stage2_packed), ("stage2_scale", qt.stage2_scale),
                   ("stage2_gmin", qt.stage2_gmin)]
    entry["_parts"], blob = _blob(arrays)
    return entry, blob


def raw_entry(tensor: torch.Tensor) -> Tuple[dict, bytes]:
    """Manifest entry and uncompressed bytes of a raw tensor
    (container.py:223-242): bf16 goes to disk as float32."""
    t = tensor.detach().to("cpu").contiguous()
    orig = str(t.dtype).replace("torch.", "")
    if t.dtype == torch.bfloat16:
        t = t.to(torch.float32)
    a = t.numpy()
    return ({"kind": "raw", "orig_shape": list(tensor.shape), "orig_torch_dtype": orig, "np_dtype": str(a.dtype),
             "_data_shape": list(a.shape)}, a.tobytes())


# ---------------------------------------------------------------------------
# writer
# ---------------------------------------------------------------------------

class ContainerWriter:
    """Appends one compressed frame per tensor; the manifest and footer are
    written by close() (container.py:245-308)."""

    def __init__(self, path):
        self.path = str(path)
        self._f = open(self.path, "wb")
        self._pos = 0
        self._manifest = {"format": FORMAT, "format_version": CONTAINER_FORMAT_VERSION, "tensors": {}}

    def add_precompressed(self, name: str, entry: dict, frame: bytes) -> None:
        entry = dict(entry)
        off = self._pos
        self._f.write(frame)
        self._pos += len(frame)
        if entry["kind"] == "quant":
            entry["segments_v2"] = {"blob": {"offset": off, "length": len(frame)}, "parts": entry.pop("_parts")}
        else:
            entry["segments"] = {"data": {"offset": off, "length": len(frame), "np_dtype": entry["np_dtype"],
                                          "shape": entry.pop("_data_shape")}}
        self._manifest["tensors"][name] = entry

    def add_quantized(self, name: str, qt: QuantizedTensor, rel_error: Optional[float] = None,
                      escalated: Optional[bool] = None, force_fp32_compute: bool = False,
                      level: int = ZSTD_LEVEL) -> None:
        entry, blob = quantized_entry(qt, rel_error, escalated, force_fp32_compute)
        self.add_precompressed(name, entry, _zstd.compress(blob, level))

    def add_raw(self, name: str, tensor: torch.Tensor, level: int = ZSTD_LEVEL) -> None:
        entry, blob = raw_entry(tensor)
        self.add_precompressed(name, entry, _zstd.compress(blob, level))

    def close(self) -> None:
        if self._f.closed:
            return
        m = json.dumps(self._manifest).encode("utf-8")
        self._f.write(m)
        self._f.write(struct.pack("<Q", len(m)))
        self._f.write(MAGIC)
        self._f.close()

    def __enter__(self):
        return self

    def __exit__(self, exc_type, exc, tb):
        if exc_type is None:
            self.close()
        else:
            self._f.close()


# ---------------------------------------------------------------------------
# reader
# ---------------------------------------------------------------------------

class ContainerReader:
    """Reads the manifest from the footer and decompresses one tensor's frame
    on demand through a read-only mmap (container.py:315-507)."""

    def __init__(self, path):
        self.path = str(path)
        self._f = open(self.path, "rb")
        size = os.fstat(self._f.fileno()).st_size
        if size < 16:
            raise ValueError(f"{path} is not a tensorshrink container (too short)")
        self._f.seek(size - 16)
        tail = self._f.read(16)
        if tail[8:] != MAGIC:
            raise ValueError(f"{path} is not a tensorshrink container (bad magic footer)")
        (mlen,) = struct.unpack("<Q", tail[:8])
        if mlen > size - 16:
            raise ValueError(f"{path}: manifest length {mlen} exceeds the file")
        self._f.seek(size - 16 - mlen)
        self.manifest = json.loads(self._f.read(mlen).decode("utf-8"))
        if self.manifest.get("format") != FORMAT:
            raise ValueError(f"{path}: unknown container format {self.manifest.get('format')!r}")
        try:
            self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        except (ValueError, OSError):
            self._mm = None

    def names(self) -> List[str]:
        return list(self.manifest["tensors"])

    def kind(self, name: str) -> str:
        return self.manifest["tensors"][name]["kind"]

    def _frame(self, offset: int, length: int) -> bytes:
        if self._mm is not None:
            return _zstd.decompress(self._mm[offset:offset + length])
        self._f.seek(offset)
        return _zstd.decompress(self._f.read(length))

    @staticmethod
    def _view(raw: bytes, m: dict, base: int = 0) -> np.ndarray:
        dt = np.dtype(m["np_dtype"])
        a = np.frombuffer(raw, dtype=dt, count=m["length"] // dt.itemsize, offset=base + m.get("offset", 0))
        return a.copy().reshape(m["shape"])

    def _read_v1(self, seg: dict) -> np.ndarray:
        raw = self._frame(seg["offset"], seg["length"])
        return self._view(raw, dict(seg, offset=0, length=len(raw)))

    def get_quantized(self, name: str) -> QuantizedTensor:
        e = self.manifest["tensors"][name]
        if e["kind"] != "quant":
            raise ValueError(f"tensor {name!r} is stored raw, not quantized")
        extra = {}
        if "segments_v2" in e:
            blob = self._frame(e["segments_v2"]["blob"]["offset"], e["segments_v2"]["blob"]["length"])
            parts = e["segments_v2"]["parts"]
            p = {k: self._view(blob, m) for k, m in parts.items()}
            if e.get("outlier_encoding") == "delta_row_v1":
                idx = decode_outliers(p["outlier_row_delta"], p["outlier_col"], e["cols"])
            else:
                idx = p["outlier_idx"]
            codebook = p.get("codebook") if e.get("companded") else None
            if e["bits"] == 6 and "stage2_packed" in p:
                extra = dict(stage2_packed=p["stage2_packed"], stage2_scale=p["stage2_scale"],
                             stage2_gmin=p["stage2_gmin"])
            packed, scale, gmin, val = p["packed"], p["scale"], p["gmin"], p["outlier_val"]
        else:  # format 1: one frame per array
            s = e["segments"]
            packed, scale, gmin = self._read_v1(s["packed"]), self._read_v1(s["scale"]), self._read_v1(s["gmin"])
            idx, val = self._read_v1(s["outlier_idx"]), self._read_v1(s["outlier_val"])
            codebook = None
        return QuantizedTensor(orig_shape=tuple(e["orig_shape"]), orig_dtype=e["orig_dtype"], bits=e["bits"],
                               group_size=e["group_size"], rows=e["rows"], cols=e["cols"],
                               padded_cols=e["padded_cols"], n_groups=e["n_groups"], packed=packed, scale=scale,
                               gmin=gmin, outlier_idx=idx, outlier_val=val, codebook=codebook, **extra)

    def get_quantized_many(self, names: Iterable[str], max_workers: Optional[int] = None
                           ) -> Dict[str, QuantizedTensor]:
        """Several tensors at once; libzstd runs outside the GIL, so the
        frames decompress in parallel threads (container.py:446-473)."""
        names = list(names)
        if self._mm is None or len(names) <= 1:
            return {n: self.get_quantized(n) for n in names}
        with ThreadPoolExecutor(max_workers=max_workers or min(32, 2 * (os.cpu_count() or 4))) as ex:
            return dict(zip(names, ex.map(self.get_quantized, names)))

    def get(self, name: str, device=None, dtype=None) -> torch.Tensor:
        """Raw tensors as stored; quantized ones dequantized (codec view)."""
        e = self.manifest["tensors"][name]
        if e["kind"] == "raw":
            t = torch.from_numpy(self._read_v1(e["segments"]["data"]))
            if e.get("orig_torch_dtype"):
                t = t.to(getattr(torch, e["orig_torch_dtype"]))
        else:
            t = dequantize_tensor(self.get_quantized(name))
        if device is not None:
            t = t.to(device)
        if dtype is not None:
            t = t.to(dtype)
        return t

    def stats(self) -> dict:
        """Tensor count, bit-width mix and sizes (container.py:475-502)."""
        orig = data = 0
        counts: Dict[str, int] = {}
        for e in self.manifest["tensors"].values():
            n = int(np.prod(e["orig_shape"])) if e["orig_shape"] else 1
            orig += n * {"float16": 2, "bfloat16": 2, "float32": 4}.get(e.get("orig_dtype", "float16"), 2)
            if e["kind"] == "quant":
                counts[str(e["bits"])] = counts.get(str(e["bits"]), 0) + 1
                data += (e["segments_v2"]["blob"]["length"] if "segments_v2" in e
                         else sum(s["length"] for s in e["segments"].values()))
            else:
                counts["raw"] = counts.get("raw", 0) + 1
                data += e["segments"]["data"]["length"]
        return {"n_tensors": len(self.manifest["tensors"]), "orig_bytes": orig,
                "container_bytes_for_tensor_data": data, "file_bytes": os.path.getsize(self.path),
                "bit_width_counts": counts}

    def close(self) -> None:
        if self._mm is not None:
            self._mm.close()
            self._mm = None
        self._f.close()

    def __enter__(self):
        return self

    def __exit__(self, exc_type, exc, tb):
        self.close()


# ---------------------------------------------------------------------------
# whole-state_dict helpers
# ---------------------------------------------------------------------------

def _eligible(name: str, t: torch.Tensor, min_numel: int, skip: Tuple[str, ...]) -> bool:
    return t.dim() >= 2 and t.numel() >= min_numel and not any(p in name.lower() for p in skip)


def save_container(state_dict: Dict[str, torch.Tensor], out_path, **quantize_kwargs) -> dict:
    """Quantize every eligible tensor of an in-memory state_dict (adaptive
    2 -> 4 -> 8 by default) and write the container (container.py:510-540)."""
    min_numel = quantize_kwargs.pop("min_numel", 16384)
    skip = tuple(quantize_kwargs.pop("skip_name_patterns", DEFAULT_CONTAINER_SKIP))
    quantize_kwargs.setdefault("allowed_bits", (2, 4, 8))
    stats = {"tensors": [], "orig_bytes": 0}
    with ContainerWriter(out_path) as w:
        for name, t in state_dict.items():
            nbytes = t.numel() * t.element_size()
            if _eligible(name, t, min_numel, skip):
                qt, err, esc = quantize_tensor_adaptive(t, **quantize_kwargs)
                w.add_quantized(name, qt, rel_error=err, escalated=esc)
                stats["tensors"].append({"name": name, "bits": qt.bits, "rel_error": err, "orig_bytes": nbytes})
            else:
                w.add_raw(name, t)
                stats["tensors"].append({"name": name, "bits": None, "rel_error": 0.0, "orig_bytes": nbytes})
            stats["orig_bytes"] += nbytes
    stats["file_bytes"] = os.path.getsize(str(out_path))
    return stats


def _shards(model_dir: Path) -> Dict[str, List[str]]:
    """{shard file: [tensor names]} of a HF safetensors checkpoint directory,
    single file or sharded with an index (container.py:547-568)."""
    from safetensors import safe_open
    index = sorted(model_dir.glob("*.safetensors.index.json"))
    if index:
        out: Dict[str, List[str]] = {}
        for t, f in json.loads(index[0].read_text(encoding="utf-8"))["weight_map"].items():
            out.setdefault(f, []).append(t)
        return out
    files = sorted(model_dir.glob("*.safetensors"))
    if not files:
        raise FileNotFoundError(f"no .safetensors files in {model_dir}")
    out = {}
    for f in files:
        with safe_open(str(f), framework="pt", device="cpu") as sf:
            out[f.name] = list(sf.keys())
    return out


def stream_quantize_safetensors_dir(model_dir, out_path, group_size: int = 128, outlier_frac: float = 0.003,
                                    error_threshold: float = 0.06, min_numel: int = 16384,
                                    skip_name_patterns: Iterable[str] = DEFAULT_CONTAINER_SKIP,
                                    progress: bool = True, parallel: bool = True, n_workers: Optional[int] = None,
                                    zstd_level: int = ZSTD_LEVEL, vram_budget_mb: Optional[float] = None) -> dict:
    """Quantize a HF safetensors checkpoint directory straight into one
    container, one tensor in memory at a time (container.py:643-834). The
    quantize runs on the GPU codec; with `parallel`, a tensor's zstd
    compression overlaps the next tensor's quantize (`n_workers` compression
    threads) instead of the reference's process pool."""
    from safetensors import safe_open
    model_dir = Path(model_dir)
    shards = _shards(model_dir)
    skip = tuple(skip_name_patterns)
    plan: Dict[str, int] = {}
    if vram_budget_mb is not None:
        ls = []
        for fname, names in shards.items():
            with safe_open(str(model_dir / fname), framework="pt", device="cpu") as sf:
                for tname in names:
                    t = sf.get_tensor(tname)
                    if not _eligible(tname, t, min_numel, skip):
                        continue
                    q4 = quantize_tensor(t, bits=4, group_size=group_size, outlier_frac=outlier_frac)
                    q8 = quantize_tensor(t, bits=8, group_size=group_size, outlier_frac=outlier_frac)
                    ls.append(LayerBitStats(tname, estimate_resident_nbytes(q4), estimate_resident_nbytes(q8),
                                            relative_error(t, q4), relative_error(t, q8)))
        plan = budget_allocate_bits(ls, vram_budget_mb * 1024 * 1024)
    per, tot_orig, tot_packed = [], 0, 0
    pool = ThreadPoolExecutor(max_workers=n_workers or 4) if parallel else None
    pending = []  # (future, name, entry) in write order

    def drain(keep: int):
        while len(pending) > keep:
            fut, n, e = pending.pop(0)
            w.add_precompressed(n, e, fut.result())

    with ContainerWriter(out_path) as w:
        for fname, names in shards.items():
            with safe_open(str(model_dir / fname), framework="pt", device="cpu") as sf:
                for tname in names:
                    t = sf.get_tensor(tname)
                    nbytes = t.numel() * t.element_size()
                    if _eligible(tname, t, min_numel, skip):
                        if tname in plan:
                            qt = quantize_tensor(t, bits=plan[tname], group_size=group_size,
                                                 outlier_frac=outlier_frac)
                            err, esc = relative_error(t, qt), plan[tname] == 8
                        else:
                            qt, err, esc = quantize_tensor_adaptive(t, group_size=group_size,
                                                                    outlier_frac=outlier_frac,
                                                                    error_threshold=error_threshold,
                                                                    allowed_bits=(2, 4, 8))
                        entry, blob = quantized_entry(qt, rel_error=err, escalated=esc)
                        bits, packed = qt.bits, qt.compressed_nbytes()
                    else:
                        entry, blob = raw_entry(t)
                        bits, packed, err = None, nbytes, 0.0
                    if pool is not None:
                        pending.append((pool.submit(_zstd.compress, blob, zstd_level), tname, entry))
                        drain(2 * (n_workers or 4))
                    else:
                        w.add_precompressed(tname, entry, _zstd.compress(blob, zstd_level))
                    per.append({"name": tname, "shard": fname, "shape": list(t.shape), "bits": bits,
                                "rel_error": err, "orig_bytes": nbytes, "packed_bytes": packed})
                    tot_orig += nbytes
                    tot_packed += packed
                    if progress:
                        tag = f"{bits}b" if bits else "raw"
                        print(f"  [{tag:>4s}] {tname:65s} {nbytes / 1e6:9.2f}MB -> {packed / 1e6:9.2f}MB"
                              + (f"  err={err:.4f}" if bits else ""))
                    del t
        drain(0)
    if pool is not None:
        pool.shutdown()
    return {"n_tensors": len(per), "orig_bytes": tot_orig, "packed_bytes_pre_entropy_coding": tot_packed,
            "container_file_bytes": os.path.getsize(str(out_path)), "tensors": per}
