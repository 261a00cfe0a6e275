"""The .tsk container on the CPU: file layout (footer, manifest, one zstd frame
per tensor, parts packed back to back), round trips of the reference's own
QuantizedTensors (the golden cases), the delta-row outlier encoding, raw
entries, format-1 files, and files assembled here byte by byte from the
layout alone.

The compressed bytes are "parity unpinned": the reference's `zstandard`
package is not in this image and zstd's output depends on its version and
threading; what is pinned is the decompressed content and the manifest."""
import json
import struct

import numpy as np
import pytest
import torch

from golden_io import QT_FIELDS, case_names, load_case
from oracle import codec_ref as O
from tensorshrink_amd import _zstd
from tensorshrink_amd.codec import QuantizedTensor
from tensorshrink_amd.container import (MAGIC, ContainerReader, ContainerWriter, decode_outliers, encode_outliers)

PART_ORDER = ("packed", "scale", "gmin", "outlier_row_delta", "outlier_col", "outlier_val")


def _golden_qt(name):
    spec, res, d, w = load_case(name)
    m = res["meta"]
    kw = {f: d["qt_" + f] for f in QT_FIELDS if "qt_" + f in d.files}
    qt = QuantizedTensor(orig_shape=tuple(w.shape), orig_dtype=m["orig_dtype"], bits=m["bits"],
                         group_size=m["group_size"], rows=m["rows"], cols=m["cols"], padded_cols=m["padded_cols"],
                         n_groups=m["n_groups"], **kw)
    return qt, d


def _parse(path):
    """The container read with nothing but the layout: footer, manifest, frames."""
    raw = open(path, "rb").read()
    assert raw[-8:] == MAGIC
    (n,) = struct.unpack("<Q", raw[-16:-8])
    manifest = json.loads(raw[-16 - n:-16].decode("utf-8"))
    return raw, manifest


def _as_dict(qt):
    q = {f: getattr(qt, f) for f in QT_FIELDS if getattr(qt, f) is not None}
    q["_meta"] = dict(bits=qt.bits, group_size=qt.group_size, rows=qt.rows, cols=qt.cols,
                      padded_cols=qt.padded_cols, n_groups=qt.n_groups, orig_dtype=qt.orig_dtype)
    return q


@pytest.mark.parametrize("name", case_names())
def test_golden_round_trip(tmp_path, name):
    """Every stored part comes back bit for bit; outliers come back
    stable-sorted by row; DQ codes are not stored, so the tensor reads back
    with its f16 scale/gmin as the reference's reader returns it."""
    qt, d = _golden_qt(name)
    path = tmp_path / "m.tsk"
    with ContainerWriter(path) as w:
        w.add_quantized("w", qt, rel_error=0.25, escalated=False)
    with ContainerReader(path) as r:
        back = r.get_quantized("w")
        e = r.manifest["tensors"]["w"]
    for f in ("packed", "scale", "gmin", "codebook", "stage2_packed", "stage2_scale", "stage2_gmin"):
        a, b = getattr(qt, f), getattr(back, f)
        assert (a is None) == (b is None), f
        if a is not None:
            assert a.dtype == b.dtype and a.shape == b.shape, f
            np.testing.assert_array_equal(a.view(np.uint8), b.view(np.uint8), err_msg=f)
    assert back.dq_scale_codes is None and back.smooth_scale is None
    order = np.argsort(qt.outlier_idx.astype(np.int64) // qt.cols, kind="stable")
    np.testing.assert_array_equal(back.outlier_idx, qt.outlier_idx[order])
    np.testing.assert_array_equal(back.outlier_val.view(np.uint16), qt.outlier_val[order].view(np.uint16))
    assert back.outlier_idx.dtype == np.int32
    assert (back.orig_shape, back.orig_dtype, back.bits, back.group_size, back.rows, back.cols, back.padded_cols,
            back.n_groups) == (qt.orig_shape, qt.orig_dtype, qt.bits, qt.group_size, qt.rows, qt.cols,
                               qt.padded_cols, qt.n_groups)
    assert e["n_outliers"] == qt.n_outliers() and e["rel_error"] == 0.25 and e["escalated"] is False
    assert e["outlier_encoding"] == "delta_row_v1" and e["kind"] == "quant"
    assert e.get("companded", False) == (qt.codebook is not None)
    # the read-back tensor dequantizes to the reference's own output (non-DQ)
    if qt.dq_scale_codes is None:
        deq = O.dequantize_rvq(_as_dict(back)) if qt.bits == 6 else O.dequantize(_as_dict(back), "f32")
        np.testing.assert_array_equal(deq.view(np.uint32), d["deq_f32"].view(np.uint32))


def test_manifest_and_layout(tmp_path):
    """The frames sit back to back from offset 0, the manifest follows them,
    the footer is u64 LE length + magic; each blob holds its parts in write
    order with no gaps."""
    qt, _ = _golden_qt("nf4_dq_g64")
    qt2, _ = _golden_qt("pad_u2_g32")
    path = tmp_path / "m.tsk"
    with ContainerWriter(path) as w:
        w.add_quantized("a.weight", qt, force_fp32_compute=True)
        w.add_raw("a.bias", torch.arange(7, dtype=torch.float16))
        w.add_quantized("b.weight", qt2)
    raw, man = _parse(path)
    assert man["format"] == "tensorshrink-v1" and man["format_version"] == 2
    assert list(man["tensors"]) == ["a.weight", "a.bias", "b.weight"]
    pos = 0
    for name, e in man["tensors"].items():
        seg = e["segments_v2"]["blob"] if e["kind"] == "quant" else e["segments"]["data"]
        assert seg["offset"] == pos, name
        pos += seg["length"]
        frame = raw[seg["offset"]:seg["offset"] + seg["length"]]
        assert frame[:4] == b"\x28\xb5\x2f\xfd"  # zstd frame magic
        blob = _zstd.decompress(frame)
        if e["kind"] == "quant":
            parts = e["segments_v2"]["parts"]
            names = list(PART_ORDER) + (["codebook"] if e.get("companded") else [])
            assert list(parts) == names
            off = 0
            for p in names:
                assert parts[p]["offset"] == off
                off += parts[p]["length"]
                assert parts[p]["length"] == int(np.prod(parts[p]["shape"], dtype=np.int64)) * \
                    np.dtype(parts[p]["np_dtype"]).itemsize
            assert off == len(blob)
            assert set(e) >= {"orig_shape", "orig_dtype", "bits", "group_size", "rows", "cols", "padded_cols",
                              "n_groups", "n_outliers", "rel_error", "escalated", "force_fp32_compute"}
            assert "_parts" not in e
        else:
            assert e["orig_torch_dtype"] == "float16" and e["np_dtype"] == "float16"
            assert np.frombuffer(blob, np.float16).tolist() == list(range(7))
    assert pos == len(raw) - 16 - len(json.dumps(man).encode())
    assert man["tensors"]["a.weight"]["force_fp32_compute"] is True
    assert man["tensors"]["b.weight"]["force_fp32_compute"] is False
    assert "segments" not in man["tensors"]["a.weight"]


def _hand_v2(path, entries):
    """A format-2 container written from the layout description alone."""
    body, tensors = bytearray(), {}
    for name, (meta, parts) in entries.items():
        blob, pm = bytearray(), {}
        for pn, a in parts:
            pm[pn] = {"offset": len(blob), "length": a.nbytes, "np_dtype": str(a.dtype), "shape": list(a.shape)}
            blob += a.tobytes()
        frame = _zstd.compress(bytes(blob), 3)
        tensors[name] = dict(meta, segments_v2={"blob": {"offset": len(body), "length": len(frame)}, "parts": pm})
        body += frame
    m = json.dumps({"format": "tensorshrink-v1", "format_version": 2, "tensors": tensors}).encode()
    open(path, "wb").write(bytes(body) + m + struct.pack("<Q", len(m)) + MAGIC)


def test_reads_hand_built_v2(tmp_path):
    rng = np.random.default_rng(1)
    packed = rng.integers(0, 256, (3, 4), dtype=np.uint8)
    scale = rng.random((3, 1)).astype(np.float16)
    gmin = (-rng.random((3, 1))).astype(np.float16)
    # outliers at (0, 5), (0, 1), (2, 7): rows 0, 0, 2 -> deltas 0, 0, 2
    meta = dict(kind="quant", orig_shape=[3, 8], orig_dtype="float16", bits=4, group_size=8, rows=3, cols=8,
                padded_cols=8, n_groups=1, n_outliers=3, rel_error=None, escalated=None, force_fp32_compute=False,
                outlier_encoding="delta_row_v1")
    parts = [("packed", packed), ("scale", scale), ("gmin", gmin),
             ("outlier_row_delta", np.array([0, 0, 2], np.uint16)), ("outlier_col", np.array([5, 1, 7], np.uint16)),
             ("outlier_val", np.array([1.5, -2.0, 3.0], np.float16))]
    legacy = dict(meta, outlier_encoding=None)
    legacy_parts = parts[:3] + [("outlier_idx", np.array([5, 1, 23], np.int32)), parts[5]]
    _hand_v2(tmp_path / "h.tsk", {"x": (meta, parts), "y": (legacy, legacy_parts)})
    with ContainerReader(tmp_path / "h.tsk") as r:
        for n in ("x", "y"):
            q = r.get_quantized(n)
            assert q.outlier_idx.tolist() == [5, 1, 23]
            assert q.outlier_val.tolist() == [1.5, -2.0, 3.0]
            np.testing.assert_array_equal(q.packed, packed)
            np.testing.assert_array_equal(q.scale.view(np.uint16), scale.view(np.uint16))
            assert q.codebook is None
        st = r.stats()
    assert st["n_tensors"] == 2 and st["bit_width_counts"] == {"4": 2} and st["orig_bytes"] == 2 * 24 * 2


def test_reads_format_1(tmp_path):
    """Format 1: one frame per array under "segments" (file offsets)."""
    arrays = {"packed": np.arange(16, dtype=np.uint8).reshape(2, 8), "scale": np.ones((2, 1), np.float16),
              "gmin": np.zeros((2, 1), np.float16), "outlier_idx": np.array([9], np.int32),
              "outlier_val": np.array([4.0], np.float16)}
    body, segs = bytearray(), {}
    for k, a in arrays.items():
        f = _zstd.compress(a.tobytes(), 1)
        segs[k] = {"offset": len(body), "length": len(f), "np_dtype": str(a.dtype), "shape": list(a.shape)}
        body += f
    raw = torch.tensor([[1.0, 2.0]], dtype=torch.float32)
    f = _zstd.compress(raw.numpy().tobytes(), 1)
    rseg = {"data": {"offset": len(body), "length": len(f), "np_dtype": "float32", "shape": [1, 2]}}
    body += f
    man = {"format": "tensorshrink-v1", "format_version": 1, "tensors": {
        "q": dict(kind="quant", orig_shape=[2, 16], orig_dtype="float16", bits=4, group_size=16, rows=2, cols=16,
                  padded_cols=16, n_groups=1, segments=segs),
        "r": dict(kind="raw", orig_shape=[1, 2], np_dtype="float32", segments=rseg)}}
    m = json.dumps(man).encode()
    (tmp_path / "v1.tsk").write_bytes(bytes(body) + m + struct.pack("<Q", len(m)) + MAGIC)
    with ContainerReader(tmp_path / "v1.tsk") as r:
        q = r.get_quantized("q")
        assert q.outlier_idx.tolist() == [9] and q.packed.tolist() == arrays["packed"].tolist()
        assert r.get("r").tolist() == [[1.0, 2.0]] and r.get("r").dtype == torch.float32
        with pytest.raises(ValueError):
            r.get_quantized("r")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32, torch.int64])
def test_raw_round_trip(tmp_path, dtype):
    t = (torch.randn(5, 3) * 100).to(dtype)
    with ContainerWriter(tmp_path / "r.tsk") as w:
        w.add_raw("t", t)
    raw, man = _parse(tmp_path / "r.tsk")
    e = man["tensors"]["t"]
    assert e["orig_torch_dtype"] == str(dtype).replace("torch.", "")
    assert e["np_dtype"] == ("float32" if dtype == torch.bfloat16 else str(dtype).replace("torch.", ""))
    with ContainerReader(tmp_path / "r.tsk") as r:
        back = r.get("t")
        assert r.kind("t") == "raw" and r.names() == ["t"]
    assert back.dtype == dtype and torch.equal(back, t)


def test_outlier_encoding():
    cols = 10
    idx = np.array([95, 3, 41, 7, 40, 99], np.int32)  # rows 9, 0, 4, 0, 4, 9
    val = np.arange(6).astype(np.float16)
    delta, col, v, dt = encode_outliers(idx, val, cols)
    assert dt == "uint16" and delta.dtype == np.uint16
    assert delta.tolist() == [0, 0, 4, 0, 5, 0]          # rows 0, 0, 4, 4, 9, 9
    assert col.tolist() == [3, 7, 1, 0, 5, 9]            # stable: top-k order kept within a row
    assert v.tolist() == [1, 3, 2, 4, 0, 5]
    assert decode_outliers(delta, col, cols).tolist() == [3, 7, 41, 40, 95, 99]
    # a column past u16 -> u32 parts
    d2, c2, _, dt2 = encode_outliers(np.array([70000], np.int32), np.ones(1, np.float16), 70001)
    assert dt2 == "uint32" and d2.dtype == np.uint32 and c2.tolist() == [70000]
    # a row jump past u16 -> u32 parts
    d3, c3, _, dt3 = encode_outliers(np.array([0, 70000 * 4 + 1], np.int32), np.ones(2, np.float16), 4)
    assert dt3 == "uint32" and d3.tolist() == [0, 70000]
    assert decode_outliers(d3, c3, 4).tolist() == [0, 280001]
    e = encode_outliers(np.zeros(0, np.int32), np.zeros(0, np.float16), 8)
    assert e[0].size == 0 and decode_outliers(e[0], e[1], 8).dtype == np.int32


def test_rejects_non_container(tmp_path):
    (tmp_path / "x.tsk").write_bytes(b"not a container at all")
    with pytest.raises(ValueError, match="magic"):
        ContainerReader(tmp_path / "x.tsk")
    (tmp_path / "y.tsk").write_bytes(b"\x00" * 4)
    with pytest.raises(ValueError):
        ContainerReader(tmp_path / "y.tsk")


def test_get_quantized_many(tmp_path):
    qts = {n: _golden_qt(n)[0] for n in ("u4_g128", "u8_g128", "nf2_dq_g64", "lm4_g128")}
    with ContainerWriter(tmp_path / "m.tsk") as w:
        for n, q in qts.items():
            w.add_quantized(n, q)
    with ContainerReader(tmp_path / "m.tsk") as r:
        many = r.get_quantized_many(list(qts), max_workers=4)
        one = {n: r.get_quantized(n) for n in qts}
        st = r.stats()
    for n in qts:
        np.testing.assert_array_equal(many[n].packed, one[n].packed)
        np.testing.assert_array_equal(many[n].outlier_idx, one[n].outlier_idx)
    assert st["bit_width_counts"] == {"4": 2, "8": 1, "2": 1}


@pytest.mark.parametrize("n", [0, 1, 1000, 3 << 20])
def test_zstd_frames(n):
    data = np.random.default_rng(n).integers(0, 4, n, dtype=np.uint8).tobytes()
    f = _zstd.compress(data, 12)
    assert f[:4] == b"\x28\xb5\x2f\xfd"
    assert _zstd.decompress(f) == data
    assert _zstd.decompress(_zstd.compress(data, 3, threads=1)) == data
