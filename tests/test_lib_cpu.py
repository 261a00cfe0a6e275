"""The C-ABI library without a GPU: it loads, exports every declared symbol,
and its host-side functions (exact top-k replay, Lloyd-Max fit) agree with the
oracle. CPU only."""
import os
import re

import numpy as np
import pytest
import torch

import recipes
from oracle import codec_ref as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _lib():
    from tensorshrink_amd import _lib as L
    if not os.path.exists(L.LIB_PATH):
        pytest.skip("libtensorshrink_hip.so not built")
    return L, L.load()


def test_exports_every_declared_symbol():
    L, lib = _lib()
    header = open(os.path.join(ROOT, "include", "tensorshrink_hip.h")).read()
    names = set(re.findall(r"^\s*(?:const\s+char\s*\*|int|size_t)\s+(ts_\w+)\s*\(", header, re.M))
    assert len(names) >= 20
    for n in sorted(names):
        assert hasattr(lib, n), n
        assert n in L.PROTOTYPES, f"{n} has no ctypes prototype"


def test_status_strings():
    L, lib = _lib()
    assert lib.ts_status_str(L.TS_OK) == b"ok"
    assert b"covered" in lib.ts_status_str(L.TS_NOT_COVERED)
    assert b"gfx950" in lib.ts_version()


def _select(lib, cidx, cval, n, k):
    oi = np.empty(k, np.int64)
    ov = np.empty(k, np.float32)
    cidx = np.ascontiguousarray(cidx, np.int64)
    cval = np.ascontiguousarray(cval, np.float32)
    rc = lib.ts_topk_select(cidx.ctypes.data, cval.ctypes.data, len(cidx), n, k, oi.ctypes.data, ov.ctypes.data)
    return rc, oi, ov


def _prefix_filter(a, k):
    """The GPU candidate rule restated on the CPU: [0, k) plus, in segment
    [k 2^(s-1), k 2^s), values above a lower bound of the k-th largest of the
    preceding prefix (here: that exact value, the tightest valid bound), and NaN."""
    n = a.shape[0]
    keep = np.zeros(n, bool)
    keep[:k] = True
    start = k
    while start < n:
        end = min(2 * start, n)
        kth = np.partition(a[:start], start - k)[start - k]
        keep[start:end] = (a[start:end] > kth) | np.isnan(a[start:end])
        start = end
    return keep


# The replay keys the heap by the values' f16 bits when every value is a
# non-negative f16 ("gauss", "ties", "f16sub"), by bf16 bits when every value
# is a bf16 ("bf16"), by float bits for other non-negative streams ("f32",
# "f32ties"), and runs the packed float heap for signed ones ("signed") and
# the std:: calls with NaN ("nan").
@pytest.mark.parametrize("n,k,kind", [(200000, 200, "gauss"), (120000, 1500, "ties"), (65536, 1024, "ties"),
                                      (5000, 600, "ties"), (5000, 4999, "gauss"), (100000, 300, "nan"),
                                      (120000, 1500, "bf16"), (200000, 200, "f32"), (120000, 1500, "f32ties"),
                                      (120000, 1500, "f16sub"), (120000, 1500, "signed")])
def test_topk_select_replay(n, k, kind):
    L, lib = _lib()
    g = torch.Generator().manual_seed(n ^ k)
    if kind == "ties":
        a = (torch.randint(-30, 31, (n,), generator=g).float() / 30).to(torch.float16).float().abs().numpy()
    elif kind == "bf16":  # beyond f16's range
        a = (torch.randn(n, generator=g) * 1e6).to(torch.bfloat16).float().abs().numpy()
    elif kind == "f32":
        a = torch.randn(n, generator=g).abs().numpy()
    elif kind == "f32ties":
        a = (torch.randint(-30, 31, (n,), generator=g).float() * 1.1 / 30).abs().numpy()
        assert (a.view(np.uint32) & 0xFFFF).any()
    elif kind == "f16sub":  # f16 subnormals, many ties
        a = (torch.randn(n, generator=g) * 3e-7).to(torch.float16).float().abs().numpy()
    elif kind == "signed":
        a = torch.randn(n, generator=g).to(torch.float16).float().numpy()
    else:
        a = torch.randn(n, generator=g).to(torch.float16).float().abs().numpy()
    if kind == "nan":  # NaN ranks above every number (the std:: path)
        a[[7, 5000, 77777]] = np.nan
    tv, ti = torch.topk(torch.from_numpy(a), k)
    if kind == "signed":  # topk of the values themselves: torch.topk is the reference
        ov_ref, oi_ref = tv.numpy(), ti.numpy()
    else:
        ov_ref, oi_ref = O.topk_abs(a, k)
        np.testing.assert_array_equal(oi_ref, ti.numpy())
    rc, oi, ov = _select(lib, np.arange(n), a, n, k)
    assert rc == 0
    np.testing.assert_array_equal(oi, oi_ref)
    np.testing.assert_array_equal(ov, ov_ref)
    if k * 64 <= n:
        keep = _prefix_filter(a, k)
        assert keep.sum() < n
        rc, oi2, ov2 = _select(lib, np.nonzero(keep)[0], a[keep], n, k)
        assert rc == 0
        np.testing.assert_array_equal(oi2, oi_ref)
    else:
        # the nth_element regime needs the whole array
        rc, _, _ = _select(lib, np.arange(n - 1), a[:-1], n, k)
        assert rc == L.TS_BAD_ARG


@pytest.mark.parametrize("kind", ["ties", "gauss", "bf16", "f32"])
def test_clamp_threshold_from_candidates(kind):
    """quantize_tensor takes the clamp threshold min(top-k |w|) as the k-th
    largest candidate (np.partition) while the replay runs: every element above
    the k-th largest |w| is a candidate, so the two agree on filtered streams."""
    L, lib = _lib()
    n, k = 120000, 1500
    g = torch.Generator().manual_seed(7 + len(kind))
    if kind == "ties":
        a = (torch.randint(-30, 31, (n,), generator=g).float() / 30).to(torch.float16).float().abs().numpy()
    elif kind == "bf16":
        a = (torch.randn(n, generator=g) * 1e6).to(torch.bfloat16).float().abs().numpy()
    elif kind == "f32":
        a = torch.randn(n, generator=g).abs().numpy()
    else:
        a = torch.randn(n, generator=g).to(torch.float16).float().abs().numpy()
    keep = _prefix_filter(a, k)
    ci, cv = np.nonzero(keep)[0], a[keep]
    rc, oi, ov = _select(lib, ci, cv, n, k)
    assert rc == 0
    assert float(np.partition(cv, cv.shape[0] - k)[cv.shape[0] - k]) == float(ov.min())
    assert float(ov.min()) == float(np.sort(a)[n - k])


def test_topk_select_rejects_bad_stream():
    L, lib = _lib()
    a = np.random.default_rng(1).random(10000).astype(np.float32)
    rc, _, _ = _select(lib, np.arange(1, 10000), a[1:], 10000, 10)
    assert rc == L.TS_BAD_ARG


@pytest.mark.parametrize("levels,m", [(4, 30000), (16, 50000), (4, 7)])
def test_lloyd_max_host_matches_oracle(levels, m):
    L, lib = _lib()
    rng = np.random.default_rng(levels + m)
    x = (rng.standard_t(5, m) * 0.5 + 1.5).astype(np.float32)
    nl = max(1, min(levels, m))
    init = torch.linspace(float(x.min()), float(x.max()), nl).numpy()
    out = np.empty(nl, np.float32)
    assert lib.ts_lloyd_max_fit_host(x.ctypes.data, m, init.ctypes.data, nl, 12, out.ctypes.data) == 0
    ref = O.lloyd_max_fit(x, levels, None)
    np.testing.assert_array_equal(out.view(np.uint32), ref.view(np.uint32))


def test_no_gpu_fails_loudly():
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    import tensorshrink_amd as ts
    with pytest.raises(RuntimeError, match="GPU"):
        ts.quantize_tensor(recipes.gaussian_weight(8, 128, 0))


def test_forward_workspace_bytes():
    """Host-only sizing of the large-M forward workspace: 0 at decode sizes,
    else the dequantized layer (rows x cols x 2) plus the GEMM library's
    32 MiB; 0 for an invalid layer view. No GPU call."""
    import ctypes
    L, lib = _lib()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced by the sizing call
    q = L.QLayer()
    q.bits, q.group_size, q.rows, q.cols = 4, 128, 14336, 4096
    q.padded_cols, q.n_groups = 4096, 32
    q.packed = q.scale = q.gmin = fake
    q.packed_stride = 2048
    for M in (1, 16):
        assert lib.ts_forward_workspace_bytes(ctypes.byref(q), M) == 0
    need = lib.ts_forward_workspace_bytes(ctypes.byref(q), 17)
    assert need == 14336 * 4096 * 2 + (32 << 20)
    assert lib.ts_forward_workspace_bytes(ctypes.byref(q), 2048) == need
    q.n_groups = 31  # inconsistent view
    assert lib.ts_forward_workspace_bytes(ctypes.byref(q), 2048) == 0


def test_forward_partials_bytes():
    """Host-only sizing of the fused prefill kernel's K-split workspace,
    k_split x M x rows x 4 bytes: 0 at decode sizes, where unsplit tiles fill
    the CUs and where K is too short to split; the split counts the launch
    plan picks for few tiles and for 256 x 256 tiles that two splits let fill
    the CUs; always below the GEMM path's workspace. No GPU call."""
    import ctypes
    L, lib = _lib()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced by the sizing call

    def layer(rows, cols, bits=4, codebook=False):
        q = L.QLayer()
        q.bits, q.group_size, q.rows, q.cols = bits, 128, rows, cols
        q.padded_cols, q.n_groups = cols, cols // 128
        q.packed = q.scale = q.gmin = fake
        if codebook:
            q.codebook = fake
        q.packed_stride = cols * bits // 8
        return q

    def splits(rows, cols, M, **kw):
        n = lib.ts_forward_partials_bytes(ctypes.byref(layer(rows, cols, **kw)), M)
        assert n % (4 * M * rows) == 0
        k = n // (4 * M * rows)
        if n:
            assert 2 <= k <= 8
            assert n < lib.ts_forward_workspace_bytes(ctypes.byref(layer(rows, cols, **kw)), M)
        return k

    # down projection at M = 256: 32 tiles of 256 x 128
    assert splits(4096, 14336, 256) == 8
    assert splits(4096, 14336, 256, bits=8, codebook=True) == 8
    # ... and at M = 2048 (config 4): 128 tiles of 256 x 256, two splits
    assert splits(4096, 14336, 2048, bits=8, codebook=True) == 2
    # k / v at M = 2048: 64 tiles of 256 x 128
    assert splits(1024, 4096, 2048) == 4
    # 512 x 8192 at M = 160: 8 tiles, 128 k-steps
    assert splits(512, 8192, 160) == 8
    # tiles filling the CUs: 14336 x 4096 at M = 2048 (448 tiles of 256 x 256)
    assert splits(14336, 4096, 2048) == 0
    # decode sizes: up to 16 rows, and up to 32 (24 for K > 8192) on layers
    # of at most 256 row tiles with codes of at most 6 bits
    for M in (1, 16, 17, 32):
        assert splits(4096, 4096, M) == 0
    assert splits(4096, 14336, 24) == 0
    assert splits(4096, 14336, 25) > 0
    assert splits(4096, 4096, 33) > 0
    # 8-bit layers and taller layers take the prefill kernel from 17 rows
    assert splits(4096, 4096, 17, bits=8, codebook=True) > 0
    assert splits(8192, 4096, 17) > 0
    # too few k-steps to split (256 columns = 4 k-steps)
    assert splits(4096, 256, 300) == 0
