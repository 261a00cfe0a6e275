"""Host-side API surface: config, budget allocator, size accounting. CPU only."""
import numpy as np
import pytest

import tensorshrink_amd as ts


def test_config_defaults_and_roundtrip():
    c = ts.TensorShrinkConfig()
    assert (c.bits, c.group_size, c.outlier_frac, c.double_quant, c.nf_quant, c.dq_group_size) == \
        (4, 128, 0.001, True, True, 256)
    d = c.to_dict()
    assert d["quant_method"] == "tensorshrink"
    c2 = ts.TensorShrinkConfig.from_dict(d)
    assert c2.to_dict() == d
    with pytest.raises(ValueError):
        ts.TensorShrinkConfig(bits=2)
    with pytest.raises(NotImplementedError):
        ts.TensorShrinkConfig(vram_budget_mb=100)
    assert c.update(bits=8, nonsense=1) == {"nonsense": 1} and c.bits == 8
    kw = ts.TensorShrinkConfig().quantize_kwargs()
    assert kw["nf_quant"] and kw["double_quant"]


def test_budget_allocate_bits():
    S = ts.LayerBitStats
    stats = [S("a", 100, 200, 0.10, 0.01), S("b", 100, 300, 0.10, 0.05), S("c", 100, 150, 0.05, 0.05)]
    assert ts.budget_allocate_bits(stats, 300) == {"a": 4, "b": 4, "c": 4}
    assert ts.budget_allocate_bits(stats, 400) == {"a": 8, "b": 4, "c": 4}
    assert ts.budget_allocate_bits(stats, 10_000) == {"a": 8, "b": 8, "c": 4}


def test_quantized_tensor_nbytes():
    q = ts.QuantizedTensor(orig_shape=(4, 256), orig_dtype="float16", bits=4, group_size=128, rows=4, cols=256,
                           padded_cols=256, n_groups=2, packed=np.zeros((4, 128), np.uint8),
                           scale=np.zeros((4, 2), np.float16), gmin=np.zeros((4, 2), np.float16),
                           outlier_idx=np.zeros(3, np.int32), outlier_val=np.zeros(3, np.float16))
    assert q.n_outliers() == 3
    assert q.compressed_nbytes() == 512 + 12 + 6 + 16 + 16
    assert ts.estimate_resident_nbytes(q) == 512 + 3 * 10 + 32
    assert q.orig_nbytes() == 4 * 256 * 2


def test_bad_bits_rejected_before_gpu():
    import torch
    with pytest.raises(ValueError):
        ts.quantize_tensor(torch.zeros(4, 4), bits=3)
    with pytest.raises(ValueError):
        ts.quantize_tensor(torch.zeros(4, 4), bits=6, companded=True)
    with pytest.raises(ValueError):
        ts.quantize_tensor_gpu(torch.zeros(4, 4), bits=6)


def test_kernel_api_not_covered_on_cpu():
    import torch
    x = torch.zeros(1, 128, dtype=torch.bfloat16)
    p = torch.zeros(4, 64, dtype=torch.uint8)
    s = torch.zeros(4, 1, dtype=torch.float16)
    assert ts.fused_quantized_linear(x, p, s, s, None, 4, 128, 128, 4, torch.bfloat16) is None
    assert ts.dequantize_weight(p, s, s, 4, 4, 128, 128, 1) is None
    assert ts.apply_outlier_correction(torch.zeros(1, 4), x, torch.zeros(1, dtype=torch.int32),
                                       torch.zeros(1, dtype=torch.int32), torch.zeros(1, dtype=torch.float16)) is None
