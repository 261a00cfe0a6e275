"""from_pretrained(quantization_config=TensorShrinkConfig(...)) on a tiny
Qwen2 checkpoint written here (random init, fp16, q/k/v with biases).

CPU: the loader plumbing, with the quantize step replaced by a stand-in that
keeps the weight it was handed: which layers are targeted (quantize_module's
eligibility: size and skip patterns), that every target receives exactly its
checkpoint weight and bias (biases arrive before weights in transformers 5's
sorted key order), that the rest loads untouched, and that a target left
unquantized fails loudly.
GPU: the real plugin; every replaced layer equals quantize_module's layer on
the dense model with the same settings, buffer for buffer, and so does the
model's output."""
import pytest
import torch
import torch.nn as nn

transformers = pytest.importorskip("transformers")


def _checkpoint(tmp_path, seed=0):
    from transformers import Qwen2Config, Qwen2ForCausalLM
    cfg = Qwen2Config(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=2, vocab_size=128)
    torch.manual_seed(seed)
    m = Qwen2ForCausalLM(cfg).to(torch.float16)
    with torch.no_grad():
        for n, p in m.named_parameters():
            if n.endswith("bias"):
                p.normal_(0, 0.05)
    d = tmp_path / "ckpt"
    m.save_pretrained(str(d))
    return m, d


TARGETS = {f"model.layers.{i}.{s}" for i in range(2) for s in
           ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
            "mlp.up_proj", "mlp.down_proj")}


class _Stand(nn.Module):
    def __init__(self, w, b):
        super().__init__()
        self.register_buffer("w", w.clone())
        self.bias = None if b is None else b.clone()
        self.packed = w
        self.bits = 4

    def dense_equiv_nbytes(self, itemsize=2):
        return self.w.numel() * itemsize

    def packed_nbytes(self):
        return self.w.numel() // 4


@pytest.fixture
def stand_in(monkeypatch):
    import tensorshrink_amd as ts
    from tensorshrink_amd import hf_integration as H
    from tensorshrink_amd import modules as M
    ts.TensorShrinkConfig()  # registers the plugin
    import transformers.quantizers.auto as A
    monkeypatch.setattr(H, "_quantize_linear", lambda cfg, w, b, name: (_Stand(w, b), None, False))
    monkeypatch.setattr(M, "QuantLinear", _Stand)
    monkeypatch.setattr(A.AUTO_QUANTIZER_MAPPING["tensorshrink"], "validate_environment", lambda *a, **k: None)
    return ts


def test_loader_plumbing(tmp_path, stand_in):
    from transformers import AutoModelForCausalLM
    ts = stand_in
    dense, d = _checkpoint(tmp_path)
    q = AutoModelForCausalLM.from_pretrained(str(d), quantization_config=ts.TensorShrinkConfig(verbose=False))
    got = {n for n, m in q.named_modules() if isinstance(m, _Stand)}
    assert got == TARGETS
    for n in TARGETS:
        s, ref = q.get_submodule(n), dense.get_submodule(n)
        assert torch.equal(s.w, ref.weight), n
        assert (s.bias is None) == (ref.bias is None), n
        if ref.bias is not None:
            assert torch.equal(s.bias, ref.bias), n
    for n in ("model.embed_tokens.weight", "lm_head.weight", "model.layers.0.input_layernorm.weight",
              "model.norm.weight"):
        assert torch.equal(q.state_dict()[n], dense.state_dict()[n]), n
    assert q.is_tensorshrink_quantized and q.config.quantization_config.bits == 4


def test_loader_skip_patterns(tmp_path, stand_in):
    from transformers import AutoModelForCausalLM
    ts = stand_in
    _, d = _checkpoint(tmp_path)
    cfg = ts.TensorShrinkConfig(verbose=False, modules_to_not_convert=["mlp"], min_numel=40000)
    q = AutoModelForCausalLM.from_pretrained(str(d), quantization_config=cfg)
    got = {n for n, m in q.named_modules() if isinstance(m, _Stand)}
    # mlp excluded by name; k/v (128 x 256 = 32768 < 40000) by size
    assert got == {n for n in TARGETS if "mlp" not in n and "k_proj" not in n and "v_proj" not in n}


def test_loader_fails_loudly(tmp_path, stand_in, monkeypatch):
    from transformers import AutoModelForCausalLM
    from tensorshrink_amd import hf_integration as H
    ts = stand_in

    def boom(cfg, w, b, name):
        raise RuntimeError("quantize failed")
    monkeypatch.setattr(H, "_quantize_linear", boom)
    _, d = _checkpoint(tmp_path)
    with pytest.raises(RuntimeError, match="conversion|not quantized"):
        AutoModelForCausalLM.from_pretrained(str(d), quantization_config=ts.TensorShrinkConfig(verbose=False))


def test_config_registration():
    import tensorshrink_amd as ts
    import transformers.quantizers.auto as A
    c = ts.TensorShrinkConfig(bits=8, adaptive=True)
    assert A.AUTO_QUANTIZATION_CONFIG_MAPPING["tensorshrink"] is ts.TensorShrinkConfig
    assert A.AUTO_QUANTIZER_MAPPING["tensorshrink"].__name__ == "TensorShrinkHfQuantizer"
    qz = A.AutoHfQuantizer.from_config(c, pre_quantized=False)
    assert qz.is_serializable() is False and qz.is_trainable is False
    assert qz.update_dtype(None) == torch.float16 and qz.update_dtype(torch.bfloat16) == torch.bfloat16
    c2 = A.AutoQuantizationConfig.from_dict(c.to_dict())
    assert isinstance(c2, ts.TensorShrinkConfig) and c2.bits == 8 and c2.adaptive


@pytest.mark.gpu
@pytest.mark.parametrize("kw", [dict(), dict(bits=8, double_quant=False, nf_quant=False),
                                dict(adaptive=True, error_threshold=0.09), dict(force_fp32_patterns=("down",))])
def test_from_pretrained_matches_quantize_module(tmp_path, kw):
    from transformers import AutoModelForCausalLM
    import tensorshrink_amd as ts
    dense, d = _checkpoint(tmp_path)
    q = AutoModelForCausalLM.from_pretrained(str(d), quantization_config=ts.TensorShrinkConfig(verbose=False, **kw),
                                             device_map="cuda")
    ref = AutoModelForCausalLM.from_pretrained(str(d), dtype=torch.float16)
    mkw = {k: v for k, v in kw.items()}
    ts.quantize_module(ref, verbose=False, **mkw)
    ref = ref.cuda()
    qs = {n: m for n, m in q.named_modules() if isinstance(m, ts.QuantLinear)}
    rs = {n: m for n, m in ref.named_modules() if isinstance(m, ts.QuantLinear)}
    assert set(qs) == set(rs) == TARGETS
    for n in TARGETS:
        a, b = qs[n].state_dict(), rs[n].state_dict()
        assert sorted(a) == sorted(b), n
        for k in a:
            assert torch.equal(a[k], b[k]), (n, k)
        assert qs[n].force_fp32_compute == rs[n].force_fp32_compute == ("down" in n and "force_fp32_patterns" in kw)
    ids = torch.randint(0, 128, (2, 9), generator=torch.Generator().manual_seed(3)).cuda()
    with torch.no_grad():
        assert torch.equal(q(ids).logits, ref(ids).logits)
