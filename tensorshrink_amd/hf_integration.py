"""transformers `from_pretrained(..., quantization_config=TensorShrinkConfig(...))`.

The quantizer plugin of hf_integration.py:198-465: every eligible nn.Linear
weight is quantized as the checkpoint reader hands it over and the layer is
replaced by a QuantLinear on the GPU right then, so the dense model never
exists in memory as a whole. Eligibility is quantize_module's (min_numel plus
skip patterns, extended by `modules_to_not_convert`), evaluated on the
meta-device model before any weight is read; quantize arguments are the
config's (fixed `bits`, or the adaptive 2 -> 4 -> 8 chain with
`error_threshold`), so a model loaded this way equals quantize_module applied
to the dense model with the same settings.

Two generations of transformers' quantizer hooks are served by one class:
- transformers >= 5: `param_needs_quantization` marks a target layer's
  weight and bias, and `get_quantize_ops()` returns the conversion op the
  loader calls with each materialized tensor;
- transformers 4.x (the hooks the reference implements):
  `check_quantized_param` / `create_quantized_param`.

The quantize runs on the GPU codec inline, on the loader's thread (a tensor
takes milliseconds there), instead of the reference's CPU thread pool;
`quantize_workers` is accepted and not needed. As in the reference,
`vram_budget_mb` is refused by TensorShrinkConfig (the budget plan needs all
layers first: stream_quantize_safetensors_dir + load_quantized_module cover
it) and a model loaded this way is not serializable through save_pretrained
(save_quant_module writes the .tsk container instead).
"""
from __future__ import annotations

from typing import Any, Dict, List, Optional

import torch
import torch.nn as nn

_INSTALLED = False


def _quantize_linear(cfg, w: torch.Tensor, bias: Optional[torch.Tensor], module_name: str):
    """One checkpoint weight -> (QuantLinear on the current GPU, rel_error or
    None, escalated); hf_integration.py:270-295 / 371-399."""
    from .codec import quantize_tensor, quantize_tensor_adaptive
    from .modules import QuantLinear
    if cfg.adaptive:
        qt, err, esc = quantize_tensor_adaptive(
            w, group_size=cfg.group_size, outlier_frac=cfg.outlier_frac, error_threshold=cfg.error_threshold,
            allowed_bits=(2, 4, 8), companded=cfg.companded, double_quant=cfg.double_quant,
            dq_group_size=cfg.dq_group_size, nf_quant=cfg.nf_quant)
    else:
        qt = quantize_tensor(w, bits=cfg.bits, group_size=cfg.group_size, outlier_frac=cfg.outlier_frac,
                             companded=cfg.companded, double_quant=cfg.double_quant, dq_group_size=cfg.dq_group_size,
                             nf_quant=cfg.nf_quant)
        err, esc = None, False
    f32 = any(p in module_name.lower() for p in cfg.force_fp32_patterns)
    q = QuantLinear(qt, bias, max_dequant_rows=cfg.max_dequant_rows, force_fp32_compute=f32,
                    fast_dequant=cfg.fast_dequant, use_triton=cfg.use_triton)
    return q, err, esc


class _Loader:
    """The quantizer's state: the target layer names, biases that arrive
    before their weight, and totals for the summary line."""

    def __init__(self, cfg):
        self.cfg = cfg
        self.targets: set = set()  # "<module>.weight" keys to quantize
        self.pending_bias: Dict[str, Optional[torch.Tensor]] = {}
        self.model = None
        self.n_replaced = self.orig_bytes = self.packed_bytes = 0

    def prepare(self, model: nn.Module) -> None:
        from .modules import _iter_target_linears
        cfg = self.cfg
        if cfg.cache_budget_mb > 0 or cfg.host_cache_budget_mb > 0:
            raise NotImplementedError("WeightCache is not part of the tensorshrink_amd path")
        skip = tuple(cfg.skip_name_patterns) + tuple(cfg.modules_to_not_convert or ())
        self.targets = {f"{n}.weight" for n, _ in _iter_target_linears(model, cfg.min_numel, skip)}
        self.model = model
        model.config.quantization_config = cfg

    def needs(self, param_name: str) -> bool:
        if param_name in self.targets:
            return True
        return param_name.endswith(".bias") and param_name[:-len("bias")] + "weight" in self.targets

    def take(self, param_name: str, value: Optional[torch.Tensor]) -> None:
        """A target weight or bias from the checkpoint (hf_integration.py:354-401)."""
        from .modules import QuantLinear, _set_module_by_name
        if param_name.endswith(".bias"):
            name = param_name[:-len(".bias")]
            mod = self.model.get_submodule(name)
            b = None if value is None else value.detach()
            if isinstance(mod, QuantLinear):
                if b is None:
                    mod._buffers.pop("bias", None)
                    mod.bias = None
                elif "bias" in mod._buffers:
                    mod.bias = b.to(mod.packed.device)
                else:
                    mod.__dict__.pop("bias", None)
                    mod.register_buffer("bias", b.to(mod.packed.device))
                    mod._rebuild_cache()
            else:
                self.pending_bias[name] = b
            return
        name = param_name[:-len(".weight")]
        w = value.detach()
        q, err, esc = _quantize_linear(self.cfg, w, self.pending_bias.pop(name, None), name)
        q._is_hf_initialized = True
        _set_module_by_name(self.model, name, q)
        self.n_replaced += 1
        self.orig_bytes += q.dense_equiv_nbytes(itemsize=w.element_size())
        self.packed_bytes += q.packed_nbytes()
        if self.cfg.verbose:
            print(f"  [{q.bits}b{'*' if esc else ''}] {name:60s}" + (f" err={err:.4f}" if err is not None else ""))

    def finish(self, model: nn.Module) -> nn.Module:
        from .modules import QuantLinear
        left = sorted(k for k in self.targets
                      if not isinstance(model.get_submodule(k[:-len(".weight")]), QuantLinear))
        if left:
            raise RuntimeError(f"tensorshrink: {len(left)} target layers were not quantized while loading "
                               f"(first: {left[0]}); see the loader's conversion errors")
        model.is_tensorshrink_quantized = True
        if self.cfg.verbose and self.orig_bytes > 0:
            print(f"  tensorshrink: replaced {self.n_replaced} layers, {self.orig_bytes / 1e6:.1f}MB -> "
                  f"{self.packed_bytes / 1e6:.1f}MB ({self.orig_bytes / max(1, self.packed_bytes):.2f}x)")
        return model


def _install() -> None:
    """Registers TensorShrinkConfig and the quantizer in transformers'
    dispatch tables, once (hf_integration.py:198-214, 461-465)."""
    global _INSTALLED
    if _INSTALLED:
        return
    try:
        import transformers.quantizers.auto as auto_mod
        from transformers.quantizers.base import HfQuantizer
    except Exception as exc:  # pragma: no cover - the image ships transformers
        raise ImportError(f"the transformers integration needs `transformers` and `accelerate`: {exc!r}") from exc
    from .config import TensorShrinkConfig

    v5 = hasattr(HfQuantizer, "param_needs_quantization")

    class TensorShrinkHfQuantizer(HfQuantizer):
        requires_parameters_quantization = True  # transformers 4.x
        requires_calibration = False
        required_packages = None

        def __init__(self, quantization_config, **kwargs):
            super().__init__(quantization_config, **kwargs)
            self._ld = _Loader(quantization_config)

        def validate_environment(self, *args, **kwargs):
            try:
                import accelerate  # noqa: F401
            except ImportError as e:
                raise ImportError("from_pretrained(quantization_config=TensorShrinkConfig(...)) needs `accelerate`") \
                    from e
            if not torch.cuda.is_available():
                raise RuntimeError("TensorShrinkConfig quantizes onto a ROCm GPU: none is available")

        def update_dtype(self, dtype):  # transformers 5
            return torch.float16 if dtype is None else dtype

        def update_torch_dtype(self, torch_dtype):  # transformers 4.x
            return torch.float16 if torch_dtype is None else torch_dtype

        def _process_model_before_weight_loading(self, model, **kwargs):
            self._ld.prepare(model)
            return model

        def _process_model_after_weight_loading(self, model, **kwargs):
            return self._ld.finish(model)

        # -- transformers 5 --------------------------------------------------
        def param_needs_quantization(self, model, param_name: str, **kwargs) -> bool:
            return self._ld.needs(param_name)

        def get_quantize_ops(self):
            from transformers.core_model_loading import ConversionOps
            ld = self._ld

            class _Quantize(ConversionOps):
                def convert(self, input_dict, full_layer_name=None, missing_keys=None, **kwargs):
                    for key, value in input_dict.items():
                        value = value[0] if isinstance(value, (list, tuple)) else value
                        name = full_layer_name if len(input_dict) == 1 and full_layer_name else key
                        ld.take(name, value)
                        if missing_keys is not None:
                            missing_keys.discard(name)
                    return {}

            return _Quantize()

        # -- transformers 4.x (hf_integration.py:341-401) -----------------------
        def check_quantized_param(self, model, param_value, param_name, state_dict, **kwargs) -> bool:
            return self._ld.needs(param_name)

        def create_quantized_param(self, model, param_value, param_name, target_device, state_dict,
                                   unexpected_keys: Optional[List[str]] = None):
            self._ld.take(param_name, param_value)

        if v5:
            def is_serializable(self, *args, **kwargs) -> bool:
                return False
        else:
            @property
            def is_serializable(self) -> bool:
                return False

        @property
        def is_trainable(self) -> bool:
            return False

    auto_mod.AUTO_QUANTIZATION_CONFIG_MAPPING["tensorshrink"] = TensorShrinkConfig
    auto_mod.AUTO_QUANTIZER_MAPPING["tensorshrink"] = TensorShrinkHfQuantizer
    _INSTALLED = True
