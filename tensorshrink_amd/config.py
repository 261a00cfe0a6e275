"""TensorShrinkConfig: the quantization_config surface of hf_integration.py:77-195.

Same fields, defaults, validation and dict/JSON round trip. Constructing one
registers the quantizer plugin (tensorshrink_amd.hf_integration) with
transformers, so it can be passed to `from_pretrained(quantization_config=...)`.
"""
from __future__ import annotations

import json
from enum import Enum
from typing import Any, Dict, Optional, Tuple

from .codec import DEFAULT_DQ_GROUP_SIZE
from .modules import DEFAULT_MAX_DEQUANT_ROWS, DEFAULT_MIN_NUMEL, DEFAULT_SKIP_PATTERNS


class TensorShrinkQuantizationMethod(str, Enum):
    TENSORSHRINK = "tensorshrink"


class TensorShrinkConfig:
    def __init__(self, bits: int = 4, group_size: int = 128, outlier_frac: float = 0.001, adaptive: bool = False,
                 error_threshold: float = 0.10, min_numel: Optional[int] = None,
                 skip_name_patterns: Optional[Tuple[str, ...]] = None, force_fp32_patterns: Tuple[str, ...] = (),
                 max_dequant_rows=None, cache_budget_mb: float = 0.0, host_cache_budget_mb: float = 0.0,
                 fast_dequant: bool = True, use_triton: bool = True, vram_budget_mb: Optional[float] = None,
                 quantize_workers: Optional[int] = 4, verbose: bool = True, companded: bool = False,
                 double_quant: bool = True, dq_group_size: Optional[int] = None, nf_quant: bool = True, **kwargs):
        from .hf_integration import _install
        _install()  # registers the quantizer with transformers, once
        self.quant_method = TensorShrinkQuantizationMethod.TENSORSHRINK
        self.bits = bits
        self.group_size = group_size
        self.outlier_frac = outlier_frac
        self.adaptive = adaptive
        self.error_threshold = error_threshold
        self.min_numel = DEFAULT_MIN_NUMEL if min_numel is None else min_numel
        self.skip_name_patterns = DEFAULT_SKIP_PATTERNS if skip_name_patterns is None else tuple(skip_name_patterns)
        self.force_fp32_patterns = tuple(p.lower() for p in force_fp32_patterns)
        self.max_dequant_rows = DEFAULT_MAX_DEQUANT_ROWS if max_dequant_rows is None else max_dequant_rows
        self.cache_budget_mb = cache_budget_mb
        self.host_cache_budget_mb = host_cache_budget_mb
        self.fast_dequant = fast_dequant
        self.use_triton = use_triton
        self.vram_budget_mb = vram_budget_mb
        self.quantize_workers = quantize_workers
        self.verbose = verbose
        self.companded = companded
        self.double_quant = double_quant
        self.dq_group_size = DEFAULT_DQ_GROUP_SIZE if dq_group_size is None else dq_group_size
        self.nf_quant = nf_quant
        self.modules_to_not_convert = kwargs.pop("modules_to_not_convert", None)
        self.post_init()

    def post_init(self):
        if self.bits not in (4, 8):
            raise ValueError(f"TensorShrinkConfig.bits must be 4 or 8, got {self.bits}")
        if self.group_size <= 0:
            raise ValueError(f"TensorShrinkConfig.group_size must be positive, got {self.group_size}")
        if self.vram_budget_mb is not None:
            raise NotImplementedError("TensorShrinkConfig.vram_budget_mb isn't supported through from_pretrained")

    def to_dict(self) -> Dict[str, Any]:
        d = dict(self.__dict__)
        d["quant_method"] = self.quant_method.value
        return d

    def to_diff_dict(self) -> Dict[str, Any]:
        return self.to_dict()

    def to_json_string(self, use_diff: bool = True) -> str:
        return json.dumps(self.to_dict(), indent=2, sort_keys=True) + "\n"

    def __iter__(self):
        yield from self.to_dict().items()

    def __repr__(self) -> str:
        return f"TensorShrinkConfig {self.to_json_string()}"

    def update(self, **kwargs) -> Dict[str, Any]:
        unused = {}
        for k, v in kwargs.items():
            if hasattr(self, k):
                setattr(self, k, v)
            else:
                unused[k] = v
        return unused

    @classmethod
    def from_dict(cls, config_dict: Dict[str, Any], return_unused_kwargs: bool = False, **kwargs):
        d = dict(config_dict)
        d.pop("quant_method", None)
        cfg = cls(**d)
        unused = cfg.update(**kwargs)
        return (cfg, unused) if return_unused_kwargs else cfg

    def quantize_kwargs(self) -> Dict[str, Any]:
        """The quantize_module arguments this config stands for."""
        return dict(bits=self.bits, group_size=self.group_size, outlier_frac=self.outlier_frac,
                    adaptive=self.adaptive, error_threshold=self.error_threshold, min_numel=self.min_numel,
                    skip_name_patterns=self.skip_name_patterns, max_dequant_rows=self.max_dequant_rows,
                    force_fp32_patterns=self.force_fp32_patterns, quantize_workers=self.quantize_workers,
                    verbose=self.verbose, companded=self.companded, double_quant=self.double_quant,
                    dq_group_size=self.dq_group_size, nf_quant=self.nf_quant)
