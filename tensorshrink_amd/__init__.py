"""tensorshrink_amd: the GOAP quantized-linear path of tensorshrink, native to
MI355X (gfx950): HIP kernels behind a C ABI (libtensorshrink_hip.so), driven
from PyTorch-ROCm host code with the reference's public API."""
from .codec import (
    DEFAULT_DQ_GROUP_SIZE,
    DEFAULT_ERROR_THRESHOLD,
    DEFAULT_GROUP_SIZE,
    DEFAULT_OUTLIER_FRAC,
    LayerBitStats,
    QuantizedTensor,
    budget_allocate_bits,
    dequantize_tensor,
    estimate_resident_nbytes,
    quantize_tensor,
    quantize_tensor_adaptive,
    relative_error,
)
from .config import TensorShrinkConfig
from .container import ContainerReader, ContainerWriter, save_container, stream_quantize_safetensors_dir
from .gpu_quantize import quantize_module_gpu, quantize_tensor_gpu, quantize_tensor_gpu_adaptive
from .graphs import CUDAGraphQuantModel
from .kernels import apply_outlier_correction, dequantize_weight, fused_quantized_linear
from .modules import (DEFAULT_SKIP_PATTERNS, T5_EXTRA_SKIP_PATTERNS, QuantLinear, load_quantized_module,
                      quantize_module, save_quant_module)
from .streaming import StreamingQuantModel, stream_offload_module

__version__ = "0.4.0+mi355x"
