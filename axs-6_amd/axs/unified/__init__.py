"""AXS-6 unified NF5 API on MI355X (gfx950) HIP kernels.

The names of the reference's ``axs.unified`` (``axs/unified/__init__.py:80-127``)
for the NF5 hot path: quantizer core, autograd ops, drop-in modules, backend
selection and the bf16 mixed-precision linear.  ``AXS6Linear`` aliases
``AXSLinearUnified``.  The reference's Triton entry points keep their names
(``has_triton``, ``triton_fused_fake_quantize``, ``triton_fused_linear``) as
aliases of the HIP ones so existing call sites keep working; they run the
HIP kernels, not Triton.  The training pipeline (``AXSTrainingPipelineUnified``,
``AmaxEMA``) runs its gradient unscale, overflow check and clipping as one
fused device pass.  The distributed gradient hooks are not part of this
package (the NF5 gradient codec is, in ``axs.unified.distributed``).
"""
from axs.unified.backend import (
    BackendType,
    accelerated_fake_quantize,
    accelerated_linear,
    accelerated_matmul,
    backend_info,
    clear_int8_weight_cache,
    detect_best_backend,
    get_backend,
    set_backend,
)
from axs.unified.functional_unified import (
    axs_linear_group_unified,
    axs_linear_unified,
    axs_matmul_unified,
    fake_quantize_unified,
)
from axs.unified.hip_kernels import has_hip, hip_fused_fake_quantize, hip_fused_linear
from axs.unified.mixed_precision import (
    AXSLinearMixedPrecision,
    axs_linear_mixed_precision,
    convert_to_axs_mixed_precision,
    estimate_memory_savings,
)
from axs.unified.modules_unified import (
    AXS6Linear,
    AXSEmbeddingUnified,
    AXSLayerNormUnified,
    AXSLinearUnified,
    AXSMultiheadAttentionUnified,
    convert_to_axs_unified,
)
from axs.unified.training_unified import AmaxEMA, AXSTrainingPipelineUnified
from axs.unified.quantize_unified import (
    FUSED_NF5_LUT,
    NF5_CODEBOOK,
    REVERSE_NF5_LUT,
    dequantize_unified,
    fused_fake_quantize,
    quantization_error_unified,
    quantize_unified,
    quantize_unified_with_fq,
)

# Reference entry-point names (axs/unified/triton_kernels.py:57,295,385), served by HIP.
has_triton = has_hip
triton_fused_fake_quantize = hip_fused_fake_quantize
triton_fused_linear = hip_fused_linear

__all__ = [
    "fused_fake_quantize",
    "quantize_unified",
    "quantize_unified_with_fq",
    "dequantize_unified",
    "quantization_error_unified",
    "FUSED_NF5_LUT",
    "NF5_CODEBOOK",
    "REVERSE_NF5_LUT",
    "fake_quantize_unified",
    "axs_linear_unified",
    "axs_linear_group_unified",
    "axs_matmul_unified",
    "AXSLinearUnified",
    "AXS6Linear",
    "AXSLayerNormUnified",
    "AXSEmbeddingUnified",
    "AXSMultiheadAttentionUnified",
    "convert_to_axs_unified",
    "BackendType",
    "accelerated_fake_quantize",
    "accelerated_linear",
    "accelerated_matmul",
    "backend_info",
    "clear_int8_weight_cache",
    "detect_best_backend",
    "get_backend",
    "set_backend",
    "has_hip",
    "hip_fused_fake_quantize",
    "hip_fused_linear",
    "has_triton",
    "triton_fused_fake_quantize",
    "triton_fused_linear",
    "AXSLinearMixedPrecision",
    "axs_linear_mixed_precision",
    "convert_to_axs_mixed_precision",
    "estimate_memory_savings",
    "AXSTrainingPipelineUnified",
    "AmaxEMA",
]
