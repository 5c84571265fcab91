"""AXS-6 unified NF5 API on the MI355X HIP kernels (interim export list)."""
from axs.unified.backend import (  # noqa: F401
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
from axs.unified.hip_kernels import has_hip, hip_fused_fake_quantize  # noqa: F401
from axs.unified.quantize_unified import (  # noqa: F401
    FUSED_NF5_LUT,
    NF5_CODEBOOK,
    REVERSE_NF5_LUT,
    dequantize_unified,
    fused_fake_quantize,
    quantization_error_unified,
    quantize_unified,
    quantize_unified_with_fq,
)
