"""NF5 quantiser: tables, fused fake-quantize, quantize / dequantize.

Same public names, signatures and results as the reference's
``axs/unified/quantize_unified.py`` (``NF5_CODEBOOK`` :61, ``FUSED_NF5_LUT``
:96, ``_LUT_MAX_IDX`` :97, ``REVERSE_NF5_LUT`` :114, ``fused_fake_quantize``
:121, ``quantize_unified`` :211, ``dequantize_unified`` :285,
``quantization_error_unified`` :315), computed by the gfx950 kernels of
libaxs6.so.  The tables below are the library's own (the values the kernels
use), so host and device can never disagree.

All compute functions take device tensors; a CPU tensor raises
``RuntimeError`` (there is no host fallback).
"""
from __future__ import annotations

import math
from typing import Literal

import torch

from axs import _lib
from axs.core import DEFAULT_BLOCK_SIZE, VALID_BLOCK_SIZES, AXSTensor
from axs.unified import hip_kernels as _hk

NF5_CODEBOOK, FUSED_NF5_LUT, REVERSE_NF5_LUT, LOG2_BAND = _lib.host_tables()
_LUT_MAX_IDX: int = FUSED_NF5_LUT.shape[0] - 1  # 1023


def fused_fake_quantize(
    tensor: torch.Tensor,
    block_size: int = DEFAULT_BLOCK_SIZE,
    rounding: Literal["nearest", "stochastic"] = "nearest",
) -> torch.Tensor:
    """NF5 fake-quantize (quantize and immediately dequantize) per block of
    ``block_size`` values along the last dim.

    Per block: power-of-two scale ``2**(floor(log2(amax)) + 1)`` (1 for an
    all-zero block), normalise, gather from the 1024-entry fused LUT at
    ``trunc(n * 1023)`` (dithered by +-0.5 LUT steps for ``"stochastic"``),
    denormalise and restore the sign.  Output has the input's shape and
    dtype; arithmetic is float32.
    """
    return _hk.hip_fused_fake_quantize(tensor, block_size, rounding)


def quantize_unified(
    tensor: torch.Tensor,
    block_size: int = DEFAULT_BLOCK_SIZE,
    rounding: Literal["nearest", "stochastic"] = "nearest",
) -> AXSTensor:
    """Quantize to the AXS-6 NF5 fields (8-bit shared exponents, signs,
    5-bit magnitude codes)."""
    assert block_size in VALID_BLOCK_SIZES
    exps, codes, signs, _ = _hk.hip_quantize(tensor, block_size, rounding)
    return AXSTensor(
        shared_exponents=exps,
        signs=signs,
        magnitudes=codes,
        block_size=block_size,
        original_shape=tensor.shape,
        num_blocks=exps.shape[1],
    )


def quantize_unified_with_fq(
    tensor: torch.Tensor,
    block_size: int = DEFAULT_BLOCK_SIZE,
    rounding: Literal["nearest", "stochastic"] = "nearest",
    *,
    seed: int | None = None,
) -> tuple[AXSTensor, torch.Tensor]:
    """One pass producing both ``quantize_unified(tensor)`` and
    ``fused_fake_quantize(tensor)`` (the latter in the input's dtype)."""
    assert block_size in VALID_BLOCK_SIZES
    exps, codes, signs, fq = _hk.hip_quantize(tensor, block_size, rounding,
                                              with_fake_quantized=True, seed=seed)
    q = AXSTensor(shared_exponents=exps, signs=signs, magnitudes=codes, block_size=block_size,
                  original_shape=tensor.shape, num_blocks=exps.shape[1])
    return q, fq


def dequantize_unified(axs_tensor: AXSTensor) -> torch.Tensor:
    """Reconstruct float32 values ``+-codebook[code] * 2**(e - 127)``."""
    shape = axs_tensor.original_shape
    cols = shape[-1]
    rows = math.prod(shape[:-1])
    y = _hk.hip_dequantize(axs_tensor.shared_exponents, axs_tensor.magnitudes, axs_tensor.signs,
                           rows, cols, axs_tensor.block_size)
    return y.reshape(shape)


def quantization_error_unified(
    original: torch.Tensor,
    block_size: int = DEFAULT_BLOCK_SIZE,
) -> dict[str, float]:
    """MSE / RMSE / max and mean abs error / SNR (dB) of NF5 fake-quantization."""
    reconstructed = fused_fake_quantize(original, block_size=block_size)
    error = (original - reconstructed).float()
    mse = error.pow(2).mean().item()
    signal_power = original.float().pow(2).mean().item()
    return {
        "mse": mse,
        "rmse": math.sqrt(mse),
        "max_abs_error": error.abs().max().item(),
        "mean_abs_error": error.abs().mean().item(),
        "signal_to_noise_db": 10 * math.log10(signal_power / max(mse, 1e-45)),
    }
