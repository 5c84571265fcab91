"""AXS-6 format constants and the AXSTensor container.

Same names and values as the reference's ``axs/core.py:32-41`` (the format
is fixed by them) and the same ``AXSTensor`` fields and derived properties
(``axs/core.py:160-206``), which is what ``quantize_unified`` returns.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

AXS6_MANTISSA_BITS: int = 5
AXS6_SIGN_BITS: int = 1
AXS6_VALUE_BITS: int = AXS6_SIGN_BITS + AXS6_MANTISSA_BITS  # 6
AXS6_EXPONENT_BITS: int = 8
AXS6_CONFIG_BITS: int = 2
AXS6_HEADER_BITS: int = AXS6_EXPONENT_BITS + AXS6_CONFIG_BITS  # 10
AXS6_MAX_MAGNITUDE: int = (1 << AXS6_MANTISSA_BITS) - 1  # 31
AXS6_EXPONENT_BIAS: int = 127
DEFAULT_BLOCK_SIZE: int = 32
VALID_BLOCK_SIZES: tuple[int, ...] = (8, 16, 32)


@dataclass
class AXSTensor:
    """A tensor in AXS-6 NF5 form: per-block shared exponents plus per-value
    sign and 5-bit magnitude code.

    shared_exponents: uint8 ``(*batch, num_blocks)``
    signs:            bool  ``(*batch, num_blocks, block_size)``
    magnitudes:       uint8 ``(*batch, num_blocks, block_size)``
    """

    shared_exponents: torch.Tensor
    signs: torch.Tensor
    magnitudes: torch.Tensor
    block_size: int
    original_shape: torch.Size
    num_blocks: int

    @property
    def effective_bits_per_value(self) -> float:
        return AXS6_VALUE_BITS + AXS6_HEADER_BITS / self.block_size

    @property
    def compression_ratio_vs_fp32(self) -> float:
        return 32.0 / self.effective_bits_per_value

    @property
    def compression_ratio_vs_fp8(self) -> float:
        return 8.0 / self.effective_bits_per_value

    @property
    def memory_bytes(self) -> int:
        numel = 1
        for s in self.original_shape:
            numel *= s
        bits = numel * AXS6_VALUE_BITS + (numel // self.block_size) * AXS6_HEADER_BITS
        return math.ceil(bits / 8)
