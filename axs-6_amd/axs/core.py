"""AXS-6 format constants, the AXSBlock byte form and the AXSTensor container.

Same names and values as the reference's ``axs/core.py:32-41`` (the format
is fixed by them), the same ``BlockConfig`` codes and ``AXSBlock`` fields,
properties and byte layout (``axs/core.py:44-152``), and the same
``AXSTensor`` fields and derived properties (``axs/core.py:160-206``), which
is what ``quantize_unified`` returns.  ``AXSBlock`` is the host form of one
block; ``axs.blocks`` writes and reads whole tensors of these records on the
GPU.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from enum import IntEnum

import numpy as np
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


class BlockConfig(IntEnum):
    """The 2-bit mode field of a block header (axs/core.py:44-50).  Every
    encoder writes DENSE; no decoder interprets the other modes."""

    DENSE = 0b00
    SPARSE = 0b01
    HIGH_PREC = 0b10
    RESERVED = 0b11


def _payload_bytes(block_size: int) -> int:
    return (block_size * AXS6_VALUE_BITS + 7) // 8


@dataclass
class AXSBlock:
    """One encoded block: biased shared exponent (scale 2^(e-127)), mode,
    per-value sign (True = negative) and 5-bit magnitude code.

    Byte form (``to_bytes``, axs/core.py:97-119): the 16-bit little-endian
    header ``shared_exponent << 2 | config``, then the values
    ``q_i = sign_i << 5 | magnitude_i`` as one little-endian bit string,
    q_i in bits [6i, 6i + 6), padded with zero bits to whole bytes --
    2 + ceil(6B / 8) bytes, 26 for B = 32.
    """

    shared_exponent: int
    config: BlockConfig
    signs: np.ndarray
    magnitudes: np.ndarray
    block_size: int = DEFAULT_BLOCK_SIZE

    @property
    def scale(self) -> float:
        return math.ldexp(1.0, self.shared_exponent - AXS6_EXPONENT_BIAS)

    @property
    def total_bits(self) -> int:
        return AXS6_HEADER_BITS + self.block_size * AXS6_VALUE_BITS

    @property
    def bits_per_value(self) -> float:
        return self.total_bits / self.block_size

    def to_bytes(self) -> bytes:
        header = (int(self.shared_exponent) << 2) | int(self.config)
        word = 0
        for i in range(self.block_size):
            word |= ((int(bool(self.signs[i])) << 5) | int(self.magnitudes[i])) << (AXS6_VALUE_BITS * i)
        n = _payload_bytes(self.block_size)
        word &= (1 << (8 * n)) - 1
        return header.to_bytes(2, byteorder="little") + word.to_bytes(n, byteorder="little")

    @classmethod
    def from_bytes(cls, data: bytes, block_size: int = DEFAULT_BLOCK_SIZE) -> "AXSBlock":
        """Inverse of ``to_bytes`` (axs/core.py:121-152); bytes past the
        block's record are ignored, a short record raises IndexError."""
        n = _payload_bytes(block_size)
        if len(data) < 2 + n:
            raise IndexError(f"AXSBlock.from_bytes: a block of {block_size} values needs {2 + n} bytes, "
                             f"got {len(data)}")
        header = int.from_bytes(bytes(data[:2]), byteorder="little")
        word = int.from_bytes(bytes(data[2:2 + n]), byteorder="little")
        q = np.array([(word >> (AXS6_VALUE_BITS * i)) & 0x3F for i in range(block_size)], dtype=np.uint8)
        return cls(shared_exponent=header >> 2, config=BlockConfig(header & 0x03),
                   signs=(q >> 5).astype(bool), magnitudes=q & 0x1F, block_size=block_size)


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
