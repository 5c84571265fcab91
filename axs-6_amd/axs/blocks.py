"""Whole tensors in the AXSBlock byte form, written and read on the GPU.

The reference serialises one block at a time on the host
(``AXSBlock.to_bytes`` / ``from_bytes``, axs/core.py:97-152; the host form is
``axs.core.AXSBlock``).  Here a tensor's blocks become the concatenation of
those records in one HIP kernel pass each way (libaxs6.so):

* per block (blocks in row-major order over the last dim, a ragged last block
  zero-padded): the 16-bit little-endian header ``e << 2 | config`` with
  config DENSE, then the 6-bit values ``sign << 5 | code``, low bits first,
  ``2 + 3 * block_size / 4`` bytes in all (26 for 32 values);
* the codes are NF5 (quantize_unified's exponent rule and reverse LUT, nearest
  rounding); decoding gives ``+-codebook[code] * 2^(e - 127)``, i.e.
  dequantize_unified, and ignores the config field as the reference's decoder
  does.

``records[i * rec : (i + 1) * rec]`` of the returned buffer equals
``AXSBlock(e_i, DENSE, signs_i, codes_i, block_size).to_bytes()``.
"""
from __future__ import annotations

import torch

from axs import _lib
from axs.core import DEFAULT_BLOCK_SIZE, VALID_BLOCK_SIZES, AXSTensor
from axs.unified.hip_kernels import _on_device, _require_device, as_rows, components

__all__ = ["block_bytes", "record_bytes", "encode_blocks", "decode_blocks", "axs_tensor_to_bytes",
           "axs_tensor_from_bytes"]


def _check_block(block_size: int) -> None:
    assert block_size in VALID_BLOCK_SIZES, f"block_size must be one of {VALID_BLOCK_SIZES}"


def record_bytes(block_size: int = DEFAULT_BLOCK_SIZE) -> int:
    """Bytes of one block's record."""
    _check_block(block_size)
    return 2 + block_size * 3 // 4


def block_bytes(rows: int, cols: int, block_size: int = DEFAULT_BLOCK_SIZE) -> int:
    """Bytes of the records of a (rows, cols) tensor."""
    nblk = (cols + block_size - 1) // block_size
    return rows * nblk * record_bytes(block_size)


def _shape_rows(shape) -> tuple[torch.Size, int, int]:
    shape = torch.Size(shape)
    cols = shape[-1] if len(shape) else 1
    rows = shape.numel() // cols if cols else 0
    return shape, rows, cols


def encode_blocks(tensor: torch.Tensor, block_size: int = DEFAULT_BLOCK_SIZE) -> torch.Tensor:
    """uint8 records of ``tensor`` (quantize + to_bytes in one pass)."""
    _require_device(tensor, "encode_blocks")
    _check_block(block_size)
    x, rows, cols = as_rows(tensor)
    buf = torch.empty((block_bytes(rows, cols, block_size),), dtype=torch.uint8, device=x.device)
    if buf.numel():
        with _on_device(x):
            _lib.call("axs6_nf5_pack_blocks", x.data_ptr(), _lib.DTYPE_CODE[x.dtype], rows, cols, block_size,
                      buf.data_ptr(), _lib.stream_of(x))
    return buf


def decode_blocks(data: torch.Tensor, shape, block_size: int = DEFAULT_BLOCK_SIZE) -> torch.Tensor:
    """float32 tensor of ``shape`` from records (from_bytes + dequantize in
    one pass).  ``data`` must hold exactly the records of ``shape``."""
    _require_device(data, "decode_blocks")
    _check_block(block_size)
    shape, rows, cols = _shape_rows(shape)
    need = block_bytes(rows, cols, block_size)
    if data.numel() * data.element_size() != need:
        raise ValueError(f"data has {data.numel() * data.element_size()} bytes, expected {need} "
                         f"for shape {tuple(shape)}")
    b = data.contiguous().view(torch.uint8).reshape(-1)
    y = torch.empty((rows, cols), dtype=torch.float32, device=b.device)
    if y.numel():
        with _on_device(b):
            _lib.call("axs6_nf5_unpack_blocks", b.data_ptr(), rows, cols, block_size, y.data_ptr(),
                      _lib.stream_of(b))
    return y.reshape(shape)


def axs_tensor_to_bytes(t: AXSTensor) -> torch.Tensor:
    """uint8 records of an AXSTensor's blocks (``AXSBlock.to_bytes`` of each
    block, concatenated)."""
    bs = t.block_size
    _check_block(bs)
    nblk = t.num_blocks
    rows = t.shared_exponents.numel() // nblk if nblk else 0
    e, c, s = components(t.shared_exponents, t.magnitudes, t.signs, rows, nblk, bs, "axs_tensor_to_bytes")
    buf = torch.empty((rows * nblk * record_bytes(bs),), dtype=torch.uint8, device=c.device)
    if buf.numel():
        with _on_device(c):
            _lib.call("axs6_nf5_blocks_from_codes", e.data_ptr(), c.data_ptr(), _lib.ptr(s), rows, nblk, bs,
                      buf.data_ptr(), _lib.stream_of(c))
    return buf


def axs_tensor_from_bytes(data: torch.Tensor, original_shape, block_size: int = DEFAULT_BLOCK_SIZE) -> AXSTensor:
    """AXSTensor of ``original_shape`` from its records (``AXSBlock.from_bytes``
    of each block), laid out as quantize_unified lays it out: exponents
    (rows, nblk), signs and codes (rows, nblk, block_size) over the shape's
    flattened leading dims.  The exponent is the header's 8-bit field
    (bits 2..9)."""
    _require_device(data, "axs_tensor_from_bytes")
    _check_block(block_size)
    shape, rows, cols = _shape_rows(original_shape)
    nblk = (cols + block_size - 1) // block_size
    need = rows * nblk * record_bytes(block_size)
    if data.numel() * data.element_size() != need:
        raise ValueError(f"data has {data.numel() * data.element_size()} bytes, expected {need} "
                         f"for shape {tuple(shape)}")
    b = data.contiguous().view(torch.uint8).reshape(-1)
    dev = b.device
    exps = torch.empty((rows, nblk), dtype=torch.uint8, device=dev)
    codes = torch.empty((rows, nblk, block_size), dtype=torch.uint8, device=dev)
    signs = torch.empty((rows, nblk, block_size), dtype=torch.uint8, device=dev)
    if need:
        with _on_device(b):
            _lib.call("axs6_nf5_blocks_to_codes", b.data_ptr(), rows, nblk, block_size, exps.data_ptr(),
                      codes.data_ptr(), signs.data_ptr(), _lib.stream_of(b))
    return AXSTensor(shared_exponents=exps, signs=signs.view(torch.bool), magnitudes=codes, block_size=block_size,
                     original_shape=shape, num_blocks=nblk)
