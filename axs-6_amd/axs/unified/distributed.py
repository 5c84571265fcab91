"""NF5 gradient wire format on the GPU.

The reference's ``axs.unified.distributed`` (axs/unified/distributed.py)
holds a gradient codec -- AXS-6 components and a 6.25-bit flat buffer -- and
DDP communication hooks built on it.  This module provides the codec with the
reference's function names, signatures and layouts, each a single HIP kernel
pass (libaxs6.so), plus a fused tensor <-> buffer pair.  The communication
hooks (``axs6_gradient_hook``, ``axs6_gradient_hook_packed``,
``AXS6GradCompressor``) move the buffer through collectives over several
GPUs; they are not part of this one-GPU build.

Buffer layout (``_pack_to_flat_buffer``, distributed.py:147-198): per block of
``block_size`` values, one byte of shared exponent then ``block_size * 3 / 4``
bytes of 6-bit codes ``(sign << 5) | nf5_code``, four codes per three bytes,
low bits first; 25 bytes per 32 values.  Returned as int8, like the reference.
"""
from __future__ import annotations

import torch

from axs import _lib
from axs.core import DEFAULT_BLOCK_SIZE, VALID_BLOCK_SIZES
from axs.unified.hip_kernels import _on_device, _require_device, as_rows, components, hip_dequantize, hip_quantize

__all__ = [
    "_pack_gradient",
    "_unpack_gradient",
    "_pack_to_flat_buffer",
    "_unpack_from_flat_buffer",
    "pack_gradient_to_buffer",
    "unpack_buffer_to_gradient",
    "wire_bytes",
]


def wire_bytes(rows: int, cols: int, block_size: int = DEFAULT_BLOCK_SIZE) -> int:
    """Size in bytes of the flat buffer of a (rows, cols) tensor."""
    assert block_size in VALID_BLOCK_SIZES, f"block_size must be one of {VALID_BLOCK_SIZES}"
    nblk = (cols + block_size - 1) // block_size
    return rows * nblk * (1 + block_size * 3 // 4)


def _pack_gradient(tensor: torch.Tensor, block_size: int = DEFAULT_BLOCK_SIZE):
    """(shared_exponents u8 (rows, nblk), signs bool (rows, nblk, bs),
    magnitudes u8 (rows, nblk, bs), original_shape) -- distributed.py:70-115
    (nearest rounding, quantize_unified's exponent rule)."""
    exps, codes, signs, _ = hip_quantize(tensor, block_size, "nearest")
    return exps, signs, codes, tensor.shape


def _unpack_gradient(shared_exponents: torch.Tensor, signs: torch.Tensor, magnitudes: torch.Tensor,
                     original_shape: torch.Size, block_size: int = DEFAULT_BLOCK_SIZE) -> torch.Tensor:
    """float32 tensor of ``original_shape`` -- distributed.py:118-144."""
    rows = magnitudes.shape[0]
    cols = original_shape[-1] if len(original_shape) else 1
    y = hip_dequantize(shared_exponents, magnitudes, signs, rows, cols, block_size)
    return y.reshape(original_shape)


def _pack_to_flat_buffer(shared_exponents: torch.Tensor, signs: torch.Tensor,
                         magnitudes: torch.Tensor) -> torch.Tensor:
    """Flat int8 buffer of the components -- distributed.py:147-198."""
    _require_device(magnitudes, "_pack_to_flat_buffer")
    rows, nblk, block_size = magnitudes.shape
    assert block_size % 4 == 0, f"block_size must be divisible by 4, got {block_size}"
    e, c, s = components(shared_exponents, magnitudes, signs, rows, nblk, block_size, "_pack_to_flat_buffer")
    buf = torch.empty((rows * nblk * (1 + block_size * 3 // 4),), dtype=torch.uint8, device=c.device)
    if buf.numel():
        with _on_device(c):
            _lib.call("axs6_nf5_wire_from_codes", e.data_ptr(), c.data_ptr(), _lib.ptr(s), rows, nblk,
                      block_size, buf.data_ptr(), _lib.stream_of(c))
    return buf.view(torch.int8)


def _unpack_from_flat_buffer(buffer: torch.Tensor, rows: int, num_blocks: int, block_size: int):
    """(shared_exponents u8, signs bool, magnitudes u8) -- distributed.py:201-232."""
    _require_device(buffer, "_unpack_from_flat_buffer")
    assert block_size in VALID_BLOCK_SIZES, f"block_size must be one of {VALID_BLOCK_SIZES}"
    need = rows * num_blocks * (1 + block_size * 3 // 4)
    if buffer.numel() != need:
        raise ValueError(f"buffer has {buffer.numel()} bytes, expected {need}")
    b = buffer.contiguous().view(torch.uint8)
    dev = b.device
    exps = torch.empty((rows, num_blocks), dtype=torch.uint8, device=dev)
    codes = torch.empty((rows, num_blocks, block_size), dtype=torch.uint8, device=dev)
    signs = torch.empty((rows, num_blocks, block_size), dtype=torch.uint8, device=dev)
    if need:
        with _on_device(b):
            _lib.call("axs6_nf5_wire_to_codes", b.data_ptr(), rows, num_blocks, block_size, exps.data_ptr(),
                      codes.data_ptr(), signs.data_ptr(), _lib.stream_of(b))
    return exps, signs.view(torch.bool), codes


def pack_gradient_to_buffer(tensor: torch.Tensor, block_size: int = DEFAULT_BLOCK_SIZE) -> torch.Tensor:
    """``_pack_to_flat_buffer(*_pack_gradient(tensor)[:3])`` in one kernel
    pass: reads the tensor once, writes 25 bytes per 32 values."""
    fn = "pack_gradient_to_buffer"
    _require_device(tensor, fn)
    assert block_size in VALID_BLOCK_SIZES, f"block_size must be one of {VALID_BLOCK_SIZES}"
    x, rows, cols = as_rows(tensor)
    buf = torch.empty((wire_bytes(rows, cols, block_size),), dtype=torch.uint8, device=x.device)
    if buf.numel():
        with _on_device(x):
            _lib.call("axs6_nf5_pack_wire", x.data_ptr(), _lib.DTYPE_CODE[x.dtype], rows, cols, block_size,
                      buf.data_ptr(), _lib.stream_of(x))
    return buf.view(torch.int8)


def unpack_buffer_to_gradient(buffer: torch.Tensor, shape: torch.Size | tuple,
                              block_size: int = DEFAULT_BLOCK_SIZE) -> torch.Tensor:
    """float32 tensor of ``shape`` from a buffer of ``pack_gradient_to_buffer``
    (``_unpack_gradient(*_unpack_from_flat_buffer(...))`` in one pass)."""
    fn = "unpack_buffer_to_gradient"
    _require_device(buffer, fn)
    assert block_size in VALID_BLOCK_SIZES, f"block_size must be one of {VALID_BLOCK_SIZES}"
    shape = torch.Size(shape)
    cols = shape[-1] if len(shape) else 1
    rows = shape.numel() // cols if cols else 0
    need = wire_bytes(rows, cols, block_size)
    if buffer.numel() != need:
        raise ValueError(f"buffer has {buffer.numel()} bytes, expected {need} for shape {tuple(shape)}")
    b = buffer.contiguous().view(torch.uint8)
    y = torch.empty((rows, cols), dtype=torch.float32, device=b.device)
    if y.numel():
        with _on_device(b):
            _lib.call("axs6_nf5_unpack_wire", b.data_ptr(), rows, cols, block_size, y.data_ptr(), _lib.stream_of(b))
    return y.reshape(shape)
