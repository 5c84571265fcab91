"""CPU oracle for the NF5 hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or the timed
CPU baseline), never as the thing measured or shipped.  The product package
``axs`` (under ``axs-6_amd/``) never imports it.

Contents:
  * ``liboracle.so`` (built from ``nf5_oracle.c`` by ``make -C oracle``): a
    scalar C restatement of the reference's eager NF5 operations
    (``axs/unified/quantize_unified.py:50-308``), wrapped below for numpy.
  * :func:`wire_pack` / :func:`wire_unpack`: the reference's 6.25-bit gradient
    buffer layout (``axs/unified/distributed.py:147-232``).
  * :func:`block_pack` / :func:`block_unpack`: the concatenated
    ``AXSBlock.to_bytes`` / ``from_bytes`` records (``axs/core.py:97-152``).
  * :func:`linear_reference`: the fp64 product of fake-quantized operands
    that the quantized-linear kernels are compared to
    (``axs/unified/functional_unified.py:107-170``).
  * :mod:`oracle.eager_torch`: the reference's op sequence in torch eager,
    timed on the host as the CPU baseline.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)


def build() -> str:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_build_tables.argtypes = [_f32p, _f32p, _u8p]
        L.oracle_floor_log2.argtypes = [ctypes.c_float]
        L.oracle_floor_log2.restype = ctypes.c_float
        L.oracle_floor_log2_batch.argtypes = [_f32p, _f32p, ctypes.c_int64]
        L.oracle_fake_quantize.argtypes = [_f32p, _f32p, ctypes.c_int64, ctypes.c_int64,
                                           ctypes.c_int, _f32p]
        L.oracle_quantize.argtypes = [_f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                      _f32p, _u8p, _u8p, _u8p]
        L.oracle_dequantize.argtypes = [_u8p, _u8p, _u8p, _f32p, ctypes.c_int64,
                                        ctypes.c_int64, ctypes.c_int]
        L.oracle_uniform.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int64, _f32p]
        _lib = L
    return _lib


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t) if a is not None else None


def tables() -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(codebook[32] f32, lut[1024] f32, reverse_lut[1024] u8)."""
    cb = np.zeros(32, np.float32)
    lut = np.zeros(1024, np.float32)
    rev = np.zeros(1024, np.uint8)
    lib().oracle_build_tables(_p(cb, _f32p), _p(lut, _f32p), _p(rev, _u8p))
    return cb, lut, rev


def floor_log2(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().oracle_floor_log2_batch(_p(x, _f32p), _p(out, _f32p), x.size)
    return out


def _as_2d(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim == 0:
        x = x.reshape(1, 1)
    return x.reshape(-1, x.shape[-1])


def uniform(seed: int, offset: int, n: int) -> np.ndarray:
    u = np.empty(n, np.float32)
    lib().oracle_uniform(ctypes.c_uint64(seed), ctypes.c_uint64(offset), n, _p(u, _f32p))
    return u


def fake_quantize(x: np.ndarray, block_size: int = 32, u: np.ndarray | None = None) -> np.ndarray:
    """fused_fake_quantize on float32 input (any shape, blocks along the last dim).

    ``u`` (same number of elements as ``x``) replaces torch.rand_like for
    rounding="stochastic"; None means rounding="nearest".
    """
    shape = np.shape(x)
    x2 = _as_2d(x)
    y = np.empty_like(x2)
    up = None
    if u is not None:
        u = np.ascontiguousarray(u, dtype=np.float32).reshape(-1)
        assert u.size == x2.size
        up = _p(u, _f32p)
    lib().oracle_fake_quantize(_p(x2, _f32p), _p(y, _f32p), x2.shape[0], x2.shape[1],
                               block_size, up)
    return y.reshape(shape)


def quantize(x: np.ndarray, block_size: int = 32, u: np.ndarray | None = None):
    """quantize_unified -> (exponents u8 (R, nblk), codes u8 (R, nblk, bs), signs bool)."""
    x2 = _as_2d(x)
    R, C = x2.shape
    nblk = (C + block_size - 1) // block_size
    exps = np.empty((R, nblk), np.uint8)
    codes = np.empty((R, nblk, block_size), np.uint8)
    signs = np.empty((R, nblk, block_size), np.uint8)
    up = None
    if u is not None:
        u = np.ascontiguousarray(u, dtype=np.float32).reshape(-1)
        up = _p(u, _f32p)
    lib().oracle_quantize(_p(x2, _f32p), R, C, block_size, up, _p(exps, _u8p),
                          _p(codes, _u8p), _p(signs, _u8p))
    return exps, codes, signs.astype(bool)


def dequantize(exps: np.ndarray, codes: np.ndarray, signs: np.ndarray, cols: int,
               block_size: int = 32) -> np.ndarray:
    exps = np.ascontiguousarray(exps, dtype=np.uint8)
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    s = np.ascontiguousarray(signs, dtype=np.uint8)
    R = exps.shape[0]
    y = np.empty((R, cols), np.float32)
    lib().oracle_dequantize(_p(exps, _u8p), _p(codes, _u8p), _p(s, _u8p), _p(y, _f32p),
                            R, cols, block_size)
    return y


def wire_pack(exps: np.ndarray, codes: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """_pack_to_flat_buffer (axs/unified/distributed.py:147-198): per block, the
    exponent byte then the 6-bit codes (sign << 5 | code) packed four per three
    bytes with the reference's shifts and masks (:178-183).  uint8 [R*nblk*rec]."""
    R, nblk, bs = codes.shape
    assert bs % 4 == 0
    q = codes.astype(np.int32) | (np.asarray(signs).astype(np.int32) << 5)
    q = q.reshape(R, nblk, bs // 4, 4)
    c0, c1, c2, c3 = q[..., 0], q[..., 1], q[..., 2], q[..., 3]
    b0 = (c0 & 0x3F) | ((c1 & 0x03) << 6)
    b1 = ((c1 >> 2) & 0x0F) | ((c2 & 0x0F) << 4)
    b2 = ((c2 >> 4) & 0x03) | ((c3 & 0x3F) << 2)
    vals = np.stack([b0, b1, b2], axis=-1).reshape(R, nblk, bs * 3 // 4).astype(np.uint8)
    out = np.zeros((R, nblk, 1 + bs * 3 // 4), np.uint8)
    out[:, :, 0] = exps
    out[:, :, 1:] = vals
    return out.reshape(-1)


def wire_unpack(buf: np.ndarray, rows: int, nblk: int, bs: int):
    """_unpack_from_flat_buffer (distributed.py:201-232): (exps, codes, signs)."""
    b = np.asarray(buf).view(np.uint8).reshape(rows, nblk, 1 + bs * 3 // 4)
    exps = b[:, :, 0].copy()
    v = b[:, :, 1:].reshape(rows, nblk, bs // 4, 3).astype(np.int32)
    b0, b1, b2 = v[..., 0], v[..., 1], v[..., 2]
    c0 = b0 & 0x3F
    c1 = ((b0 >> 6) & 0x03) | ((b1 & 0x0F) << 2)
    c2 = ((b1 >> 4) & 0x0F) | ((b2 & 0x03) << 4)
    c3 = (b2 >> 2) & 0x3F
    q = np.stack([c0, c1, c2, c3], axis=-1).reshape(rows, nblk, bs)
    return exps, (q & 0x1F).astype(np.uint8), ((q >> 5) & 1).astype(bool)


def block_pack(exps: np.ndarray, codes: np.ndarray, signs: np.ndarray,
               configs: np.ndarray | None = None) -> np.ndarray:
    """AXSBlock.to_bytes (axs/core.py:97-119) of every block, concatenated:
    the 2-byte little-endian header ``e << 2 | config`` then the 6-bit values
    ``sign << 5 | code`` emitted low bit first (the reference's bit
    accumulator, here as unpackbits/packbits in little bit order) and padded
    to whole bytes.  uint8 [R * nblk * (2 + ceil(6 bs / 8))]."""
    R, nblk, bs = codes.shape
    q = (codes.astype(np.uint8) & 0x1F) | (np.asarray(signs).astype(np.uint8) << 5)
    bits = np.unpackbits(q.reshape(R, nblk, bs, 1), axis=-1, bitorder="little")[..., :6]
    bits = bits.reshape(R, nblk, bs * 6)
    pad = (-bits.shape[-1]) % 8
    if pad:
        bits = np.concatenate([bits, np.zeros((R, nblk, pad), np.uint8)], axis=-1)
    payload = np.packbits(bits, axis=-1, bitorder="little")
    cfg = np.zeros((R, nblk), np.int64) if configs is None else np.asarray(configs, np.int64)
    header = (np.asarray(exps, np.int64) << 2) | cfg
    out = np.empty((R, nblk, 2 + payload.shape[-1]), np.uint8)
    out[:, :, 0] = header & 0xFF
    out[:, :, 1] = header >> 8
    out[:, :, 2:] = payload
    return out.reshape(-1)


def block_unpack(buf: np.ndarray, rows: int, nblk: int, bs: int):
    """AXSBlock.from_bytes (axs/core.py:121-152) of every record:
    (exps, codes, signs, configs), exps = header >> 2."""
    nb = (6 * bs + 7) // 8
    b = np.asarray(buf).view(np.uint8).reshape(rows, nblk, 2 + nb)
    header = b[:, :, 0].astype(np.int64) | (b[:, :, 1].astype(np.int64) << 8)
    bits = np.unpackbits(b[:, :, 2:], axis=-1, bitorder="little")[..., :6 * bs]
    q = np.packbits(bits.reshape(rows, nblk, bs, 6), axis=-1, bitorder="little")[..., 0]
    return header >> 2, (q & 0x1F).astype(np.uint8), ((q >> 5) & 1).astype(bool), (header & 3).astype(np.uint8)


def linear_reference(xq: np.ndarray, wq: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    """Y = Xq . Wq^T (+ b) in float64 -- the exact product the fp32 reference
    (F.linear of fake-quantized operands, functional_unified.py:123)
    approximates; kernels are held to rel-L2 against it."""
    y = np.asarray(xq, np.float64) @ np.asarray(wq, np.float64).T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    return y


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b.ravel())
    return float(np.linalg.norm((a - b).ravel()) / (den if den > 0 else 1.0))
