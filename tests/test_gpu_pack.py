"""Bit-level parity of the GEMM operand packing (`axs6_nf5_pack_rows`).

The packed operand of a row r of x is fully determined by the NF5 format:
    S[r] = max over the row's finite nonzero blocks of e1 - 15   (0 if none),
    out[r, c] = fp16(v[r, c] * 2^-S[r])   for c < cols,   0 for cols <= c < cols_pad,
where 2^e1 is the block's FQ scale (e1 = floor_log2(amax) + 1, the
exponent rule of quantize_unified.py:154-160 restated in the oracle) and v is
FQ(x) (mode 1, fused_fake_quantize, quantize_unified.py:121-204) or x itself
(mode 0).  The expected bits are built here from the oracle's FQ values and
exponents with numpy's correctly rounded float32 ldexp and float16 casts; the
kernel must match them exactly.  Row widths cover every launch shape of the
packing kernel (one wave per row; 256, 512 and 768 threads per row), with odd
row counts so a workgroup is left with a single row.

The same S (with column exponents) and the tensor-wide maximum come from the
tiled statistics pass of the backward (`axs6_nf5_row_stats`), at row counts
and widths that exercise its 16-, 32- and 64-row tiles and ragged edges.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
BS = 32


def _data(rows: int, cols: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    x[rng.random((rows, cols)) < 0.01] *= 100.0
    if rows >= 8:
        x[1] = 0.0                                  # no finite nonzero block: S = 0
        x[2] *= np.float32(1e-38)                   # subnormal inputs
        x[3, ::7] *= np.float32(1e35)               # huge finite blocks: exponents near the top
        x[4, 5] = np.inf                            # an infinite block (FQ gives NaN/0 there)
        x[5, 40 % cols] = np.nan                    # a NaN block
        x[6] = np.float32(2.0 ** -130)              # scale exponents at the bottom
    return x


def _expected(x: np.ndarray, mode: int, cols_pad: int, colx: np.ndarray | None = None,
              u: np.ndarray | None = None, elem=None) -> tuple[np.ndarray, np.ndarray]:
    """Packed bits and row shifts; mode 1 FQ with nearest rounding, 2 with the
    dither u, 0 raw; colx optional per-column exponents.  `elem` (torch.bfloat16
    or torch.float16) is the input's element type: the FQ values are rounded to
    it first, as the reference's fake-quantize returns them for such a tensor."""
    rows, cols = x.shape
    v = oracle.fake_quantize(x, BS, u if mode == 2 else None) if mode else x.astype(np.float32)
    if mode and elem is not None:
        v = torch.from_numpy(v).to(elem).float().numpy()
    a = np.abs(x).reshape(rows, cols // BS, BS)
    with np.errstate(invalid="ignore"):
        amax = a.max(axis=2)                        # NaN where the block holds a NaN
    finite = np.isfinite(amax) & (amax > 0)
    e1 = oracle.floor_log2(np.where(finite, amax, 1.0)).astype(np.int64) + 1
    ok = finite & (e1 < 128)                        # 2^e1 finite in float32
    cx = np.zeros(cols, np.int64) if colx is None else colx.astype(np.int64)
    cblk = cx.reshape(cols // BS, BS).max(axis=1)
    lo = np.iinfo(np.int64).min // 2
    tmax = np.where(ok, e1 + cblk[None, :], lo).max(axis=1)
    shift = np.where(tmax == lo, 0, tmax - 15).astype(np.int32)
    with np.errstate(over="ignore", invalid="ignore"):
        scaled = np.ldexp(v.astype(np.float32), cx[None, :] - shift.astype(np.int64)[:, None]).astype(np.float32)
        packed = np.zeros((rows, cols_pad), np.float16)
        packed[:, :cols] = scaled.astype(np.float16)
    return packed, shift


def _pack(x: torch.Tensor, mode: int, cols_pad: int, colx: torch.Tensor | None = None, seed: int = 0,
          offset: int = 0):
    from axs import _lib

    rows, cols = x.shape
    out = torch.full((rows, cols_pad), float("nan"), dtype=torch.float16, device=DEV)   # padding must be written
    shift = torch.full((rows,), -12345, dtype=torch.int32, device=DEV)
    _lib.call("axs6_nf5_pack_rows", x.data_ptr(), _lib.DTYPE_CODE[x.dtype], rows, cols, BS, mode, seed, offset,
              _lib.ptr(colx), out.data_ptr(), cols_pad, cols_pad, shift.data_ptr(), None, _lib.stream_of(x))
    torch.cuda.synchronize()
    return out.cpu().numpy(), shift.cpu().numpy()


def _assert_bits(got: np.ndarray, want: np.ndarray, what: str):
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn), f"{what}: NaN positions differ"
    g = got.view(np.uint16)[~gn]
    w = want.view(np.uint16)[~wn]
    bad = np.flatnonzero(g != w)
    assert bad.size == 0, f"{what}: {bad.size} values differ, first {g[bad[:4]]} vs {w[bad[:4]]}"


# row lengths cover every thread shape of the kernel (one wave per row with
# 1, 2 or 4 vectors; 256 x 2/4, 768 x 2/4, 512 x 4/8 threads x vectors), the
# boundaries between them, and rows past the register-resident 16384
# (statistics pass + tiled pack)
@pytest.mark.parametrize("cols", [32, 256, 512, 1024, 1056, 1536, 2048, 4096, 6144, 8192, 8224, 11008, 12288, 12320,
                                  16384, 16416, 20000, 65536])
@pytest.mark.parametrize("rows", [37, 1])
def test_pack_rows_f32_bitexact(rows, cols):
    print(f"[pack_rows f32 {rows}x{cols}]", flush=True)
    x = _data(rows, cols, cols + rows)
    cols_pad = (cols + 63) // 64 * 64
    got, shift = _pack(torch.from_numpy(x).to(DEV), 1, cols_pad)
    want, wshift = _expected(x, 1, cols_pad)
    assert np.array_equal(shift, wshift)
    _assert_bits(got, want, f"f32 {rows}x{cols}")


# bf16 widths over every thread shape, up to the register-resident 32768 and past it
@pytest.mark.parametrize("cols", [256, 2080, 2560, 4096, 8192, 11008, 16384, 16416, 24576, 32768, 32800, 40000])
def test_pack_rows_bf16_bitexact(cols):
    print(f"[pack_rows bf16 37x{cols}]", flush=True)
    xb = torch.from_numpy(_data(37, cols, 5 + cols)).to(torch.bfloat16)
    x = xb.float().numpy()
    cols_pad = (cols + 63) // 64 * 64
    got, shift = _pack(xb.to(DEV), 1, cols_pad)
    want, wshift = _expected(x, 1, cols_pad, elem=torch.bfloat16)
    assert np.array_equal(shift, wshift)
    _assert_bits(got, want, f"bf16 37x{cols}")


# f16 inputs: FQ values rounded to f16 first (past 65504 -> inf, as torch's
# cast of the reference's fp32 FQ result), in registers and past them
@pytest.mark.parametrize("cols", [256, 4096, 32800])
def test_pack_rows_f16_bitexact(cols):
    print(f"[pack_rows f16 37x{cols}]", flush=True)
    x = _data(37, cols, 7 + cols)
    x = np.clip(x, -6e4, 6e4)
    x[8, :32] = 65000.0                         # FQ: lut[1014..] * 2^16 = 65536 -> inf in f16
    x[9, :32] = np.float32(3e-5)                # FQ values in the f16 subnormal range
    xh = torch.from_numpy(x).to(torch.float16)
    cols_pad = (cols + 63) // 64 * 64
    got, shift = _pack(xh.to(DEV), 1, cols_pad)
    want, wshift = _expected(xh.float().numpy(), 1, cols_pad, elem=torch.float16)
    assert np.array_equal(shift, wshift)
    assert np.isinf(want[8, :32].astype(np.float32)).any()
    _assert_bits(got, want, f"f16 37x{cols}")


def test_pack_rows_bf16_stochastic_bitexact():
    """Stochastic FQ of bf16 rows (the backward's dY in bf16): dither, then
    the bf16 rounding of the FQ value, then the fp16 packing."""
    cols = 4096
    xb = torch.from_numpy(_data(37, cols, 77)).to(torch.bfloat16)
    seed, offset = 0xABCDEF, 99
    cols_pad = cols
    got, shift = _pack(xb.to(DEV), 2, cols_pad, None, seed, offset)
    x = xb.float().numpy()
    want, wshift = _expected(x, 2, cols_pad, None, oracle.uniform(seed, offset, x.size).reshape(x.shape),
                             elem=torch.bfloat16)
    assert np.array_equal(shift, wshift)
    _assert_bits(got, want, "bf16 stochastic")


@pytest.mark.parametrize("cols", [256, 11008])
def test_pack_rows_raw_mode_bitexact(cols):
    """Mode 0 (no FQ, the general matmul's operands): the values themselves."""
    rng = np.random.default_rng(cols)
    x = (rng.standard_normal((21, cols)) * 3).astype(np.float32)
    cols_pad = (cols + 63) // 64 * 64
    got, shift = _pack(torch.from_numpy(x).to(DEV), 0, cols_pad)
    want, wshift = _expected(x, 0, cols_pad)
    assert np.array_equal(shift, wshift)
    _assert_bits(got, want, f"raw 21x{cols}")


@pytest.mark.parametrize("cols", [4096, 12320, 20000, 40960])
def test_pack_rows_stochastic_colx_bitexact(cols):
    """Mode 2 (dither counters offset + r * cols + c) with per-column
    exponents, in registers and past the register-resident length."""
    print(f"[pack_rows stochastic colx 37x{cols}]", flush=True)
    rng = np.random.default_rng(cols + 1)
    x = _data(37, cols, 9 + cols)
    colx = rng.integers(-6, 7, cols).astype(np.int32)
    seed, offset = 0x5EED0123, 12345
    cols_pad = (cols + 63) // 64 * 64
    got, shift = _pack(torch.from_numpy(x).to(DEV), 2, cols_pad, torch.from_numpy(colx).to(DEV), seed, offset)
    want, wshift = _expected(x, 2, cols_pad, colx, oracle.uniform(seed, offset, x.size).reshape(x.shape))
    assert np.array_equal(shift, wshift)
    _assert_bits(got, want, f"stochastic colx 37x{cols}")


def test_pack_rows_long_padding():
    """Past the register-resident length: zero columns up to a cols_pad beyond
    64 * ceil(cols / 64); a cols_pad short of that is refused (the tiled pack
    writes zeros up to it)."""
    from axs import _lib

    cols = 20000
    x = _data(5, cols, 4)
    got, shift = _pack(torch.from_numpy(x).to(DEV), 1, 20224)
    want, wshift = _expected(x, 1, 20224)
    assert np.array_equal(shift, wshift)
    _assert_bits(got, want, "long, cols_pad 20224")
    with pytest.raises(_lib.LibraryError, match="cols_pad"):
        _pack(torch.from_numpy(x).to(DEV), 1, 20000)


def _stats_expected(x: np.ndarray, colx: np.ndarray, rowx: np.ndarray):
    rows, cols = x.shape
    a = np.abs(x).reshape(rows, cols // BS, BS)
    with np.errstate(invalid="ignore"):
        amax = a.max(axis=2)
    finite = np.isfinite(amax) & (amax > 0)
    e1 = oracle.floor_log2(np.where(finite, amax, 1.0)).astype(np.int64) + 1
    ok = finite & (e1 < 128)
    lo = np.iinfo(np.int64).min // 2
    cblk = colx.astype(np.int64).reshape(cols // BS, BS).max(axis=1)
    tmax = np.where(ok, e1 + cblk[None, :], lo).max(axis=1)
    shift = np.where(tmax == lo, 0, tmax - 15).astype(np.int32)
    rmax = np.where(ok, e1, lo).max(axis=1)
    g = np.where(rmax == lo, lo, rmax + rowx.astype(np.int64)).max()
    return shift, (np.iinfo(np.int32).min if g == lo else int(g))


@pytest.mark.parametrize("rows,cols,dtype", [(37, 256, torch.float32), (37, 11008, torch.float32),
                                             (300, 1056, torch.float32), (64, 4096, torch.bfloat16),
                                             (50, 11008, torch.bfloat16), (8192, 11008, torch.float32),
                                             (8192, 1024, torch.float32), (129, 16416, torch.float16)], ids=str)
def test_row_stats_bitexact(rows, cols, dtype):
    from axs import _lib

    print(f"[row_stats {dtype} {rows}x{cols}]", flush=True)
    rng = np.random.default_rng(rows + cols)
    x = torch.from_numpy(_data(rows, cols, 3 + cols)).to(dtype)
    xf = x.float().numpy()
    colx = rng.integers(-3, 4, cols).astype(np.int32)
    rowx = rng.integers(-5, 6, rows).astype(np.int32)
    want_shift, want_g = _stats_expected(xf, colx, rowx)
    xd, cd, rd = x.to(DEV), torch.from_numpy(colx).to(DEV), torch.from_numpy(rowx).to(DEV)
    ws = torch.empty(_lib.lib().axs6_nf5_row_stats_workspace(rows, cols), dtype=torch.uint8, device=DEV)
    shift = torch.full((rows,), -12345, dtype=torch.int32, device=DEV)
    g = torch.full((1,), 777, dtype=torch.int32, device=DEV)
    _lib.call("axs6_nf5_row_stats", xd.data_ptr(), _lib.DTYPE_CODE[dtype], rows, cols, BS, cd.data_ptr(),
              shift.data_ptr(), rd.data_ptr(), g.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(xd))
    torch.cuda.synchronize()
    assert np.array_equal(shift.cpu().numpy(), want_shift)
    assert g.item() == want_g
    # without column exponents: the row pack's S
    _lib.call("axs6_nf5_row_stats", xd.data_ptr(), _lib.DTYPE_CODE[dtype], rows, cols, BS, None,
              shift.data_ptr(), None, None, ws.data_ptr(), ws.numel(), _lib.stream_of(xd))
    torch.cuda.synchronize()
    _, pack_shift = _pack(xd, 0, (cols + 63) // 64 * 64)
    assert np.array_equal(shift.cpu().numpy(), pack_shift)
