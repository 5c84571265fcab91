"""GPU parity of the NF5 wire format (axs/unified/distributed.py:70-232):
the fused quantize+pack kernel, the fused unpack+dequantize kernel and the
component-level packers, bit-exact against the oracle's quantize/dequantize
and its restatement of the buffer layout."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from conftest import bits_equal

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _data(shape, seed, outliers=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g)
    if outliers:
        m = torch.rand(*shape, generator=g) < 0.01
        x[m] *= 100.0
    return x


def _edge_rows(bs):
    rows = [np.zeros(64, np.float32), np.full(64, -0.0, np.float32), np.full(64, 1.0, np.float32)]
    r = np.linspace(-1, 1, 64).astype(np.float32)
    r[3] = np.nan
    rows.append(r)
    r = np.linspace(-1, 1, 64).astype(np.float32)
    r[5] = np.inf
    r[40] = -np.inf
    rows.append(r)
    rows.append((np.linspace(-1, 1, 64) * 1e-40).astype(np.float32))      # subnormal blocks
    rows.append((np.linspace(-1, 1, 64) * 3e38).astype(np.float32))       # exponent clamp at 255
    rows.append((np.linspace(-1, 1, 64) * 2.0 ** -130).astype(np.float32))  # exponent clamp at 0
    return np.stack(rows)


def _oracle_buffer(x2: np.ndarray, bs: int) -> np.ndarray:
    exps, codes, signs = oracle.quantize(x2, bs)
    return oracle.wire_pack(exps, codes, signs)


# (64, 256), (300, 512), (7, 96), (1, 8): rows tile into whole blocks (the
# vector kernels; 300 x 512 ends in a partial workgroup iteration, 7 x 96 in a
# partial tile whose record bytes end mid 16-byte chunk); the others are
# ragged for some block sizes (the vector kernels' row-geometry mode: tiles
# spanning many short rows, rows of 4100 with four-value loads, rows of 777
# and 4095 with one-value loads)
@pytest.mark.parametrize("bs", [8, 16, 32])
@pytest.mark.parametrize("shape", [(64, 256), (300, 512), (7, 96), (37, 100), (5, 33), (1, 8),
                                   (300, 4100), (129, 777), (40, 4095)], ids=str)
def test_pack_wire_bitexact(bs, shape):
    from axs.unified.distributed import pack_gradient_to_buffer, unpack_buffer_to_gradient

    x = _data(shape, 7 * bs + shape[1])
    buf = pack_gradient_to_buffer(x.to(DEV), bs)
    assert np.array_equal(buf.cpu().numpy().view(np.uint8), _oracle_buffer(x.numpy(), bs))
    y = unpack_buffer_to_gradient(buf, shape, bs).cpu().numpy()
    exps, codes, signs = oracle.quantize(x.numpy(), bs)
    assert bits_equal(y, oracle.dequantize(exps, codes, signs, shape[1], bs))


@pytest.mark.parametrize("bs", [8, 32])
def test_wire_unaligned_pointers(bs):
    """Pointers off the vector kernels' alignment take the general kernels:
    same bytes and values."""
    from axs import _lib

    rows, cols = 40, 128
    x = _data((rows, cols + 1), 21 + bs)[:, 1:].contiguous()
    nbytes = _lib.lib().axs6_nf5_wire_bytes(rows, cols, bs)
    want = _oracle_buffer(x.numpy(), bs)
    xs = torch.zeros(rows * cols + 1, device=DEV)
    xs[1:] = x.reshape(-1).to(DEV)                       # input 4 bytes past a 16-byte boundary
    raw = torch.zeros(nbytes + 16, dtype=torch.uint8, device=DEV)
    st = _lib.stream_of(xs)
    _lib.call("axs6_nf5_pack_wire", xs[1:].data_ptr(), _lib.F32, rows, cols, bs, raw[3:].data_ptr(), st)
    torch.cuda.synchronize()
    assert np.array_equal(raw[3:3 + nbytes].cpu().numpy(), want)
    y = torch.zeros(rows * cols + 1, device=DEV)
    _lib.call("axs6_nf5_unpack_wire", raw[3:].data_ptr(), rows, cols, bs, y[1:].data_ptr(), st)
    torch.cuda.synchronize()
    exps, codes, signs = oracle.quantize(x.numpy(), bs)
    assert bits_equal(y[1:].cpu().numpy().reshape(rows, cols), oracle.dequantize(exps, codes, signs, cols, bs))


@pytest.mark.parametrize("bs", [8, 16, 32])
def test_pack_wire_edge_cases(bs):
    from axs.unified.distributed import pack_gradient_to_buffer, unpack_buffer_to_gradient

    x = _edge_rows(bs)
    buf = pack_gradient_to_buffer(torch.from_numpy(x).to(DEV), bs)
    assert np.array_equal(buf.cpu().numpy().view(np.uint8), _oracle_buffer(x, bs))
    y = unpack_buffer_to_gradient(buf, x.shape, bs).cpu().numpy()
    exps, codes, signs = oracle.quantize(x, bs)
    assert bits_equal(y, oracle.dequantize(exps, codes, signs, x.shape[1], bs))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bs,cols", [(32, 320), (8, 328), (16, 100), (32, 4100), (8, 777)])
def test_pack_wire_16bit_inputs(dtype, bs, cols):
    from axs.unified.distributed import pack_gradient_to_buffer

    x = _data((48, cols), 3 + bs).to(dtype)
    got = pack_gradient_to_buffer(x.to(DEV), bs).cpu().numpy().view(np.uint8)
    assert np.array_equal(got, _oracle_buffer(x.float().numpy(), bs))


def test_components_round_trip_and_match_fused():
    from axs.unified import distributed as d

    x = _data((3, 40, 96), 11).to(DEV)
    exps, signs, mags, shape = d._pack_gradient(x, 32)
    buf = d._pack_to_flat_buffer(exps, signs, mags)
    assert buf.dtype == torch.int8 and buf.numel() == 3 * 40 * 3 * 25
    assert torch.equal(buf, d.pack_gradient_to_buffer(x, 32))
    e2, s2, m2 = d._unpack_from_flat_buffer(buf, 120, 3, 32)
    assert torch.equal(e2, exps) and torch.equal(s2, signs) and torch.equal(m2, mags)
    y = d._unpack_gradient(e2, s2, m2, shape, 32)
    assert y.shape == x.shape
    assert torch.equal(y, d.unpack_buffer_to_gradient(buf, shape, 32))
    want = oracle.dequantize(*oracle.quantize(x.cpu().numpy().reshape(120, 96), 32), 96, 32)
    assert bits_equal(y.cpu().numpy().reshape(120, 96), want)


def test_wire_full_size_round_trip():
    """8192 x 4096 (the FQ benchmark shape): unpack(pack(x)) equals the
    dequantized quantize of x, bit for bit; the buffer is 25/128 of the f32 size."""
    from axs.unified import distributed as d
    from axs.unified.hip_kernels import hip_dequantize, hip_quantize

    print("[wire 8192x4096]", flush=True)
    g = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn(8192, 4096, device=DEV, generator=g)
    buf = d.pack_gradient_to_buffer(x, 32)
    assert buf.numel() * 128 == x.numel() * 4 * 25
    y = d.unpack_buffer_to_gradient(buf, x.shape, 32)
    e, c, s, _ = hip_quantize(x, 32)
    want = hip_dequantize(e, c, s, 8192, 4096, 32)
    assert torch.equal(y.view(torch.int32), want.view(torch.int32))
    # sampled rows against the oracle as well
    rows = torch.randperm(8192, generator=torch.Generator().manual_seed(1))[:64].to(DEV)
    xs = x[rows].cpu().numpy()
    assert np.array_equal(d.pack_gradient_to_buffer(x[rows], 32).cpu().numpy().view(np.uint8),
                          _oracle_buffer(xs, 32))
