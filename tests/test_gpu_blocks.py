"""GPU parity of the AXSBlock byte form (axs/core.py:97-152) written and read
for whole tensors (axs.blocks, libaxs6.so): the fused quantize+serialise
kernel, the fused deserialise+dequantize kernel and the component-level
converters, bit-exact against the oracle's quantize/dequantize and its
restatement of the record layout, and against the product's host AXSBlock."""
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


def _edge_rows():
    rows = [np.zeros(64, np.float32), np.full(64, -0.0, np.float32), np.full(64, 1.0, np.float32)]
    r = np.linspace(-1, 1, 64).astype(np.float32)
    r[3] = np.nan
    rows.append(r)
    r = np.linspace(-1, 1, 64).astype(np.float32)
    r[5] = np.inf
    r[40] = -np.inf
    rows.append(r)
    rows.append((np.linspace(-1, 1, 64) * 1e-40).astype(np.float32))       # subnormal blocks
    rows.append((np.linspace(-1, 1, 64) * 3e38).astype(np.float32))        # exponent clamp at 255
    rows.append((np.linspace(-1, 1, 64) * 2.0 ** -130).astype(np.float32))  # exponent clamp at 0
    return np.stack(rows)


def _oracle_records(x2: np.ndarray, bs: int) -> np.ndarray:
    exps, codes, signs = oracle.quantize(x2, bs)
    return oracle.block_pack(exps, codes, signs)


def _oracle_values(x2: np.ndarray, bs: int) -> np.ndarray:
    exps, codes, signs = oracle.quantize(x2, bs)
    return oracle.dequantize(exps, codes, signs, x2.shape[1], bs)


# whole-block rows (vector kernels, with partial tiles and partial workgroup
# iterations) and ragged rows (general kernels), as for the wire format
@pytest.mark.parametrize("bs", [8, 16, 32])
@pytest.mark.parametrize("shape", [(64, 256), (300, 512), (7, 96), (37, 100), (5, 33), (1, 8),
                                   (300, 4100), (129, 777)], ids=str)
def test_encode_decode_bitexact(bs, shape):
    from axs.blocks import decode_blocks, encode_blocks

    print(f"[blocks bs={bs} shape={shape}]", flush=True)
    x = _data(shape, 5 * bs + shape[1])
    buf = encode_blocks(x.to(DEV), bs)
    assert buf.dtype == torch.uint8
    assert np.array_equal(buf.cpu().numpy(), _oracle_records(x.numpy(), bs))
    y = decode_blocks(buf, shape, bs).cpu().numpy()
    assert bits_equal(y, _oracle_values(x.numpy(), bs))


@pytest.mark.parametrize("bs", [8, 16, 32])
def test_edge_cases(bs):
    from axs.blocks import decode_blocks, encode_blocks

    x = _edge_rows()
    buf = encode_blocks(torch.from_numpy(x).to(DEV), bs)
    assert np.array_equal(buf.cpu().numpy(), _oracle_records(x, bs))
    assert bits_equal(decode_blocks(buf, x.shape, bs).cpu().numpy(), _oracle_values(x, bs))


@pytest.mark.parametrize("bs", [8, 32])
def test_unaligned_pointers(bs):
    """Pointers off the vector kernels' alignment take the general kernels:
    same bytes and values."""
    from axs import _lib

    rows, cols = 40, 128
    x = _data((rows, cols), 31 + bs)
    nbytes = _lib.lib().axs6_nf5_block_bytes(rows, cols, bs)
    assert nbytes == rows * cols // bs * (2 + bs * 3 // 4)
    xs = torch.zeros(rows * cols + 1, device=DEV)
    xs[1:] = x.reshape(-1).to(DEV)                       # input 4 bytes past a 16-byte boundary
    raw = torch.zeros(nbytes + 16, dtype=torch.uint8, device=DEV)
    st = _lib.stream_of(xs)
    _lib.call("axs6_nf5_pack_blocks", xs[1:].data_ptr(), _lib.F32, rows, cols, bs, raw[3:].data_ptr(), st)
    torch.cuda.synchronize()
    assert np.array_equal(raw[3:3 + nbytes].cpu().numpy(), _oracle_records(x.numpy(), bs))
    y = torch.zeros(rows * cols + 1, device=DEV)
    _lib.call("axs6_nf5_unpack_blocks", raw[3:].data_ptr(), rows, cols, bs, y[1:].data_ptr(), st)
    torch.cuda.synchronize()
    assert bits_equal(y[1:].cpu().numpy().reshape(rows, cols), _oracle_values(x.numpy(), bs))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bs,cols", [(32, 320), (8, 328), (16, 100)])
def test_16bit_inputs(dtype, bs, cols):
    from axs.blocks import encode_blocks

    x = _data((48, cols), 9 + bs).to(dtype)
    got = encode_blocks(x.to(DEV), bs).cpu().numpy()
    assert np.array_equal(got, _oracle_records(x.float().numpy(), bs))


def test_axs_tensor_round_trip_and_host_blocks():
    """quantize_unified -> axs_tensor_to_bytes equals the fused encoder and,
    record by record, the host AXSBlock.to_bytes; axs_tensor_from_bytes gives
    back the AXSTensor, and dequantize_unified of it the decoder's values."""
    from axs.blocks import axs_tensor_from_bytes, axs_tensor_to_bytes, decode_blocks, encode_blocks
    from axs.core import AXSBlock, BlockConfig
    from axs.unified.quantize_unified import dequantize_unified, quantize_unified

    x = _data((3, 40, 96), 13).to(DEV)
    q = quantize_unified(x, 32)
    buf = axs_tensor_to_bytes(q)
    assert buf.numel() == 120 * 3 * 26
    assert torch.equal(buf, encode_blocks(x, 32))
    recs = buf.cpu().numpy().reshape(120, 3, 26)
    e = q.shared_exponents.cpu().numpy()
    s = q.signs.cpu().numpy()
    c = q.magnitudes.cpu().numpy()
    for r in range(0, 120, 17):
        for j in range(3):
            blk = AXSBlock(int(e[r, j]), BlockConfig.DENSE, s[r, j], c[r, j], 32)
            assert blk.to_bytes() == recs[r, j].tobytes()
    q2 = axs_tensor_from_bytes(buf, x.shape, 32)
    assert q2.original_shape == x.shape and q2.num_blocks == 3 and q2.block_size == 32
    assert torch.equal(q2.shared_exponents, q.shared_exponents)
    assert torch.equal(q2.magnitudes, q.magnitudes) and torch.equal(q2.signs, q.signs)
    y = dequantize_unified(q2)
    assert torch.equal(y.view(torch.int32), decode_blocks(buf, x.shape, 32).view(torch.int32))


def test_decode_ignores_config_and_padding_bits():
    """Records whose header carries a non-DENSE config or set padding bits
    (bits 10..15) decode as the DENSE record of the same exponent: the
    reference's decoder reads no config, and the exponent is the 8-bit field."""
    from axs.blocks import axs_tensor_from_bytes, decode_blocks, encode_blocks

    x = _data((16, 64), 3).to(DEV)
    buf = encode_blocks(x, 32)
    want = decode_blocks(buf, x.shape, 32)
    recs = buf.clone().view(16 * 2, 26)
    recs[:, 0] |= torch.arange(32, device=DEV, dtype=torch.uint8) % 4          # config 0..3
    recs[:, 1] |= 0xFC                                                         # padding bits set
    got = decode_blocks(recs.reshape(-1), x.shape, 32)
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))
    q = axs_tensor_from_bytes(recs.reshape(-1), x.shape, 32)
    assert torch.equal(q.shared_exponents, axs_tensor_from_bytes(buf, x.shape, 32).shared_exponents)


def test_size_errors_and_empty():
    from axs.blocks import axs_tensor_from_bytes, decode_blocks, encode_blocks

    with pytest.raises(ValueError, match="bytes"):
        decode_blocks(torch.zeros(25, dtype=torch.uint8, device=DEV), (1, 32))
    with pytest.raises(ValueError, match="bytes"):
        axs_tensor_from_bytes(torch.zeros(27, dtype=torch.uint8, device=DEV), (1, 32))
    assert encode_blocks(torch.zeros(0, 64, device=DEV)).numel() == 0
    assert decode_blocks(torch.zeros(0, dtype=torch.uint8, device=DEV), (0, 64)).shape == (0, 64)


def test_full_size_round_trip():
    """8192 x 4096 (the FQ benchmark shape): decode(encode(x)) equals the
    dequantized quantize of x bit for bit, and equals the wire format's round
    trip; the records are 26/128 of the f32 size."""
    from axs.blocks import decode_blocks, encode_blocks
    from axs.unified import distributed as d
    from axs.unified.hip_kernels import hip_dequantize, hip_quantize

    print("[blocks 8192x4096]", flush=True)
    g = torch.Generator(device=DEV).manual_seed(6)
    x = torch.randn(8192, 4096, device=DEV, generator=g)
    buf = encode_blocks(x, 32)
    assert buf.numel() * 128 == x.numel() * 4 * 26
    y = decode_blocks(buf, x.shape, 32)
    e, c, s, _ = hip_quantize(x, 32)
    want = hip_dequantize(e, c, s, 8192, 4096, 32)
    assert torch.equal(y.view(torch.int32), want.view(torch.int32))
    wire = d.unpack_buffer_to_gradient(d.pack_gradient_to_buffer(x, 32), x.shape, 32)
    assert torch.equal(y.view(torch.int32), wire.view(torch.int32))
    rows = torch.randperm(8192, generator=torch.Generator().manual_seed(2))[:64].to(DEV)
    assert np.array_equal(encode_blocks(x[rows], 32).cpu().numpy(), _oracle_records(x[rows].cpu().numpy(), 32))


def test_short_or_host_fields_raise():
    """AXSTensor fields smaller than their shape claims, or on another device,
    raise before any kernel reads them."""
    from axs.blocks import axs_tensor_to_bytes
    from axs.core import AXSTensor
    from axs.unified import distributed as d
    from axs.unified.quantize_unified import dequantize_unified, quantize_unified

    q = quantize_unified(_data((8, 64), 4).to(DEV), 32)
    short = AXSTensor(q.shared_exponents[:4], q.signs, q.magnitudes, 32, q.original_shape, q.num_blocks)
    with pytest.raises(ValueError, match="too small"):
        dequantize_unified(short)
    host = AXSTensor(q.shared_exponents.cpu(), q.signs, q.magnitudes, 32, q.original_shape, q.num_blocks)
    with pytest.raises(RuntimeError, match="shared_exponents"):
        axs_tensor_to_bytes(host)
    with pytest.raises(ValueError, match="too small"):
        d._pack_to_flat_buffer(q.shared_exponents, q.signs.reshape(-1)[:10], q.magnitudes)
