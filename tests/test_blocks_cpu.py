"""The AXSBlock byte form (axs/core.py:44-152): the oracle's restatement and
the product's host ``AXSBlock``, pinned independently of either formula --
hand-computed bytes of a known block, every header value against the
little-endian 16-bit word, the payload against the wire format's payload
(whose layout ``test_wire_cpu`` pins over all 64^4 code quadruples; both
formats carry the same little-endian 6-bit stream), and round trips."""
from __future__ import annotations

import numpy as np
import pytest

import oracle


def _random_blocks(seed, rows, nblk, bs):
    rng = np.random.default_rng(seed)
    exps = rng.integers(0, 256, (rows, nblk), dtype=np.uint8)
    codes = rng.integers(0, 32, (rows, nblk, bs), dtype=np.uint8)
    signs = rng.integers(0, 2, (rows, nblk, bs)).astype(bool)
    return exps, codes, signs


# codes 1, 2, 3, 4 (signs 0, 1, 0, 1) then 31, 0, 17, 5 (signs 1, 0, 0, 0), exponent 130:
# header 130 << 2 = 0x0208 -> 0x08, 0x02; payload as worked out in test_wire_cpu
KNOWN = [0x08, 0x02, 0x81, 0x38, 0x90, 0x3F, 0x10, 0x15]
K_CODES = np.array([1, 2, 3, 4, 31, 0, 17, 5], np.uint8)
K_SIGNS = np.array([0, 1, 0, 1, 1, 0, 0, 0], bool)


def test_oracle_known_block():
    buf = oracle.block_pack(np.array([[130]], np.uint8), K_CODES.reshape(1, 1, 8), K_SIGNS.reshape(1, 1, 8))
    assert buf.tolist() == KNOWN
    e, c, s, cfg = oracle.block_unpack(buf, 1, 1, 8)
    assert e.tolist() == [[130]] and cfg.tolist() == [[0]]
    assert np.array_equal(c[0, 0], K_CODES) and np.array_equal(s[0, 0], K_SIGNS)


def test_product_block_known_bytes_and_properties():
    from axs.core import AXSBlock, BlockConfig

    b = AXSBlock(130, BlockConfig.DENSE, K_SIGNS, K_CODES, 8)
    assert list(b.to_bytes()) == KNOWN
    assert b.scale == 8.0 and b.total_bits == 10 + 48 and b.bits_per_value == 58 / 8
    b2 = AXSBlock.from_bytes(bytes(KNOWN), 8)
    assert b2.shared_exponent == 130 and b2.config is BlockConfig.DENSE and b2.block_size == 8
    assert b2.signs.dtype == bool and b2.magnitudes.dtype == np.uint8
    assert np.array_equal(b2.signs, K_SIGNS) and np.array_equal(b2.magnitudes, K_CODES)
    assert AXSBlock(127, BlockConfig.DENSE, K_SIGNS, K_CODES, 8).scale == 1.0
    assert AXSBlock(0, BlockConfig.DENSE, np.zeros(32, bool), np.zeros(32, np.uint8)).bits_per_value == 6.3125


def test_every_header_value():
    from axs.core import AXSBlock, BlockConfig

    e = np.repeat(np.arange(256), 4).reshape(-1, 1)
    cfg = np.tile(np.arange(4), 256).reshape(-1, 1)
    codes = np.zeros((1024, 1, 8), np.uint8)
    buf = oracle.block_pack(e, codes, codes.astype(bool), cfg).reshape(1024, 8)
    word = (e[:, 0] << 2) | cfg[:, 0]
    assert np.array_equal(buf[:, 0], word & 0xFF) and np.array_equal(buf[:, 1], word >> 8)
    assert not buf[:, 2:].any()
    ee, _, _, cc = oracle.block_unpack(buf.reshape(-1), 1024, 1, 8)
    assert np.array_equal(ee[:, 0], e[:, 0]) and np.array_equal(cc[:, 0], cfg[:, 0])
    for i in range(0, 1024, 37):
        blk = AXSBlock(int(e[i, 0]), BlockConfig(int(cfg[i, 0])), np.zeros(8, bool), np.zeros(8, np.uint8), 8)
        assert blk.to_bytes() == bytes(buf[i])


@pytest.mark.parametrize("bs", [8, 16, 32])
def test_payload_equals_wire_payload(bs):
    exps, codes, signs = _random_blocks(bs, 40, 5, bs)
    blocks = oracle.block_pack(exps, codes, signs).reshape(40, 5, 2 + bs * 3 // 4)
    wire = oracle.wire_pack(exps, codes, signs).reshape(40, 5, 1 + bs * 3 // 4)
    assert np.array_equal(blocks[..., 2:], wire[..., 1:])
    e, c, s, cfg = oracle.block_unpack(blocks.reshape(-1), 40, 5, bs)
    assert np.array_equal(e, exps) and np.array_equal(c, codes) and np.array_equal(s, signs)
    assert not cfg.any()


@pytest.mark.parametrize("bs", [8, 16, 32])
def test_product_block_matches_oracle(bs):
    from axs.core import AXSBlock, BlockConfig

    exps, codes, signs = _random_blocks(100 + bs, 1, 24, bs)
    want = oracle.block_pack(exps, codes, signs).reshape(24, -1)
    for j in range(24):
        blk = AXSBlock(int(exps[0, j]), BlockConfig.DENSE, signs[0, j], codes[0, j], bs)
        data = blk.to_bytes()
        assert data == bytes(want[j])
        back = AXSBlock.from_bytes(data + b"\xff", bs)        # trailing bytes are ignored
        assert back.shared_exponent == exps[0, j] and back.config is BlockConfig.DENSE
        assert np.array_equal(back.magnitudes, codes[0, j]) and np.array_equal(back.signs, signs[0, j])


def test_from_bytes_short_record_raises():
    from axs.core import AXSBlock

    with pytest.raises(IndexError):
        AXSBlock.from_bytes(bytes(25), 32)


def test_record_sizes():
    from axs.blocks import block_bytes, record_bytes

    assert [record_bytes(b) for b in (8, 16, 32)] == [8, 14, 26]
    assert block_bytes(3, 33, 32) == 3 * 2 * 26
    assert block_bytes(2, 16, 8) == 2 * 2 * 8
    with pytest.raises(AssertionError):
        record_bytes(12)


def test_device_codec_rejects_cpu_tensors():
    import torch

    from axs import blocks

    with pytest.raises(RuntimeError, match="CUDA"):
        blocks.encode_blocks(torch.zeros(4, 32))
    with pytest.raises(RuntimeError, match="CUDA"):
        blocks.decode_blocks(torch.zeros(26, dtype=torch.uint8), (1, 32))
