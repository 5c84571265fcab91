"""The 6.25-bit wire layout of the oracle (restating
axs/unified/distributed.py:147-232), pinned independently of the
reference's shift/mask formulas: hand-computed bytes for a known block, and
for every one of the 64^4 code quadruples the three bytes equal the
little-endian bytes of the 24-bit word q0 | q1<<6 | q2<<12 | q3<<18, and
unpacking returns the codes.  Plus the Python API surface of the codec."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle


def test_known_block_bytes():
    # one block of 8 values: codes 1, 2, 3, 4 (signs 0, 1, 0, 1) then 31, 0, 17, 5 (signs 1, 0, 0, 0)
    codes = np.array([[[1, 2, 3, 4, 31, 0, 17, 5]]], np.uint8)
    signs = np.array([[[0, 1, 0, 1, 1, 0, 0, 0]]], bool)
    exps = np.array([[130]], np.uint8)
    buf = oracle.wire_pack(exps, codes, signs)
    # q = 1, 34, 3, 36 -> word 1 | 34<<6 | 3<<12 | 36<<18 = 0x9038 81 -> bytes 0x81, 0x38, 0x90
    # q = 63, 0, 17, 5 -> word 63 | 0 | 17<<12 | 5<<18 = 0x15103F -> bytes 0x3F, 0x10, 0x15
    assert buf.tolist() == [130, 0x81, 0x38, 0x90, 0x3F, 0x10, 0x15]
    e, c, s = oracle.wire_unpack(buf, 1, 1, 8)
    assert e.tolist() == [[130]] and np.array_equal(c, codes) and np.array_equal(s, signs)


def test_every_code_quadruple_is_little_endian_24_bit():
    # 2^24 quadruples in chunks of 2^21 (one 4-value block per quadruple)
    for start in range(0, 64 ** 4, 1 << 21):
        q = np.arange(start, start + (1 << 21), dtype=np.int32)
        quads = np.stack([(q >> (6 * i)) & 63 for i in range(4)], axis=-1)        # (N, 4)
        codes = (quads & 31).astype(np.uint8).reshape(-1, 1, 4)
        signs = ((quads >> 5) & 1).astype(bool).reshape(-1, 1, 4)
        exps = np.zeros((codes.shape[0], 1), np.uint8)
        buf = oracle.wire_pack(exps, codes, signs).reshape(-1, 4)
        word = q   # q0 | q1<<6 | q2<<12 | q3<<18 is the counter itself
        want = np.stack([word & 255, (word >> 8) & 255, (word >> 16) & 255], axis=-1).astype(np.uint8)
        assert np.array_equal(buf[:, 1:], want), start
        e, c, s = oracle.wire_unpack(buf.reshape(-1), codes.shape[0], 1, 4)
        assert np.array_equal(c, codes) and np.array_equal(s, signs), start


def test_record_sizes():
    from axs.unified.distributed import wire_bytes

    assert wire_bytes(1, 32, 32) == 25
    assert wire_bytes(3, 33, 32) == 3 * 2 * 25
    assert wire_bytes(2, 16, 8) == 2 * 2 * 7
    assert wire_bytes(1, 16, 16) == 13


def test_codec_names_and_cpu_tensor_error():
    from axs.unified import distributed as d

    for name in ("_pack_gradient", "_unpack_gradient", "_pack_to_flat_buffer", "_unpack_from_flat_buffer",
                 "pack_gradient_to_buffer", "unpack_buffer_to_gradient"):
        assert callable(getattr(d, name))
    with pytest.raises(RuntimeError, match="CUDA"):
        d.pack_gradient_to_buffer(torch.zeros(4, 32))
