"""The C-ABI library loads, exports every entry point include/axs6.h
declares, carries the same constant tables as the oracle, and rejects bad
arguments before touching a device (no compute calls: runs without a GPU)."""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest
import torch  # noqa: F401  (loads the HIP runtime libaxs6 binds to)

import oracle
from axs import _lib
from conftest import ROOT, bits_equal


def declared_symbols() -> list[str]:
    names = []
    for f in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if f.endswith(".h"):
            text = open(os.path.join(ROOT, "include", f)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names += re.findall(r"\b(axs6_\w+)\s*\(", text)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = declared_symbols()
    assert "axs6_nf5_fake_quantize" in names
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_every_declared_symbol_has_a_binding_signature():
    names = set(declared_symbols()) - {"axs6_version", "axs6_last_error"}
    assert names <= set(_lib._SIGNATURES), sorted(names - set(_lib._SIGNATURES))


def test_version_string():
    assert "gfx950" in _lib.version()


def test_tables_match_oracle():
    cb, lut, rev, band = _lib.host_tables()
    ocb, olut, orev = oracle.tables()
    assert bits_equal(cb.numpy(), ocb)
    assert bits_equal(lut.numpy(), olut)
    assert np.array_equal(rev.numpy(), orev)
    # band[k+149]: floats just below 2^k whose floor(log2) is k, by the oracle
    want = np.zeros(278, np.uint8)
    for k in range(-148, 129):
        top = (k + 127) << 23 if k >= -126 else 1 << (k + 149)
        xs = np.arange(max(top - 64, 1), top, dtype=np.uint32)[::-1].view(np.float32)
        fl = oracle.floor_log2(xs)
        n = 0
        for v in fl:
            if v == k:
                n += 1
            else:
                break
        want[k + 149] = n
    assert np.array_equal(band.numpy(), want)
    assert band[127 + 149] == 44 and band[0 + 149] == 0


def test_band_matches_torch_log2_directly():
    _, _, _, band = _lib.host_tables()
    for k in (-130, -126, -100, -64, -63, -4, -2, 3, 8, 9, 17, 33, 64, 65, 127, 128):
        top = (k + 127) << 23 if k >= -126 else 1 << (k + 149)
        c = int(band[k + 149])
        inside = np.array([top - m for m in range(1, c + 1)], np.uint32).view(np.float32)
        outside = np.array([top - c - 1], np.uint32).view(np.float32)
        if c:
            assert np.all(torch.floor(torch.log2(torch.from_numpy(inside))).numpy() == k)
        assert torch.floor(torch.log2(torch.from_numpy(outside))).item() == k - 1


def _status(name, *args):
    fn = getattr(_lib.lib(), name)
    rc = fn(*args)
    return rc, _lib.lib().axs6_last_error().decode()


def test_invalid_arguments_rejected_without_device():
    rc, msg = _status("axs6_nf5_fake_quantize", 1, 1, 0, 4, 32, 17, 0, 0, 0, None, None)
    assert rc == 1 and "block_size" in msg
    rc, msg = _status("axs6_nf5_fake_quantize", 1, 1, 9, 4, 32, 32, 0, 0, 0, None, None)
    assert rc == 1 and "dtype" in msg
    rc, msg = _status("axs6_nf5_fake_quantize", 1, 1, 0, -1, 32, 32, 0, 0, 0, None, None)
    assert rc == 1 and "negative" in msg
    rc, msg = _status("axs6_nf5_fake_quantize", None, None, 0, 4, 32, 32, 0, 0, 0, None, None)
    assert rc == 1 and "null" in msg
    # empty tensors are a no-op, not an error
    rc, _ = _status("axs6_nf5_fake_quantize", None, None, 0, 0, 32, 32, 0, 0, 0, None, None)
    assert rc == 0
    rc, msg = _status("axs6_nf5_quantize", 1, 0, 4, 32, 12, 0, 0, 0, 1, 1, None, None, None, None)
    assert rc == 1 and "block_size" in msg
    rc, msg = _status("axs6_nf5_dequantize", 1, 1, None, 1, 4, 32, 7, None)
    assert rc == 1


def test_layer_norm_arguments_rejected_without_device():
    rc, msg = _status("axs6_layer_norm_forward", 16, 7, 4, 8, None, None, 1e-5, 16, None, None, None)
    assert rc == 1 and "dtype" in msg
    rc, msg = _status("axs6_layer_norm_forward", 16, 0, -1, 8, None, None, 1e-5, 16, None, None, None)
    assert rc == 1 and "negative" in msg
    rc, msg = _status("axs6_layer_norm_forward", None, 0, 4, 8, None, None, 1e-5, None, None, None, None)
    assert rc == 1 and "null" in msg
    rc, msg = _status("axs6_layer_norm_forward", 16, 0, 4, 8, None, None, -1.0, 16, None, None, None)
    assert rc == 1 and "eps" in msg
    # element-misaligned pointers (2 bytes into a float32 buffer)
    rc, msg = _status("axs6_layer_norm_forward", 18, 0, 4, 8, None, None, 1e-5, 16, None, None, None)
    assert rc == 1 and "aligned" in msg
    # empty rows or columns: nothing to do
    assert _status("axs6_layer_norm_forward", None, 0, 0, 8, None, None, 1e-5, None, None, None, None)[0] == 0
    ws = _lib.lib().axs6_layer_norm_backward_workspace(1000, 256)
    assert ws == 63 * 2 * 256 * 4   # one partial row pair per 16 rows
    assert _lib.lib().axs6_layer_norm_backward_workspace(-1, 4) == -1
    rc, msg = _status("axs6_layer_norm_backward", 16, 16, 0, 1000, 256, 16, 16, None, 16, 16, 16, 16, ws - 4, None)
    assert rc == 1 and "workspace" in msg
    rc, msg = _status("axs6_layer_norm_backward", None, 16, 0, 1000, 256, 16, 16, None, 16, 16, 16, 16, ws, None)
    assert rc == 1 and "null" in msg


def test_error_raises_runtime_error():
    with pytest.raises(RuntimeError, match="block_size"):
        _lib.call("axs6_nf5_fake_quantize", 1, 1, 0, 4, 32, 17, 0, 0, 0, None, None)


def test_backward_workspace_query_with_empty_dimensions():
    """No rows (M = 0) or an empty contraction (K = 0) is a normal query,
    not a division by a zero tile count."""
    L = _lib.lib()
    for M, N, K in ((0, 512, 256), (0, 4096, 4096), (64, 512, 0), (8192, 4096, 0), (0, 0, 0)):
        ws = L.axs6_nf5_linear_backward_workspace(M, N, K, 1, 1, 1)
        assert ws >= 0
    # K = 0 still needs the bias-gradient partials, nothing for dX / dW
    assert L.axs6_nf5_linear_backward_workspace(64, 512, 0, 1, 1, 0) <= \
        L.axs6_nf5_linear_backward_workspace(64, 512, 0, 1, 1, 1)


def test_leading_dimensions_checked_without_device():
    # pack_rows: ld_out below cols_pad would overlap rows and write the last
    # row's padding past the buffer
    rc, msg = _status("axs6_nf5_pack_rows", 256, 0, 4, 128, 32, 1, 0, 0, None, 256, 64, 128, 256, None, None)
    assert rc == 1 and "ld_out" in msg
    # GEMM: ldo below N
    rc, msg = _status("axs6_gemm_f16_nt", 256, 64, 256, 64, 64, 64, 64, None, None, None, 256, 32, 0, None)
    assert rc == 1 and "ldo" in msg


def test_noalloc_backward_rejects_shapes_beyond_its_scratch_without_device():
    """The allocation-free backward refuses a shape whose workspace exceeds
    its fixed scratch before it looks up a device or launches anything."""
    L = _lib.lib()
    limit = 64 << 20
    M, N, K = 8192, 4096, 11008
    assert L.axs6_nf5_linear_backward_workspace(M, N, K, 1, 1, 1) > limit
    p = 256   # never dereferenced: the size check comes first
    rc, msg = _status("axs6_nf5_linear_backward_noalloc", p, 0, M, N, K, 32, 1, 0, 0, p, p, p, p, p, p, p,
                      None, None)
    assert rc == 2 and "scratch" in msg
    # dX alone at this shape still exceeds it
    rc, msg = _status("axs6_nf5_linear_backward_noalloc", p, 0, M, N, K, 32, 0, 0, 0, p, p, p, p, p, None,
                      None, None, None)
    assert rc == 2 and "scratch" in msg
    # argument checks are the workspace entry point's
    rc, msg = _status("axs6_nf5_linear_backward_noalloc", p, 0, 64, 50, 64, 32, 0, 0, 0, p, p, p, p, p, p, p,
                      None, None)
    assert rc == 1 and "multiples of 4" in msg
    # nothing requested, or no rows: a no-op
    rc, _ = _status("axs6_nf5_linear_backward_noalloc", p, 0, 0, 64, 64, 32, 0, 0, 0, p, p, p, p, p, p, p,
                    None, None)
    assert rc == 0


def test_fused_linear_split_x_rule_without_device():
    """The host-only query behind fused_forward's two-launch path, (M, N, K)."""
    f = _lib.lib().axs6_nf5_fused_linear_split_x
    # X past both LDS stagings of FQ(X) and K >= 1024: the two-launch path
    assert f(16, 4096, 4096, _lib.F32) == 1 and f(32, 4096, 4096, _lib.F32) == 1
    assert f(17, 300, 2080, _lib.F32) == 1 and f(9, 4096, 4096, _lib.F32) == 1
    # the streamed decode form (M <= 2) or the MFMA form's staging holds X
    assert f(1, 4096, 4096, _lib.F32) == 0 and f(8, 4096, 4096, _lib.F32) == 0
    assert f(2, 4096, 8192, _lib.F32) == 0
    # every input dtype (the arranged FQ(X) is f32 either way)
    assert f(16, 4096, 4096, _lib.BF16) == 1 and f(32, 4096, 4096, _lib.F16) == 1
    assert f(128, 1024, 1024, _lib.F32) == 1 and f(64, 2048, 1024, _lib.F32) == 1
    # short contractions, empty or unaligned shapes, unknown dtypes
    assert f(128, 1024, 992, _lib.F32) == 0 and f(32, 4096, 512, _lib.F32) == 0
    assert f(16, 4096, 4096, 7) == 0
    assert f(0, 4096, 4096, _lib.F32) == 0 and f(16, 4096, 4100, _lib.F32) == 0


def test_fused_linear_split_workspace_and_arguments_without_device():
    """The arranged-X workspace is 16 * ceil(M / 16) * K floats; the split
    entry rejects a missing or unaligned workspace before any device work."""
    ws = _lib.lib().axs6_nf5_fused_linear_split_workspace
    assert ws(1, 4096) == 16 * 4096 * 4 and ws(16, 64) == 16 * 64 * 4
    assert ws(17, 2080) == 32 * 2080 * 4 and ws(40, 8192) == 48 * 8192 * 4
    assert ws(0, 64) == 0 and ws(16, 0) == 0 and ws(-1, 64) == 0
    name = "axs6_nf5_fused_linear_split"
    fake = 4096       # never dereferenced: the checks fail first
    rc, msg = _status(name, fake, fake, None, fake, None, _lib.F32, 32, 64, 2048, 32, 1, None)
    assert rc == 1 and "x_arranged" in msg
    rc, msg = _status(name, fake, fake, None, fake, fake + 4, _lib.F32, 32, 64, 2048, 32, 1, None)
    assert rc == 1 and "x_arranged" in msg
    rc, msg = _status(name, fake, fake, None, fake, fake, _lib.F32, 32, 64, 2050, 32, 1, None)
    assert rc == 1 and "multiple of 32" in msg
    rc, msg = _status(name, fake, fake, None, fake, fake, _lib.F32, 32, 64, 2048, 16, 1, None)
    assert rc == 1 and "block_size" in msg
    rc, _ = _status(name, fake, fake, None, fake, None, _lib.F32, 0, 64, 2048, 32, 1, None)
    assert rc == 0      # nothing to compute
