"""Host-side behaviour of the axs.unified drop-in API that needs no GPU:
names, error behaviour (reference tests: tests/test_triton_kernels.py:268-280,
tests/test_triton_fused_linear.py:217-231, tests/test_backend.py:116-167,
424-435), module construction and conversion."""
from __future__ import annotations

import os
from unittest import mock

import pytest
import torch
import torch.nn as nn

import oracle
from conftest import bits_equal

REFERENCE_ALL = [
    "fused_fake_quantize", "quantize_unified", "dequantize_unified", "quantization_error_unified",
    "FUSED_NF5_LUT", "NF5_CODEBOOK", "REVERSE_NF5_LUT", "fake_quantize_unified", "axs_linear_unified",
    "axs_matmul_unified", "AXSLinearUnified", "AXSLayerNormUnified", "AXSEmbeddingUnified",
    "AXSMultiheadAttentionUnified", "convert_to_axs_unified", "BackendType", "accelerated_fake_quantize",
    "accelerated_linear", "accelerated_matmul", "backend_info", "clear_int8_weight_cache",
    "detect_best_backend", "get_backend", "set_backend", "has_triton", "triton_fused_fake_quantize",
    "triton_fused_linear", "AXSLinearMixedPrecision", "axs_linear_mixed_precision",
    "convert_to_axs_mixed_precision", "estimate_memory_savings",
]


@pytest.fixture(autouse=True)
def _reset_backend():
    yield
    from axs.unified import backend

    backend._active_backend = None


def test_reference_names_exported():
    import axs.unified as u

    missing = [n for n in REFERENCE_ALL if not hasattr(u, n)]
    assert not missing, missing
    assert u.AXS6Linear is u.AXSLinearUnified


def test_tables_match_oracle():
    from axs.unified import FUSED_NF5_LUT, NF5_CODEBOOK, REVERSE_NF5_LUT

    cb, lut, rev = oracle.tables()
    assert NF5_CODEBOOK.shape == (32,) and FUSED_NF5_LUT.shape == (1024,)
    assert bits_equal(NF5_CODEBOOK.numpy(), cb)
    assert bits_equal(FUSED_NF5_LUT.numpy(), lut)
    assert (REVERSE_NF5_LUT.numpy() == rev).all()
    from axs.unified.quantize_unified import _LUT_MAX_IDX

    assert _LUT_MAX_IDX == 1023


@pytest.mark.parametrize("fn_name", ["fused_fake_quantize", "triton_fused_fake_quantize",
                                     "accelerated_fake_quantize", "fake_quantize_unified",
                                     "quantize_unified"])
def test_cpu_tensor_raises_cuda_error(fn_name):
    import axs.unified as u

    with pytest.raises(RuntimeError, match="CUDA"):
        getattr(u, fn_name)(torch.randn(8, 32))


def test_linear_cpu_tensor_raises_cuda_error():
    import axs.unified as u

    x, w = torch.randn(4, 64), torch.randn(16, 64)
    with pytest.raises(RuntimeError, match="CUDA"):
        u.triton_fused_linear(x, w)
    with pytest.raises(RuntimeError, match="CUDA"):
        u.accelerated_linear(x, w)
    with pytest.raises(RuntimeError, match="CUDA"):
        u.AXSLinearUnified(64, 16)(x)


class _FakeCuda(torch.Tensor):
    pass


def _fake_cuda():
    t = torch.randn(4, 64)
    t = t.as_subclass(_FakeCuda)
    return t


@pytest.fixture(autouse=False)
def _patch_is_cuda():
    with mock.patch.object(_FakeCuda, "is_cuda", new_callable=mock.PropertyMock, return_value=True):
        yield


def test_invalid_block_size_asserts(_patch_is_cuda):
    from axs.unified.hip_kernels import hip_fused_fake_quantize

    with pytest.raises(AssertionError):
        hip_fused_fake_quantize(_fake_cuda(), 17, "nearest")


def test_invalid_rounding_rejected(_patch_is_cuda):
    from axs.unified.hip_kernels import hip_fused_fake_quantize

    with pytest.raises(ValueError, match="rounding"):
        hip_fused_fake_quantize(_fake_cuda(), 32, "up")


def test_block_32_check_precedes_device_work(_patch_is_cuda):
    from axs.unified.hip_kernels import hip_fused_linear

    with pytest.raises(ValueError, match="block_size=32"):
        hip_fused_linear(_fake_cuda(), _fake_cuda(), None, 16)


def test_backend_selection():
    from axs.unified.backend import BackendType, detect_best_backend, get_backend, set_backend

    with mock.patch.dict(os.environ, {"AXS6_BACKEND": ""}):
        assert detect_best_backend() == BackendType.HIP
    for name in ("eager", "compiled", "int8", "triton", "hip"):
        with mock.patch.dict(os.environ, {"AXS6_BACKEND": f"  {name.upper()} "}):
            assert detect_best_backend() == BackendType(name)
    with mock.patch.dict(os.environ, {"AXS6_BACKEND": "bogus"}):
        assert detect_best_backend() == BackendType.HIP
    set_backend("EAGER")
    assert get_backend() == BackendType.EAGER
    set_backend(BackendType.TRITON)
    assert get_backend() == BackendType.TRITON
    with pytest.raises(ValueError):
        set_backend("nonexistent")


def test_backend_info_keys():
    from axs.unified.backend import backend_info

    info = backend_info()
    for key in ("active_backend", "cuda_available", "triton_kernel", "int8_tensorcore", "torch_compile",
                "gpu_name", "compute_capability", "lut_cached_devices", "hip_library", "hip_kernel"):
        assert key in info
    assert "gfx950" in info["hip_library"]
    assert info["cuda_available"] is False and info["hip_kernel"] is False


def test_modules_construct_like_reference():
    import axs.unified as u

    lin = u.AXSLinearUnified(96, 48, bias=True, block_size=16, quantize_input=False, quantize_grad=False)
    assert lin.weight.shape == (48, 96) and lin.bias.shape == (48,)
    assert "block_size=16" in repr(lin) and "quant_input=False" in repr(lin)
    bound = 1 / 96 ** 0.5
    assert lin.bias.abs().max() <= bound
    assert lin.weight.abs().max() <= bound + 1e-6          # kaiming_uniform(a=sqrt5) bound
    nb = u.AXSLinearUnified(8, 8, bias=False)
    assert nb.bias is None
    ln = u.AXSLayerNormUnified(32)
    x = torch.randn(2, 32)
    assert torch.allclose(ln(x), torch.nn.functional.layer_norm(x, [32]))
    emb = u.AXSEmbeddingUnified(10, 32, padding_idx=0)
    assert (emb.weight[0] == 0).all()
    mha = u.AXSMultiheadAttentionUnified(64, 4)
    assert isinstance(mha.q_proj, u.AXSLinearUnified) and mha.head_dim == 16
    mp = u.AXSLinearMixedPrecision(32, 16)
    assert "mixed_precision=bf16" in repr(mp)


def test_warmup_bypass_runs_plain_linear_on_cpu():
    import axs.unified as u

    lin = u.AXSLinearUnified(32, 8)
    lin._warmup_active = True
    x = torch.randn(3, 32)
    assert torch.allclose(lin(x), torch.nn.functional.linear(x, lin.weight, lin.bias))


def test_convert_to_axs_unified():
    import axs.unified as u

    model = nn.Sequential(nn.Embedding(20, 32), nn.Linear(32, 64), nn.LayerNorm(64), nn.ReLU(),
                          nn.Sequential(nn.Linear(64, 16)))
    conv = u.convert_to_axs_unified(model, block_size=16, skip_layers={"4.0"})
    assert isinstance(conv[0], u.AXSEmbeddingUnified)
    assert isinstance(conv[1], u.AXSLinearUnified) and conv[1].block_size == 16
    assert isinstance(conv[2], u.AXSLayerNormUnified)
    assert isinstance(conv[4][0], nn.Linear)                 # skipped
    assert torch.equal(conv[1].weight, model[1].weight)
    assert isinstance(model[1], nn.Linear)                   # deep copy by default
    mp = u.convert_to_axs_mixed_precision(conv)
    assert isinstance(mp[1], u.AXSLinearMixedPrecision) and isinstance(mp[4][0], u.AXSLinearMixedPrecision)
    est = u.estimate_memory_savings(mp, batch_size=4, seq_len=8)
    assert est["savings_ratio"] > 1.0


def test_axstensor_properties():
    from axs.core import AXSTensor

    t = AXSTensor(torch.zeros(2, 4, dtype=torch.uint8), torch.zeros(2, 4, 32, dtype=torch.bool),
                  torch.zeros(2, 4, 32, dtype=torch.uint8), 32, torch.Size([2, 128]), 4)
    assert t.effective_bits_per_value == pytest.approx(6 + 10 / 32)
    assert t.memory_bytes == (256 * 6 + 8 * 10 + 7) // 8


def test_bias_vector_broadcasts_like_f_linear():
    """The fused path's bias check (host logic, no device work): one value or
    N values as (N,) / (1, N) are accepted and expanded to N float32 values,
    as F.linear broadcasts them; other lengths raise instead of reaching the
    kernel, which reads N values."""
    import torch.nn.functional as F

    from axs.unified.hip_linear import _bias_vector

    x, w = torch.randn(3, 4), torch.randn(5, 4)
    for b in (torch.randn(5), torch.randn(1), torch.randn(()), torch.randn(1, 5)):
        v = _bias_vector(b, 5, "t")
        assert v.shape == (5,) and v.dtype == torch.float32 and v.is_contiguous()
        assert torch.equal(F.linear(x, w, b), F.linear(x, w, v))
    assert _bias_vector(None, 5, "t") is None
    for b in (torch.randn(3), torch.randn(6), torch.randn(5, 1), torch.randn(2, 5)):
        with pytest.raises(RuntimeError):
            F.linear(x, w, b)
        with pytest.raises(RuntimeError, match="does not broadcast"):
            _bias_vector(b, 5, "t")
