"""The C++ autograd node of the quantized linear (axs._C.linear, used by
axs_linear_unified) against the Python-level autograd Function
(_AXSLinearUnifiedFunction over hip_linear.forward_train / backward): the
same seed sequence gives bit-identical outputs and gradients, over dtypes,
ragged shapes, bias and no bias, and gradients for a subset of inputs."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _run(fn, x, w, b, g, needs):
    xs = x.clone().requires_grad_(needs[0])
    ws = w.clone().requires_grad_(needs[1])
    bs = None if b is None else b.clone().requires_grad_(needs[2])
    torch.manual_seed(11)
    out = fn(xs, ws, bs)
    out.backward(g)
    return out.detach(), [None if t is None else t.grad for t in (xs, ws, bs)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(2, 37, 96, 80), (1, 256, 128, 64), (3, 5, 40, 33)], ids=str)
@pytest.mark.parametrize("bias", [True, False])
def test_node_matches_python_function(dtype, shape, bias):
    from axs.unified import functional_unified as fu

    B, M, K, N = shape
    print(f"[ext {dtype} {shape} bias={bias}]", flush=True)
    gen = torch.Generator().manual_seed(B * M + K)
    x = torch.randn(B, M, K, generator=gen).to(DEV, dtype)
    w = (torch.randn(N, K, generator=gen) / K ** 0.5).to(DEV, dtype)
    b = torch.randn(N, generator=gen).to(DEV, dtype) if bias else None
    g = torch.randn(B, M, N, generator=gen).to(DEV, dtype)
    needs = (True, True, bias)
    y1, g1 = _run(lambda a, c, d: fu.axs_linear_unified(a, c, d, 32, True, True), x, w, b, g, needs)
    y2, g2 = _run(lambda a, c, d: fu._AXSLinearUnifiedFunction.apply(a, c, d, 32, True, True), x, w, b, g, needs)
    assert y1.dtype == dtype and torch.equal(y1, y2)
    for a, c in zip(g1, g2):
        assert (a is None) == (c is None)
        if a is not None:
            assert a.dtype == c.dtype and torch.equal(a, c)


def test_partial_gradients_and_no_grad():
    from axs.unified import functional_unified as fu

    gen = torch.Generator().manual_seed(4)
    x = torch.randn(64, 128, generator=gen).to(DEV)
    w = torch.randn(96, 128, generator=gen).to(DEV)
    b = torch.randn(96, generator=gen).to(DEV)
    g = torch.randn(64, 96, generator=gen).to(DEV)
    for needs in ((True, False, False), (False, True, False), (False, False, True), (True, True, True)):
        y1, g1 = _run(lambda a, c, d: fu.axs_linear_unified(a, c, d), x, w, b, g, needs)
        y2, g2 = _run(lambda a, c, d: fu._AXSLinearUnifiedFunction.apply(a, c, d, 32, True, True), x, w, b, g,
                      needs)
        assert torch.equal(y1, y2)
        for want, a, c in zip(needs, g1, g2):
            assert (a is not None) == want and (c is not None) == want
            if want:
                assert torch.equal(a, c)
    with torch.no_grad():
        y = fu.axs_linear_unified(x, w, b)
    assert not y.requires_grad and torch.equal(y, y1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float64])
@pytest.mark.parametrize("shape", [(3, 40, 96), (7, 33), (1, 8)], ids=str)
def test_fq_node(dtype, shape):
    """fake_quantize_unified (the C++ node axs._C.fq_ste) gives the bits of
    hip_fused_fake_quantize (pinned against the oracle by the FQ tests) and of
    the Python _FusedQuantizeSTE, in the input's dtype and shape, and its
    backward hands back the incoming gradient itself."""
    from axs.unified import functional_unified as fu
    from axs.unified.hip_kernels import hip_fused_fake_quantize

    gen = torch.Generator().manual_seed(sum(shape))
    x = (torch.randn(*shape, generator=gen) * 3).to(DEV, dtype)
    g = torch.randn(*shape, generator=gen).to(DEV, dtype)
    for bs in (8, 32):
        xs = x.clone().requires_grad_(True)
        y = fu.fake_quantize_unified(xs, bs, "nearest")
        assert y.dtype == dtype and y.shape == x.shape and y.requires_grad
        want = hip_fused_fake_quantize(x, bs, "nearest")
        assert torch.equal(y.detach(), want)
        assert torch.equal(fu._FusedQuantizeSTE.apply(x.clone().requires_grad_(True), bs, "nearest").detach(), want)
        (gx,) = torch.autograd.grad(y, xs, g)
        assert gx.data_ptr() == g.data_ptr()
    # stochastic: the seed comes from torch's default CPU generator, as in the function
    torch.manual_seed(21)
    y1 = fu.fake_quantize_unified(x, 32, "stochastic")
    torch.manual_seed(21)
    y2 = hip_fused_fake_quantize(x, 32, "stochastic")
    assert torch.equal(y1, y2)
    # a non-contiguous view is quantized as its contiguous copy
    if len(shape) == 3:
        xt = x.transpose(0, 1)
        assert torch.equal(fu.fake_quantize_unified(xt, 32, "nearest"),
                           hip_fused_fake_quantize(xt.contiguous(), 32, "nearest"))


def test_fq_node_empty_and_errors():
    from axs.unified import functional_unified as fu

    assert fu.fake_quantize_unified(torch.zeros(0, 64, device=DEV)).shape == (0, 64)
    assert fu.fake_quantize_unified(torch.zeros(4, 0, device=DEV)).shape == (4, 0)
    with pytest.raises(AssertionError):
        fu.fake_quantize_unified(torch.zeros(4, 64, device=DEV), 12)
    with pytest.raises(ValueError):
        fu.fake_quantize_unified(torch.zeros(4, 64, device=DEV), 32, "up")
