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
