"""API edges of the quantized linear and matmul against the reference's
semantics, on the GPU:

* the bias broadcasts as in the reference's F.linear (one value, or N
  values) and any other length raises instead of being read past its end
  (fused small-output kernel, packed path, autograd node);
* float64 inputs come back as float64 (the reference's fused and eager
  linears return ``result.to(orig_dtype)`` / F.linear of float64 FQ values,
  ``triton_kernels.py:432,482``), with dX float64 too;
* ``axs_matmul_unified`` with batched operands ``a (*, M, K) @ b (*, K, N)``
  and 1-D operands, as the reference's torch.matmul of the FQ values
  (``functional_unified.py:204-227``).

Bar: rel-L2 <= 1e-3 against the fp64 product of the C oracle's FQ values."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TOL = 1e-3


def _inputs(M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(M, K, generator=g), torch.randn(N, K, generator=g) * K ** -0.5, torch.randn(N, generator=g)


def _ref(x, w, b):
    xq = oracle.fake_quantize(x.float().numpy(), 32).astype(np.float64)
    wq = oracle.fake_quantize(w.float().numpy(), 32).astype(np.float64)
    return xq @ wq.T + (0.0 if b is None else np.broadcast_to(b.double().numpy().reshape(-1), (wq.shape[0],)))


# (M, N): M*N <= 128K takes the fused kernel, more the packed path
@pytest.mark.parametrize("M,N", [(8, 64), (512, 384)])
def test_bias_broadcast_and_length_errors(M, N):
    from axs.unified import hip_linear
    from axs.unified.functional_unified import axs_linear_unified

    x, w, _ = _inputs(M, N, 256, M + N)
    xd, wd = x.to(DEV), w.to(DEV)
    for b in (torch.tensor([0.75]), torch.tensor(-1.5), torch.randn(1, N)):
        want = _ref(x, w, b)
        assert oracle.rel_l2(hip_linear.linear_forward(xd, wd, b.to(DEV)).cpu().numpy(), want) < TOL
        assert oracle.rel_l2(hip_linear.forward_train(xd, wd, b.to(DEV), 32, True)[0].cpu().numpy(), want) < TOL
        y = axs_linear_unified(xd, wd, b.to(DEV))
        assert oracle.rel_l2(y.detach().cpu().numpy(), want) < TOL
    for bad in (torch.randn(N - 1), torch.randn(N + 3), torch.randn(N, 1), torch.randn(2, N)):
        with pytest.raises(RuntimeError, match="does not broadcast"):
            hip_linear.linear_forward(xd, wd, bad.to(DEV))
        with pytest.raises(RuntimeError, match="does not broadcast"):
            hip_linear.forward_train(xd, wd, bad.to(DEV), 32, True)
        with pytest.raises(RuntimeError, match="does not broadcast"):
            axs_linear_unified(xd, wd, bad.to(DEV))


@pytest.mark.parametrize("M,N", [(4, 96), (300, 640)])
def test_float64_in_float64_out(M, N):
    from axs.unified import hip_kernels, hip_linear
    from axs.unified.functional_unified import axs_linear_unified

    x, w, b = _inputs(M, N, 512, 7 * M)
    want = _ref(x, w, b)
    xd, wd, bd = x.double().to(DEV), w.double().to(DEV), b.double().to(DEV)
    for y in (hip_linear.linear_forward(xd, wd, bd), hip_kernels.hip_fused_linear(xd, wd, bd),
              hip_linear.forward_train(xd, wd, bd, 32, True)[0]):
        assert y.dtype == torch.float64
        assert oracle.rel_l2(y.cpu().numpy(), want) < TOL
    xg = xd.clone().requires_grad_(True)
    wg = wd.clone().requires_grad_(True)
    y = axs_linear_unified(xg, wg, bd, 32, True, False)
    assert y.dtype == torch.float64
    dy = torch.randn(M, N, generator=torch.Generator().manual_seed(3), dtype=torch.float64)
    y.backward(dy.to(DEV))
    assert xg.grad.dtype == torch.float64 and wg.grad.dtype == torch.float64
    wq = oracle.fake_quantize(w.numpy(), 32).astype(np.float64)
    xq = oracle.fake_quantize(x.numpy(), 32).astype(np.float64)
    # quantize_grad=False: dY as given (rounded to the float32 compute type)
    d = dy.float().double().numpy()
    assert oracle.rel_l2(xg.grad.cpu().numpy(), d @ wq) < TOL
    assert oracle.rel_l2(wg.grad.cpu().numpy(), d.T @ xq) < TOL


def _mm_ref(a, b):
    """torch.matmul of the oracle's FQ values (blocks along each operand's
    last dim), in fp64."""
    aq = torch.from_numpy(oracle.fake_quantize(a.numpy(), 32)).double()
    bq = torch.from_numpy(oracle.fake_quantize(b.numpy(), 32)).double()
    return torch.matmul(aq, bq).numpy()


@pytest.mark.parametrize("sa,sb", [((2, 3, 40, 96), (3, 96, 72)), ((5, 33, 64), (64, 48)),
                                   ((4, 1, 17, 128), (6, 128, 20)), ((96,), (2, 96, 24)),
                                   ((3, 10, 64), (64,)), ((64,), (64,)), ((1, 8, 32), (4, 32, 8))])
def test_axs_matmul_unified_batched(sa, sb):
    from axs.unified import accelerated_matmul
    from axs.unified.functional_unified import axs_matmul_unified

    g = torch.Generator().manual_seed(sum(sa) + sum(sb))
    a = torch.randn(*sa, generator=g)
    b = torch.randn(*sb, generator=g)
    want = _mm_ref(a, b)
    got = axs_matmul_unified(a.to(DEV), b.to(DEV))
    assert got.shape == torch.matmul(a, b).shape and got.dtype == torch.float32
    aq = torch.from_numpy(oracle.fake_quantize(a.numpy(), 32))
    bq = torch.from_numpy(oracle.fake_quantize(b.numpy(), 32))

    def close(y):
        if want.size >= 16:
            return oracle.rel_l2(y, want) < TOL
        # a lone dot product can cancel, which makes its relative error
        # ill-posed: bound it by the scale of its terms, sum |a_i b_i|
        scale = torch.matmul(aq.abs().double(), bq.abs().double()).numpy()
        return np.max(np.abs(y - want) / scale) < TOL

    assert close(got.cpu().numpy()), (sa, sb)
    # the GEMM alone (accelerated_matmul: no NF5 step) on the same FQ values
    got2 = accelerated_matmul(aq.to(DEV), bq.to(DEV))
    assert got2.shape == got.shape
    assert close(got2.cpu().numpy()), (sa, sb)


def test_axs_matmul_unified_dtype_and_errors():
    from axs.unified.functional_unified import axs_matmul_unified

    g = torch.Generator().manual_seed(1)
    a = torch.randn(2, 16, 64, generator=g)
    b = torch.randn(2, 64, 32, generator=g)
    y = axs_matmul_unified(a.to(DEV, torch.bfloat16), b.to(DEV, torch.bfloat16))
    assert y.dtype == torch.bfloat16
    want = _mm_ref(a.bfloat16().float(), b.bfloat16().float())
    assert oracle.rel_l2(y.float().cpu().numpy(), want) < 5e-3   # bf16 output rounding
    with pytest.raises(RuntimeError, match="do not contract"):
        axs_matmul_unified(a.to(DEV), torch.randn(2, 63, 32, device=DEV))
