"""bf16 mixed-precision linear (``AXSLinearMixedPrecision`` /
``axs_linear_mixed_precision``) against a CPU restatement of the reference's
``_AXSLinearBF16Function`` (axs/unified/mixed_precision.py:96-153 in the
reference):

  forward   Xq = bf16(FQ(bf16(X))), Wq = bf16(FQ(bf16(W))),
            Y  = bf16(Xq . Wq^T + bf16(b))           (fp32 accumulation)
  backward  dYq = bf16(FQ_stochastic(bf16(dY)))      (or bf16(dY))
            dX = bf16(dYq . Wq),  dW = dYq^T . Xq in fp32,
            db = sum of the unquantized dY in fp32.

FQ values come from the C oracle (with the library's dither draws for the
stochastic dY: the seed is torch's CPU generator draw at the backward).

Tolerances, per output:
  * bf16 outputs (Y, dX): at least 99% of elements bit-identical to the
    exact (fp64) result rounded to bf16 -- the remaining ones are fp32
    accumulation-order flips of the last bf16 bit -- and rel-L2 <= 2e-3
    against the exact result (the bf16 rounding of the output itself is
    ~1e-3);
  * dW (fp32 from bf16 operands, every product exact): rel-L2 <= 1e-5;
  * db: rel-L2 <= 1e-6."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _bf16_fq(t: torch.Tensor, u: np.ndarray | None = None) -> torch.Tensor:
    """The reference's FQ of a bf16 tensor: fp32 arithmetic, result cast to bf16."""
    v = oracle.fake_quantize(t.float().numpy(), 32, u)
    return torch.from_numpy(v).to(torch.bfloat16)


def _check_bf16(got: torch.Tensor, exact: np.ndarray, what: str):
    got = got.detach().cpu()
    want = torch.from_numpy(exact.astype(np.float32)).to(torch.bfloat16)
    same = (got.view(torch.int16) == want.view(torch.int16)).float().mean().item()
    err = oracle.rel_l2(got.float().numpy(), exact)
    print(f"  {what}: {same:.5f} bit-identical to bf16(exact), rel-L2 {err:.3e}", flush=True)
    assert same >= 0.99, f"{what}: only {same:.4f} of the elements equal bf16(exact)"
    assert err <= 2e-3, f"{what}: rel-L2 {err:.3e}"


def _gauss(shape, seed, scale=1.0):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)) * scale


@pytest.mark.parametrize("M,K,N", [(4096, 4096, 4096), (2048, 768, 3072), (2048, 3072, 768), (96, 200, 64)])
@pytest.mark.parametrize("qgrad", [False, True], ids=["exact_dy", "stochastic_dy"])
def test_mixed_precision_linear_vs_reference_restatement(M, K, N, qgrad):
    from axs.unified.mixed_precision import axs_linear_mixed_precision

    print(f"[bf16 linear {M}x{K}x{N} qgrad={qgrad}]", flush=True)
    x = _gauss((M, K), 1)
    w = _gauss((N, K), 2, K ** -0.5)
    b = _gauss((N,), 3)
    dy = _gauss((M, N), 4)
    xd, wd, bd = (t.to(DEV).requires_grad_(True) for t in (x, w, b))
    y = axs_linear_mixed_precision(xd, wd, bd, 32, True, qgrad)
    assert y.dtype == torch.bfloat16 and y.shape == (M, N)
    torch.manual_seed(77)                       # the backward's dither seed comes from here
    y.backward(dy.to(DEV))
    torch.manual_seed(77)
    seed = int(torch.randint(0, 2**62, (1,)).item())

    g = torch.Generator().manual_seed(9)
    rm = torch.randperm(M, generator=g)[:256] if M > 256 else torch.arange(M)
    rn = torch.randperm(N, generator=g)[:256] if N > 256 else torch.arange(N)
    xq = _bf16_fq(x.bfloat16()).double()
    wq = _bf16_fq(w.bfloat16()).double()
    b16 = b.bfloat16().double()
    y_exact = (xq[rm] @ wq.T + b16).numpy()
    _check_bf16(y[rm.to(DEV)], y_exact, "Y")

    dyb = dy.bfloat16()
    u = oracle.uniform(seed, 0, dy.numel()).reshape(dy.shape) if qgrad else None
    dyq = (_bf16_fq(dyb, u) if qgrad else dyb).double()
    assert xd.grad.dtype == torch.float32 and wd.grad.dtype == torch.float32
    _check_bf16(xd.grad[rm.to(DEV)].bfloat16(), (dyq[rm] @ wq).numpy(), "dX")
    e_dw = oracle.rel_l2(wd.grad[rn.to(DEV)].cpu().numpy(), (dyq[:, rn].T @ xq).numpy())
    # autograd hands the backward dY cast to the output's dtype (bf16)
    e_db = oracle.rel_l2(bd.grad.cpu().numpy(), dyb.double().sum(0).numpy())
    print(f"  dW rel-L2 {e_dw:.3e}, db rel-L2 {e_db:.3e}", flush=True)
    assert e_dw <= 1e-5 and e_db <= 1e-6


def test_bf16_linear_backward_operands():
    """The quantized linear on bf16 tensors (the unified path with a bf16
    model): dX leaves the GEMM in bf16 and dW is the fp32 product of the
    bf16 operands, returned in the weight's dtype."""
    from axs.unified import hip_linear

    M, K, N = 128, 256, 96
    x = _gauss((M, K), 5).bfloat16()
    w = _gauss((N, K), 6, 0.1).bfloat16()
    dy = _gauss((M, N), 7).bfloat16()
    _, saved = hip_linear.forward_train(x.to(DEV), w.to(DEV), None, 32, True)
    dx, dw, db = hip_linear.backward(dy.to(DEV), saved, 32, False, True, True, True)
    assert dx.dtype == torch.bfloat16 and dw.dtype == torch.bfloat16
    xq = _bf16_fq(x).double()
    wq = _bf16_fq(w).double()
    _check_bf16(dx, (dy.double() @ wq).numpy(), "dX (bf16 linear)")
    _check_bf16(dw, (dy.double().T @ xq).numpy(), "dW (bf16 weight)")
    assert oracle.rel_l2(db.cpu().numpy(), dy.double().sum(0).numpy()) <= 1e-6


def test_mixed_precision_module_matches_function():
    import axs.unified as u

    torch.manual_seed(4)
    lin = u.AXSLinearMixedPrecision(128, 64, quantize_grad=False).to(DEV)
    x = _gauss((32, 128), 41)
    y = lin(x.to(DEV))
    assert y.dtype == torch.bfloat16 and y.shape == (32, 64)
    xq = _bf16_fq(x.bfloat16()).double()
    wq = _bf16_fq(lin.weight.detach().cpu().bfloat16()).double()
    exact = (xq @ wq.T + lin.bias.detach().cpu().bfloat16().double()).numpy()
    _check_bf16(y, exact, "module Y")
    y.float().sum().backward()
    assert lin.weight.grad.dtype == torch.float32
    assert torch.allclose(lin.bias.grad, torch.full_like(lin.bias.grad, 32.0))
    assert "mixed_precision=bf16" in repr(lin)
