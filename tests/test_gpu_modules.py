"""GPU behaviour of the drop-in modules and autograd ops against the oracle
(reference tests: tests/test_unified.py:258-496, tests/test_mixed_precision.py:63-142)."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
from conftest import bits_equal

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TOL = 1e-3


def gauss(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g) * scale


def test_ste_gradient_is_identity():
    import axs.unified as u

    x = gauss((8, 64), 1).to(DEV).requires_grad_(True)
    y = u.fake_quantize_unified(x, 32, "nearest")
    g = gauss((8, 64), 2).to(DEV)
    (gx,) = torch.autograd.grad(y, x, g)
    assert torch.equal(gx, g)
    # the reference's STE test: d/dx sum(2*FQ(x)) == 2
    x2 = gauss((4, 32), 3).to(DEV).requires_grad_(True)
    (u.fake_quantize_unified(x2) * 2).sum().backward()
    assert torch.all(x2.grad == 2.0)


@pytest.mark.parametrize("cls_name", ["AXSLinearUnified", "AXS6Linear"])
def test_linear_module_autograd_vs_oracle(cls_name):
    import axs.unified as u

    torch.manual_seed(0)
    lin = getattr(u, cls_name)(192, 96, bias=True, quantize_grad=False).to(DEV)
    x = gauss((5, 7, 192), 11).to(DEV).requires_grad_(True)
    y = lin(x)
    assert y.shape == (5, 7, 96)
    dy = gauss((5, 7, 96), 12)
    y.backward(dy.to(DEV))
    w = lin.weight.detach().cpu().numpy()
    xq = oracle.fake_quantize(x.detach().cpu().numpy().reshape(-1, 192), 32)
    wq = oracle.fake_quantize(w, 32)
    ref = oracle.linear_reference(xq, wq, lin.bias.detach().cpu().numpy())
    assert oracle.rel_l2(y.detach().cpu().numpy().reshape(-1, 96), ref) < TOL
    d = dy.numpy().reshape(-1, 96).astype(np.float64)
    assert oracle.rel_l2(x.grad.cpu().numpy().reshape(-1, 192), d @ wq) < TOL
    assert oracle.rel_l2(lin.weight.grad.cpu().numpy(), d.T @ xq) < TOL
    assert oracle.rel_l2(lin.bias.grad.cpu().numpy(), d.sum(0)) < 1e-5


def test_linear_module_quantized_grad():
    """dY is fake-quantized with the reference's +-0.5-LUT-step dither
    (quantize_unified.py:186-189), which only moves values next to a LUT cell
    boundary: each draw sits at the NF5 noise level of the exact gradient,
    draws differ, and their mean stays within that noise level."""
    import axs.unified as u

    torch.manual_seed(1)
    lin = u.AXSLinearUnified(256, 128, bias=False).to(DEV)
    x = gauss((64, 256), 21).to(DEV)
    dy = gauss((64, 128), 22).to(DEV)
    grads = []
    for _ in range(8):
        lin.weight.grad = None
        lin(x).backward(dy)
        grads.append(lin.weight.grad.clone())
    xq = oracle.fake_quantize(x.cpu().numpy(), 32).astype(np.float64)
    exact = dy.cpu().numpy().astype(np.float64).T @ xq
    nearest = oracle.fake_quantize(dy.cpu().numpy(), 32).astype(np.float64).T @ xq
    noise = oracle.rel_l2(nearest, exact)               # NF5 quantization noise of dY
    for g in grads:
        assert oracle.rel_l2(g.cpu().numpy(), exact) < 1.5 * noise
    assert not torch.equal(grads[0], grads[1])
    mean = torch.stack(grads).mean(0).cpu().numpy().astype(np.float64)
    assert oracle.rel_l2(mean, exact) < 1.5 * noise


def test_embedding_fake_quantizes_rows():
    import axs.unified as u

    torch.manual_seed(2)
    emb = u.AXSEmbeddingUnified(50, 64, padding_idx=0).to(DEV)
    idx = torch.randint(0, 50, (4, 9), device=DEV)
    out = emb(idx)
    raw = emb.weight.detach()[idx].cpu().numpy()
    assert bits_equal(out.detach().cpu().numpy(), oracle.fake_quantize(raw, 32))
    out.sum().backward()
    assert emb.weight.grad is not None


def test_attention_module_runs_and_backprops():
    import axs.unified as u

    torch.manual_seed(3)
    mha = u.AXSMultiheadAttentionUnified(128, 4).to(DEV)
    x = gauss((2, 16, 128), 31).to(DEV).requires_grad_(True)
    mask = torch.triu(torch.full((16, 16), float("-inf"), device=DEV), diagonal=1)
    y = mha(x, x, x, attn_mask=mask)
    assert y.shape == (2, 16, 128) and torch.isfinite(y).all()
    y.pow(2).mean().backward()
    assert torch.isfinite(x.grad).all() and mha.q_proj.weight.grad is not None


def test_convert_model_and_train_step():
    import axs.unified as u

    torch.manual_seed(5)
    model = nn.Sequential(nn.Linear(64, 128), nn.LayerNorm(128), nn.GELU(), nn.Linear(128, 10)).to(DEV)
    conv = u.convert_to_axs_unified(model)
    opt = torch.optim.AdamW(conv.parameters(), lr=1e-3)
    x = gauss((256, 64), 51).to(DEV)
    target = torch.randint(0, 10, (256,), device=DEV)
    losses = []
    for _ in range(30):
        opt.zero_grad()
        loss = nn.functional.cross_entropy(conv(x), target)
        loss.backward()
        opt.step()
        losses.append(loss.item())
    assert losses[-1] < losses[0] * 0.7, losses


def test_matmul_ops():
    import axs.unified as u

    a = gauss((3, 40, 96), 61).to(DEV)
    b = gauss((96, 72), 62).to(DEV)
    got = u.accelerated_matmul(a, b).cpu().numpy()
    assert oracle.rel_l2(got, a.cpu().numpy().astype(np.float64) @ b.cpu().numpy()) < TOL
    q = u.axs_matmul_unified(a[0], b).cpu().numpy()
    ref = oracle.fake_quantize(a[0].cpu().numpy(), 32).astype(np.float64) @ oracle.fake_quantize(b.cpu().numpy(), 32)
    assert oracle.rel_l2(q, ref) < TOL


def test_quantization_quality_matches_published_figures():
    """README.md:276-280 of the reference: 4096x4096 N(0,1), block 32 ->
    MSE 0.00077, SNR 31.2 dB."""
    import axs.unified as u

    torch.manual_seed(42)
    x = torch.randn(4096, 4096, device=DEV)
    st = u.quantization_error_unified(x, 32)
    assert abs(st["mse"] - 0.00077) < 0.00002, st
    assert abs(st["signal_to_noise_db"] - 31.2) < 0.1, st
