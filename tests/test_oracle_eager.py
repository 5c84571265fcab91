"""The torch-eager restatement timed as the CPU baseline equals the C
oracle and the golden vectors bit for bit."""
from __future__ import annotations

import numpy as np
import torch

import oracle
from oracle import eager_torch
from conftest import bits_equal, load_golden


def test_eager_matches_golden_edges():
    g = load_golden("edge_cases.npz")
    x = torch.from_numpy(g["x"])
    for bs in (8, 16, 32):
        assert bits_equal(eager_torch.fake_quantize(x, bs).numpy(), g[f"fq_bs{bs}"])


def test_eager_matches_oracle_random():
    gen = torch.Generator().manual_seed(4)
    x = torch.randn(333, 257, generator=gen) * 3
    for bs in (8, 16, 32):
        assert bits_equal(eager_torch.fake_quantize(x, bs).numpy(), oracle.fake_quantize(x.numpy(), bs))


def test_eager_linear_shapes_and_values():
    gen = torch.Generator().manual_seed(5)
    x = torch.randn(64, 96, generator=gen)
    w = torch.randn(48, 96, generator=gen) / 10
    b = torch.randn(48, generator=gen)
    y, xq = eager_torch.linear_fwd(x, w, b)
    want = oracle.linear_reference(oracle.fake_quantize(x.numpy()), oracle.fake_quantize(w.numpy()), b.numpy())
    assert oracle.rel_l2(y.numpy(), want) < 1e-6
    dy = torch.randn(64, 48, generator=gen)
    dx, dw, db = eager_torch.linear_bwd(dy, xq, w, quantize_grad=False)
    assert dx.shape == x.shape and dw.shape == w.shape and db.shape == b.shape
    assert np.allclose(db.numpy(), dy.sum(0).numpy())


def test_eager_linear_backward_values_against_fp64():
    """dX = dYq . FQ(W) and dW = dYq^T . FQ(X) of the CPU restatement the
    MiniGPT parity test trains against, against fp64 products of the C
    oracle's operands (fp32 matmul: rel-L2 well under 1e-6)."""
    gen = torch.Generator().manual_seed(6)
    x = torch.randn(3, 40, 96, generator=gen)         # batched input, as in the model
    w = torch.randn(64, 96, generator=gen) / 10
    dy = torch.randn(3, 40, 64, generator=gen) * 5
    _, xq = eager_torch.linear_fwd(x, w, None)
    xq64 = oracle.fake_quantize(x.numpy()).reshape(-1, 96).astype(np.float64)
    wq64 = oracle.fake_quantize(w.numpy()).astype(np.float64)
    for quantize_grad in (False, True):
        torch.manual_seed(11)
        dx, dw, db = eager_torch.linear_bwd(dy, xq, w, quantize_grad=quantize_grad)
        if quantize_grad:
            # the stochastic FQ of dY draws torch.rand_like over the (rows, blocks, 32)
            # view; the same draws through the oracle give the same dYq
            torch.manual_seed(11)
            u = torch.rand(120, 2, 32).numpy()
            dyq = oracle.fake_quantize(dy.numpy(), 32, u)
        else:
            dyq = dy.numpy()
        dyq64 = dyq.reshape(-1, 64).astype(np.float64)
        assert dx.shape == x.shape and dw.shape == w.shape
        assert oracle.rel_l2(dx.numpy().reshape(-1, 96), dyq64 @ wq64) < 1e-6
        assert oracle.rel_l2(dw.numpy(), dyq64.T @ xq64) < 1e-6
        assert oracle.rel_l2(db.numpy(), dyq64.sum(0)) < 1e-6
