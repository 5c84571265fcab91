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
