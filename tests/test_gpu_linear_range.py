"""Range limits of the linear's fp16 operands, and NaN / inf propagation.

The GEMM contracts operands packed as fp16 rows scaled by a power of two:
X and W rows by 2^-S with S the row's largest block exponent minus 15 (so
the row's largest value is <= 2^15), dY for dX by a row shift over
(exponent + the weight's row shift), dY for dW by one tensor-wide shift.
Each packed entry v of a row with shift S is therefore stored as v' with

    |v' - v| <= 2^-11 |v| + 2^(S - 25)

(11-bit rounding in fp16's normal range; below 2^(S - 14) the subnormal
spacing 2^(S - 24) takes over, and entries under 2^(S - 25) become zero).
An entry 2^30 below its row's largest block keeps ~5 bits; one 2^40 below
is flushed to zero.  These tests check every output of crafted wide-range
operands against the error bound that follows (plus fp32 accumulation),
and pin the flush itself: an output fed only by blocks 2^40 below their
row's largest is returned as 0.  (The fused small-output kernel contracts
fp32 FQ values and has no such limit.)

NaN / inf: a NaN anywhere in a block makes the block's FQ values NaN, an
infinite block scale makes them +-inf (0 * inf = NaN where the block holds
zeros) -- quantize_unified.py:167-197 -- and the contraction then spreads
them as fp32 IEEE arithmetic does; checked against numpy's fp64 product of
the oracle's FQ operands, position by position."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
BS = 32
U11 = 2.0 ** -11


def _block_e1(x: np.ndarray) -> np.ndarray:
    """e1 per block (rows, cols/32): floor(log2(amax)) + 1 for finite nonzero
    blocks with a finite scale, else a very small sentinel."""
    R, C = x.shape
    amax = np.abs(x).reshape(R, C // BS, BS).max(axis=2)
    ok = np.isfinite(amax) & (amax > 0)
    e1 = oracle.floor_log2(np.where(ok, amax, 1.0).astype(np.float32)).astype(np.int64) + 1
    ok &= e1 < 128
    return np.where(ok, e1, -(1 << 40))


def _row_shift(x: np.ndarray, colx: np.ndarray | None = None) -> np.ndarray:
    e1 = _block_e1(x)
    if colx is not None:
        e1 = e1 + colx.reshape(-1, BS).max(axis=1)[None, :]
    t = e1.max(axis=1)
    return np.where(t < -(1 << 39), 0, t - 15)


def _err(v: np.ndarray, shift: np.ndarray) -> np.ndarray:
    """The packing bound for entries v with per-entry shift (broadcast)."""
    return U11 * np.abs(v) + np.exp2(shift.astype(np.float64) - 25)


def _contract_bound(a, ea, b, eb):
    """Bound on |a' b'^T - a b^T| for a [M, K], b [N, K] with entry bounds ea, eb,
    plus fp32 accumulation (K * 2^-24 of the absolute sum)."""
    a, b = np.abs(a), np.abs(b)
    K = a.shape[1]
    return ea @ (b + eb).T + a @ eb.T + (K + 2) * 2.0 ** -24 * ((a + ea) @ (b + eb).T)


def _wide_rows(M, K, seed, span):
    """Gaussian rows whose blocks are scaled by 2^0 ... 2^-span (block j of
    row i by 2^(-span * ((i + j) % nb) / (nb - 1)))."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(np.float32)
    nb = K // BS
    i = np.arange(M)[:, None]
    j = np.arange(nb)[None, :]
    e = -np.round(span * ((i + j) % nb) / (nb - 1)).astype(np.int64)
    return (x.reshape(M, nb, BS) * np.exp2(e)[:, :, None]).reshape(M, K).astype(np.float32)


def test_forward_wide_rows_within_bound_and_flush():
    from axs.unified import hip_linear

    M, N, K = 96, 80, 512
    x = _wide_rows(M, K, 1, 44)
    w = _wide_rows(N, K, 2, 30) * np.float32(0.05)
    xq = oracle.fake_quantize(x, BS).astype(np.float64)
    wq = oracle.fake_quantize(w, BS).astype(np.float64)
    y, _ = hip_linear.forward_train(torch.from_numpy(x).to(DEV), torch.from_numpy(w).to(DEV), None, BS, True)
    got = y.cpu().numpy().astype(np.float64)
    exact = xq @ wq.T
    sx, sw = _row_shift(x), _row_shift(w)
    bound = _contract_bound(xq, _err(xq, sx[:, None]), wq, _err(wq, sw[:, None]))
    excess = np.abs(got - exact) - bound
    print(f"  max |error| / bound {np.max(np.abs(got - exact) / np.maximum(bound, 1e-300)):.3f}", flush=True)
    assert np.all(excess <= 0), f"{int((excess > 0).sum())} outputs outside the packing bound"

    # the flush: row 0's largest block is block 0; an output whose weight row
    # is zero there and sees only blocks >= 2^40 below it comes out 0
    xs = x.copy()
    xs[0, :BS] = 1.0
    xs[0, BS:] *= np.float32(2.0 ** -40) / np.abs(xs[0, BS:]).max()
    ws = w.copy()
    ws[0, :BS] = 0.0
    y2, _ = hip_linear.forward_train(torch.from_numpy(xs).to(DEV), torch.from_numpy(ws).to(DEV), None, BS, True)
    e2 = oracle.fake_quantize(xs, BS).astype(np.float64)[0] @ oracle.fake_quantize(ws, BS).astype(np.float64)[0]
    assert e2 != 0.0 and y2[0, 0].item() == 0.0


@pytest.mark.parametrize("qgrad", [False, True], ids=["exact_dy", "stochastic_dy"])
def test_backward_wide_dy_rows_within_bound(qgrad):
    """dY rows spanning 2^40 (the dW operand's tensor-wide shift flushes the
    smallest rows' contributions) and dY blocks spanning 2^40 within a row
    (the dX operand's row shift)."""
    from axs.unified import hip_linear

    M, N, K = 256, 96, 128
    rng = np.random.default_rng(3)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.1).astype(np.float32)
    dy = _wide_rows(M, N, 4, 40)
    dy *= np.exp2(-np.round(40 * np.arange(M) / (M - 1)))[:, None].astype(np.float32)
    _, saved = hip_linear.forward_train(torch.from_numpy(x).to(DEV), torch.from_numpy(w).to(DEV), None, BS, True)
    seed = 4242
    dx, dw, _ = hip_linear.backward(torch.from_numpy(dy).to(DEV), saved, BS, qgrad, True, True, False, seed=seed)
    xq = oracle.fake_quantize(x, BS).astype(np.float64)
    wq = oracle.fake_quantize(w, BS).astype(np.float64)
    dyq = (oracle.fake_quantize(dy, BS, oracle.uniform(seed, 0, dy.size)) if qgrad else dy).astype(np.float64)
    sx, sw = saved.sx.cpu().numpy(), saved.sw.cpu().numpy()
    assert np.array_equal(sx, _row_shift(x)) and np.array_equal(sw, _row_shift(w))
    # dX = dYq . Wq: A1[m, n] = dYq * 2^(sw[n] - t[m]), t[m] = max(e1 + sw) - 15
    t = _row_shift(dy, sw)
    e_dy = U11 * np.abs(dyq) + np.exp2(t[:, None] - sw[None, :] - 25.0)
    e_wq = _err(wq, sw[:, None])
    bound_dx = _contract_bound(dyq, e_dy, wq.T, e_wq.T)
    got_dx = dx.cpu().numpy().astype(np.float64)
    assert np.all(np.abs(got_dx - dyq @ wq) <= bound_dx), "dX outside the packing bound"
    # dW = dYq^T . Xq: A2T[n, m] = dYq * 2^(sx[m] - G), G = max_m(max e1 + sx[m]) - 15
    e1 = _block_e1(dy).max(axis=1)
    G = int(np.max(np.where(e1 < -(1 << 39), -(1 << 40), e1 + sx))) - 15
    e_dyw = U11 * np.abs(dyq) + np.exp2(G - sx[:, None] - 25.0)
    e_xq = _err(xq, sx[:, None])
    bound_dw = _contract_bound(dyq.T, e_dyw.T, xq.T, e_xq.T)
    got_dw = dw.cpu().numpy().astype(np.float64)
    assert np.all(np.abs(got_dw - dyq.T @ xq) <= bound_dw), "dW outside the packing bound"
    rel = oracle.rel_l2(got_dw, dyq.T @ xq)
    print(f"  dX rel-L2 {oracle.rel_l2(got_dx, dyq @ wq):.2e}, dW rel-L2 {rel:.2e}", flush=True)
    # the dW error stays at the fp16 rounding level: the rows it flushes are
    # the ones whose contributions are ~2^-30 of the largest
    assert rel < 1e-3


@pytest.mark.parametrize("path", ["packed", "fused"])
def test_nan_and_inf_propagate_like_the_fp32_product(path):
    from axs.unified import hip_linear

    M, N, K = 64, 48, 128
    rng = np.random.default_rng(7)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.1).astype(np.float32)
    x[3, 40] = np.nan                   # NaN block -> the whole FQ block is NaN
    x[5, 70] = np.inf                   # infinite scale: +-inf, and NaN at the zeros
    x[5, 71] = 0.0
    x[9, 100] = -np.inf                 # no zero in the block: +-inf only
    x[9, 96:128] = np.abs(x[9, 96:128]) + 1.0
    x[9, 100] = -np.inf
    w[7, 0] = np.nan
    w[11, 33] = np.inf
    xd, wd = torch.from_numpy(x).to(DEV), torch.from_numpy(w).to(DEV)
    y = hip_linear.forward_train(xd, wd, None, BS, True)[0] if path == "packed" else hip_linear.fused_forward(xd, wd)
    got = y.cpu().numpy().astype(np.float64)
    xq = oracle.fake_quantize(x, BS).astype(np.float64)
    wq = oracle.fake_quantize(w, BS).astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        want = xq @ wq.T
    assert np.array_equal(np.isnan(got), np.isnan(want)), "NaN positions differ"
    assert np.array_equal(np.isposinf(got), np.isposinf(want)) and np.array_equal(np.isneginf(got), np.isneginf(want))
    assert np.isnan(got[3]).all() and np.isnan(got[:, 7]).all()
    fin = np.isfinite(want)
    assert fin.sum() > 0.8 * fin.size
    assert oracle.rel_l2(got[fin], want[fin]) < (1e-3 if path == "packed" else 1e-5)
