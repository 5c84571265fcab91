"""Seeded random sweep over the FQ, quantize/dequantize, wire and linear entry points:
shapes of 1-3 dims with row lengths from 1 to ~5000 values, the three input
dtypes, block sizes 8/16/32, nearest and stochastic rounding, and views that
start 0-7 elements into their buffer.  Each case lands on whichever kernel
the dispatch picks for it (whole-block vectors, row segments with four or one
value per lane, one block per lane group, the wire format's record tiles) and
is compared bit-exactly with the oracle, as the fixed-shape tests are; the
linear cases within rel-L2 1e-3 of the fp64 product of the oracle's FQ
operands."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from conftest import bits_equal, first_mismatch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
DTYPES = (torch.float32, torch.bfloat16, torch.float16)
N_CASES = 64


def _case(i: int):
    """Shape, dtype, block size, element offset and dither seed of case i."""
    rng = np.random.default_rng(1000 + i)
    dt = DTYPES[int(rng.integers(0, 3))]
    bs = (8, 16, 32)[int(rng.integers(0, 3))]
    kind = rng.random()
    if kind < 0.35:
        cols = bs * int(rng.integers(1, 160))                # whole blocks
    elif kind < 0.55:
        cols = 4 * int(rng.integers(16, 1200))               # four-value rows, ragged last block
    else:
        cols = int(np.exp(rng.uniform(0.0, np.log(5000.0))))
    rows = int(np.exp(rng.uniform(0.0, np.log(max(2, min(300, 300_000 // cols))))))
    lead = () if rng.random() < 0.2 else ((rows,) if rng.random() < 0.6 else (2, (rows + 1) // 2))
    shape = (*lead, cols) if lead else (cols,)
    off = int(rng.integers(0, 8)) if rng.random() < 0.5 else 0
    seed = int(rng.integers(1, 2**62)) if rng.random() < 0.4 else None
    return shape, dt, bs, off, seed, rng


def _values(shape, rng) -> np.ndarray:
    x = rng.standard_normal(shape).astype(np.float32)
    m = rng.random(shape) < 0.01
    x[m] *= 100.0
    if x.size > 8 and rng.random() < 0.3:
        flat = x.reshape(-1)
        idx = rng.choice(flat.size, size=4, replace=False)
        flat[idx] = np.array([0.0, -0.0, 1e-40, -2.0 ** -120], np.float32)
    return x


def _on_device(x: torch.Tensor, off: int) -> torch.Tensor:
    """x on the GPU as a view starting `off` elements into a larger buffer."""
    buf = torch.zeros(x.numel() + off, dtype=x.dtype, device=DEV)
    buf[off:] = x.reshape(-1).to(DEV)
    return buf[off:].view(x.shape)


def _label(i, shape, dt, bs, off, seed):
    return f"case {i}: shape={shape} {str(dt)[6:]} bs={bs} offset={off} seed={seed}"


@pytest.mark.parametrize("i", range(N_CASES))
def test_fake_quantize_sweep(i):
    from axs.unified.hip_kernels import hip_fused_fake_quantize

    shape, dt, bs, off, seed, rng = _case(i)
    print(f"[sweep fq {_label(i, shape, dt, bs, off, seed)}]", flush=True)
    x = torch.from_numpy(_values(shape, rng)).to(dt)
    xf = x.float().numpy().reshape(-1, shape[-1])
    rounding = "nearest" if seed is None else "stochastic"
    got = hip_fused_fake_quantize(_on_device(x, off), bs, rounding, seed=seed).cpu()
    u = None if seed is None else oracle.uniform(seed, 0, x.numel())
    want = torch.from_numpy(oracle.fake_quantize(xf, bs, u)).to(dt).reshape(shape)
    assert got.shape == x.shape and got.dtype == dt
    if dt == torch.float32:
        assert bits_equal(got.numpy(), want.numpy()), first_mismatch(got.numpy(), want.numpy())
    else:
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("i", range(N_CASES))
def test_quantize_dequantize_sweep(i):
    from axs.unified.hip_kernels import hip_dequantize, hip_quantize

    shape, dt, bs, off, seed, rng = _case(i)
    print(f"[sweep quantize {_label(i, shape, dt, bs, off, seed)}]", flush=True)
    x = torch.from_numpy(_values(shape, rng)).to(dt)
    cols = shape[-1]
    rows = x.numel() // cols
    xf = x.float().numpy().reshape(rows, cols)
    rounding = "nearest" if seed is None else "stochastic"
    e, c, s, fq = hip_quantize(_on_device(x, off), bs, rounding, with_fake_quantized=True, seed=seed)
    u = None if seed is None else oracle.uniform(seed, 0, x.numel())
    oe, oc, os_ = oracle.quantize(xf, bs, u)
    ge, gc, gs = (t.cpu().numpy().reshape(o.shape) for t, o in ((e, oe), (c, oc), (s, os_)))
    assert np.array_equal(ge, oe), first_mismatch(ge, oe)
    assert np.array_equal(gc, oc), first_mismatch(gc, oc)
    assert np.array_equal(gs, os_)
    want = torch.from_numpy(oracle.fake_quantize(xf, bs, u)).to(dt)
    got = fq.cpu().reshape(rows, cols)
    bits = torch.int32 if dt == torch.float32 else torch.int16
    assert torch.equal(got.view(bits), want.view(bits))
    d = hip_dequantize(e, c, s, rows, cols, bs).cpu().numpy().reshape(rows, cols)
    wd = oracle.dequantize(oe, oc, os_, cols, bs)
    assert bits_equal(d, wd), first_mismatch(d, wd)


@pytest.mark.parametrize("i", range(N_CASES))
def test_wire_sweep(i):
    """The 6.25-bit wire format through the C ABI, input and output views at
    the case's element offset: buffer bytes and unpacked values."""
    from axs import _lib

    shape, _, bs, off, _, rng = _case(i)
    print(f"[sweep wire {_label(i, shape, torch.float32, bs, off, None)}]", flush=True)
    x = torch.from_numpy(_values(shape, rng))
    cols = shape[-1]
    rows = x.numel() // cols
    xf = x.numpy().reshape(rows, cols)
    exps, codes, signs = oracle.quantize(xf, bs)
    want = oracle.wire_pack(exps, codes, signs)
    nbytes = _lib.lib().axs6_nf5_wire_bytes(rows, cols, bs)
    assert nbytes == want.size
    xd = _on_device(x, off)
    raw = torch.zeros(nbytes + 16, dtype=torch.uint8, device=DEV)
    st = _lib.stream_of(xd)
    _lib.call("axs6_nf5_pack_wire", xd.data_ptr(), _lib.F32, rows, cols, bs, raw[off:].data_ptr(), st)
    y = torch.zeros(x.numel() + off, device=DEV)
    _lib.call("axs6_nf5_unpack_wire", raw[off:].data_ptr(), rows, cols, bs, y[off:].data_ptr(), st)
    torch.cuda.synchronize()
    got = raw[off:off + nbytes].cpu().numpy()
    assert np.array_equal(got, want), first_mismatch(got, want)
    assert not raw[off + nbytes:].any() and not raw[:off].any()      # nothing written outside the buffer
    wd = oracle.dequantize(exps, codes, signs, cols, bs)
    yd = y[off:].cpu().numpy().reshape(rows, cols)
    assert bits_equal(yd, wd), first_mismatch(yd, wd)


def _linear_case(i: int):
    """M, K, N, block size, bias and dY rounding of linear case i: K and N
    mostly multiples of 4 (the kernels take them as they are, ragged last
    block included), sometimes not (padded first)."""
    rng = np.random.default_rng(5000 + i)
    M = int(np.exp(rng.uniform(0.0, np.log(600.0))))
    K, N = (int(4 * rng.integers(1, 750)) if rng.random() < 0.8 else int(rng.integers(1, 3000)) for _ in range(2))
    bs = (8, 16, 32)[int(rng.integers(0, 3))]
    return M, K, N, bs, bool(rng.random() < 0.7), bool(rng.random() < 0.5), rng


@pytest.mark.parametrize("i", range(32))
def test_linear_sweep(i):
    """Forward (training and no-grad paths) and backward of the quantized
    linear against the fp64 product of the oracle's FQ operands, rel-L2 within
    the north star's 1e-3 (db, a plain column sum, within 1e-5)."""
    from axs.unified import hip_linear

    M, K, N, bs, has_bias, qgrad, rng = _linear_case(i)
    print(f"[sweep linear case {i}: M={M} K={K} N={N} bs={bs} bias={has_bias} qgrad={qgrad}]", flush=True)
    x = torch.from_numpy(_values((M, K), rng))
    w = torch.from_numpy(rng.standard_normal((N, K)).astype(np.float32) * K ** -0.5)
    b = torch.from_numpy(rng.standard_normal(N).astype(np.float32)) if has_bias else None
    dy = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32))
    xq = oracle.fake_quantize(x.numpy(), bs).astype(np.float64)
    wq = oracle.fake_quantize(w.numpy(), bs).astype(np.float64)
    ref = xq @ wq.T + (0.0 if b is None else b.numpy().astype(np.float64))
    bd = None if b is None else b.to(DEV)
    y, saved = hip_linear.forward_train(x.to(DEV), w.to(DEV), bd, bs, True)
    assert y.shape == (M, N) and y.dtype == torch.float32
    assert oracle.rel_l2(y.cpu().numpy(), ref) < 1e-3
    y2 = hip_linear.linear_forward(x.to(DEV), w.to(DEV), bd, bs, True)
    assert oracle.rel_l2(y2.cpu().numpy(), ref) < 1e-3
    seed = 777 + i
    dx, dw, db = hip_linear.backward(dy.to(DEV), saved, bs, qgrad, True, True, has_bias, seed=seed)
    assert dx.shape == (M, K) and dw.shape == (N, K)
    if qgrad:
        # dY rows are zero-padded to whole 16-byte vectors (N4 columns) before
        # the draws, so element (m, n) takes counter m * N4 + n; the padding
        # zeros leave every block maximum unchanged
        n4 = -(-N // 4) * 4
        dyp = np.pad(dy.numpy(), ((0, 0), (0, n4 - N)))
        d2 = oracle.fake_quantize(dyp, bs, oracle.uniform(seed, 0, dyp.size))[:, :N].astype(np.float64)
    else:
        d2 = dy.numpy().astype(np.float64)
    assert oracle.rel_l2(dx.cpu().numpy(), d2 @ wq) < 1e-3
    assert oracle.rel_l2(dw.cpu().numpy(), d2.T @ xq) < 1e-3
    if has_bias:
        assert oracle.rel_l2(db.cpu().numpy(), d2.sum(0)) < 1e-5
