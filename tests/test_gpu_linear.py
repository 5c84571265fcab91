"""GPU parity of the quantized linear (fp16-MFMA GEMM on packed NF5
operands) against the fp64 product of the oracle's fake-quantized operands:
rel-L2 <= 1e-3 for outputs and gradients, plus exact
checks of the GEMM itself on fp16-representable inputs."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TOL = 1e-3   # rel-L2 tolerance of the north star for outputs and gradients


def gauss(shape, seed, scale=1.0, outliers=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * scale
    if outliers:
        m = torch.rand(*shape, generator=g) < 0.01
        x[m] *= 100.0
    return x


def _gemm(a16, b16, M, N, Kp, rexp=None, cexp=None, bias=None, out_dtype=torch.float32):
    from axs import _lib

    out = torch.empty((M, N), dtype=out_dtype, device=DEV)
    _lib.call("axs6_gemm_f16_nt", a16.data_ptr(), Kp, b16.data_ptr(), Kp, M, N, Kp, _lib.ptr(rexp),
              _lib.ptr(cexp), _lib.ptr(bias), out.data_ptr(), N, _lib.DTYPE_CODE[out_dtype],
              _lib.stream_of(a16))
    return out


# (2048, 768, 3072) and (1000, 200, 2112): small tiles with a long
# contraction (three K-slabs in flight)
@pytest.mark.parametrize("M,N,Kp", [(128, 128, 64), (256, 384, 512), (100, 72, 128), (1, 33, 64),
                                    (300, 260, 1024), (4096, 4096, 256), (2048, 768, 3072), (1000, 200, 2112)])
def test_gemm_exact_small_integers(M, N, Kp):
    # small integers are exact in fp16 and their products sum exactly in fp32
    g = torch.Generator().manual_seed(M * 7 + N)
    A = torch.randint(-8, 9, (M, Kp), generator=g).to(torch.float16)
    B = torch.randint(-8, 9, (N, Kp), generator=g).to(torch.float16)
    want = A.double() @ B.double().T
    got = _gemm(A.to(DEV), B.to(DEV), M, N, Kp).cpu().double()
    assert torch.equal(got, want), (got - want).abs().max()


def test_gemm_epilogue_exponents_bias_and_dtypes():
    M, N, Kp = 96, 160, 128
    g = torch.Generator().manual_seed(1)
    A = torch.randint(-4, 5, (M, Kp), generator=g).to(torch.float16)
    B = torch.randint(-4, 5, (N, Kp), generator=g).to(torch.float16)
    re = torch.randint(-20, 20, (M,), generator=g, dtype=torch.int32)
    ce = torch.randint(-20, 20, (N,), generator=g, dtype=torch.int32)
    bias = torch.randn(N, generator=g)
    acc = A.double() @ B.double().T
    want = (acc * torch.exp2((re[:, None] + ce[None, :]).double())).float() + bias
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        got = _gemm(A.to(DEV), B.to(DEV), M, N, Kp, re.to(DEV), ce.to(DEV), bias.to(DEV), dt).cpu()
        assert torch.equal(got, want.to(dt)), dt


@pytest.mark.parametrize("N,ldo,offset", [(161, 161, 0), (250, 256, 0), (256, 260, 1), (37, 40, 2)],
                         ids=["ragged_n", "strided", "misaligned_base", "narrow"])
def test_gemm_epilogue_ragged_and_strided_output(N, ldo, offset):
    # the staged epilogue writes 4 columns per lane: vector stores only where the
    # row segment is whole and aligned, element stores elsewhere; nothing may be
    # written outside [row, 0:N) of each output row
    from axs import _lib

    M, Kp = 300, 192
    g = torch.Generator().manual_seed(N + ldo)
    A = torch.randint(-4, 5, (M, Kp), generator=g).to(torch.float16)
    B = torch.randint(-4, 5, (N, Kp), generator=g).to(torch.float16)
    re = torch.randint(-10, 10, (M,), generator=g, dtype=torch.int32)
    ce = torch.randint(-10, 10, (N,), generator=g, dtype=torch.int32)
    bias = torch.randn(N, generator=g)
    acc = A.double() @ B.double().T
    want = (acc * torch.exp2((re[:, None] + ce[None, :]).double())).float() + bias
    # device copies held in names: the call is asynchronous and must not see freed temporaries
    Ad, Bd, red, ced, biasd = (t.to(DEV) for t in (A, B, re, ce, bias))
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        buf = torch.full((offset + M * ldo + 8,), 7.0, dtype=dt, device=DEV)
        _lib.call("axs6_gemm_f16_nt", Ad.data_ptr(), Kp, Bd.data_ptr(), Kp, M, N, Kp,
                  _lib.ptr(red), _lib.ptr(ced), _lib.ptr(biasd),
                  buf.data_ptr() + offset * buf.element_size(), ldo, _lib.DTYPE_CODE[dt], _lib.stream_of(buf))
        host = buf.cpu()
        out = host[offset:offset + M * ldo].view(M, ldo)
        assert torch.equal(out[:, :N], want.to(dt)), dt
        untouched = torch.cat([host[:offset], out[:, N:].reshape(-1), host[offset + M * ldo:]])
        assert bool((untouched == 7.0).all()), f"{dt}: wrote outside the output rows"


@pytest.mark.parametrize("M,N", [(8192, 11008), (11008, 2048)], ids=["column_cut", "row_cut"])
def test_gemm_tail_cut_exact(M, N):
    """Outputs whose 256x256 tiles leave a small last round run as two
    launches (a multiple of 256 tiles, then the remainder with smaller
    tiles), cut along columns (8192 x 11008) or rows (11008 x 2048); the
    exponents, bias and output pointers of the second part are offsets of
    the first's.  Exact on small integers, every element checked."""
    Kp = 64
    g = torch.Generator().manual_seed(M + N)
    A = torch.randint(-4, 5, (M, Kp), generator=g).to(torch.float16)
    B = torch.randint(-4, 5, (N, Kp), generator=g).to(torch.float16)
    re = torch.randint(-6, 6, (M,), generator=g, dtype=torch.int32)
    ce = torch.randint(-6, 6, (N,), generator=g, dtype=torch.int32)
    bias = torch.randint(-8, 9, (N,), generator=g).float()
    want = ((A.double() @ B.double().T) * torch.exp2((re[:, None] + ce[None, :]).double())).float() + bias
    got = _gemm(A.to(DEV), B.to(DEV), M, N, Kp, re.to(DEV), ce.to(DEV), bias.to(DEV)).cpu()
    assert torch.equal(got, want)


def _oracle_linear(x, w, b):
    xq = oracle.fake_quantize(x.numpy(), 32)
    wq = oracle.fake_quantize(w.numpy(), 32)
    return xq, wq, oracle.linear_reference(xq, wq, None if b is None else b.numpy())


# K 20000 (f32) is past the row pack's register-resident length: statistics
# pass + tiled pack
@pytest.mark.parametrize("M,K,N", [(64, 256, 128), (100, 96, 64), (2048, 768, 3072), (2048, 3072, 768),
                                   (4096, 4096, 4096), (64, 20000, 96)])
def test_linear_forward_vs_oracle(M, K, N):
    from axs.unified import hip_linear

    print(f"[linear fwd {M}x{K}x{N}]", flush=True)
    x = gauss((M, K), 11, outliers=True)
    w = gauss((N, K), 12, scale=K ** -0.5)
    b = gauss((N,), 13)
    _, _, ref = _oracle_linear(x, w, b)
    y = hip_linear.linear_forward(x.to(DEV), w.to(DEV), b.to(DEV), 32, True).cpu().numpy()
    err = oracle.rel_l2(y, ref)
    print(f"  rel-L2 {err:.3e}", flush=True)
    assert err < TOL


@pytest.mark.parametrize("M,K,N", [(8192, 4096, 11008), (8192, 11008, 4096)])
def test_linear_forward_config4_rows(M, K, N):
    """Full-size forward; the fp64 reference is evaluated on 256 sampled rows."""
    from axs.unified import hip_linear

    print(f"[linear fwd {M}x{K}x{N}]", flush=True)
    x = gauss((M, K), 21, outliers=True)
    w = gauss((N, K), 22, scale=K ** -0.5)
    y = hip_linear.linear_forward(x.to(DEV), w.to(DEV), None, 32, True)
    rows = torch.randperm(M, generator=torch.Generator().manual_seed(0))[:256]
    xq = oracle.fake_quantize(x[rows].numpy(), 32)
    wq = oracle.fake_quantize(w.numpy(), 32)
    err = oracle.rel_l2(y[rows.to(DEV)].cpu().numpy(), oracle.linear_reference(xq, wq))
    print(f"  rel-L2 {err:.3e}", flush=True)
    assert err < TOL


# Three shapes run split-K GEMMs: dW of one 256x256 tile over 128 K-steps (32
# splits); dW over a ragged 5000-row contraction (16 uneven splits); dX of one
# tile over a 4096-wide contraction (16 splits).  K 20000 packs its forward
# operands in two passes (rows past the register-resident length).
@pytest.mark.parametrize("M,K,N", [(64, 256, 128), (100, 96, 64), (2048, 768, 3072), (2048, 3072, 768),
                                   (8192, 256, 256), (5000, 160, 96), (256, 256, 4096), (96, 20000, 64)])
@pytest.mark.parametrize("qgrad", [False, True], ids=["exact_dy", "stochastic_dy"])
def test_linear_backward_vs_oracle(M, K, N, qgrad):
    from axs.unified import hip_linear

    print(f"[linear bwd {M}x{K}x{N} qgrad={qgrad}]", flush=True)
    x = gauss((M, K), 31, outliers=True)
    w = gauss((N, K), 32, scale=K ** -0.5)
    b = gauss((N,), 33)
    dy = gauss((M, N), 34)
    xq, wq, _ = _oracle_linear(x, w, b)
    _, saved = hip_linear.forward_train(x.to(DEV), w.to(DEV), b.to(DEV), 32, True)
    seed = 987654321
    dx, dw, db = hip_linear.backward(dy.to(DEV), saved, 32, qgrad, True, True, True, seed=seed)
    dyq = oracle.fake_quantize(dy.numpy(), 32, oracle.uniform(seed, 0, dy.numel())) if qgrad else dy.numpy()
    dx_ref = dyq.astype(np.float64) @ wq.astype(np.float64)
    dw_ref = dyq.astype(np.float64).T @ xq.astype(np.float64)
    db_ref = dyq.astype(np.float64).sum(0)
    e = (oracle.rel_l2(dx.cpu().numpy(), dx_ref), oracle.rel_l2(dw.cpu().numpy(), dw_ref),
         oracle.rel_l2(db.cpu().numpy(), db_ref))
    print(f"  rel-L2 dX {e[0]:.3e} dW {e[1]:.3e} db {e[2]:.3e}", flush=True)
    assert e[0] < TOL and e[1] < TOL and e[2] < 1e-5


@pytest.mark.parametrize("M,K,N", [(8192, 4096, 11008), (8192, 11008, 4096)])
def test_linear_backward_config4_sampled(M, K, N):
    """Full-size fwd+bwd with stochastic dY; dX checked on 128 sampled rows,
    dW on 128 sampled rows, db in full."""
    from axs.unified import hip_linear

    print(f"[linear bwd {M}x{K}x{N}]", flush=True)
    x = gauss((M, K), 41)
    w = gauss((N, K), 42, scale=K ** -0.5)
    dy = gauss((M, N), 43)
    _, saved = hip_linear.forward_train(x.to(DEV), w.to(DEV), None, 32, True)
    seed = 1234
    dx, dw, db = hip_linear.backward(dy.to(DEV), saved, 32, True, True, True, True, seed=seed)
    dyq = oracle.fake_quantize(dy.numpy(), 32, oracle.uniform(seed, 0, dy.numel())).astype(np.float64)
    g = torch.Generator().manual_seed(5)
    rm = torch.randperm(M, generator=g)[:128].numpy()
    rn = torch.randperm(N, generator=g)[:128].numpy()
    wq = oracle.fake_quantize(w.numpy(), 32).astype(np.float64)
    xq = oracle.fake_quantize(x.numpy(), 32).astype(np.float64)
    e_dx = oracle.rel_l2(dx.cpu().numpy()[rm], dyq[rm] @ wq)
    e_dw = oracle.rel_l2(dw.cpu().numpy()[rn], dyq[:, rn].T @ xq)
    e_db = oracle.rel_l2(db.cpu().numpy(), dyq.sum(0))
    print(f"  rel-L2 dX {e_dx:.3e} dW {e_dw:.3e} db {e_db:.3e}", flush=True)
    assert e_dx < TOL and e_dw < TOL and e_db < 1e-5


@pytest.mark.parametrize("need", [(False, False, True), (False, True, True), (True, False, True), (True, True, False)],
                         ids=["db", "dw_db", "dx_db", "dx_dw"])
def test_linear_backward_gradient_subsets(need):
    """Each subset of (dX, dW, db): the bias reduction runs inside the
    operand-transpose launch, or alone when nothing is transposed."""
    from axs.unified import hip_linear

    M, K, N = 300, 160, 96
    x = gauss((M, K), 41, outliers=True)
    w = gauss((N, K), 42, scale=K ** -0.5)
    b = gauss((N,), 43)
    dy = gauss((M, N), 44)
    xq, wq, _ = _oracle_linear(x, w, b)
    _, saved = hip_linear.forward_train(x.to(DEV), w.to(DEV), b.to(DEV), 32, True)
    dx, dw, db = hip_linear.backward(dy.to(DEV), saved, 32, False, *need)
    d = dy.numpy().astype(np.float64)
    for got, want, on in ((dx, d @ wq.astype(np.float64), need[0]), (dw, d.T @ xq.astype(np.float64), need[1]),
                          (db, d.sum(0), need[2])):
        assert (got is None) == (not on)
        if on:
            assert oracle.rel_l2(got.cpu().numpy(), want) < (1e-5 if got.dim() == 1 else TOL)


def test_linear_ragged_and_3d():
    from axs.unified import hip_linear

    x = gauss((3, 7, 50), 51)
    w = gauss((70, 50), 52, scale=0.2)
    b = gauss((70,), 53)
    xq, wq, ref = _oracle_linear(x.reshape(-1, 50), w, b)
    y, saved = hip_linear.forward_train(x.to(DEV), w.to(DEV), b.to(DEV), 32, True)
    assert y.shape == (3, 7, 70)
    assert oracle.rel_l2(y.reshape(-1, 70).cpu().numpy(), ref) < TOL
    dy = gauss((3, 7, 70), 54)
    dx, dw, db = hip_linear.backward(dy.to(DEV), saved, 32, False, True, True, True)
    d2 = dy.reshape(-1, 70).numpy().astype(np.float64)
    assert dx.shape == x.shape and dw.shape == w.shape and db.shape == b.shape
    assert oracle.rel_l2(dx.reshape(-1, 50).cpu().numpy(), d2 @ wq) < TOL
    assert oracle.rel_l2(dw.cpu().numpy(), d2.T @ xq) < TOL


@pytest.mark.parametrize("bs", [8, 16])
def test_linear_small_blocks(bs):
    from axs.unified import hip_linear

    x = gauss((96, 128), 61)
    w = gauss((64, 128), 62, scale=0.1)
    xq = oracle.fake_quantize(x.numpy(), bs)
    wq = oracle.fake_quantize(w.numpy(), bs)
    y = hip_linear.linear_forward(x.to(DEV), w.to(DEV), None, bs, True)
    assert oracle.rel_l2(y.cpu().numpy(), oracle.linear_reference(xq, wq)) < TOL


def test_linear_bf16_inputs():
    from axs.unified import hip_linear

    x = gauss((128, 256), 71).bfloat16()
    w = (gauss((192, 256), 72) / 16).bfloat16()
    y = hip_linear.linear_forward(x.to(DEV), w.to(DEV), None, 32, True)
    assert y.dtype == torch.bfloat16
    xq = oracle.fake_quantize(x.float().numpy(), 32)
    wq = oracle.fake_quantize(w.float().numpy(), 32)
    assert oracle.rel_l2(y.float().cpu().numpy(), oracle.linear_reference(xq, wq)) < 5e-3


def test_linear_without_input_quantization():
    from axs.unified import hip_linear

    x = gauss((64, 128), 81)
    w = gauss((32, 128), 82, scale=0.1)
    y = hip_linear.linear_forward(x.to(DEV), w.to(DEV), None, 32, False)
    ref = oracle.linear_reference(x.numpy(), oracle.fake_quantize(w.numpy(), 32))
    assert oracle.rel_l2(y.cpu().numpy(), ref) < TOL


def test_matmul_vs_float64():
    from axs.unified import hip_linear

    a = gauss((5, 33, 70), 91)
    b = gauss((70, 45), 92)
    got = hip_linear.matmul(a.to(DEV), b.to(DEV)).cpu().numpy()
    want = a.numpy().astype(np.float64) @ b.numpy().astype(np.float64)
    assert got.shape == (5, 33, 45)
    assert oracle.rel_l2(got, want) < TOL


# K and N that are multiples of 4 (f32) / 8 (bf16) but not of the block size
# go to the kernels as they are (a ragged last NF5 block, zero-padded by the
# kernels; K = 20004 takes the two-pass pack of long rows); other lengths are
# padded to such a multiple first (K 50, N 70).
@pytest.mark.parametrize("M,K,N", [(64, 100, 100), (96, 1004, 36), (33, 20004, 44), (70, 50, 70)], ids=str)
@pytest.mark.parametrize("qgrad", [False, True], ids=["exact_dy", "stochastic_dy"])
def test_linear_ragged_k_n(M, K, N, qgrad):
    from axs.unified import hip_linear

    print(f"[linear ragged {M}x{K}x{N} qgrad={qgrad}]", flush=True)
    x = gauss((M, K), 41, outliers=True)
    w = gauss((N, K), 42, scale=K ** -0.5)
    b = gauss((N,), 43)
    dy = gauss((M, N), 44)
    xq, wq, ref = _oracle_linear(x, w, b)
    y, saved = hip_linear.forward_train(x.to(DEV), w.to(DEV), b.to(DEV), 32, True)
    assert y.shape == (M, N) and y.is_contiguous()
    assert oracle.rel_l2(y.cpu().numpy(), ref) < TOL
    seed = 24680
    dx, dw, db = hip_linear.backward(dy.to(DEV), saved, 32, qgrad, True, True, True, seed=seed)
    assert dx.shape == (M, K) and dw.shape == (N, K) and db.shape == (N,)
    dyq = oracle.fake_quantize(dy.numpy(), 32, oracle.uniform(seed, 0, dy.numel())) if qgrad else dy.numpy()
    d2 = dyq.astype(np.float64)
    if N % 4 == 0:
        # dY goes to the kernels unpadded: the stochastic draws follow its own layout
        assert oracle.rel_l2(dx.cpu().numpy(), d2 @ wq.astype(np.float64)) < TOL
        assert oracle.rel_l2(dw.cpu().numpy(), d2.T @ xq.astype(np.float64)) < TOL
        assert oracle.rel_l2(db.cpu().numpy(), d2.sum(0)) < 1e-5
    elif not qgrad:
        assert oracle.rel_l2(dx.cpu().numpy(), d2 @ wq.astype(np.float64)) < TOL
        assert oracle.rel_l2(dw.cpu().numpy(), d2.T @ xq.astype(np.float64)) < TOL


@pytest.mark.parametrize("K,N", [(1000, 1000), (1004, 40)], ids=["k1000", "k1004_padded"])
def test_linear_bf16_ragged_k(K, N):
    from axs.unified import hip_linear

    x = gauss((64, K), 75).bfloat16()
    w = (gauss((N, K), 76) / 16).bfloat16()
    y = hip_linear.linear_forward(x.to(DEV), w.to(DEV), None, 32, True)
    assert y.dtype == torch.bfloat16 and y.shape == (64, N)
    xq = oracle.fake_quantize(x.float().numpy(), 32)
    wq = oracle.fake_quantize(w.float().numpy(), 32)
    assert oracle.rel_l2(y.float().cpu().numpy(), oracle.linear_reference(xq, wq)) < 5e-3
