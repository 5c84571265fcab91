"""The single-launch fused linear (``axs6_nf5_fused_linear``): NF5 FQ of
each 32-wide K tile as it is loaded and an fp32 contraction, the
reference's ``triton_fused_linear`` / ``_nf5_fq_linear_kernel``
(triton_kernels.py:185-282,385-482 in the reference), which its
``accelerated_linear`` selects for M*N <= 128K outputs.

Bar: the products are those of the fp32 FQ values, so against the fp64
product of the C oracle's FQ operands rel-L2 <= 1e-5 (fp32 accumulation;
measured ~1e-7).  16-bit inputs: the FQ of the 16-bit values stays fp32 and
only Y is rounded, as in the reference's fused kernel: >= 99% of Y
bit-identical to the exact result rounded to the dtype, the rest one ulp
(fp32 accumulation order)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TOL = 1e-5


def _inputs(lead, K, N, seed, outliers=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*lead, K, generator=g)
    if outliers:
        x[torch.rand(*lead, K, generator=g) < 0.01] *= 100.0
    w = torch.randn(N, K, generator=g) * K ** -0.5
    b = torch.randn(N, generator=g)
    return x, w, b


def _exact(x, w, b, quantize_input=True):
    K = x.shape[-1]
    x2 = x.reshape(-1, K).float().numpy()
    xq = oracle.fake_quantize(x2, 32) if quantize_input else x2
    wq = oracle.fake_quantize(w.float().numpy(), 32)
    y = oracle.linear_reference(xq, wq, None if b is None else b.float().numpy())
    return y.reshape(*x.shape[:-1], w.shape[0])


# decode-like (M 1..32, K = N = 4096), square-ish, wide/short, ragged N and K
@pytest.mark.parametrize("lead,K,N", [((1,), 4096, 4096), ((7,), 4096, 4096), ((8,), 4096, 4096),
                                      ((16,), 2048, 1024), ((16,), 8192, 512), ((32,), 4096, 4096),
                                      ((128,), 1024, 1024), ((256,), 512, 512), ((362,), 4096, 362),
                                      ((64,), 256, 2048), ((512,), 4096, 256), ((5,), 96, 13), ((3, 7), 160, 33),
                                      ((2, 4, 8), 32, 64),
                                      # the MFMA decode form's largest LDS stagings: 16 x (2208 + 4),
                                      # 8 x (4096 + 4) and 1 x (35552 + 4) floats, just under its
                                      # 139 KiB (159.3 KiB with the static LDS); 16 x 2240 is the first
                                      # shape past it
                                      ((16,), 2208, 1024), ((16,), 2240, 1024), ((8,), 4096, 2048),
                                      ((1,), 35552, 64)])
def test_fused_linear_f32_vs_fp64(lead, K, N):
    from axs.unified import hip_linear

    print(f"[fused linear {lead} K={K} N={N}]", flush=True)
    x, w, b = _inputs(lead, K, N, K + N)
    y = hip_linear.fused_forward(x.to(DEV), w.to(DEV), b.to(DEV))
    assert y.shape == (*lead, N) and y.dtype == torch.float32
    err = oracle.rel_l2(y.cpu().numpy(), _exact(x, w, b))
    print(f"  rel-L2 {err:.2e}", flush=True)
    assert err <= TOL


# The streamed decode form (M <= 2, FQ(X) within 48 KiB of LDS): one weight
# row per wave, or two waves per row (K split) for short or very tall weights;
# K not a multiple of its 512-value step, a single partial step, rows past N
# in the last workgroup, zeros in W and X (the masked magnitudes), the largest
# contractions it takes (M 1: 12288, M 2: 6144) and the first it leaves to
# the MFMA form.
@pytest.mark.parametrize("m,K,N", [(1, 4096, 4096), (2, 4096, 4096), (1, 4096, 1024), (2, 4096, 1024),
                                   (1, 4000, 4000), (2, 544, 4097), (1, 32, 7), (2, 96, 13), (1, 8192, 6500),
                                   (1, 12288, 300), (2, 6144, 300), (1, 12320, 64), (2, 6176, 64), (1, 1024, 1)])
def test_fused_linear_decode_form(m, K, N):
    from axs.unified import hip_linear

    print(f"[fused decode m={m} K={K} N={N}]", flush=True)
    x, w, b = _inputs((m,), K, N, 3 * K + N)
    w[:, 5::7] = 0.0                  # zeros inside blocks
    w[N // 2, :] = 0.0                # a zero row
    x[:, : K // 4] = 0.0              # a zero run of X
    y = hip_linear.fused_forward(x.to(DEV), w.to(DEV), b.to(DEV))
    err = oracle.rel_l2(y.cpu().numpy(), _exact(x, w, b))
    print(f"  rel-L2 {err:.2e}", flush=True)
    assert err <= TOL
    # repeat: same bits (fixed reduction order)
    assert torch.equal(hip_linear.fused_forward(x.to(DEV), w.to(DEV), b.to(DEV)), y)


@pytest.mark.parametrize("m", [1, 2, 3, 20])
def test_fused_linear_special_blocks(m):
    """Blocks the short FQ sequence does not cover take the general one
    (m 1, 2: the decode form's per-step fallback; m 3: the MFMA form; m 20:
    the two-launch path, X arranged first): a NaN
    block (the whole row's output NaN), an inf block, a row of 1e-33 values
    (every block's e1 below -100), a row scaled by 1e30, a block with
    subnormals beside normal values."""
    from axs.unified import hip_linear

    K, N = 2048, 1024
    x, w, b = _inputs((m,), K, N, 77, outliers=False)
    w[3, 100] = float("nan")
    w[4, 64:96] = w[4, 64:96].abs()
    w[4, 70] = float("inf")
    w[5] *= 1e-33
    w[6] *= 1e30
    w[7, 0:32] = 1e-41
    w[7, 3] = 0.5
    y = hip_linear.fused_forward(x.to(DEV), w.to(DEV), b.to(DEV)).cpu().numpy().astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):   # the NaN and inf blocks' products
        want = _exact(x, w, b)
    assert np.array_equal(np.isnan(y), np.isnan(want)), (np.isnan(y).sum(), np.isnan(want).sum())
    assert np.array_equal(np.isinf(y), np.isinf(want))
    assert np.array_equal(np.sign(y[np.isinf(y)]), np.sign(want[np.isinf(want)]))
    assert np.isnan(y[:, 3]).all()
    fin = np.isfinite(want).all(axis=0)
    for c in (5, 6, 7):                # the special rows, each against its own scale
        assert fin[c] and oracle.rel_l2(y[:, c], want[:, c]) <= TOL, c
    assert oracle.rel_l2(y[:, fin], want[:, fin]) <= TOL


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [1, 2, 3, 20])
def test_fused_linear_special_blocks_16bit(dt, m):
    """The same special blocks with 16-bit operands (FQ of the upcast values,
    Y rounded to the dtype): a NaN block, an inf block, a row far above and a
    row far below unit scale (f16: within its range), subnormals beside normal
    values."""
    from axs.unified import hip_linear

    K, N = 2048, 1024
    x, w, b = _inputs((m,), K, N, 78, outliers=False)
    big, small, sub = (1e30, 1e-33, 1e-41) if dt == torch.bfloat16 else (1e3, 1e-3, 1e-7)
    w[3, 100] = float("nan")
    w[4, 64:96] = w[4, 64:96].abs()
    w[4, 70] = float("inf")
    w[5] *= small
    w[6] *= big
    w[7, 0:32] = sub
    w[7, 3] = 0.5
    x, w = x.to(dt), w.to(dt)
    y = hip_linear.fused_forward(x.to(DEV), w.to(DEV), b.to(DEV)).cpu()
    assert y.dtype == dt
    y = y.double().numpy()
    with np.errstate(invalid="ignore", over="ignore"):
        want = _exact(x.float(), w.float(), b)
    assert np.array_equal(np.isnan(y), np.isnan(want)), (np.isnan(y).sum(), np.isnan(want).sum())
    assert np.array_equal(np.isinf(y), np.isinf(want))
    assert np.isnan(y[:, 3]).all()
    fin = np.isfinite(want).all(axis=0)
    tol = 4e-3 if dt == torch.bfloat16 else 5e-4
    for c in (5, 6, 7):
        assert fin[c] and oracle.rel_l2(y[:, c], want[:, c]) <= tol, c
    assert oracle.rel_l2(y[:, fin], want[:, fin]) <= tol


@pytest.mark.parametrize("m,K,N", [(9, 4096, 4096), (16, 4096, 4096), (32, 4096, 4096), (64, 2048, 512),
                                   (17, 2080, 300), (40, 8192, 64), (128, 1024, 1024), (200, 1056, 100)])
def test_fused_linear_split_x_is_bit_identical(m, K, N):
    """Where the library advises it (axs6_nf5_fused_linear_split_x: K >= 1024,
    X past both LDS stagings), fused_forward takes the two-launch entry: FQ(X)
    once into the contraction's read order (rows past M zero to the 16-row
    block), then the contraction on it.  The output equals the single launch
    bit for bit, and the oracle's fp64 product to the usual bar; so does the
    entry with quantize_input 0 (X arranged as given)."""
    from axs import _lib
    from axs.unified import hip_linear

    print(f"[fused split m={m} K={K} N={N}]", flush=True)
    x, w, b = _inputs((m,), K, N, 5 * K + m)
    assert _lib.lib().axs6_nf5_fused_linear_split_x(m, N, K, _lib.F32) == 1
    y = hip_linear.fused_forward(x.to(DEV), w.to(DEV), b.to(DEV))
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    st = torch.cuda.current_stream().cuda_stream
    for qx in (1, 0):
        one = torch.empty(m, N, device=DEV)
        _lib.call("axs6_nf5_fused_linear", xd.data_ptr(), wd.data_ptr(), bd.data_ptr(), one.data_ptr(), _lib.F32,
                  m, N, K, 32, qx, st)
        if qx:
            assert torch.equal(y, one)
        # a workspace of NaNs: every word the contraction reads is written first
        xa = torch.full((_lib.lib().axs6_nf5_fused_linear_split_workspace(m, K) // 4,), float("nan"), device=DEV)
        two = torch.empty(m, N, device=DEV)
        _lib.call("axs6_nf5_fused_linear_split", xd.data_ptr(), wd.data_ptr(), bd.data_ptr(), two.data_ptr(),
                  xa.data_ptr(), _lib.F32, m, N, K, 32, qx, st)
        assert torch.equal(two, one), qx
    assert oracle.rel_l2(y.cpu().numpy(), _exact(x, w, b)) <= TOL


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("m,K,N", [(512, 1024, 1024), (512, 64, 1024), (256, 512, 1024), (256, 128, 1024),
                                   (64, 256, 512), (16, 256, 256), (48, 32, 40)])
def test_fused_linear_split_entry_every_tiling(m, K, N, dt):
    """axs6_nf5_fused_linear_split called directly, at shapes the advice never
    picks, so that each tiling of the MFMA form runs on arranged X: 32 x 64
    tiles (4 K-splitting waves, then 1), 32 x 32 (8, then 2), 32 x 16 with 4
    waves, 16 x 16 with 4, and a single K tile; f32 and bf16 weights (two
    16-byte loads per lane and tile, or one).  Bit-identical to the single
    launch, which takes the same tiling; both against the fp64 product (the
    64- and 128-thread tilings once staged only part of the FQ tables)."""
    from axs import _lib

    print(f"[fused split entry {dt} m={m} K={K} N={N}]", flush=True)
    x, w, b = _inputs((m,), K, N, 11 * K + m)
    x, w = x.to(dt), w.to(dt)
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    code = _lib.DTYPE_CODE[dt]
    st = torch.cuda.current_stream().cuda_stream
    one = torch.empty(m, N, device=DEV, dtype=dt)
    _lib.call("axs6_nf5_fused_linear", xd.data_ptr(), wd.data_ptr(), bd.data_ptr(), one.data_ptr(), code, m, N, K,
              32, 1, st)
    xa = torch.full((_lib.lib().axs6_nf5_fused_linear_split_workspace(m, K) // 4,), float("nan"), device=DEV)
    two = torch.empty(m, N, device=DEV, dtype=dt)
    _lib.call("axs6_nf5_fused_linear_split", xd.data_ptr(), wd.data_ptr(), bd.data_ptr(), two.data_ptr(),
              xa.data_ptr(), code, m, N, K, 32, 1, st)
    exact = _exact(x.float(), w.float(), b)
    assert oracle.rel_l2(one.float().cpu().numpy(), exact) <= (TOL if dt == torch.float32 else 4e-3)
    assert torch.equal(two, one)


@pytest.mark.parametrize("m", [1, 2])
def test_fused_linear_split_entry_streamed_rows(m):
    """At one and two rows the single launch streams the weight (VALU
    products, per-lane partial sums), so the split entry's MFMA contraction
    agrees with it to fp32 rounding rather than bit for bit: both against the
    fp64 product to the usual bar."""
    from axs import _lib

    K, N = 4096, 1024
    x, w, b = _inputs((m,), K, N, 13 * m)
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    st = torch.cuda.current_stream().cuda_stream
    one = torch.empty(m, N, device=DEV)
    _lib.call("axs6_nf5_fused_linear", xd.data_ptr(), wd.data_ptr(), bd.data_ptr(), one.data_ptr(), _lib.F32, m, N,
              K, 32, 1, st)
    xa = torch.full((_lib.lib().axs6_nf5_fused_linear_split_workspace(m, K) // 4,), float("nan"), device=DEV)
    two = torch.empty(m, N, device=DEV)
    _lib.call("axs6_nf5_fused_linear_split", xd.data_ptr(), wd.data_ptr(), bd.data_ptr(), two.data_ptr(),
              xa.data_ptr(), _lib.F32, m, N, K, 32, 1, st)
    exact = _exact(x, w, b)
    assert oracle.rel_l2(one.cpu().numpy(), exact) <= TOL
    assert oracle.rel_l2(two.cpu().numpy(), exact) <= TOL


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,K,N", [(16, 4096, 4096), (40, 2048, 200), (33, 4096, 1024)])
def test_fused_linear_split_16bit_is_bit_identical(dt, m, K, N):
    """16-bit inputs take the two-launch path too: the arranged FQ(X) is f32,
    the values the single launch computes from the 16-bit X, so Y (rounded
    to the input's dtype) equals the single launch's bit for bit."""
    from axs import _lib
    from axs.unified import hip_linear

    print(f"[fused split {dt} m={m} K={K} N={N}]", flush=True)
    x, w, b = _inputs((m,), K, N, 7 * K + m)
    xd, wd, bd = x.to(DEV, dt), w.to(DEV, dt), b.to(DEV)
    code = _lib.DTYPE_CODE[dt]
    assert _lib.lib().axs6_nf5_fused_linear_split_x(m, N, K, code) == 1
    y = hip_linear.fused_forward(xd, wd, bd)
    one = torch.empty(m, N, device=DEV, dtype=dt)
    _lib.call("axs6_nf5_fused_linear", xd.data_ptr(), wd.data_ptr(), bd.data_ptr(), one.data_ptr(), code, m, N, K,
              32, 1, torch.cuda.current_stream().cuda_stream)
    assert y.dtype == dt and torch.equal(y, one)
    ref = _exact(xd.float().cpu(), wd.float().cpu(), b)
    assert oracle.rel_l2(y.float().cpu().numpy(), ref) <= (4e-3 if dt == torch.bfloat16 else 5e-4)


@pytest.mark.parametrize("m,K,N", [(1, 4096, 1024), (2, 8192, 300), (16, 4096, 1024), (5, 512, 512)])
def test_fused_linear_in_graph_replays(m, K, N):
    """fused_forward recorded in a HIP graph (the streamed decode form, its
    two-waves-per-row split, X quantized first, the MFMA form): every replay,
    with eager work between them, equals the eager call bit for bit."""
    from axs.unified import hip_linear

    x, w, b = _inputs((m,), K, N, 31 * m + K)
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    eager = hip_linear.fused_forward(xd, wd, bd)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        hip_linear.fused_forward(xd, wd, bd)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = hip_linear.fused_forward(xd, wd, bd)
    for i in range(3):
        scratch = torch.randn(1 << 20, device=DEV) * (i + 1)     # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), i
        del scratch


@pytest.mark.parametrize("K", [33, 50, 100, 127, 255])
def test_fused_linear_ragged_k(K):
    from axs.unified import hip_linear

    x, w, b = _inputs((64,), K, 32, K)
    y = hip_linear.fused_forward(x.to(DEV), w.to(DEV), None)
    assert oracle.rel_l2(y.cpu().numpy(), _exact(x, w, None)) <= TOL


def test_fused_linear_raw_input_and_no_bias():
    from axs.unified import hip_linear

    for m in (96, 3, 2, 1):
        x, w, b = _inputs((m,), 1024, 768, 9)
        y = hip_linear.fused_forward(x.to(DEV), w.to(DEV), None, quantize_input=False)
        assert oracle.rel_l2(y.cpu().numpy(), _exact(x, w, None, quantize_input=False)) <= TOL, m


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [48, 4, 2, 1])
def test_fused_linear_16bit(dt, m):
    from axs.unified import hip_linear

    x, w, b = _inputs((m,), 2048, 1024, 11, outliers=False)
    x, w = x.to(dt), w.to(dt)
    y = hip_linear.fused_forward(x.to(DEV), w.to(DEV), b.to(DEV))
    assert y.dtype == dt
    exact = _exact(x.float(), w.float(), b)
    want = torch.from_numpy(exact.astype(np.float32)).to(dt)
    got = y.cpu()
    same = (got.view(torch.int16) == want.view(torch.int16)).float().mean().item()
    print(f"  {dt}: {same:.5f} bit-identical to the rounded exact product", flush=True)
    assert same >= 0.99
    assert oracle.rel_l2(got.float().numpy(), exact) <= (4e-3 if dt == torch.bfloat16 else 5e-4)


def test_fused_linear_fq_is_bit_exact_with_the_fq_kernel():
    """With W = c I, c = 0.99999994 (the largest float below 1: its block
    scale is 1 and its LUT cell the top code, so FQ(W) = I exactly), Y is
    FQ(X) itself: the fused kernel's FQ of X must equal the oracle's bit for
    bit."""
    from axs.unified import hip_linear

    K = 256
    g = torch.Generator().manual_seed(2)
    x = torch.randn(40, K, generator=g) * torch.exp2(torch.randint(-30, 30, (40, 1), generator=g).float())
    eye = torch.eye(K) * 0.99999994
    assert np.array_equal(oracle.fake_quantize(eye.numpy(), 32), np.eye(K, dtype=np.float32))
    y = hip_linear.fused_forward(x.to(DEV), eye.to(DEV), None)
    want = oracle.fake_quantize(x.numpy(), 32)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))
    # at most 16 rows: FQ(X) staged once in LDS (the streamed decode form at
    # 1 and 2 rows, the MFMA form's LDS staging up to 16), same bits
    for m in (1, 2, 5, 16):
        ym = hip_linear.fused_forward(x[:m].to(DEV), eye.to(DEV), None)
        assert np.array_equal(ym.cpu().numpy().view(np.uint32), want[:m].view(np.uint32)), m


def test_linear_forward_dispatches_small_outputs_to_the_fused_kernel(monkeypatch):
    from axs.unified import hip_linear

    calls = []
    real = hip_linear.fused_forward
    monkeypatch.setattr(hip_linear, "fused_forward", lambda *a, **k: calls.append(1) or real(*a, **k))
    x, w, b = _inputs((32,), 4096, 4096, 1)
    y = hip_linear.linear_forward(x.to(DEV), w.to(DEV), b.to(DEV), 32, True)        # 131072 outputs: fused
    assert calls == [1]
    assert oracle.rel_l2(y.cpu().numpy(), _exact(x, w, b)) <= TOL
    x2, w2, _ = _inputs((33,), 256, 4096, 2)
    hip_linear.linear_forward(x2.to(DEV), w2.to(DEV), None, 32, True)                # 135168: packed path
    hip_linear.linear_forward(x.to(DEV), w.to(DEV), None, 16, True)                  # block 16: packed path
    assert calls == [1]


def test_fused_linear_errors():
    from axs import _lib
    from axs.unified import hip_linear

    with pytest.raises(RuntimeError, match="CUDA"):
        hip_linear.fused_forward(torch.randn(4, 32), torch.randn(8, 32))
    x = torch.randn(4, 64, device=DEV)
    w = torch.randn(8, 64, device=DEV)
    y = torch.empty(4, 8, device=DEV)
    with pytest.raises(_lib.LibraryError, match="block_size=32"):
        _lib.call("axs6_nf5_fused_linear", x.data_ptr(), w.data_ptr(), None, y.data_ptr(), 0, 4, 8, 64, 16, 1,
                  _lib.stream_of(x))
    with pytest.raises(_lib.LibraryError, match="multiple of 32"):
        _lib.call("axs6_nf5_fused_linear", x.data_ptr(), w.data_ptr(), None, y.data_ptr(), 0, 4, 8, 48, 32, 1,
                  _lib.stream_of(x))
