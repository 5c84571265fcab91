"""The forward that packs the operands while it contracts them
(``axs6_nf5_linear_forward_stream``, the no-grad ``linear_forward`` above the
fused threshold).

Its packed values carry a power-of-two shift per (row, 512-wide K-chunk)
instead of per row; where both keep every packed value in fp16's normal range
each value is the two-launch path's value times a power of two, and the
accumulators are rescaled by exact powers of two, so Y must equal the
two-launch forward (``axs6_nf5_linear_forward``) bit for bit -- including
rows whose shift rises along K (the rescale path), 16-bit inputs, block
sizes 8/16/32 and NaN/inf blocks (raw X, whose small values can fall into
fp16's subnormal range, against the oracle).  Against the oracle: rel-L2 <= 1e-3
of the fp64 product of the FQ operands (config 3 on sampled rows).  Every
test also checks that no launch timed out waiting for a chunk."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _gauss(shape, seed, scale=1.0, outliers=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * scale
    if outliers:
        x[torch.rand(*shape, generator=g) < 0.01] *= 100.0
    return x


def _ws(M, N, K, dtype=torch.float32):
    from axs import _lib

    return int(_lib.lib().axs6_nf5_linear_forward_stream_workspace(M, N, K, _lib.DTYPE_CODE[dtype]))


def _stream(x, w, b=None, bs=32, qx=True):
    """The streamed kernel through the C ABI (raises if the shape does not qualify)."""
    from axs import _lib

    M, K = x.shape
    N = w.shape[0]
    nbytes = _ws(M, N, K, x.dtype)
    assert nbytes > 0, (M, N, K)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    y = torch.empty((M, N), dtype=x.dtype, device=DEV)
    _lib.call("axs6_nf5_linear_forward_stream", x.data_ptr(), w.data_ptr(), _lib.ptr(b), y.data_ptr(),
              _lib.DTYPE_CODE[x.dtype], M, N, K, bs, int(qx), ws.data_ptr(), nbytes, _lib.stream_of(x))
    return y


def _two_launch(x, w, b=None, bs=32, qx=True):
    from axs.unified import hip_linear

    return hip_linear.forward_train(x, w, b, bs, qx)[0]


def _no_timeouts():
    from axs import _lib

    flag = ctypes.c_int32(0)
    _lib.call("axs6_nf5_linear_stream_error", ctypes.byref(flag))
    assert flag.value == 0, "a streamed forward timed out waiting for a chunk"


def _bits_equal(a, b):
    return torch.equal(a.view(torch.int32) if a.dtype == torch.float32 else a.view(torch.int16),
                       b.view(torch.int32) if b.dtype == torch.float32 else b.view(torch.int16))


# K: 512 (one chunk, nothing streamed), 1024, 4096 (8 chunks), 4100 (a ragged
# last chunk and NF5 block); M, N: whole and partial 256-row tiles
@pytest.mark.parametrize("M,K,N", [(4096, 4096, 4096), (4096, 1024, 4096), (4096, 512, 4096), (4096, 4100, 4096),
                                   (4000, 2048, 4092), (2048, 1536, 8192), (3840, 1024, 4096)])
def test_stream_equals_two_launch_bitwise(M, K, N):
    print(f"[stream linear {M}x{K}x{N}]", flush=True)
    x = _gauss((M, K), M + K, outliers=True).to(DEV)
    w = (_gauss((N, K), N + 7) * K ** -0.5).to(DEV)
    b = _gauss((N,), 3).to(DEV)
    got = _stream(x, w, b)
    want = _two_launch(x, w, b)
    torch.cuda.synchronize()
    _no_timeouts()
    assert _bits_equal(got, want), (got - want).abs().max().item()


def test_stream_config3_vs_oracle_and_dispatch():
    """Config 3 (4096^3, X ~ N(0,1), W ~ N(0, 1/sqrt(K)), bias zero): equal to
    the public no-grad entry point (the two-launch forward) and, on sampled
    rows, within rel-L2 1e-3 of the fp64 product of the oracle's FQ operands."""
    from axs.unified import hip_linear

    M = K = N = 4096
    x = _gauss((M, K), 11)
    w = _gauss((N, K), 12) * K ** -0.5
    b = torch.zeros(N)
    assert _ws(M, N, K) > 0
    y = _stream(x.to(DEV), w.to(DEV), b.to(DEV))
    assert _bits_equal(y, hip_linear.linear_forward(x.to(DEV), w.to(DEV), b.to(DEV), 32, True))
    rows = np.random.default_rng(0).choice(M, 96, replace=False)
    xq = oracle.fake_quantize(x.numpy()[rows], 32)
    wq = oracle.fake_quantize(w.numpy(), 32)
    want = oracle.linear_reference(xq, wq, b.numpy())
    err = oracle.rel_l2(y[torch.from_numpy(rows).to(DEV)].cpu().numpy(), want)
    print(f"  rel-L2 on 96 sampled rows {err:.2e}", flush=True)
    assert err < 1e-3
    _no_timeouts()


def test_stream_rising_shifts_rescale_exactly():
    """Rows whose magnitude grows along K (each 512-wide chunk 2^2 above the
    previous, some rows 2^4 more from K = 2048; every 7th W row likewise):
    the running shift rises past the first chunk's headroom, so the tile's
    accumulators are rescaled at chunk boundaries -- exactly, hence bit for
    bit the two-launch result (the 18 binades of growth keep every block of
    these rows in fp16's normal range under both paths' shifts)."""
    M, K, N = 4096, 4096, 4096
    x = _gauss((M, K), 21)
    w = _gauss((N, K), 22) * K ** -0.5
    grow = torch.exp2(2.0 * (torch.arange(K) // 512).float())
    x = x * grow
    w[::7] = w[::7] * grow
    x[5::97, 2048:] *= 2.0 ** 4
    w[3::101, 1024:] *= 2.0 ** 4
    xd, wd = x.to(DEV), w.to(DEV)
    got = _stream(xd, wd)
    want = _two_launch(xd, wd)
    torch.cuda.synchronize()
    _no_timeouts()
    assert _bits_equal(got, want), (got - want).abs().max().item()
    rows = np.arange(5, M, 97)[:40]
    ref = oracle.linear_reference(oracle.fake_quantize(x.numpy()[rows], 32), oracle.fake_quantize(w.numpy(), 32))
    assert oracle.rel_l2(got[torch.from_numpy(rows).to(DEV)].cpu().numpy(), ref) < 1e-3


def test_stream_wide_row_spread_vs_oracle():
    """Rows spanning 2^40 along K (the last chunks 2^40 above the first, so the
    running shift rises by ~40 at one boundary and the accumulators of every
    tile are rescaled by 2^-40): within the north star's rel-L2 of the
    oracle."""
    M, K, N = 4096, 4096, 4096
    x = _gauss((M, K), 23)
    w = _gauss((N, K), 24) * K ** -0.5
    x[:, 3072:] *= 2.0 ** 40
    got = _stream(x.to(DEV), w.to(DEV))
    torch.cuda.synchronize()
    _no_timeouts()
    rows = np.arange(0, M, 61)[:48]
    xq = oracle.fake_quantize(x.numpy()[rows], 32).astype(np.float64)
    wq = oracle.fake_quantize(w.numpy(), 32).astype(np.float64)
    ref = xq @ wq.T
    assert oracle.rel_l2(got[torch.from_numpy(rows).to(DEV)].cpu().numpy(), ref) < 1e-3


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bs", [8, 16, 32])
def test_stream_16bit_and_block_sizes(dt, bs):
    M, K, N = 4096, 2048, 4096
    x = _gauss((M, K), 31 + bs).to(dt).to(DEV)
    w = (_gauss((N, K), 32) * K ** -0.5).to(dt).to(DEV)
    got = _stream(x, w, None, bs)
    want = _two_launch(x, w, None, bs)
    torch.cuda.synchronize()
    _no_timeouts()
    assert got.dtype == dt and _bits_equal(got, want)


@pytest.mark.parametrize("bs", [8, 16])
def test_stream_f32_block_sizes_and_raw_x(bs):
    M, K, N = 4096, 1536, 4096
    x = _gauss((M, K), 41, outliers=True).to(DEV)
    w = (_gauss((N, K), 42) * K ** -0.5).to(DEV)
    assert _bits_equal(_stream(x, w, None, bs), _two_launch(x, w, None, bs))
    # raw X is not bounded below by its block maximum (FQ values are, by
    # 2^-7), so the first chunk's 4 binades of headroom can leave its
    # smallest values in fp16's subnormal range, where the two paths' shifts
    # round differently: checked against the oracle instead
    raw = _stream(x, w, None, 32, qx=False)
    rows = np.arange(0, M, 83)[:48]
    ref = oracle.linear_reference(x.cpu().numpy()[rows], oracle.fake_quantize(w.cpu().numpy(), 32))
    assert oracle.rel_l2(raw[torch.from_numpy(rows).to(DEV)].cpu().numpy(), ref) < 1e-3
    torch.cuda.synchronize()
    _no_timeouts()


def test_stream_special_blocks_match_two_launch():
    """NaN and inf blocks (and an all-zero row) give the same NaN / inf
    positions and the same finite values as the two-launch path."""
    M, K, N = 4096, 2048, 4096
    x = _gauss((M, K), 51)
    w = _gauss((N, K), 52) * K ** -0.5
    x[17, 600] = float("nan")
    x[300, 1500] = float("inf")
    x[301, :] = 0.0
    w[40, 1030] = float("-inf")
    xd, wd = x.to(DEV), w.to(DEV)
    got, want = _stream(xd, wd), _two_launch(xd, wd)
    torch.cuda.synchronize()
    _no_timeouts()
    assert torch.equal(torch.isnan(got), torch.isnan(want))
    fin = torch.isfinite(want)
    assert torch.equal(torch.isfinite(got), fin)
    assert torch.equal(got[fin], want[fin])


def test_stream_repeated_calls_and_graph_replays():
    """Back-to-back launches reuse the counter sets (each launch leaves its set
    at zero) and give the same bits; so do replays of a recorded graph, with
    eager launches between them."""
    M = K = N = 4096
    x = _gauss((M, K), 61, outliers=True).to(DEV)
    w = (_gauss((N, K), 62) * K ** -0.5).to(DEV)
    first = _stream(x, w)
    for _ in range(20):
        again = _stream(x, w)
    torch.cuda.synchronize()
    assert _bits_equal(first, again)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _stream(x, w)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        yg = _stream(x, w)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert _bits_equal(yg, first)
        assert _bits_equal(_stream(x, w), first)
    _no_timeouts()


def test_stream_shape_rule():
    """Shapes outside one round of 256x256 tiles (or with too many rows per
    workgroup to pack) report no workspace and are refused; the public entry
    point then takes the two-launch forward."""
    from axs import _lib

    assert _ws(8192, 8192, 4096) == 0          # 1024 tiles: more than one round
    assert _ws(512, 512, 4096) == 0            # 4 tiles: 256 rows per workgroup to pack
    assert _ws(4096, 4096, 64 * 1024) == 0     # more than 64 chunks
    x = torch.randn(512, 256, device=DEV)
    w = torch.randn(512, 256, device=DEV)
    y = torch.empty(512, 512, device=DEV)
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=DEV)
    with pytest.raises(_lib.LibraryError, match="one round"):
        _lib.call("axs6_nf5_linear_forward_stream", x.data_ptr(), w.data_ptr(), None, y.data_ptr(), 0, 512, 512,
                  256, 32, 1, ws.data_ptr(), 1 << 20, _lib.stream_of(x))
