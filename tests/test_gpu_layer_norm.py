"""AXSLayerNormUnified on the HIP LayerNorm kernels (csrc/layer_norm.hip):
forward and backward against float64 LayerNorm on the CPU (torch's
F.layer_norm in double) and beside torch's own GPU F.layer_norm in the same
dtype, over the kernels' launch forms (one wave per row, a workgroup per row,
the generic streaming form for ragged, unaligned and long rows), 16-bit
inputs, several normalized dims, empty inputs, determinism and graph replay.
The reference module calls F.layer_norm (axs/unified/modules_unified.py:
120-144)."""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    d = torch.linalg.vector_norm(a - b)
    n = torch.linalg.vector_norm(b)
    return float(d / n) if n > 0 else float(d)


def _module(shape, dtype, seed=0):
    from axs.unified import AXSLayerNormUnified

    m = AXSLayerNormUnified(shape).to(DEV, dtype)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        m.weight.copy_(1.0 + 0.5 * torch.randn(m.weight.shape, generator=g))
        m.bias.copy_(0.3 * torch.randn(m.bias.shape, generator=g))
    return m


def _run(m, x, dy):
    xd = x.to(DEV).requires_grad_(True)
    y = m(xd)
    y.backward(dy.to(DEV))
    return y.detach(), xd.grad, m.weight.grad, m.bias.grad


def _reference(m, x, dy):
    """float64 F.layer_norm on the CPU with the module's parameters."""
    xd = x.double().requires_grad_(True)
    w = m.weight.detach().double().cpu().requires_grad_(True)
    b = m.bias.detach().double().cpu().requires_grad_(True)
    y = F.layer_norm(xd, m.normalized_shape, w, b, m.eps)
    y.backward(dy.double())
    return y.detach(), xd.grad, w.grad, b.grad


# (input shape, normalized dims): one wave per row (cols <= 1024 f32), a
# workgroup per row, the generic form (ragged, long), several normalized dims
SHAPES = [
    ((8192, 256), 1),
    ((64, 1024), 1),
    ((33, 4096), 1),
    ((7, 8192), 1),
    ((10, 1000), 1),
    ((10, 1001), 1),
    ((5, 20000), 1),
    ((3, 17, 96), 1),
    ((4, 8, 16, 12), 2),
    ((1, 4), 1),
    ((300, 3), 1),
]
TOL = {torch.float32: 2e-6, torch.bfloat16: 8e-3, torch.float16: 1e-3}


@pytest.mark.parametrize("shape,nd", SHAPES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_layer_norm_matches_float64(shape, nd, dtype):
    print(f"[layer_norm {shape} nd={nd} {dtype}]", flush=True)
    g = torch.Generator().manual_seed(1)
    x = (torch.randn(shape, generator=g) * 3.0 + 0.7).to(dtype)
    dy = torch.randn(shape, generator=g).to(dtype)
    m = _module(list(shape[-nd:]), dtype)
    got = _run(m, x, dy)
    want = _reference(m, x.double(), dy.double())
    # torch's own GPU LayerNorm in the same dtype, for scale
    mt = _module(list(shape[-nd:]), dtype)
    xt = x.to(DEV).requires_grad_(True)
    yt = F.layer_norm(xt, mt.normalized_shape, mt.weight, mt.bias, mt.eps)
    yt.backward(dy.to(DEV))
    torch_err = [_rel(yt, want[0]), _rel(xt.grad, want[1]), _rel(mt.weight.grad, want[2]),
                 _rel(mt.bias.grad, want[3])]
    errs = [_rel(a, b) for a, b in zip(got, want)]
    print(f"  rel-L2 y/dx/dgamma/dbeta {['%.1e' % e for e in errs]} (torch's: {['%.1e' % e for e in torch_err]})",
          flush=True)
    for name, e, te in zip(("y", "dx", "dgamma", "dbeta"), errs, torch_err):
        assert e <= max(TOL[dtype], 2 * te), (name, e, te)
    assert got[0].dtype == dtype and got[1].dtype == dtype and got[2].dtype == dtype


def test_layer_norm_unaligned_view():
    """A view off 16-byte alignment takes the kernels as it is (contiguous
    copy of a sliced view) and non-contiguous inputs are copied first."""
    g = torch.Generator().manual_seed(2)
    base = torch.randn(64, 257, generator=g)
    x = base[:, 1:]                       # non-contiguous
    dy = torch.randn(64, 256, generator=g)
    m = _module([256], torch.float32)
    got = _run(m, x, dy)
    want = _reference(m, x.contiguous(), dy)
    for a, b in zip(got, want):
        assert _rel(a, b) <= 2e-6
    # a contiguous buffer whose start is 4 bytes off 16-byte alignment
    flat = torch.randn(1 + 32 * 256, generator=g)
    xd = flat.to(DEV)[1:].view(32, 256)
    assert xd.data_ptr() % 16 != 0
    y = m(xd)
    ref = F.layer_norm(xd.double().cpu(), [256], m.weight.double().cpu(), m.bias.double().cpu(), m.eps)
    assert _rel(y, ref) <= 2e-6


def test_layer_norm_deterministic_and_extremes():
    """Bit-identical on repeat (fixed reduction orders); a constant row gives
    y = beta exactly; a row far from zero keeps its variance."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(512, 768, generator=g)
    x[0] = 5.0                            # constant row
    x[1] = 1e4 + torch.randn(768, generator=g)   # large mean, unit variance
    dy = torch.randn(512, 768, generator=g)
    m = _module([768], torch.float32)
    a = _run(m, x, dy)
    m.weight.grad = None
    m.bias.grad = None
    b = _run(m, x, dy)
    for u, v in zip(a, b):
        assert torch.equal(u, v)
    assert torch.equal(a[0][0], m.bias.detach())
    want = _reference(m, x.double(), dy.double())
    # a row near 1e4: its mean is an fp32 number with ulp 2^-10, which bounds
    # any fp32 LayerNorm; held to torch's own GPU LayerNorm on the same data
    # (the statistics about the row's first value keep the variance: a plain
    # fp32 sum of 768 values near 1e4 would lose ~1e-3 of the mean)
    mt = _module([768], torch.float32)
    xt = x.to(DEV).requires_grad_(True)
    yt = F.layer_norm(xt, [768], mt.weight, mt.bias, mt.eps)
    yt.backward(dy.to(DEV))
    ty, tx = _rel(yt[1], want[0][1]), _rel(xt.grad, want[1])
    print(f"  offset row: y {_rel(a[0][1], want[0][1]):.1e} (torch {ty:.1e}); dx {_rel(a[1], want[1]):.1e} "
          f"(torch {tx:.1e})", flush=True)
    assert _rel(a[0][1], want[0][1]) <= max(2 * ty, 1e-5)
    assert _rel(a[1], want[1]) <= max(2 * tx, 1e-5)


def test_layer_norm_empty_and_no_affine_grads():
    from axs.unified import AXSLayerNormUnified

    m = AXSLayerNormUnified(64).to(DEV)
    x = torch.zeros(0, 64, device=DEV, requires_grad=True)
    y = m(x)
    y.sum().backward()
    assert y.shape == (0, 64)
    assert torch.equal(m.weight.grad, torch.zeros(64, device=DEV))
    assert torch.equal(m.bias.grad, torch.zeros(64, device=DEV))
    # parameters frozen: only dx is computed
    m.weight.requires_grad_(False)
    m.bias.requires_grad_(False)
    x = torch.randn(16, 64, device=DEV, requires_grad=True)
    m(x).sum().backward()
    assert x.grad is not None and torch.isfinite(x.grad).all()


def test_layer_norm_in_graph_replays():
    """Forward + backward recorded in a HIP graph: every replay matches the
    eager result (no memset nodes: the column reduction writes every output)."""
    g = torch.Generator().manual_seed(4)
    m = _module([256], torch.float32)
    x = torch.randn(1024, 256, generator=g).to(DEV)
    dy = torch.randn(1024, 256, generator=g).to(DEV)
    xs = x.clone().requires_grad_(True)

    def step():
        m.weight.grad = None
        m.bias.grad = None
        xs.grad = None
        y = m(xs)
        y.backward(dy)
        return y

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    eager_y = step().detach().clone()
    eager = (xs.grad.clone(), m.weight.grad.clone(), m.bias.grad.clone())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = step()
    for i in range(3):
        with torch.no_grad():
            x.mul_(1.0)        # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager_y), i
        assert torch.equal(xs.grad, eager[0]) and torch.equal(m.weight.grad, eager[1])
        assert torch.equal(m.bias.grad, eager[2])


def test_module_runs_the_hip_kernels():
    """On the GPU the module's forward is the extension's autograd node (the
    HIP kernels), not F.layer_norm; on the CPU it is F.layer_norm."""
    from axs.unified import AXSLayerNormUnified

    m = AXSLayerNormUnified(128).to(DEV)
    y = m(torch.randn(4, 128, device=DEV, requires_grad=True))
    assert "LayerNormFunction" in y.grad_fn.name(), y.grad_fn.name()
    mc = AXSLayerNormUnified(128)
    yc = mc(torch.randn(4, 128, requires_grad=True))
    assert "LayerNorm" in yc.grad_fn.name() and "LayerNormFunction" not in yc.grad_fn.name(), yc.grad_fn.name()
