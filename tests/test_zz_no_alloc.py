"""The allocation-free backward (axs6_nf5_linear_backward_noalloc, the
library's fixed per-device scratch) against the workspace entry point
(axs6_nf5_linear_backward): the same kernels on the same inputs, so dX, dW
and db must be bit-identical.  Two calls in a row, the second smaller, so
the second reads scratch the first left behind."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import bits_equal, first_mismatch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _case(M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    w = torch.randn(N, K, generator=g) / K ** 0.5
    dy = torch.randn(M, N, generator=g)
    m = torch.rand(M, N, generator=g) < 0.01
    dy[m] *= 100.0
    return x.to(DEV), w.to(DEV), dy.to(DEV)


def _backward(entry, saved, dy, quantize_grad, seed):
    from axs import _lib

    M, N, K = saved.M, saved.N, saved.K
    dx = torch.full((M, K), float("nan"), device=DEV)
    dw = torch.full((N, K), float("nan"), device=DEV)
    db = torch.full((N,), float("nan"), device=DEV)
    head = (dy.data_ptr(), _lib.F32, M, N, K, 32, int(quantize_grad), seed, 0,
            saved.xq.data_ptr(), saved.sx.data_ptr(), saved.wq.data_ptr(), saved.sw.data_ptr(),
            dx.data_ptr(), dw.data_ptr(), db.data_ptr())
    st = _lib.stream_of(dy)
    if entry == "workspace":
        nbytes = int(_lib.lib().axs6_nf5_linear_backward_workspace(M, N, K, 1, 1, 1))
        ws = torch.empty((nbytes,), dtype=torch.uint8, device=DEV)
        _lib.call("axs6_nf5_linear_backward", *head, ws.data_ptr(), nbytes, None, st)
    else:
        _lib.call("axs6_nf5_linear_backward_noalloc", *head, None, st)
    torch.cuda.synchronize()
    return dx.cpu().numpy(), dw.cpu().numpy(), db.cpu().numpy()


@pytest.mark.parametrize("quantize_grad", [True, False])
def test_noalloc_backward_matches_workspace_backward(quantize_grad):
    from axs.unified import hip_linear

    # the second shape is smaller, and ragged against the tiles
    for (M, N, K), seed in (((2048, 768, 3072), 11), ((200, 96, 320), 12)):
        print(f"noalloc backward M={M} N={N} K={K} quantize_grad={quantize_grad}", flush=True)
        x, w, dy = _case(M, N, K, seed)
        _, saved = hip_linear.forward_train(x, w, None, 32, True)
        want = _backward("workspace", saved, dy, quantize_grad, seed)
        got = _backward("noalloc", saved, dy, quantize_grad, seed)
        for name, a, b in zip(("dx", "dw", "db"), got, want):
            assert not np.isnan(b).any(), name
            assert bits_equal(a, b), f"{name} at {(M, N, K)}: {first_mismatch(a, b)}"


def test_noalloc_backward_refuses_oversized_shapes_on_device():
    from axs import _lib
    from axs.unified import hip_linear

    M, N, K = 4096, 4096, 4096      # 129.5 MiB of workspace
    x, w, dy = _case(M, N, K, 5)
    _, saved = hip_linear.forward_train(x, w, None, 32, True)
    dx = torch.zeros((M, K), device=DEV)
    with pytest.raises(RuntimeError, match="scratch"):
        _lib.call("axs6_nf5_linear_backward_noalloc", dy.data_ptr(), _lib.F32, M, N, K, 32, 1, 0, 0,
                  saved.xq.data_ptr(), saved.sx.data_ptr(), saved.wq.data_ptr(), saved.sw.data_ptr(),
                  dx.data_ptr(), None, None, None, _lib.stream_of(dy))
    torch.cuda.synchronize()
    assert torch.count_nonzero(dx).item() == 0   # nothing was launched
