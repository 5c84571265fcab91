"""The torch extension axs._C (csrc/torch_ext.cpp) loads beside libaxs6.so,
exports the fake-quantize's and the linear's entry points, draws dither seeds exactly as the Python
wrappers do (torch.randint(0, 2**62, (1,)) on the default CPU generator),
and rejects host tensors with the reference's CUDA error."""
from __future__ import annotations

import pytest
import torch


def test_extension_loads_and_exports():
    from axs import _lib

    C = _lib.ext()
    for name in ("fq", "fq_ste", "linear", "linear_fwd", "linear_bwd", "graph_counter", "graph_counter_advance",
                 "next_seed"):
        assert callable(getattr(C, name)), name


def test_seed_draw_matches_python():
    from axs import _lib
    from axs.unified import hip_kernels

    C = _lib.ext()
    for s in (0, 5, 123):
        torch.manual_seed(s)
        a = [C.next_seed() for _ in range(3)]
        torch.manual_seed(s)
        b = [hip_kernels.next_seed() for _ in range(3)]
        assert a == b


def test_host_tensors_raise_cuda_error():
    from axs import _lib

    C = _lib.ext()
    x, w = torch.randn(4, 64), torch.randn(16, 64)
    with pytest.raises(RuntimeError, match="CUDA"):
        C.linear(x, w, None, 32, True, True)
    with pytest.raises(RuntimeError, match="CUDA"):
        C.linear_fwd(x, w, None, 32, True)


def test_fq_host_tensor_raises_before_the_extension():
    """fake_quantize_unified checks its arguments in Python first, with the
    reference's exception types."""
    from axs.unified import functional_unified as fu

    x = torch.randn(4, 64)
    with pytest.raises(RuntimeError, match="CUDA"):
        fu.fake_quantize_unified(x)
