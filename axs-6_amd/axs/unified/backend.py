"""Backend selection API and the accelerated entry points.

Keeps the reference's names and behaviour surface
(``axs/unified/backend.py``: ``BackendType`` :79, ``detect_best_backend``
:128, ``get_backend`` / ``set_backend`` :156-180, ``accelerated_fake_quantize``
:495, ``accelerated_linear`` :540, ``accelerated_matmul`` :621,
``backend_info`` :678, ``clear_int8_weight_cache`` :694) so existing callers
keep working, but there is exactly one compute path: the gfx950 HIP kernels
of libaxs6.so.  The enum keeps the reference's values (plus ``HIP``) and the
``AXS6_BACKEND`` override is still honoured (case- and space-insensitive),
yet whichever value is active, device tensors go to the HIP kernels; there
is no Triton, torch.compile, INT8 or eager variant to fall back to, and a
failing kernel raises instead of silently switching backends.
"""
from __future__ import annotations

import enum
import logging
import os
from typing import Literal

import torch

from axs import _lib
from axs.core import DEFAULT_BLOCK_SIZE
from axs.unified import hip_kernels as _hk

logger = logging.getLogger(__name__)


class BackendType(enum.Enum):
    """Backend names accepted by set_backend / AXS6_BACKEND.  All of them
    execute on the single HIP path."""

    EAGER = "eager"
    COMPILED = "compiled"
    INT8 = "int8"
    TRITON = "triton"
    HIP = "hip"


_VALID = tuple(b.value for b in BackendType)
_active_backend: BackendType | None = None

# Per-device table residency, reported by backend_info (the library keeps
# the LUT resident on each device it has run on).
_LUT_CACHE: dict[torch.device, bool] = {}


def _has_cuda() -> bool:
    return torch.cuda.is_available()


def _has_hip_kernel() -> bool:
    return _hk.has_hip()


def detect_best_backend() -> BackendType:
    """``AXS6_BACKEND`` if set to a known name, else HIP."""
    env = os.environ.get("AXS6_BACKEND", "").lower().strip()
    if env in _VALID:
        return BackendType(env)
    return BackendType.HIP


def get_backend() -> BackendType:
    global _active_backend
    if _active_backend is None:
        _active_backend = detect_best_backend()
        logger.info("AXS-6 backend: %s", _active_backend.value)
    return _active_backend


def set_backend(backend: str | BackendType) -> None:
    """Select a backend name (``"eager"``, ``"compiled"``, ``"int8"``,
    ``"triton"`` or ``"hip"``); raises ValueError for unknown names."""
    global _active_backend
    if isinstance(backend, str):
        backend = BackendType(backend.lower().strip())
    _active_backend = backend
    logger.info("AXS-6 backend set to: %s", backend.value)


def accelerated_fake_quantize(
    tensor: torch.Tensor,
    block_size: int = DEFAULT_BLOCK_SIZE,
    rounding: Literal["nearest", "stochastic"] = "nearest",
) -> torch.Tensor:
    """NF5 fake-quantize on the HIP path."""
    note_device(tensor)
    return _hk.hip_fused_fake_quantize(tensor, block_size, rounding)


def note_device(tensor: torch.Tensor) -> None:
    """Resolves the active backend (once) and records the tensor's device
    as holding the tables (reported by backend_info)."""
    get_backend()
    if tensor.is_cuda:
        _LUT_CACHE.setdefault(tensor.device, True)


def accelerated_linear(
    input: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    block_size: int = DEFAULT_BLOCK_SIZE,
    quantize_input: bool = True,
) -> torch.Tensor:
    """``FQ(input) @ FQ(weight).T + bias`` with the fused HIP linear."""
    get_backend()
    from axs.unified import hip_linear

    return hip_linear.linear_forward(input, weight, bias, block_size, quantize_input)


def accelerated_matmul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """``a (*, K) @ b (K, N)`` in float32 on the HIP GEMM (operands are taken
    as given; no NF5 step)."""
    get_backend()
    from axs.unified import hip_linear

    return hip_linear.matmul(a, b)


def backend_info() -> dict[str, object]:
    """Diagnostic info about the active backend and the HIP library."""
    try:
        version = _lib.version()
        lib_ok = True
    except _lib.LibraryError:
        version, lib_ok = None, False
    cuda = _has_cuda()
    props = torch.cuda.get_device_properties(torch.cuda.current_device()) if cuda else None
    return {
        "active_backend": get_backend().value,
        "cuda_available": cuda,
        "hip_kernel": lib_ok and cuda,
        "hip_library": version,
        "gcn_arch": getattr(props, "gcnArchName", None) if props is not None else None,
        "triton_kernel": False,
        "int8_tensorcore": False,
        "torch_compile": False,
        "gpu_name": torch.cuda.get_device_name() if cuda else None,
        "compute_capability": torch.cuda.get_device_capability() if cuda else None,
        "lut_cached_devices": [str(d) for d in _LUT_CACHE],
    }


def clear_int8_weight_cache() -> None:
    """Kept for API compatibility: the HIP path keeps no INT8 weight cache."""
    from axs.unified import hip_linear

    hip_linear.clear_weight_cache()
