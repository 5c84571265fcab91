"""Autograd ops: NF5 fake-quantize with a straight-through gradient and the
AXS-6 quantized linear / matmul.

Mirrors ``axs/unified/functional_unified.py`` of the reference
(``_FusedQuantizeSTE`` :38-60, ``fake_quantize_unified`` :63-82,
``_AXSLinearUnifiedFunction`` :89-170, ``axs_linear_unified`` :173-197,
``axs_matmul_unified`` :204-227): same signatures, same gradient semantics.
The linear runs on the HIP kernels of libaxs6.so: NF5 fake-quantize fused
with the fp16 operand packing, then an MFMA GEMM (``axs.unified.hip_linear``).
"""
from __future__ import annotations

from typing import Literal

import torch

from axs import _lib
from axs.core import DEFAULT_BLOCK_SIZE
from axs.unified import backend as _backend
from axs.unified import hip_kernels as _hk
from axs.unified import hip_linear
from axs.unified.backend import accelerated_fake_quantize as _accel_fq


class _FusedQuantizeSTE(torch.autograd.Function):
    """Forward: NF5 fake-quantize.  Backward: the incoming gradient, unchanged.

    ``fake_quantize_unified`` runs the same operation as a C++ autograd node
    (``axs._C.fq_ste``), without this class's Python forward and backward."""

    @staticmethod
    def forward(ctx, tensor: torch.Tensor, block_size: int, rounding: str) -> torch.Tensor:  # type: ignore[override]
        return _accel_fq(tensor, block_size=block_size, rounding=rounding)  # type: ignore[arg-type]

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):  # type: ignore[override]
        return grad_output, None, None


def fake_quantize_unified(
    tensor: torch.Tensor,
    block_size: int = DEFAULT_BLOCK_SIZE,
    rounding: Literal["nearest", "stochastic"] = "nearest",
) -> torch.Tensor:
    """NF5 fake-quantize with a straight-through gradient: the backward
    hands the incoming gradient back unchanged."""
    stochastic = _hk.fq_checks(tensor, block_size, rounding, "fake_quantize_unified")
    _backend.note_device(tensor)
    return _lib.ext().fq_ste(tensor, block_size, stochastic)


class _AXSLinearUnifiedFunction(torch.autograd.Function):
    """Y = FQ(X) FQ(W)^T + b.

    Backward (straight-through): dY is fake-quantized with stochastic
    rounding when ``quantize_grad``; dX = dYq FQ(W), dW = dYq^T FQ(X),
    db = sum of dYq over the batch dims.  The fp16 operands packed in the
    forward are kept for the backward instead of the fp32 FQ(X) the
    reference saves (half the activation memory; FQ(W) is not recomputed).
    """

    @staticmethod
    def forward(ctx, input, weight, bias, block_size, quantize_input, quantize_grad):  # type: ignore[override]
        out, saved = hip_linear.forward_train(input, weight, bias, block_size, quantize_input)
        ctx.save_for_backward(*saved.tensors())
        ctx.meta = saved.meta()
        ctx.block_size = block_size
        ctx.quantize_grad = quantize_grad
        ctx.has_bias = bias is not None
        return out

    @staticmethod
    def backward(ctx, grad_output):  # type: ignore[override]
        saved = hip_linear.Saved.restore(ctx.saved_tensors, ctx.meta)
        need_x, need_w, need_b = ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.needs_input_grad[2]
        dx, dw, db = hip_linear.backward(
            grad_output, saved, ctx.block_size, ctx.quantize_grad,
            need_x, need_w, need_b and ctx.has_bias)
        return dx, dw, db, None, None, None


def axs_linear_unified(
    input: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    block_size: int = DEFAULT_BLOCK_SIZE,
    quantize_input: bool = True,
    quantize_grad: bool = True,
) -> torch.Tensor:
    """AXS-6 quantized linear: ``input (*, in) -> (*, out)``.  Runs as one C++
    autograd node (the same forward and backward as
    ``_AXSLinearUnifiedFunction``, whose Python class is kept for callers
    that use it directly)."""
    return hip_linear.linear_autograd(input, weight, bias, block_size, quantize_input, quantize_grad)


def axs_linear_group_unified(
    input: torch.Tensor,
    weights: list[torch.Tensor] | tuple[torch.Tensor, ...],
    biases: list[torch.Tensor | None] | tuple[torch.Tensor | None, ...] | None = None,
    block_size: int = DEFAULT_BLOCK_SIZE,
    quantize_input: bool = True,
    quantize_grad: bool = True,
) -> tuple[torch.Tensor, ...]:
    """Several quantized linears of one input -- ``(axs_linear_unified(input,
    w_i, b_i) for each i)``, e.g. the q/k/v projections of self-attention --
    as one: the weights stacked along the output dim, so the input is packed
    once and forward and backward each run one linear (one GEMM per
    direction instead of one per weight).  Each output equals its own
    ``axs_linear_unified`` forward bit for bit (same operand rows, same
    contraction order); in the backward the input gradient is the contraction
    over all stacked outputs at once, and the stochastic rounding of the
    output gradient draws one stream for the stacked rows (both within the
    linear's tolerance).  This function is this library's; the reference runs
    the projections one by one (``modules_unified.py:235-243``)."""
    weights = list(weights)
    if not weights:
        return ()
    biases = [None] * len(weights) if biases is None else list(biases)
    if len(biases) != len(weights):
        raise ValueError(f"axs_linear_group_unified: {len(weights)} weights but {len(biases)} biases")
    if len(weights) == 1:
        return (axs_linear_unified(input, weights[0], biases[0], block_size, quantize_input, quantize_grad),)
    sizes = [w.shape[0] for w in weights]
    w = torch.cat(weights, 0)
    if all(b is None for b in biases):
        b = None
    else:
        b = torch.cat([bi if bi is not None else torch.zeros(n, dtype=w.dtype, device=w.device)
                       for bi, n in zip(biases, sizes)])
    y = axs_linear_unified(input, w, b, block_size, quantize_input, quantize_grad)
    return tuple(y.split(sizes, dim=-1))


def axs_matmul_unified(
    a: torch.Tensor,
    b: torch.Tensor,
    block_size: int = DEFAULT_BLOCK_SIZE,
    quantize_inputs: bool = True,
) -> torch.Tensor:
    """``FQ(a) @ FQ(b)`` (blocks along each operand's last dim, as the
    reference) on the HIP GEMM; no autograd.  ``a (*, M, K)``, ``b (*, K, N)``
    with torch.matmul's broadcasting; the result has the operands' dtype, as
    the reference's torch.matmul of the FQ values."""
    dtype = torch.promote_types(a.dtype, b.dtype)
    if quantize_inputs:
        a = _accel_fq(a, block_size, "nearest")
        b = _accel_fq(b, block_size, "nearest")
    out = hip_linear.matmul(a, b)
    return out.to(dtype) if dtype.is_floating_point and out.dtype != dtype else out
