"""bf16 mixed-precision AXS-6 linear.

Mirrors ``axs/unified/mixed_precision.py`` of the reference
(``_AXSLinearBF16Function`` :65-155, ``axs_linear_mixed_precision`` :158,
``AXSLinearMixedPrecision`` :193-269, ``convert_to_axs_mixed_precision``
:277-349, ``estimate_memory_savings`` :357-401), with its arithmetic:

* forward (:96-108): input and weight cast to bf16, fake-quantized (fp32
  arithmetic, result rounded to bf16), contracted with fp32 accumulation,
  plus the bias rounded to bf16, output rounded to bf16;
* backward (:128-153): dY cast to bf16 and stochastically fake-quantized
  (rounded to bf16); dX = dYq . FQ(W) rounded to bf16; dW = dYq^T . FQ(X) in
  fp32 from the bf16 operands; db = the column sums of the *unquantized*
  dY in fp32.

The contractions run on the fp16-MFMA quantized-linear kernels: the packing
rounds bf16 inputs' FQ values to bf16, and a bf16 value times a power of two
is exact in fp16, so the MFMAs see the reference's bf16 operands and
accumulate in fp32 like its bf16 GEMM.
"""
from __future__ import annotations

import copy
import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from axs.core import DEFAULT_BLOCK_SIZE
from axs.unified import hip_linear


class _AXSLinearBF16Function(torch.autograd.Function):
    @staticmethod
    def forward(ctx, input, weight, bias, block_size, quantize_input, quantize_grad):  # type: ignore[override]
        # the reference adds the bias as bf16 (F.linear(input_q, weight_q, bias.to(bf16)))
        b16 = bias.to(torch.bfloat16) if bias is not None else None
        out, saved = hip_linear.forward_train(input.to(torch.bfloat16), weight.to(torch.bfloat16), b16,
                                              block_size, quantize_input)
        saved.w_dtype = torch.float32     # dW stays fp32 for the fp32 master weight
        ctx.save_for_backward(*saved.tensors())
        ctx.meta = saved.meta()
        ctx.block_size = block_size
        ctx.quantize_grad = quantize_grad
        ctx.has_bias = bias is not None
        return out

    @staticmethod
    def backward(ctx, grad_output):  # type: ignore[override]
        saved = hip_linear.Saved.restore(ctx.saved_tensors, ctx.meta)
        need_x, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        dx, dw, _ = hip_linear.backward(grad_output.to(torch.bfloat16), saved, ctx.block_size,
                                        ctx.quantize_grad, need_x, need_w, False)
        db = None
        if ctx.has_bias and ctx.needs_input_grad[2]:
            db = grad_output.float().sum(dim=tuple(range(grad_output.ndim - 1)))
        return dx, dw, db, None, None, None


def axs_linear_mixed_precision(
    input: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    block_size: int = DEFAULT_BLOCK_SIZE,
    quantize_input: bool = True,
    quantize_grad: bool = True,
) -> torch.Tensor:
    """AXS-6 quantized linear with bf16 compute; returns bf16."""
    return _AXSLinearBF16Function.apply(input, weight, bias, block_size, quantize_input, quantize_grad)


class AXSLinearMixedPrecision(nn.Module):
    """``nn.Linear`` replacement: fp32 master weights, bf16 compute and output."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True,
                 block_size: int = DEFAULT_BLOCK_SIZE, quantize_input: bool = True,
                 quantize_grad: bool = True) -> None:
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.block_size = block_size
        self.quantize_input = quantize_input
        self.quantize_grad = quantize_grad
        self.weight = nn.Parameter(torch.empty(out_features, in_features))
        if bias:
            self.bias = nn.Parameter(torch.empty(out_features))
        else:
            self.register_parameter("bias", None)
        self._warmup_active: bool = False
        self.reset_parameters()

    def reset_parameters(self) -> None:
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        if self.bias is not None:
            bound = 1 / math.sqrt(self.weight.shape[1])
            nn.init.uniform_(self.bias, -bound, bound)

    def forward(self, input: torch.Tensor) -> torch.Tensor:
        if self._warmup_active:
            return F.linear(input.to(torch.bfloat16), self.weight.to(torch.bfloat16),
                            self.bias.to(torch.bfloat16) if self.bias is not None else None)
        return axs_linear_mixed_precision(input, self.weight, self.bias, self.block_size,
                                          self.quantize_input, self.quantize_grad)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, block_size={self.block_size}, "
                f"quant_input={self.quantize_input}, quant_grad={self.quantize_grad}, "
                f"mixed_precision=bf16")


def convert_to_axs_mixed_precision(
    model: nn.Module,
    block_size: int = DEFAULT_BLOCK_SIZE,
    quantize_input: bool = True,
    quantize_grad: bool = True,
    skip_layers: set[str] | None = None,
    inplace: bool = False,
) -> nn.Module:
    """Replace ``nn.Linear`` and ``AXSLinearUnified`` children with
    :class:`AXSLinearMixedPrecision`, copying weights as fp32."""
    from axs.unified.modules_unified import AXSLinearUnified

    if not inplace:
        model = copy.deepcopy(model)
    skip = set(skip_layers or ())

    def _convert(module: nn.Module, prefix: str = "") -> None:
        for name, child in module.named_children():
            full = f"{prefix}.{name}" if prefix else name
            if full in skip:
                continue
            if isinstance(child, (nn.Linear, AXSLinearUnified)):
                new = AXSLinearMixedPrecision(child.in_features, child.out_features,
                                              bias=child.bias is not None, block_size=block_size,
                                              quantize_input=quantize_input, quantize_grad=quantize_grad)
                new.weight.data.copy_(child.weight.data.float())
                if child.bias is not None:
                    new.bias.data.copy_(child.bias.data.float())
                setattr(module, name, new.to(child.weight.device))
            else:
                _convert(child, full)

    _convert(model)
    return model


def estimate_memory_savings(model: nn.Module, batch_size: int = 1, seq_len: int = 1) -> dict[str, float]:
    """Activation memory of fp32 (input_q + weight_q saved) versus bf16 with
    weight recomputation (input_q only), over the model's mixed-precision
    linears, in MiB."""
    fp32_bytes = 0
    bf16_bytes = 0
    for m in model.modules():
        if isinstance(m, AXSLinearMixedPrecision):
            act = batch_size * seq_len * m.in_features
            fp32_bytes += (act + m.out_features * m.in_features) * 4
            bf16_bytes += act * 2
    fp32_mb = fp32_bytes / (1024 * 1024)
    bf16_mb = bf16_bytes / (1024 * 1024)
    return {"fp32_mb": round(fp32_mb, 2), "bf16_recomp_mb": round(bf16_mb, 2),
            "savings_ratio": round(fp32_mb / bf16_mb, 1) if bf16_mb > 0 else float("inf")}
