"""Drop-in modules on the HIP NF5 path.

Same classes, constructor arguments, parameters and forward semantics as the
reference's ``axs/unified/modules_unified.py``:

* ``AXSLinearUnified`` (:43-113) -- ``nn.Linear`` replacement, kaiming-uniform
  init, ``_warmup_active`` bypass; ``AXS6Linear`` is an alias (the name the
  benchmark configuration uses);
* ``AXSLayerNormUnified`` (:120-148) -- plain LayerNorm (no quantization);
* ``AXSEmbeddingUnified`` (:151-189) -- lookup, then NF5 fake-quantize of the
  gathered rows;
* ``AXSMultiheadAttentionUnified`` (:192-264) -- quantized q/k/v/out
  projections, fp32 scores, stochastic NF5 fake-quantize of the softmax
  probabilities;
* ``convert_to_axs_unified`` (:271-368) -- swaps ``nn.Linear`` /
  ``nn.LayerNorm`` / ``nn.Embedding`` for the modules above, keeping weights.
  (The reference also converts its deprecated V1/V2 layer classes, which do
  not exist here.)
"""
from __future__ import annotations

import copy
import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from axs import _lib
from axs.core import DEFAULT_BLOCK_SIZE
from axs.unified.functional_unified import axs_linear_group_unified, axs_linear_unified, fake_quantize_unified

# input dtypes whose LayerNorm runs on the HIP kernels
_LN_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


class AXSLinearUnified(nn.Module):
    """``nn.Linear`` with NF5 fake-quantized weight and input (and stochastic
    fake-quantized output gradient), on the gfx950 quantized-linear kernels."""

    def __init__(
        self,
        in_features: int,
        out_features: int,
        bias: bool = True,
        block_size: int = DEFAULT_BLOCK_SIZE,
        quantize_input: bool = True,
        quantize_grad: bool = True,
    ) -> None:
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
            return F.linear(input, self.weight, self.bias)
        return axs_linear_unified(input, self.weight, self.bias, self.block_size,
                                  self.quantize_input, self.quantize_grad)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, block_size={self.block_size}, "
                f"quant_input={self.quantize_input}, quant_grad={self.quantize_grad}")


AXS6Linear = AXSLinearUnified


class AXSLayerNormUnified(nn.Module):
    """LayerNorm without output quantization (the next linear quantizes its
    input), ``modules_unified.py:120-144``.  On the GPU, for float32, bfloat16
    or float16 input with parameters of the same dtype, forward and backward
    run on this library's HIP kernels (one autograd node; the statistics and
    the parameter gradients in float32, reduced in a fixed order); CPU tensors
    and other dtype combinations take ``F.layer_norm``, as the reference does
    everywhere."""

    def __init__(self, normalized_shape: int | list[int], eps: float = 1e-5) -> None:
        super().__init__()
        if isinstance(normalized_shape, int):
            normalized_shape = [normalized_shape]
        self.normalized_shape = list(normalized_shape)
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(self.normalized_shape))
        self.bias = nn.Parameter(torch.zeros(self.normalized_shape))

    def forward(self, input: torch.Tensor) -> torch.Tensor:
        if (input.is_cuda and input.dtype in _LN_DTYPES and self.weight.dtype == input.dtype
                and self.bias.dtype == input.dtype):
            return _lib.ext().layer_norm(input, self.weight, self.bias, len(self.normalized_shape), self.eps)
        return F.layer_norm(input, self.normalized_shape, self.weight, self.bias, self.eps)


class AXSEmbeddingUnified(nn.Module):
    """Embedding lookup followed by NF5 fake-quantize of the gathered rows only."""

    def __init__(
        self,
        num_embeddings: int,
        embedding_dim: int,
        padding_idx: int | None = None,
        block_size: int = DEFAULT_BLOCK_SIZE,
    ) -> None:
        super().__init__()
        self.num_embeddings = num_embeddings
        self.embedding_dim = embedding_dim
        self.padding_idx = padding_idx
        self.block_size = block_size
        self.weight = nn.Parameter(torch.empty(num_embeddings, embedding_dim))
        nn.init.normal_(self.weight)
        if padding_idx is not None:
            with torch.no_grad():
                self.weight[padding_idx].fill_(0)
        self._warmup_active: bool = False

    def forward(self, input: torch.Tensor) -> torch.Tensor:
        raw = F.embedding(input, self.weight, self.padding_idx)
        if self._warmup_active:
            return raw
        return fake_quantize_unified(raw, self.block_size, "nearest")


class AXSMultiheadAttentionUnified(nn.Module):
    """Multi-head attention with AXS-6 projections; scores in fp32; the
    post-softmax probabilities are NF5 fake-quantized with stochastic rounding."""

    def __init__(
        self,
        embed_dim: int,
        num_heads: int,
        dropout: float = 0.0,
        bias: bool = True,
        block_size: int = DEFAULT_BLOCK_SIZE,
    ) -> None:
        super().__init__()
        assert embed_dim % num_heads == 0, "embed_dim must be divisible by num_heads"
        self.embed_dim = embed_dim
        self.num_heads = num_heads
        self.head_dim = embed_dim // num_heads
        self.block_size = block_size
        self.dropout = dropout
        self.q_proj = AXSLinearUnified(embed_dim, embed_dim, bias=bias, block_size=block_size)
        self.k_proj = AXSLinearUnified(embed_dim, embed_dim, bias=bias, block_size=block_size)
        self.v_proj = AXSLinearUnified(embed_dim, embed_dim, bias=bias, block_size=block_size)
        self.out_proj = AXSLinearUnified(embed_dim, embed_dim, bias=bias, block_size=block_size)
        self.scale = self.head_dim ** -0.5

    def _projections(self, query, key, value):
        """q, k, v: in self-attention (one input tensor) the three projections
        run as one grouped linear (the input packed once, one GEMM per
        direction), else one by one as the reference does -- also when a
        projection has hooks, which see only calls of the module itself."""
        p = (self.q_proj, self.k_proj, self.v_proj)
        grouped = (query is key and key is value and all(type(m) is AXSLinearUnified for m in p)
                   and not any(m._warmup_active or m._forward_hooks or m._forward_pre_hooks for m in p)
                   and len({(m.block_size, m.quantize_input, m.quantize_grad) for m in p}) == 1)
        if not grouped:
            return self.q_proj(query), self.k_proj(key), self.v_proj(value)
        m = p[0]
        return axs_linear_group_unified(query, [x.weight for x in p], [x.bias for x in p], m.block_size,
                                        m.quantize_input, m.quantize_grad)

    def forward(self, query, key, value, attn_mask=None):
        B, T = query.shape[0], query.shape[1]
        qp, kp, vp = self._projections(query, key, value)
        q = qp.reshape(B, T, self.num_heads, self.head_dim).transpose(1, 2)
        k = kp.reshape(B, key.shape[1], self.num_heads, self.head_dim).transpose(1, 2)
        v = vp.reshape(B, value.shape[1], self.num_heads, self.head_dim).transpose(1, 2)
        scores = torch.matmul(q, k.transpose(-2, -1)) * self.scale
        if attn_mask is not None:
            scores = scores + attn_mask
        probs = F.softmax(scores, dim=-1)
        if self.dropout > 0 and self.training:
            probs = F.dropout(probs, p=self.dropout)
        probs = fake_quantize_unified(probs, self.block_size, "stochastic")
        out = torch.matmul(probs, v).transpose(1, 2).reshape(B, T, self.embed_dim)
        return self.out_proj(out)


def convert_to_axs_unified(
    model: nn.Module,
    block_size: int = DEFAULT_BLOCK_SIZE,
    quantize_input: bool = True,
    quantize_grad: bool = True,
    skip_layers: set[str] | None = None,
    inplace: bool = False,
) -> nn.Module:
    """Replace ``nn.Linear`` / ``nn.LayerNorm`` / ``nn.Embedding`` children with
    the unified AXS-6 modules, copying weights; ``skip_layers`` names
    (dotted paths) are left alone; RMSNorm and other norms are not touched."""
    if not inplace:
        model = copy.deepcopy(model)
    skip = set(skip_layers or ())

    def _convert(module: nn.Module, prefix: str = "") -> None:
        for name, child in module.named_children():
            full = f"{prefix}.{name}" if prefix else name
            if full in skip:
                continue
            if isinstance(child, nn.Linear):
                new = AXSLinearUnified(child.in_features, child.out_features, bias=child.bias is not None,
                                       block_size=block_size, quantize_input=quantize_input,
                                       quantize_grad=quantize_grad)
                new.weight.data.copy_(child.weight.data)
                if child.bias is not None:
                    new.bias.data.copy_(child.bias.data)
                setattr(module, name, new.to(child.weight.device))
            elif isinstance(child, nn.LayerNorm):
                new = AXSLayerNormUnified(list(child.normalized_shape), eps=child.eps)
                if child.weight is not None:
                    new.weight.data.copy_(child.weight.data)
                if child.bias is not None:
                    new.bias.data.copy_(child.bias.data)
                setattr(module, name, new.to(child.weight.device if child.weight is not None else "cpu"))
            elif isinstance(child, nn.Embedding):
                new = AXSEmbeddingUnified(child.num_embeddings, child.embedding_dim,
                                          padding_idx=child.padding_idx, block_size=block_size)
                new.weight.data.copy_(child.weight.data)
                setattr(module, name, new.to(child.weight.device))
            elif isinstance(child, getattr(nn, "RMSNorm", ())):
                continue
            else:
                _convert(child, full)

    _convert(model)
    return model
