"""The reference's eager CPU path, restated op for op in torch -- TEST
INFRASTRUCTURE / CPU BASELINE ONLY.

``bench.py``'s ``cpu_baseline`` leg times these functions on the GPU box's
host cores: they issue the same sequence of full-tensor torch operations as
the reference's eager path (pad, reshape, sign, abs, amax, clamp, log2,
floor, exp2, masked_fill, divide, clamp, multiply, int32 cast, clamp, int64
index, gather, two multiplies, trim, cast), so their time is the time of the
reference's CPU eager path on that host.  ``tests/test_oracle_eager.py``
holds them bit-identical to the C oracle and the golden vectors.

  fake_quantize  -> axs/unified/quantize_unified.py:121-204
  linear_fwd     -> axs/unified/functional_unified.py:107-131 (CPU: fp32 F.linear)
  linear_bwd     -> axs/unified/functional_unified.py:134-170 (CPU: fp32 matmul,
                    axs/unified/backend.py:644-645)
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

import oracle

_cb, _lut, _rev = oracle.tables()
LUT = torch.from_numpy(_lut.copy())
LUT_MAX_IDX = 1023


def fake_quantize(x: torch.Tensor, block_size: int = 32, rounding: str = "nearest") -> torch.Tensor:
    shape, dtype = x.shape, x.dtype
    flat = x.reshape(-1, x.shape[-1]).float()
    cols = flat.shape[-1]
    pad = (block_size - cols % block_size) % block_size
    if pad:
        flat = F.pad(flat, (0, pad))
    nblk = flat.shape[-1] // block_size
    blocks = flat.reshape(-1, nblk, block_size)
    sgn = blocks.sign()
    mag = blocks.abs()
    amax = mag.amax(dim=-1, keepdim=True)
    scale = torch.exp2(amax.clamp(min=1e-45).log2().floor() + 1.0)
    scale = scale.masked_fill(amax == 0, 1.0)
    n = (mag / scale).clamp(0.0, 1.0)
    if rounding == "stochastic":
        n = n + (torch.rand_like(n) - 0.5) / LUT_MAX_IDX
    idx = (n * LUT_MAX_IDX).to(torch.int32).clamp(0, LUT_MAX_IDX)
    out = sgn * LUT[idx.long()] * scale
    out = out.reshape(-1, nblk * block_size)
    if pad:
        out = out[:, :cols]
    return out.reshape(shape).to(dtype)


def linear_fwd(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None, block_size: int = 32):
    """Returns (Y, Xq): FQ(W), FQ(X), F.linear in fp32."""
    wq = fake_quantize(w, block_size)
    xq = fake_quantize(x, block_size)
    return F.linear(xq, wq, b), xq


def linear_bwd(dy: torch.Tensor, xq: torch.Tensor, w: torch.Tensor, block_size: int = 32,
               quantize_grad: bool = True):
    """Returns (dX, dW, db) with the reference's CPU operations."""
    wq = fake_quantize(w, block_size)
    if quantize_grad:
        dy = fake_quantize(dy, block_size, "stochastic")
    dx = torch.matmul(dy, wq)
    dw = torch.matmul(dy.reshape(-1, dy.shape[-1]).t().contiguous(), xq.reshape(-1, xq.shape[-1]))
    db = dy.sum(dim=tuple(range(dy.ndim - 1)))
    return dx, dw, db
