"""BASELINE config 5 workload: a MiniGPT training step with every nn.Linear
replaced by the AXS-6 quantized linear.

Architecture of the reference's example trainer (examples/pretrain_gpt.py:57-67
for the dimensions, :91-170 for the model): token embedding + learned position
embedding, 4 pre-LN decoder blocks (causal self-attention, GELU FFN), final LN
and an LM head; d_model 256, 4 heads, FFN 1024, vocab 256, context 128.
Differences, chosen so that "every nn.Linear" is meaningful and the run is
deterministic up to the gradient dither:
  * attention uses explicit q/k/v/o nn.Linear layers (nn.MultiheadAttention's
    fused in-projection is not an nn.Linear, and its forward reads
    out_proj.weight directly, so converting it would quantize nothing); the
    q/k/v layers of the one input run as one stacked linear, as
    nn.MultiheadAttention's in-projection does (fp32: one F.linear over the
    stacked weights; AXS-6: the library's grouped linear, the input packed
    once), while the CPU reference restatement runs them one by one;
  * dropout 0 and no weight tying (the head is its own nn.Linear).

Two builds of the same model and initial weights:
  * :func:`build_axs` -- ``axs.unified.convert_to_axs_unified`` (the product:
    Linear -> AXSLinearUnified, Embedding -> AXSEmbeddingUnified, LayerNorm ->
    AXSLayerNormUnified), trained on the GPU;
  * :func:`build_reference` -- test-side modules that restate the reference's
    eager CPU path (oracle.eager_torch, itself pinned to the reference by the
    golden vectors): FQ(W), FQ(X), fp32 F.linear forward; stochastic FQ(dY),
    fp32 matmuls backward (axs/unified/functional_unified.py:107-170,
    axs/unified/backend.py:644-645); FQ of the gathered embedding rows with an
    identity backward (axs/unified/modules_unified.py:151-189).
The oracle is the checker here; the product path never calls it.

Data: one fixed batch of 64 sequences of 129 tokens drawn uniformly from the
vocabulary (seeded), inputs tokens[:, :-1], targets tokens[:, 1:] -- the model
memorises it, as in the reference's training benchmark
(benchmarks/benchmark_triton.py:76-102, which also reuses one batch).
Optimiser: AdamW, lr 3e-4, torch defaults otherwise, fp32 master weights.
"""
from __future__ import annotations

import math
import time
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F


@dataclass
class GPTConfig:
    vocab_size: int = 256
    context_len: int = 128
    embed_dim: int = 256
    num_heads: int = 4
    num_layers: int = 4
    ff_dim: int = 1024
    batch: int = 64
    lr: float = 3e-4


class CausalSelfAttention(nn.Module):
    def __init__(self, c: GPTConfig) -> None:
        super().__init__()
        self.h = c.num_heads
        self.hd = c.embed_dim // c.num_heads
        self.q_proj = nn.Linear(c.embed_dim, c.embed_dim)
        self.k_proj = nn.Linear(c.embed_dim, c.embed_dim)
        self.v_proj = nn.Linear(c.embed_dim, c.embed_dim)
        self.out_proj = nn.Linear(c.embed_dim, c.embed_dim)

    def _qkv(self, x: torch.Tensor) -> tuple[torch.Tensor, ...]:
        """The three projections of the one input as one stacked linear: a
        plain fp32 F.linear over the stacked weights for nn.Linear layers, the
        library's grouped quantized linear for AXS-6 ones (the input packed
        once); the CPU reference restatement runs them one by one, as the
        reference does.  Every layer keeps its own weight and bias."""
        ps = (self.q_proj, self.k_proj, self.v_proj)
        if all(type(p) is nn.Linear for p in ps):
            y = F.linear(x, torch.cat([p.weight for p in ps]), torch.cat([p.bias for p in ps]))
            return y.split(x.shape[-1], dim=-1)
        if all(type(p).__name__ == "AXSLinearUnified" for p in ps) and not any(p._warmup_active for p in ps):
            from axs.unified import axs_linear_group_unified

            q = ps[0]
            return axs_linear_group_unified(x, [p.weight for p in ps], [p.bias for p in ps], q.block_size,
                                            q.quantize_input, q.quantize_grad)
        return tuple(p(x) for p in ps)

    def forward(self, x: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
        B, T, D = x.shape
        qp, kp, vp = self._qkv(x)
        q = qp.reshape(B, T, self.h, self.hd).transpose(1, 2)
        k = kp.reshape(B, T, self.h, self.hd).transpose(1, 2)
        v = vp.reshape(B, T, self.h, self.hd).transpose(1, 2)
        # fp32 attention; the transposed operand is made contiguous before the
        # batched product
        s = torch.matmul(q, k.transpose(-2, -1).contiguous()) * (self.hd ** -0.5) + mask
        p = F.softmax(s, dim=-1)
        o = torch.matmul(p, v).transpose(1, 2).reshape(B, T, D)
        return self.out_proj(o)


class Block(nn.Module):
    def __init__(self, c: GPTConfig) -> None:
        super().__init__()
        self.ln1 = nn.LayerNorm(c.embed_dim)
        self.attn = CausalSelfAttention(c)
        self.ln2 = nn.LayerNorm(c.embed_dim)
        self.fc1 = nn.Linear(c.embed_dim, c.ff_dim)
        self.fc2 = nn.Linear(c.ff_dim, c.embed_dim)

    def forward(self, x: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
        x = x + self.attn(self.ln1(x), mask)
        return x + self.fc2(F.gelu(self.fc1(self.ln2(x))))


class MiniGPT(nn.Module):
    def __init__(self, c: GPTConfig) -> None:
        super().__init__()
        self.c = c
        self.token_embed = nn.Embedding(c.vocab_size, c.embed_dim)
        self.pos_embed = nn.Parameter(torch.randn(1, c.context_len, c.embed_dim) * 0.02)
        self.blocks = nn.ModuleList([Block(c) for _ in range(c.num_layers)])
        self.ln_f = nn.LayerNorm(c.embed_dim)
        self.head = nn.Linear(c.embed_dim, c.vocab_size, bias=False)
        for m in self.modules():
            if isinstance(m, nn.Linear):
                nn.init.normal_(m.weight, std=0.02)
                if m.bias is not None:
                    nn.init.zeros_(m.bias)
            elif isinstance(m, nn.Embedding):
                nn.init.normal_(m.weight, std=0.02)

    def forward(self, idx: torch.Tensor) -> torch.Tensor:
        T = idx.shape[1]
        mask = torch.triu(torch.full((T, T), float("-inf"), device=idx.device), diagonal=1)
        x = self.token_embed(idx) + self.pos_embed[:, :T, :]
        for b in self.blocks:
            x = b(x, mask)
        return self.head(self.ln_f(x))


def base_model(seed: int = 0, c: GPTConfig | None = None) -> MiniGPT:
    """fp32 model with seeded initial weights (CPU)."""
    torch.manual_seed(seed)
    return MiniGPT(c or GPTConfig())


def batch(seed: int = 1, c: GPTConfig | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    c = c or GPTConfig()
    g = torch.Generator().manual_seed(seed)
    tok = torch.randint(0, c.vocab_size, (c.batch, c.context_len + 1), generator=g)
    return tok[:, :-1].contiguous(), tok[:, 1:].contiguous()


def build_axs(seed: int = 0, device: str = "cuda", c: GPTConfig | None = None) -> nn.Module:
    from axs.unified import convert_to_axs_unified

    return convert_to_axs_unified(base_model(seed, c)).to(device)


# ---- CPU restatement of the reference's eager modules (test side) -----------

class _RefLinearFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, b, quantize_grad):
        from oracle import eager_torch

        y, xq = eager_torch.linear_fwd(x, w, b)
        ctx.save_for_backward(xq, w)
        ctx.has_bias = b is not None
        ctx.quantize_grad = quantize_grad
        return y

    @staticmethod
    def backward(ctx, dy):
        from oracle import eager_torch

        xq, w = ctx.saved_tensors
        dx, dw, db = eager_torch.linear_bwd(dy, xq, w, 32, ctx.quantize_grad)
        return dx, dw, (db if ctx.has_bias else None), None


class _RefFQ(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        from oracle import eager_torch

        return eager_torch.fake_quantize(x, 32)

    @staticmethod
    def backward(ctx, g):
        return g


class RefLinear(nn.Module):
    def __init__(self, lin: nn.Linear, quantize_grad: bool = True) -> None:
        super().__init__()
        self.weight = nn.Parameter(lin.weight.detach().clone())
        self.bias = None if lin.bias is None else nn.Parameter(lin.bias.detach().clone())
        self.quantize_grad = quantize_grad

    def forward(self, x):
        return _RefLinearFn.apply(x, self.weight, self.bias, self.quantize_grad)


class RefEmbedding(nn.Module):
    def __init__(self, emb: nn.Embedding) -> None:
        super().__init__()
        self.weight = nn.Parameter(emb.weight.detach().clone())

    def forward(self, idx):
        return _RefFQ.apply(F.embedding(idx, self.weight))


def build_reference(seed: int = 0, quantize_grad: bool = True, c: GPTConfig | None = None) -> nn.Module:
    """The same initial model, with the reference's eager NF5 path (CPU)."""
    model = base_model(seed, c)

    def swap(mod: nn.Module) -> None:
        for name, child in mod.named_children():
            if isinstance(child, nn.Linear):
                setattr(mod, name, RefLinear(child, quantize_grad))
            elif isinstance(child, nn.Embedding):
                setattr(mod, name, RefEmbedding(child))
            else:
                swap(child)

    swap(model)
    return model


# ---- training loop ----------------------------------------------------------

def train(model: nn.Module, x: torch.Tensor, y: torch.Tensor, steps: int, lr: float = 3e-4,
          warmup: int = 0, sync=None, capturable: bool = False, fused: bool = False) -> tuple[list[float], float]:
    """AdamW steps on one batch.  Returns (loss per step, ms per timed step).
    The first ``warmup`` steps are untimed but part of the curve.
    ``capturable`` selects AdamW's device-side step arithmetic (the form a
    graph-replayed step uses); ``fused`` selects torch's fused AdamW (one
    multi-tensor update kernel, device-side step counts) instead of the
    default multi-tensor form."""
    opt = torch.optim.AdamW(model.parameters(), lr=lr, capturable=capturable, fused=fused)
    losses = []
    t0 = None
    for i in range(steps):
        if i == warmup:
            if sync:
                sync()
            t0 = time.perf_counter()
        logits = model(x)
        loss = F.cross_entropy(logits.reshape(-1, logits.shape[-1]), y.reshape(-1))
        opt.zero_grad(set_to_none=True)
        loss.backward()
        opt.step()
        losses.append(loss.detach())
    if sync:
        sync()
    ms = (time.perf_counter() - t0) * 1e3 / max(steps - warmup, 1) if t0 is not None else float("nan")
    return [float(v) for v in losses], ms


def train_graphed(model: nn.Module, x: torch.Tensor, y: torch.Tensor, steps: int, lr: float = 3e-4,
                  warmup: int = 3, fused: bool = False) -> tuple[list[float], float]:
    """The same AdamW training, with the step recorded once in a HIP graph and
    replayed: forward, loss, backward and the optimiser update run as one
    graph launch (AdamW with capturable state; ``fused`` selects torch's fused
    AdamW, whose one update kernel replaces the capturable multi-tensor form's
    two per-parameter broadcast divisions).  The first ``warmup`` steps run
    eagerly on a side stream (they initialise the optimiser state and the
    allocator pools) and are part of the loss curve; the replays are timed.
    Stochastic FQ calls inside the graph read a device counter the library
    advances after each of them, so every replay draws a fresh dither.
    Returns (loss per step, ms per replayed step)."""
    opt = torch.optim.AdamW(model.parameters(), lr=lr, capturable=True, fused=fused)

    def step():
        logits = model(x)
        loss = F.cross_entropy(logits.reshape(-1, logits.shape[-1]), y.reshape(-1))
        loss.backward()
        opt.step()
        return loss

    losses = []
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(warmup):
            opt.zero_grad(set_to_none=True)
            losses.append(step().detach().clone())
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    opt.zero_grad(set_to_none=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_loss = step()
    n = steps - warmup
    hist = torch.empty(n, device=x.device)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(n):
        graph.replay()
        hist[i].copy_(static_loss)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / max(n, 1)
    return [float(v) for v in losses] + hist.tolist(), ms


UNIFORM_LOSS = math.log(256.0)


if __name__ == "__main__":
    # `python tests/minigpt.py --steps 15`: the eager AXS training loop on the
    # GPU (for kernel traces of one training step)
    import argparse
    import os
    import sys

    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "axs-6_amd"))
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=15)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--graph", action="store_true", help="record the step in a HIP graph and replay it")
    ap.add_argument("--fused-adamw", action="store_true", help="torch's fused AdamW")
    a = ap.parse_args()
    xb, yb = batch(1)
    torch.manual_seed(5)
    m = build_axs(0, "cuda")
    if a.graph:
        losses, ms = train_graphed(m, xb.cuda(), yb.cuda(), a.steps, warmup=a.warmup, fused=a.fused_adamw)
    else:
        losses, ms = train(m, xb.cuda(), yb.cuda(), a.steps, warmup=a.warmup, sync=torch.cuda.synchronize,
                           fused=a.fused_adamw)
    print(f"minigpt {'graph' if a.graph else 'eager'}: {ms:.3f} ms/step over {a.steps - a.warmup} steps, "
          f"loss {losses[0]:.4f} -> {losses[-1]:.4f}", flush=True)
