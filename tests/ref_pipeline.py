"""Test-side restatement of the reference's training step
(axs/unified/training_unified.py:192-292) with plain torch operations: the
per-parameter unscale (``grad.div_(loss_scale)``, :224-227), the
per-parameter inf/NaN check (``_check_overflow``, :287-292), the overflow
back-off (:230-245), ``clip_grad_norm_`` (:248-252), the optimiser and
scheduler steps and the loss-scale growth (:265-270).  It is the checker for
``axs.unified.AXSTrainingPipelineUnified`` and the timing comparison in
bench.py; the product never calls it."""
from __future__ import annotations

from typing import Any, Callable

import torch
import torch.nn as nn


class RefPipeline:
    def __init__(self, model: nn.Module, optimizer, scheduler=None, warmup_steps: int = 0,
                 loss_scale_init: float = 2.0 ** 16, loss_scale_growth_interval: int = 2000,
                 loss_scale_backoff: float = 0.5, loss_scale_growth: float = 2.0,
                 max_grad_norm: float = 1.0) -> None:
        self.model = model
        self.optimizer = optimizer
        self.scheduler = scheduler
        self.warmup_steps = warmup_steps
        self.loss_scale = loss_scale_init
        self.growth_interval = loss_scale_growth_interval
        self.backoff = loss_scale_backoff
        self.growth = loss_scale_growth
        self.max_grad_norm = max_grad_norm
        self._steps_since_scale_change = 0
        self._total_steps = 0
        self._overflow_count = 0

    def _set_warmup(self, active: bool) -> None:
        for m in self.model.modules():
            if hasattr(m, "_warmup_active"):
                m._warmup_active = active

    def _check_overflow(self) -> bool:
        for p in self.model.parameters():
            if p.grad is not None:
                if torch.any(torch.isinf(p.grad)) or torch.any(torch.isnan(p.grad)):
                    return True
        return False

    def training_step(self, inputs: Any, loss_fn: Callable[..., torch.Tensor]) -> dict[str, Any]:
        self.model.train()
        self.optimizer.zero_grad()
        warmup = self._total_steps < self.warmup_steps
        self._set_warmup(warmup)
        output = self.model(inputs)
        loss = loss_fn(output, inputs)
        (loss * self.loss_scale).backward()
        for p in self.model.parameters():
            if p.grad is not None:
                p.grad.data.div_(self.loss_scale)
        if self._check_overflow():
            self.loss_scale *= self.backoff
            self._steps_since_scale_change = 0
            self._overflow_count += 1
            self.optimizer.zero_grad()
            return {"loss": loss.item(), "loss_scale": self.loss_scale, "grad_norm": 0.0, "overflow": True,
                    "step": self._total_steps, "warmup": warmup}
        grad_norm = torch.nn.utils.clip_grad_norm_(self.model.parameters(), self.max_grad_norm)
        grad_norm_val = grad_norm.item() if isinstance(grad_norm, torch.Tensor) else grad_norm
        self.optimizer.step()
        if self.scheduler is not None:
            self.scheduler.step()
        self._steps_since_scale_change += 1
        if self._steps_since_scale_change >= self.growth_interval:
            self.loss_scale *= self.growth
            self._steps_since_scale_change = 0
        self._total_steps += 1
        return {"loss": loss.item(), "loss_scale": self.loss_scale, "grad_norm": grad_norm_val, "overflow": False,
                "step": self._total_steps, "warmup": warmup}
