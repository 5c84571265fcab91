"""AXS-6 unified training pipeline on the GPU.

The reference's ``axs.unified.training_unified`` (axs/unified/training_unified.py)
wraps a training step with skip-first-N warm-up, loss scaling with overflow
back-off, gradient clipping, an optional amax EMA, step metrics and
checkpointing.  Its step unscales every gradient with its own kernel, checks
every gradient for inf/NaN with two host-synchronising reductions per
parameter (``_check_overflow``, :287-292), then runs ``clip_grad_norm_`` and
reads the norm back -- on the order of 2 x (number of parameters) host
round trips per step.

Here the same class and API, with the unscale, the overflow count and the
global-norm clip done by ``axs6_multi_tensor_unscale_clip`` (libaxs6.so):
one pass over all gradients, a fixed-order reduction and a device-side clip,
then a single 4-value read (norm, clip coefficient, non-finite count, loss)
per step.  The decisions that follow (skip the optimiser step on overflow,
back off or grow the loss scale) are the reference's, made on that read.

Differences, on purpose:
  * the global norm is summed in a fixed order (per-workgroup fp32 partials,
    then fp64), so it is deterministic; torch's clip_grad_norm_ (per-tensor
    norms, then the norm of norms) differs from it in the last bits;
  * ``load_checkpoint`` uses ``torch.load(weights_only=True)`` -- model,
    optimiser, scheduler and RNG states load; an ``extra`` dict holding
    arbitrary Python objects does not (pass ``weights_only=False`` for files
    you wrote yourself);
  * gradients must be CUDA tensors (no CPU path, like every entry point of
    this package).
"""
from __future__ import annotations

import ctypes
import logging
import math
from pathlib import Path
from typing import Any, Callable

import torch
import torch.nn as nn
from torch.optim import Optimizer

from axs import _lib
from axs.unified.modules_unified import AXSEmbeddingUnified, AXSLinearUnified

logger = logging.getLogger(__name__)

__all__ = ["AmaxEMA", "AXSTrainingPipelineUnified", "unscale_and_clip_", "GradUnscaler"]


def _get_warmup_types() -> tuple[type, ...]:
    """Module types carrying a ``_warmup_active`` flag (training_unified.py:43-58)."""
    from axs.unified.mixed_precision import AXSLinearMixedPrecision

    return (AXSLinearUnified, AXSEmbeddingUnified, AXSLinearMixedPrecision)


class AmaxEMA:
    """Exponential moving average of per-tensor amax values
    (training_unified.py:63-108): ``update`` blends a new amax in with
    ``decay``; ``get_scale`` is the power of two ``2^(floor(log2 amax) + 1)``."""

    def __init__(self, decay: float = 0.999) -> None:
        self.decay = decay
        self._values: dict[str, float] = {}

    def update(self, name: str, amax: float) -> None:
        if name not in self._values:
            self._values[name] = amax
        else:
            self._values[name] = self.decay * self._values[name] + (1.0 - self.decay) * amax

    def get_amax(self, name: str, default: float = 1.0) -> float:
        return self._values.get(name, default)

    def get_scale(self, name: str, default: float = 1.0) -> float:
        amax = self.get_amax(name, default)
        if amax <= 0:
            return 1.0
        return 2.0 ** (math.floor(math.log2(amax)) + 1)

    def state_dict(self) -> dict[str, Any]:
        return {"decay": self.decay, "values": dict(self._values)}

    def load_state_dict(self, state: dict[str, Any]) -> None:
        self.decay = state["decay"]
        self._values = dict(state["values"])


class GradUnscaler:
    """Runs the fused unscale / overflow count / global-norm clip over a list
    of gradient tensors on one device.  Keeps its workspace between calls."""

    def __init__(self, device: torch.device) -> None:
        self.device = torch.device(device)
        self.result = torch.zeros(3, dtype=torch.float32, device=self.device)
        self._partials = torch.empty(2, dtype=torch.float32, device=self.device)

    def __call__(self, grads: list[torch.Tensor], loss_scale: float, max_norm: float,
                 clip: bool = True) -> torch.Tensor:
        """In place: g /= loss_scale, then (clip) g *= min(max_norm / (norm + 1e-6), 1)
        unless a non-finite value appeared.  Returns the device tensor
        (norm, clip coefficient, non-finite count)."""
        work, back = [], []
        for g in grads:
            if not g.is_cuda:
                raise RuntimeError("AXS-6 gradient unscale requires CUDA tensors")
            if g.device != self.device:
                raise RuntimeError(f"gradient on {g.device}, unscaler on {self.device}")
            if g.dtype not in _lib.DTYPE_CODE:
                raise TypeError(f"unsupported gradient dtype {g.dtype}")
            if g.is_contiguous():
                work.append(g)
            else:                                  # strided view: work on a copy, write it back
                c = g.contiguous()
                work.append(c)
                back.append((g, c))
        # one launch per dtype run: order the list by dtype (the norm is over all of them)
        work.sort(key=lambda t: _lib.DTYPE_CODE[t.dtype])
        n = len(work)
        ptrs = (ctypes.c_void_p * max(n, 1))(*[t.data_ptr() for t in work])
        numel = (ctypes.c_int64 * max(n, 1))(*[t.numel() for t in work])
        dts = (ctypes.c_int32 * max(n, 1))(*[_lib.DTYPE_CODE[t.dtype] for t in work])
        need = int(_lib.lib().axs6_multi_tensor_workspace(numel, n))
        if need > self._partials.numel():
            self._partials = torch.empty(need, dtype=torch.float32, device=self.device)
        with torch.cuda.device(self.device):
            st = torch.cuda.current_stream(self.device).cuda_stream
            _lib.call("axs6_multi_tensor_unscale_clip", ptrs, numel, dts, n, float(loss_scale), float(max_norm),
                      int(bool(clip)), self._partials.data_ptr(), self._partials.numel(), self.result.data_ptr(), st)
        for g, c in back:
            g.copy_(c)
        return self.result


_unscalers: dict[torch.device, GradUnscaler] = {}


def unscale_and_clip_(parameters, loss_scale: float = 1.0, max_norm: float = float("inf"),
                      clip: bool = True) -> torch.Tensor:
    """Functional form over ``parameters`` (their ``.grad``): returns the
    device tensor (total norm, clip coefficient, non-finite count)."""
    grads = [p.grad for p in parameters if p.grad is not None]
    if not grads:
        return torch.zeros(3)
    dev = grads[0].device
    u = _unscalers.get(dev)
    if u is None:
        u = _unscalers[dev] = GradUnscaler(dev)
    return u(grads, loss_scale, max_norm, clip)


class AXSTrainingPipelineUnified:
    """Training wrapper with the reference's features and API
    (training_unified.py:115-410): warm-up (quantisation bypassed for the
    first ``warmup_steps`` steps), adaptive loss scaling with overflow
    back-off, clipping at ``max_grad_norm``, optional amax EMA, step metrics,
    checkpoint save/load and a per-batch LR scheduler."""

    def __init__(
        self,
        model: nn.Module,
        optimizer: Optimizer,
        scheduler: Any | None = None,
        warmup_steps: int = 0,
        loss_scale_init: float = 2.0 ** 16,
        loss_scale_growth_interval: int = 2000,
        loss_scale_backoff: float = 0.5,
        loss_scale_growth: float = 2.0,
        max_grad_norm: float = 1.0,
        use_amax_ema: bool = False,
        amax_ema_decay: float = 0.999,
    ) -> None:
        self.model = model
        self.optimizer = optimizer
        self.scheduler = scheduler
        self.warmup_steps = warmup_steps
        self.loss_scale = loss_scale_init
        self._loss_scale_init = loss_scale_init
        self.growth_interval = loss_scale_growth_interval
        self.backoff = loss_scale_backoff
        self.growth = loss_scale_growth
        self.max_grad_norm = max_grad_norm
        self.amax_ema = AmaxEMA(decay=amax_ema_decay) if use_amax_ema else None
        self._steps_since_scale_change = 0
        self._total_steps = 0
        self._overflow_count = 0
        self._grad_norms: list[float] = []
        self._unscaler: GradUnscaler | None = None

    def _set_warmup(self, active: bool) -> None:
        warmup_types = _get_warmup_types()
        for module in self.model.modules():
            if isinstance(module, warmup_types):
                module._warmup_active = active  # type: ignore[union-attr]

    @property
    def is_warmup(self) -> bool:
        return self._total_steps < self.warmup_steps

    def _grads(self) -> list[torch.Tensor]:
        return [p.grad for p in self.model.parameters() if p.grad is not None]

    def _get_unscaler(self, grads: list[torch.Tensor]) -> GradUnscaler:
        dev = grads[0].device
        if self._unscaler is None or self._unscaler.device != dev:
            self._unscaler = GradUnscaler(dev)
        return self._unscaler

    def training_step(self, inputs: Any, loss_fn: Callable[..., torch.Tensor]) -> dict[str, Any]:
        """One step (training_unified.py:192-281).  Returns ``loss``,
        ``loss_scale``, ``grad_norm``, ``overflow``, ``step``, ``warmup``, ``lr``."""
        self.model.train()
        self.optimizer.zero_grad()
        warmup = self.is_warmup
        self._set_warmup(warmup)

        output = self.model(inputs)
        loss = loss_fn(output, inputs)
        (loss * self.loss_scale).backward()

        grads = self._grads()
        if grads:
            res = self._get_unscaler(grads)(grads, self.loss_scale, self.max_grad_norm, clip=True)
            vals = torch.cat([res, loss.detach().reshape(1).to(torch.float32)]).cpu().tolist()
        else:
            vals = [0.0, 1.0, 0.0, float(loss.detach())]
        norm, _coef, nonfinite, loss_val = vals

        if nonfinite > 0:
            self.loss_scale *= self.backoff
            self._steps_since_scale_change = 0
            self._overflow_count += 1
            self.optimizer.zero_grad()
            return {"loss": loss_val, "loss_scale": self.loss_scale, "grad_norm": 0.0, "overflow": True,
                    "step": self._total_steps, "warmup": warmup, "lr": self._current_lr()}

        self._grad_norms.append(norm)
        self.optimizer.step()
        from axs.unified.backend import clear_int8_weight_cache

        clear_int8_weight_cache()
        if self.scheduler is not None:
            self.scheduler.step()
        self._steps_since_scale_change += 1
        if self._steps_since_scale_change >= self.growth_interval:
            self.loss_scale *= self.growth
            self._steps_since_scale_change = 0
        self._total_steps += 1
        return {"loss": loss_val, "loss_scale": self.loss_scale, "grad_norm": norm, "overflow": False,
                "step": self._total_steps, "warmup": warmup, "lr": self._current_lr()}

    def _current_lr(self) -> float:
        return self.optimizer.param_groups[0]["lr"]

    def _check_overflow(self) -> bool:
        """Whether any gradient holds inf or NaN (one fused pass, no division)."""
        grads = self._grads()
        if not grads:
            return False
        res = self._get_unscaler(grads)(grads, 1.0, float("inf"), clip=False)
        return float(res[2].item()) > 0

    def save_checkpoint(self, path: str | Path, *, extra: dict[str, Any] | None = None) -> Path:
        """Model, optimiser, scheduler, loss-scale and step state, amax EMA and
        RNG states (training_unified.py:298-347)."""
        path = Path(path)
        path.parent.mkdir(parents=True, exist_ok=True)
        state: dict[str, Any] = {
            "model": self.model.state_dict(),
            "optimizer": self.optimizer.state_dict(),
            "total_steps": self._total_steps,
            "loss_scale": self.loss_scale,
            "steps_since_scale_change": self._steps_since_scale_change,
            "overflow_count": self._overflow_count,
            "warmup_steps": self.warmup_steps,
        }
        if self.scheduler is not None:
            state["scheduler"] = self.scheduler.state_dict()
        if self.amax_ema is not None:
            state["amax_ema"] = self.amax_ema.state_dict()
        state["rng"] = {
            "python": torch.random.get_rng_state(),
            "cuda": torch.cuda.get_rng_state() if torch.cuda.is_available() else None,
        }
        if extra is not None:
            state["extra"] = extra
        torch.save(state, path)
        logger.info("Saved checkpoint to %s (step %d)", path, self._total_steps)
        return path

    def load_checkpoint(self, path: str | Path, *, map_location: str | torch.device | None = None,
                        weights_only: bool = True) -> dict[str, Any]:
        """Restores what ``save_checkpoint`` wrote (training_unified.py:349-395);
        returns the ``extra`` dict (``{}`` if none)."""
        path = Path(path)
        state = torch.load(path, map_location=map_location, weights_only=weights_only)
        self.model.load_state_dict(state["model"])
        self.optimizer.load_state_dict(state["optimizer"])
        self._total_steps = state["total_steps"]
        self.loss_scale = state["loss_scale"]
        self._steps_since_scale_change = state.get("steps_since_scale_change", 0)
        self._overflow_count = state.get("overflow_count", 0)
        self.warmup_steps = state.get("warmup_steps", self.warmup_steps)
        if self.scheduler is not None and "scheduler" in state:
            self.scheduler.load_state_dict(state["scheduler"])
        if self.amax_ema is not None and "amax_ema" in state:
            self.amax_ema.load_state_dict(state["amax_ema"])
        rng = state.get("rng", {})
        if rng.get("python") is not None:
            torch.random.set_rng_state(rng["python"])
        if rng.get("cuda") is not None and torch.cuda.is_available():
            torch.cuda.set_rng_state(rng["cuda"])
        logger.info("Loaded checkpoint from %s (step %d)", path, self._total_steps)
        return state.get("extra", {})

    @property
    def stats(self) -> dict[str, Any]:
        """Training statistics (training_unified.py:397-410)."""
        recent = self._grad_norms[-100:] if self._grad_norms else [0.0]
        return {
            "total_steps": self._total_steps,
            "overflow_count": self._overflow_count,
            "current_loss_scale": self.loss_scale,
            "is_warmup": self.is_warmup,
            "warmup_steps": self.warmup_steps,
            "avg_grad_norm_recent": sum(recent) / len(recent),
            "max_grad_norm_recent": max(recent),
            "amax_ema_active": self.amax_ema is not None,
            "lr": self._current_lr(),
        }
