"""CPU tests of the training pipeline's host logic: AmaxEMA against its
defining formulas (training_unified.py:63-108), constructor defaults and
stats keys (:142-178, :397-410), checkpoint round trip (:298-395), and the
no-CPU-path rule of the gradient unscale."""
from __future__ import annotations

import math

import pytest
import torch
import torch.nn as nn


def test_amax_ema_formulas():
    from axs.unified import AmaxEMA

    e = AmaxEMA(decay=0.9)
    assert e.get_amax("w") == 1.0 and e.get_scale("w") == 2.0         # default 1.0 -> 2^(0+1)
    e.update("w", 3.0)
    assert e.get_amax("w") == 3.0                                      # first value taken as is
    e.update("w", 5.0)
    assert e.get_amax("w") == pytest.approx(0.9 * 3.0 + 0.1 * 5.0)
    assert e.get_scale("w") == 2.0 ** (math.floor(math.log2(3.2)) + 1) == 4.0
    e.update("z", 0.0)
    assert e.get_scale("z") == 1.0                                     # amax <= 0 -> 1
    e.update("p", 4.0)
    assert e.get_scale("p") == 8.0                                     # power of two: next one up
    e2 = AmaxEMA()
    e2.load_state_dict(e.state_dict())
    assert e2.decay == 0.9 and e2.get_amax("w") == e.get_amax("w")


def _pipeline(**kw):
    from axs.unified import AXSLinearUnified, AXSTrainingPipelineUnified

    torch.manual_seed(0)
    model = nn.Sequential(AXSLinearUnified(32, 64), nn.ReLU(), AXSLinearUnified(64, 8))
    opt = torch.optim.AdamW(model.parameters(), lr=1e-3)
    sched = torch.optim.lr_scheduler.StepLR(opt, step_size=10, gamma=0.5)
    return model, opt, sched, AXSTrainingPipelineUnified(model, opt, sched, **kw)


def test_pipeline_defaults_and_stats():
    _, _, _, p = _pipeline()
    assert p.loss_scale == 2.0 ** 16 and p.growth_interval == 2000 and p.backoff == 0.5 and p.growth == 2.0
    assert p.max_grad_norm == 1.0 and p.amax_ema is None and not p.is_warmup
    s = p.stats
    assert set(s) == {"total_steps", "overflow_count", "current_loss_scale", "is_warmup", "warmup_steps",
                      "avg_grad_norm_recent", "max_grad_norm_recent", "amax_ema_active", "lr"}
    _, _, _, p2 = _pipeline(warmup_steps=3, use_amax_ema=True, amax_ema_decay=0.5)
    assert p2.is_warmup and p2.amax_ema is not None and p2.amax_ema.decay == 0.5


def test_checkpoint_round_trip(tmp_path):
    model, opt, sched, p = _pipeline(use_amax_ema=True)
    p.loss_scale = 1234.0
    p._total_steps, p._steps_since_scale_change, p._overflow_count = 7, 3, 2
    p.amax_ema.update("x", 2.5)
    sched.step()
    path = p.save_checkpoint(tmp_path / "ck" / "state.pt", extra={"epoch": 4})
    want = {k: v.clone() for k, v in model.state_dict().items()}

    model2, opt2, sched2, q = _pipeline(use_amax_ema=True)
    with torch.no_grad():
        for prm in model2.parameters():
            prm.add_(1.0)
    extra = q.load_checkpoint(path)
    assert extra == {"epoch": 4}
    assert all(torch.equal(model2.state_dict()[k], v) for k, v in want.items())
    assert q.loss_scale == 1234.0 and q._total_steps == 7 and q._steps_since_scale_change == 3
    assert q._overflow_count == 2 and q.amax_ema.get_amax("x") == 2.5
    assert sched2.state_dict()["last_epoch"] == sched.state_dict()["last_epoch"]


def test_unscale_rejects_cpu_gradients():
    from axs.unified.training_unified import unscale_and_clip_

    w = nn.Parameter(torch.ones(4))
    w.grad = torch.ones(4)
    with pytest.raises(RuntimeError, match="CUDA"):
        unscale_and_clip_([w], 2.0, 1.0)


def test_reference_style_pipeline_matches_the_reference_fixture():
    """tests/ref_pipeline.py (the checker of AXSTrainingPipelineUnified and the
    bench's reference-style timing) against tests/golden/pipeline.npz, which
    the reference's own AXSTrainingPipelineUnified wrote on the same model,
    data and schedule (make_pipeline_golden.py): loss-scale growth, two
    forced overflows with back-off, clipping, SGD with momentum and a
    LambdaLR scheduler -- every returned value and the final parameters
    bit for bit."""
    import os
    import sys

    import numpy as np

    from conftest import GOLDEN, load_golden

    sys.path.insert(0, GOLDEN)
    import make_pipeline_golden as mk
    from ref_pipeline import RefPipeline

    want = load_golden("pipeline.npz")
    rows, params = mk.run(RefPipeline)
    assert np.array_equal(rows, want["steps"]), (rows, want["steps"])
    assert rows[:, 3].tolist().count(1.0) == len(mk.OVERFLOW_AT)
    for i, a in enumerate(params):
        assert np.array_equal(a.view(np.uint32), want[f"param{i}"].view(np.uint32)), i
