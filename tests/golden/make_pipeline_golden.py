"""Write the fixture that pins the test-side restatement of the reference's
training step (tests/ref_pipeline.py) to the reference itself.

Run once, in the build container where the reference is mounted:

    python tests/golden/make_pipeline_golden.py /root/reference

It imports the reference's AXSTrainingPipelineUnified
(axs/unified/training_unified.py:142-292) and runs it on a small plain-torch
model on the CPU (one thread): loss scaling, the per-parameter unscale and
overflow check with its back-off (overflow forced at two steps by a loss
that overflows once scaled), gradient clipping, the optimiser and scheduler
steps and the loss-scale growth.  Data only goes to pipeline.npz beside this
script: the inputs' seeds are fixed here, the per-step results and the final
parameters are saved.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch
import torch.nn as nn

HERE = os.path.dirname(os.path.abspath(__file__))
STEPS = 12
OVERFLOW_AT = (4, 5)          # calls of the loss function whose scaled loss overflows


def setup():
    """(model, optimizer, scheduler, inputs, loss_fn) -- identical for the
    reference and the restatement."""
    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(16, 32), nn.Tanh(), nn.Linear(32, 4))
    opt = torch.optim.SGD(model.parameters(), lr=0.1, momentum=0.9)
    sched = torch.optim.lr_scheduler.LambdaLR(opt, lambda s: 1.0 / (1.0 + 0.1 * s))
    g = torch.Generator().manual_seed(1)
    x = torch.randn(8, 16, generator=g)
    y = torch.randn(8, 4, generator=g)
    calls = [0]

    def loss_fn(out, inputs):
        calls[0] += 1
        loss = ((out - y) ** 2).mean()
        return loss * 1e35 if calls[0] in OVERFLOW_AT else loss

    return model, opt, sched, x, loss_fn


PIPELINE_ARGS = dict(warmup_steps=2, loss_scale_init=2.0 ** 16, loss_scale_growth_interval=3,
                     loss_scale_backoff=0.5, loss_scale_growth=2.0, max_grad_norm=0.5)


def run(pipeline_cls):
    torch.set_num_threads(1)
    model, opt, sched, x, loss_fn = setup()
    p = pipeline_cls(model, opt, scheduler=sched, **PIPELINE_ARGS)
    rows = []
    for _ in range(STEPS):
        r = p.training_step(x, loss_fn)
        rows.append([r["loss"], r["loss_scale"], r["grad_norm"], float(r["overflow"]), float(r["step"]),
                     float(r["warmup"])])
    params = [t.detach().numpy().copy() for t in model.parameters()]
    return np.array(rows, np.float64), params


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from axs.unified.training_unified import AXSTrainingPipelineUnified  # noqa: E402  (reference)

    rows, params = run(AXSTrainingPipelineUnified)
    np.savez_compressed(os.path.join(HERE, "pipeline.npz"), steps=rows,
                        **{f"param{i}": a for i, a in enumerate(params)})
    print("wrote pipeline.npz:", rows[:, [1, 3]].tolist())


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
