"""GPU tests of the training-step glue: the fused gradient unscale / overflow
count / global-norm clip (`axs6_multi_tensor_unscale_clip`) against torch's
own operations -- the ones the reference's training step calls
(training_unified.py:224-257: `grad.div_`, `isinf`/`isnan`,
`clip_grad_norm_`) -- and `AXSTrainingPipelineUnified` against the
test-side restatement of the reference step (tests/ref_pipeline.py)."""
from __future__ import annotations

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

import minigpt
from ref_pipeline import RefPipeline

pytestmark = pytest.mark.gpu

DEV = "cuda:0"

# sizes around the kernel's 16384-element chunk and 16-byte vectors; with the
# repeats below the list holds 66 tensors, more than one launch's table
SIZES = [1, 3, 17, 256, 1000, 16383, 16384, 16385, 65543, 4096 * 33]


def _grads(dtype, scale, seed, offset_views=True):
    g = torch.Generator(device=DEV).manual_seed(seed)
    out = []
    for rep in range(6):
        for i, n in enumerate(SIZES):
            if offset_views and (i + rep) % 3 == 0:
                # a view at an odd element offset of a larger buffer: not 16-byte aligned
                buf = torch.randn(n + 5, generator=g, device=DEV).to(dtype)
                t = buf[1 + rep % 3: 1 + rep % 3 + n]
            else:
                t = torch.randn(n, generator=g, device=DEV).to(dtype)
            out.append(t.mul_(scale) if dtype == torch.float32 else t)
    return out


def _params(grads):
    ps = []
    for t in grads:
        p = nn.Parameter(torch.empty_like(t))
        p.grad = t
        ps.append(p)
    return ps


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("loss_scale", [2.0 ** 16, 1000.0])
@pytest.mark.parametrize("max_norm", [0.5, 1e9], ids=["clipping", "no_clip"])
def test_unscale_clip_matches_torch(dtype, loss_scale, max_norm):
    from axs.unified.training_unified import unscale_and_clip_

    scale = loss_scale if dtype == torch.float32 else 1.0     # keep 16-bit gradients in range
    base = _grads(dtype, scale, 11)
    ours = [t.clone() for t in base]
    ref = [t.clone() for t in base]
    # torch, as the reference step does it: per-tensor division, then clip_grad_norm_
    # (a GPU div_ by a scalar multiplies by its fp32 reciprocal; loss scale
    # 1000 tells that apart from an IEEE division)
    for t in ref:
        t.div_(loss_scale)
    unscaled = [t.clone() for t in ref]
    total = torch.nn.utils.clip_grad_norm_(_params(ref), max_norm)

    res = unscale_and_clip_(_params(ours), loss_scale, max_norm).cpu()
    assert res[2].item() == 0
    # torch returns the norm of 16-bit gradients in that 16-bit type (~3
    # significant digits); the fused pass keeps it in fp32
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert abs(res[0].item() - total.float().item()) <= tol * total.float().item(), (res[0].item(), total.item())
    coef = torch.clamp(torch.tensor(max_norm, dtype=torch.float32) / (res[0] + 1e-6), max=1.0)
    assert res[1].item() == coef.item()
    for o, u, r in zip(ours, unscaled, ref):
        want = (u.float() * coef.to(DEV)).to(dtype) if coef.item() < 1.0 else u
        assert torch.equal(o.view(torch.int16) if dtype != torch.float32 else o.view(torch.int32),
                           want.view(torch.int16) if dtype != torch.float32 else want.view(torch.int32))
        # torch clips with its own (16-bit) norm: a coefficient ~1e-3 away moves
        # f16 subnormals (step 2^-24) by a step
        torch.testing.assert_close(o.float(), r.float(), rtol=2e-5 if dtype == torch.float32 else 1e-2,
                                   atol=4 * 2.0 ** -24 if dtype == torch.float16 else 0)


def test_unscale_counts_nonfinite_and_skips_clip():
    from axs.unified.training_unified import unscale_and_clip_

    grads = _grads(torch.float32, 1.0, 5, offset_views=False)
    grads[7][3] = float("inf")
    grads[14][0] = float("nan")
    grads[14][1] = -float("inf")
    before = [t.clone() for t in grads]
    res = unscale_and_clip_(_params(grads), 4.0, 1e-3).cpu()
    assert res[2].item() == 3
    for o, b in zip(grads, before):                          # divided, never clipped
        torch.testing.assert_close(o, b / 4.0, rtol=0, atol=0, equal_nan=True)


def _gpt(seed=0):
    c = minigpt.GPTConfig(num_layers=2, batch=16)
    return minigpt.build_axs(seed, DEV, c), c


def _run(pipe_cls, steps, quantize_grad=False, **kw):
    model, c = _gpt(0)
    if not quantize_grad:
        from axs.unified import AXSLinearUnified

        for m in model.modules():
            if isinstance(m, AXSLinearUnified):
                m.quantize_grad = False
    x, y = minigpt.batch(3, c)
    x, y = x.to(DEV), y.to(DEV)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-3)
    pipe = pipe_cls(model, opt, **kw)
    loss_fn = lambda out, inp: F.cross_entropy(out.reshape(-1, out.shape[-1]), y.reshape(-1))  # noqa: E731
    return [pipe.training_step(x, loss_fn) for _ in range(steps)], model


def test_pipeline_matches_reference_without_clipping():
    """No clipping (coefficient 1) and nearest dY: the fused path and the
    reference's per-parameter path do the same arithmetic -- the loss-scale
    division by a power of two is exact -- so the runs are bit-identical,
    loss-scale growth included."""
    from axs.unified import AXSTrainingPipelineUnified

    kw = dict(max_grad_norm=1e9, loss_scale_growth_interval=3)
    ours, m1 = _run(AXSTrainingPipelineUnified, 8, **kw)
    ref, m2 = _run(RefPipeline, 8, **kw)
    for a, b in zip(ours, ref):
        assert a["loss"] == b["loss"] and a["loss_scale"] == b["loss_scale"] and not a["overflow"]
        assert abs(a["grad_norm"] - b["grad_norm"]) <= 1e-5 * b["grad_norm"]
    assert ours[-1]["loss_scale"] == 2.0 ** 16 * 4
    for p1, p2 in zip(m1.parameters(), m2.parameters()):
        assert torch.equal(p1, p2)


def test_pipeline_matches_reference_with_clipping():
    """Clipping active on every step (max norm 0.05): the norms agree to float
    rounding (fixed-order sum against torch's norm of norms), and the
    training curves agree to 1e-3 relative over 10 steps."""
    from axs.unified import AXSTrainingPipelineUnified

    ours, _ = _run(AXSTrainingPipelineUnified, 10, max_grad_norm=0.05)
    ref, _ = _run(RefPipeline, 10, max_grad_norm=0.05)
    assert abs(ours[0]["grad_norm"] - ref[0]["grad_norm"]) <= 1e-5 * ref[0]["grad_norm"]
    assert ref[0]["grad_norm"] > 0.05
    for a, b in zip(ours, ref):
        assert abs(a["loss"] - b["loss"]) <= 1e-3 * b["loss"], (a, b)


def test_pipeline_overflow_backoff_matches_reference():
    """A loss scale beyond float32 (2^130: the backward's multiplier rounds
    to inf, so every gradient is non-finite): the steps overflow and halve
    the scale until the gradients fit, the optimiser does not step on them,
    and the sequence of overflows and scales equals the reference's."""
    from axs.unified import AXSTrainingPipelineUnified

    kw = dict(loss_scale_init=2.0 ** 130, max_grad_norm=1.0)
    ours, m1 = _run(AXSTrainingPipelineUnified, 8, **kw)
    ref, m2 = _run(RefPipeline, 8, **kw)
    assert [a["overflow"] for a in ours] == [b["overflow"] for b in ref]
    assert [a["loss_scale"] for a in ours] == [b["loss_scale"] for b in ref]
    assert ours[0]["overflow"] and ours[0]["grad_norm"] == 0.0
    first_ok = next(i for i, a in enumerate(ours) if not a["overflow"])
    assert first_ok >= 1


def test_pipeline_warmup_and_stats():
    from axs.unified import AXSTrainingPipelineUnified

    ours, _ = _run(AXSTrainingPipelineUnified, 4, warmup_steps=2)
    ref, _ = _run(RefPipeline, 4, warmup_steps=2)
    assert [a["warmup"] for a in ours] == [True, True, False, False]
    for a, b in zip(ours, ref):
        assert abs(a["loss"] - b["loss"]) <= 1e-3 * b["loss"]


def test_pipeline_matches_the_reference_fixture_on_gpu():
    """AXSTrainingPipelineUnified on the GPU against tests/golden/pipeline.npz,
    written by the reference's own pipeline on the CPU with the same model,
    data, schedule and two forced overflows: the overflow flags, loss scales
    and step counters identical; losses, gradient norms and final parameters
    within 1e-5 relative (GPU fp32 matmuls order their sums differently from
    the CPU's)."""
    import sys

    import numpy as np

    from axs.unified import AXSTrainingPipelineUnified
    from conftest import GOLDEN, load_golden

    sys.path.insert(0, GOLDEN)
    import make_pipeline_golden as mk

    want = load_golden("pipeline.npz")
    model, opt, sched, x, loss_fn = mk.setup()
    model = model.to(DEV)
    # the optimiser was built on the CPU parameters: rebuild it on the moved ones
    opt = torch.optim.SGD(model.parameters(), lr=0.1, momentum=0.9)
    sched = torch.optim.lr_scheduler.LambdaLR(opt, lambda s: 1.0 / (1.0 + 0.1 * s))
    p = AXSTrainingPipelineUnified(model, opt, scheduler=sched, **mk.PIPELINE_ARGS)
    rows = []
    xd = x.to(DEV)
    ystate = {}

    def loss_dev(out, inputs):
        # the fixture's loss (mean squared error against its fixed targets, scaled
        # at the forced-overflow calls) evaluated on the device
        ystate.setdefault("n", 0)
        ystate["n"] += 1
        g = torch.Generator().manual_seed(1)
        torch.randn(8, 16, generator=g)
        t = torch.randn(8, 4, generator=g).to(DEV)
        loss = ((out - t) ** 2).mean()
        return loss * 1e35 if ystate["n"] in mk.OVERFLOW_AT else loss

    for _ in range(mk.STEPS):
        r = p.training_step(xd, loss_dev)
        rows.append([r["loss"], r["loss_scale"], r["grad_norm"], float(r["overflow"]), float(r["step"]),
                     float(r["warmup"])])
    rows = np.array(rows, np.float64)
    ref = want["steps"]
    assert np.array_equal(rows[:, [1, 3, 4, 5]], ref[:, [1, 3, 4, 5]])
    ok = ref[:, 3] == 0
    assert np.allclose(rows[ok, 0], ref[ok, 0], rtol=1e-5, atol=0)
    assert np.allclose(rows[ok, 2], ref[ok, 2], rtol=1e-5, atol=0)
    for i, t in enumerate(model.parameters()):
        a = t.detach().cpu().numpy()
        assert np.allclose(a, want[f"param{i}"], rtol=1e-5, atol=1e-6), i
