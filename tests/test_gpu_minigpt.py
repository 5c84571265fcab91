"""MiniGPT (4 layers, d 256, 4 heads, FFN 1024, vocab 256,
context 128, batch 64) trained with AdamW (lr 3e-4, fp32 master weights), every
nn.Linear replaced by the AXS-6 linear through convert_to_axs_unified.

The 200-step loss curve of the product path on the GPU is compared with
  * the same model, initial weights and batch trained on the CPU through the
    reference's eager NF5 operations (tests/minigpt.py ``build_reference``),
    whose 200-step curves tests/golden/make_minigpt_curve.py wrote to
    tests/golden/minigpt_curve.npz: with dY taken as given (nearest) step by
    step, and with stochastically rounded dY within an envelope (the two
    sides draw different dither streams);
  * a live CPU run of the restatement over the first REF_STEPS steps (the
    fixture's path on this host);
  * the unquantized fp32 model on the GPU over the full 200 steps (the
    reference's claim: AXS-6 training tracks fp32, README.md:238-243).
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import minigpt

pytestmark = pytest.mark.gpu

STEPS = 200
REF_STEPS = 8
STEP_TOL = 2e-3        # relative, per step, GPU product path vs CPU reference (first REF_STEPS)
NEAR_STEPS = 10        # nearest dY: steps compared step by step at STEP_TOL (the
                       # runs then drift: 2.4e-3 relative at step 19, the largest gaps at
                       # steps ~35-60, back to 1e-4 once the batch is memorised)
NEAR_CURVE_TOL = 0.027  # x initial loss, |a - b| at every step, GPU vs CPU reference, both
                        # with nearest dY.  The bound is set by how far any change in the
                        # order of fp32 additions carries this curve, measured: the CPU
                        # reference restatement itself, run with 2 / 3 / 4 / 6 threads
                        # instead of the fixture's 8, misses its own fixture by 0.047 /
                        # 0.069 / 0.053 / 0.090 nats (up to 1.61%); the GPU product path
                        # 0.062 with q/k/v as three linears, 0.097 and 0.120 (2.15%, two
                        # boxes) grouped.  The bound is ~1.25x the largest of these.
CURVE_TOL = 0.025      # x initial loss, |a - b| at every step of two AXS curves with different
                       # dither streams (GPU vs CPU reference, stochastic dY: measured 0.057
                       # = 1.0%; eager vs graph-replayed: 0.099 = 1.8%)
FP32_CURVE_TOL = 0.04  # x initial loss, AXS (stochastic dY) against the fp32 model: a different
                       # trajectory, not a parity bound -- measured 0.167 = 3.0% near step 50
FINAL_TOL = 0.005      # nats, final loss (both near 0.02: the batch is memorised, so a
                       # relative bound would be ill-posed)

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "minigpt_curve.npz")


def _nearest_dy(model):
    from axs.unified import AXSLinearUnified

    for m in model.modules():
        if isinstance(m, AXSLinearUnified):
            m.quantize_grad = False
    return model


def _max_gap(a, b):
    return max(abs(u - v) for u, v in zip(a, b))


def test_minigpt_loss_curve_matches_reference_and_fp32():
    ref_curves = np.load(FIXTURE, allow_pickle=False)
    assert int(ref_curves["steps"]) == STEPS
    x, y = minigpt.batch(1)

    print("[minigpt: GPU product path, nearest dY, 200 steps]", flush=True)
    near, _ = minigpt.train(_nearest_dy(minigpt.build_axs(0, "cuda")), x.cuda(), y.cuda(), STEPS)
    ref_near = ref_curves["nearest"].tolist()
    gap = _max_gap(near, ref_near)
    windows = [round(_max_gap(near[i:i + 20], ref_near[i:i + 20]), 4) for i in range(0, STEPS, 20)]
    print(f"  loss {near[0]:.4f} -> {near[-1]:.4f}; CPU reference {ref_near[0]:.4f} -> {ref_near[-1]:.4f}; "
          f"max gap {gap:.4f}; per 20 steps {windows}", flush=True)
    # step by step while the two runs have not yet diverged (fp16 rounding of
    # the products vs fp32, amplified by NF5's quantization steps and the
    # training dynamics), then within the envelope of two dither streams
    rel = [abs(near[i] - ref_near[i]) / ref_near[i] for i in range(NEAR_STEPS)]
    print(f"  first {NEAR_STEPS} steps: max relative gap {max(rel):.2e}", flush=True)
    assert max(rel) < STEP_TOL
    assert gap < NEAR_CURVE_TOL * ref_near[0]
    assert abs(near[-1] - ref_near[-1]) < FINAL_TOL

    print("[minigpt: GPU product path, stochastic dY, 200 steps]", flush=True)
    torch.manual_seed(5)
    model = minigpt.build_axs(0, "cuda")
    gpu_losses, ms = minigpt.train(model, x.cuda(), y.cuda(), STEPS, warmup=5, sync=torch.cuda.synchronize)
    ref_st = ref_curves["stochastic"].tolist()
    gap = _max_gap(gpu_losses, ref_st)
    print(f"  {ms:.2f} ms/step, loss {gpu_losses[0]:.4f} -> {gpu_losses[-1]:.4f}; CPU reference "
          f"{ref_st[0]:.4f} -> {ref_st[-1]:.4f}; max gap {gap:.4f}", flush=True)
    assert gap < CURVE_TOL * ref_st[0]
    assert abs(gpu_losses[-1] - ref_st[-1]) < FINAL_TOL

    print("[minigpt: fp32 GPU model, 200 steps]", flush=True)
    fp32 = minigpt.base_model(0).cuda()
    fp32_losses, fp32_ms = minigpt.train(fp32, x.cuda(), y.cuda(), STEPS, warmup=5, sync=torch.cuda.synchronize)
    print(f"  {fp32_ms:.2f} ms/step, loss {fp32_losses[0]:.4f} -> {fp32_losses[-1]:.4f}", flush=True)

    print(f"[minigpt: CPU reference restatement, {REF_STEPS} steps]", flush=True)
    torch.manual_seed(6)
    ref = minigpt.build_reference(0)
    ref_losses, ref_ms = minigpt.train(ref, x, y, REF_STEPS, warmup=1)
    print(f"  {ref_ms:.0f} ms/step, losses {[round(v, 4) for v in ref_losses]}", flush=True)
    print(f"  gpu losses {[round(v, 4) for v in gpu_losses[:REF_STEPS]]}", flush=True)
    # the fixture was written by the same restatement (same seeds and draws) on
    # another host, whose thread count orders the fp32 reductions differently:
    # measured 1.6e-4 relative by step 3
    assert np.allclose(ref_losses, ref_st[:REF_STEPS], rtol=1e-3, atol=0)

    for i in range(REF_STEPS):
        rel = abs(gpu_losses[i] - ref_losses[i]) / ref_losses[i]
        assert rel < STEP_TOL, (i, gpu_losses[i], ref_losses[i])
    assert gpu_losses[-1] < gpu_losses[0] - 1.0, "training did not make progress"
    gap = _max_gap(gpu_losses, fp32_losses)
    print(f"  final loss axs {gpu_losses[-1]:.4f} fp32 {fp32_losses[-1]:.4f}; max curve gap {gap:.4f}", flush=True)
    assert gap < FP32_CURVE_TOL * fp32_losses[0]
    assert abs(gpu_losses[-1] - fp32_losses[-1]) < FINAL_TOL


def test_minigpt_every_linear_converted():
    from axs.unified import AXSEmbeddingUnified, AXSLinearUnified

    model = minigpt.build_axs(0, "cuda")
    assert not any(type(m) is torch.nn.Linear for m in model.modules())
    n_lin = sum(isinstance(m, AXSLinearUnified) for m in model.modules())
    assert n_lin == 4 * 6 + 1   # q, k, v, o, fc1, fc2 per block + head
    assert isinstance(model.token_embed, AXSEmbeddingUnified)


def test_minigpt_graph_replay_matches_eager_training():
    """The whole training step (forward, loss, backward, AdamW) recorded in one
    HIP graph and replayed trains like the eager loop.  With nearest-rounded
    dY both compute the same thing and every kernel on the path is
    deterministic, so the loss curves are bit-identical over 30 steps, for
    AdamW's capturable multi-tensor form and for its fused form (the eager
    loop uses the same form as the graph: the default form rounds
    differently, and NF5's quantization steps amplify that ulp-level
    difference to ~5e-3 of the loss within 30 steps).  With the stochastic dY
    of the default modules the two runs draw different dither streams; the
    curves then agree to the AXS-vs-fp32 curve bound."""
    x, y = minigpt.batch(1)
    xd, yd = x.cuda(), y.cuda()
    for fused in (False, True):
        print(f"[minigpt: eager vs graph-replayed, nearest dY, 30 steps, fused AdamW {fused}]", flush=True)
        eager, _ = minigpt.train(_nearest_dy(minigpt.build_axs(0, "cuda")), xd, yd, 30,
                                 capturable=True, fused=fused)
        graphed, _ = minigpt.train_graphed(_nearest_dy(minigpt.build_axs(0, "cuda")), xd, yd, 30, warmup=3,
                                           fused=fused)
        print(f"  losses {eager[0]:.5f} -> {eager[-1]:.5f}", flush=True)
        assert graphed == eager

    print("[minigpt: eager vs graph-replayed, stochastic dY, 100 steps]", flush=True)
    torch.manual_seed(5)
    eager, eager_ms = minigpt.train(minigpt.build_axs(0, "cuda"), xd, yd, 100, warmup=5,
                                    sync=torch.cuda.synchronize)
    torch.manual_seed(5)
    graphed, graph_ms = minigpt.train_graphed(minigpt.build_axs(0, "cuda"), xd, yd, 100, warmup=3)
    gap = max(abs(a - b) for a, b in zip(graphed, eager))
    print(f"  eager {eager_ms:.2f} ms/step, graph {graph_ms:.2f} ms/step; final loss {eager[-1]:.4f} vs "
          f"{graphed[-1]:.4f}; max gap {gap:.4f}", flush=True)
    assert graphed[-1] < graphed[0] - 1.0, "graph-replayed training did not make progress"
    assert gap < CURVE_TOL * eager[0]


def test_graph_replays_draw_fresh_dither():
    """A stochastic fake-quantize recorded in a graph: each replay adds the
    device counter to the seed fixed at capture, so replays differ, and each
    replay is bit-exact against the oracle given that seed."""
    import numpy as np

    import oracle
    from axs.unified import hip_kernels

    g = torch.Generator().manual_seed(3)
    xh = torch.randn(64, 256, generator=g)
    x = xh.cuda()
    hip_kernels.prepare_graph_capture(x.device)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        hip_kernels.hip_fused_fake_quantize(x, 32, "stochastic")
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    # the seed drawn at capture: the next draw of torch's CPU generator
    torch.manual_seed(29)
    seed = hip_kernels.next_seed()
    torch.manual_seed(29)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = hip_kernels.hip_fused_fake_quantize(x, 32, "stochastic")
    ctr = hip_kernels._graph_counters[x.device.index]
    seen = []
    for _ in range(3):
        c = int(ctr.item())
        graph.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        want = oracle.fake_quantize(xh.numpy(), 32, oracle.uniform(seed + c, 0, xh.numel()))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        assert int(ctr.item()) == c + 1
        seen.append(got)
    assert not np.array_equal(seen[0], seen[1])


def test_graph_counter_advances_once_per_graph():
    """Two stochastic calls recorded in one graph: the graph advances the
    device counter once, after its first stochastic call, so per replay the
    first call keys its dither with (its capture seed + c) and the second with
    (its seed + c + 1); both bit-exact against the oracle, and the counter
    moves by one per replay."""
    import numpy as np

    import oracle
    from axs.unified import hip_kernels

    g = torch.Generator().manual_seed(4)
    xh = [torch.randn(64, 256, generator=g), torch.randn(32, 128, generator=g)]
    xs = [t.cuda() for t in xh]
    hip_kernels.prepare_graph_capture(xs[0].device)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for x in xs:
            hip_kernels.hip_fused_fake_quantize(x, 32, "stochastic")
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    torch.manual_seed(31)
    seeds = [hip_kernels.next_seed(), hip_kernels.next_seed()]
    torch.manual_seed(31)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = [hip_kernels.hip_fused_fake_quantize(x, 32, "stochastic") for x in xs]
    ctr = hip_kernels._graph_counters[xs[0].device.index]
    for _ in range(3):
        c = int(ctr.item())
        graph.replay()
        torch.cuda.synchronize()
        for i, (o, x) in enumerate(zip(outs, xh)):
            want = oracle.fake_quantize(x.numpy(), 32, oracle.uniform(seeds[i] + c + i, 0, x.numel()))
            assert np.array_equal(o.cpu().numpy().view(np.uint32), want.view(np.uint32)), f"call {i}"
        assert int(ctr.item()) == c + 1
