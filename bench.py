#!/usr/bin/env python3
"""Benchmark of the AXS-6 NF5 hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-linear] [--no-minigpt]

Workload (BASELINE.json metric "NF5 fake-quant GB/s @8192x4096 fp32; AXS-6
linear TFLOP/s @4096^3 bf16"):
  * headline ("value"): NF5 fake-quantize forward + STE backward of one
    8192x4096 fp32 tensor (config 2's largest shape, N(0,1) with 1% x100
    outliers).  One step = one fake-quantize pass; the STE backward is the
    identity and launches nothing.  Algorithmic bytes per step = 8 B/elem
    (4 read + 4 written) = 268,435,456 B.
  * "linear": the fused AXS-6 linear forward at M=N=K=4096 (config 3), FLOPs
    per step = 2*M*N*K, timed the same way.
  * "linear_train": config 4, forward + backward at its four shapes
    (6*M*N*K FLOPs per step).
  * "wire": the 6.25-bit gradient wire format (quantize+pack, unpack) at
    8192x4096, GB/s, and the AXSBlock record stream (26 B per 32 values).
  * "codec": quantize (exponents, codes, signs and the FQ output) and
    dequantize at 8192x4096, GB/s.
  * "configs": the smaller config-1/2 shapes (FQ at 256^2 and 4096^2,
    quantize/dequantize at 1024^2), device time per launch.
  * "fused": the single-launch fused linear at small outputs (decode-like
    shapes), beside the packing + GEMM path.
  * "minigpt": config 5, the MiniGPT training step with every nn.Linear
    converted (ms/step and the loss curve, beside the fp32 model).
Inputs are synthetic, resident in HBM before the timed region.  K steps are
timed between device synchronisations as replays of a HIP graph holding 20
steps' kernels (every kernel runs every step; the graph removes the host
launch cost, which exceeds the 40 us kernel through the Python API); the
same K steps through the Python API and autograd are timed and reported as
eager_ms_per_step.  Device time per step comes from HIP events on the stream
the kernels run on (torch's current stream).

Prints one JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "axs-6_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0            # MI355X HBM3E, published
BF16_DENSE_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 / fp16 MFMA, published

FQ_SHAPE = (8192, 4096)
LIN_SHAPE = (4096, 4096, 4096)   # M, K, N


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return platform.processor() or "unknown"


def load_traffic(name: str, key: str = "traffic_bytes_per_launch"):
    """HBM bytes per launch measured by rocprofv3 --pmc (profiles/<name>)."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            return json.load(f).get(key)
    except (OSError, ValueError):
        return None


GRAPH_STEPS = 20   # steps captured per HIP graph


def time_steps(step, launches, steps: int, warmup: int):
    """Time `steps` steps.

    `step` is the full step through the public API (autograd included);
    `launches` issues exactly the kernels of one step (the STE backward of
    the fake-quantize launches none).  After `warmup` eager steps,
    GRAPH_STEPS steps' launches are captured into one HIP graph on a side
    stream, replayed untimed as often as the timed run will, then replayed
    until `steps` steps have run, between device synchronisations (wall
    clock) and HIP events on the launch stream (device time).  Every kernel
    runs every step; the graph only takes the per-launch host cost out of the
    loop.  Then `steps` eager steps are timed for reference.
    Returns (wall ms/step, device ms/step, eager wall ms/step)."""
    import torch

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            launches()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(GRAPH_STEPS):
            launches()
    g.replay()
    torch.cuda.synchronize()
    replays = max(1, (steps + GRAPH_STEPS - 1) // GRAPH_STEPS)
    # as many untimed replays first: the power-limited GEMM reads several
    # percent slow in the first replays after the eager warm-up, while the
    # clocks settle (4096^3 forward: 160 against 146-152 us a moment later)
    for _ in range(replays):
        g.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(replays):
        g.replay()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / (replays * GRAPH_STEPS)
    # the eager steps are timed last, with the GPU's clocks already settled by
    # the replays (timed first, right after the data was made, they read up
    # to 25% slower than the same steps a moment later)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3 / steps
    return wall_ms, ev0.elapsed_time(ev1) / (replays * GRAPH_STEPS), eager_ms


FQ_ROTATE = 4   # input buffers the cold-HBM FQ leg cycles through (4 x 128 MiB)


def bench_fq(steps: int, warmup: int):
    """The FQ step at 8192x4096 f32, timed twice.

    Cold (the headline): FQ_ROTATE inputs of 128 MiB are cycled and every
    launch of the recorded graph keeps its own output, so each launch reads an
    input last touched FQ_ROTATE launches (1 GiB of traffic) earlier and
    writes a buffer last written a whole graph earlier: 4 x 256 MiB, well
    past the 256 MiB last-level cache, so the bytes come from HBM.  A device
    copy of the same bytes runs the same rotation (the practical ceiling).
    Warm: one input replayed every step (as a training loop re-quantizing one
    tensor would), which the last-level cache partly serves."""
    import torch

    from axs.unified.functional_unified import fake_quantize_unified
    from axs.unified.hip_kernels import hip_fused_fake_quantize

    g = torch.Generator(device="cuda").manual_seed(3)
    xs = []
    for _ in range(FQ_ROTATE):
        x = torch.randn(*FQ_SHAPE, device="cuda", generator=g)
        m = torch.rand(*FQ_SHAPE, device="cuda", generator=g) < 0.01
        x[m] *= 100.0
        xs.append(x.requires_grad_(True))
    grad = torch.randn(*FQ_SHAPE, device="cuda", generator=g)
    xds = [x.detach() for x in xs]

    def rotating(fn):
        """fn over the inputs in turn; the outputs of the launches recorded
        into a graph are kept (held below), so each gets its own buffer."""
        state = {"i": 0, "keep": []}

        def call():
            i = state["i"]
            state["i"] = (i + 1) % FQ_ROTATE
            y = fn(i)
            if torch.cuda.is_current_stream_capturing():
                state["keep"].append(y)
            return y
        return call, state

    def fq_step(i):
        y = fake_quantize_unified(xs[i], 32, "nearest")
        # STE backward: hands back `grad` itself and launches nothing;
        # autograd.grad avoids accumulating into a leaf .grad (not part of the path)
        (gx,) = torch.autograd.grad(y, xs[i], grad)
        return y, gx

    _, gx = fq_step(0)
    assert gx.data_ptr() == grad.data_ptr(), "STE backward must hand back the incoming gradient"

    step, _ = rotating(fq_step)
    launches, held = rotating(lambda i: hip_fused_fake_quantize(xds[i], 32, "nearest"))
    wall_ms, gpu_ms, eager_ms = time_steps(step, launches, steps, warmup)
    held["keep"].clear()
    copy_launch, held_c = rotating(lambda i: xds[i].clone())
    _, copy_ms, _ = time_steps(copy_launch, copy_launch, steps, warmup)
    held_c["keep"].clear()

    x0 = xs[0]

    def warm_step():
        y = fake_quantize_unified(x0, 32, "nearest")
        torch.autograd.grad(y, x0, grad)

    x0d = xds[0]
    warm_wall, warm_gpu, _ = time_steps(warm_step, lambda: hip_fused_fake_quantize(x0d, 32, "nearest"),
                                        steps, warmup)
    _, warm_copy, _ = time_steps(x0d.clone, x0d.clone, steps, warmup)
    return {"wall_ms": wall_ms, "gpu_ms": gpu_ms, "eager_ms": eager_ms, "bytes": 8 * x0.numel(),
            "copy_gpu_ms": copy_ms, "warm": {"wall_ms": warm_wall, "gpu_ms": warm_gpu, "copy_gpu_ms": warm_copy}}


def bench_linear(steps: int, warmup: int, dtype=None):
    """Config 3's forward at 4096^3 (fp32 X, W, Y; or `dtype` inputs and
    output, without the per-kernel split)."""
    import torch

    from axs.unified import hip_linear

    M, K, N = LIN_SHAPE
    g = torch.Generator(device="cuda").manual_seed(4)
    X = torch.randn(M, K, device="cuda", generator=g)
    W = torch.randn(N, K, device="cuda", generator=g) * K ** -0.5
    b = torch.zeros(N, device="cuda")
    if dtype is not None:
        X, W = X.to(dtype), W.to(dtype)

    def step():
        hip_linear.linear_forward(X, W, b, 32, True)

    wall_ms, gpu_ms, eager_ms = time_steps(step, step, steps, warmup)
    if dtype is not None:
        return {"wall_ms": wall_ms, "gpu_ms": gpu_ms, "eager_ms": eager_ms, "flops": 2.0 * M * N * K}
    kern = hip_linear.last_forward_kernel_times(X, W, b, reps=max(steps, 10))
    # HBM-cold: 3 rotating (X, W) pairs (384 MiB) and a fresh Y per call
    Xs = [X] + [torch.randn(M, K, device="cuda", generator=g) for _ in range(2)]
    Ws = [W] + [torch.randn(N, K, device="cuda", generator=g) * K ** -0.5 for _ in range(2)]
    cold_ms = _timed_cold(lambda i: hip_linear.linear_forward(Xs[i % 3], Ws[i % 3], b, 32, True), 3,
                          max(steps, 12), 3)
    del Xs, Ws
    return {"wall_ms": wall_ms, "gpu_ms": gpu_ms, "eager_ms": eager_ms, "flops": 2.0 * M * N * K,
            "kernels": kern, "cold_ms": cold_ms}


def _timed_cold(fn, n_in: int, reps: int, warmup: int, keep: int = 3) -> float:
    """Device ms per call of fn(i), HBM-cold, from HIP-graph replays (so host
    time per API call, which allocates its outputs, is not mixed in): call i
    takes input set i % n_in (the caller sizes the sets past the 256 MiB
    last-level cache) and the last `keep` results stay referenced, so each
    call writes a different buffer of the graph's pool than the call before
    (a result freed at once would come back at the same address)."""
    import collections

    import torch

    held = collections.deque(maxlen=keep)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(warmup):
            held.append(fn(i))
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    held.clear()
    steps = max(reps, 2 * n_in)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(steps):
            held.append(fn(i))
    graph.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(3):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    held.clear()
    del graph
    return e0.elapsed_time(e1) / (3 * steps)


def bench_wire(reps: int = 20, warmup: int = 3):
    """NF5 wire format (the reference's 6.25-bit gradient buffer) of an
    8192x4096 f32 tensor: quantize+pack and unpack+dequantize, one kernel each.
    Algorithmic bytes: pack 4 B read + 25/32 B written per value; unpack the
    reverse.  The same for the AXSBlock record stream (26/32 B per value).
    Device time per call from HIP-graph replays, HBM-cold (_timed_cold: 3
    rotating 128 MiB inputs, 8 rotating wire buffers)."""
    import torch

    from axs import blocks
    from axs.unified import distributed as d

    g = torch.Generator(device="cuda").manual_seed(3)
    xs = [torch.randn(*FQ_SHAPE, device="cuda", generator=g) for _ in range(3)]
    bufs = [d.pack_gradient_to_buffer(xs[i % 3] * (1.0 + i), 32) for i in range(8)]
    shape = xs[0].shape
    pack_ms = _timed_cold(lambda i: d.pack_gradient_to_buffer(xs[i % 3], 32), 3, reps, warmup)
    unpack_ms = _timed_cold(lambda i: d.unpack_buffer_to_gradient(bufs[i % 8], shape, 32), 8, reps, warmup)
    nbytes = xs[0].numel() * 4 + bufs[0].numel()
    # the AXSBlock record stream (2-byte header, 26 B per 32 values): same kernels
    recs = [blocks.encode_blocks(xs[i % 3] * (1.0 + i), 32) for i in range(8)]
    bpack_ms = _timed_cold(lambda i: blocks.encode_blocks(xs[i % 3], 32), 3, reps, warmup)
    bunpack_ms = _timed_cold(lambda i: blocks.decode_blocks(recs[i % 8], shape, 32), 8, reps, warmup)
    bbytes = xs[0].numel() * 4 + recs[0].numel()
    return {"metric": "NF5 wire format GB/s @8192x4096 fp32 (quantize+pack, unpack+dequantize)",
            "cache": "cold: rotating inputs and freshly written outputs, past the 256 MiB last-level cache",
            "buffer_bytes": bufs[0].numel(), "bits_per_value": round(bufs[0].numel() * 8 / xs[0].numel(), 4),
            "pack_ms": round(pack_ms, 5), "unpack_ms": round(unpack_ms, 5),
            "pack_gbs": round(nbytes / (pack_ms * 1e-3) / 1e9, 1),
            "unpack_gbs": round(nbytes / (unpack_ms * 1e-3) / 1e9, 1),
            "axs_blocks": {"buffer_bytes": recs[0].numel(),
                           "encode_ms": round(bpack_ms, 5), "decode_ms": round(bunpack_ms, 5),
                           "encode_gbs": round(bbytes / (bpack_ms * 1e-3) / 1e9, 1),
                           "decode_gbs": round(bbytes / (bunpack_ms * 1e-3) / 1e9, 1)}}


def bench_codec(reps: int = 20, warmup: int = 3):
    """quantize_unified / dequantize_unified (the AXSTensor codec, config 1's
    operation) on an 8192x4096 f32 tensor, block 32, nearest rounding.
    Algorithmic bytes per value: quantize with the FQ output 4 read + 1 code +
    1 sign + 1/32 exponent + 4 FQ written = 10.03; dequantize 1 + 1 + 1/32
    read + 4 written = 6.03.  Device time per call from HIP-graph replays,
    HBM-cold (_timed_cold: 3 rotating 128 MiB inputs, 8 rotating code sets)."""
    import torch

    from axs.unified.hip_kernels import hip_dequantize, hip_quantize

    g = torch.Generator(device="cuda").manual_seed(4)
    xs = [torch.randn(*FQ_SHAPE, device="cuda", generator=g) for _ in range(3)]
    codes = [hip_quantize(xs[i % 3] * (1.0 + i), 32)[:3] for i in range(8)]
    rows, cols = FQ_SHAPE
    q_ms = _timed_cold(lambda i: hip_quantize(xs[i % 3], 32, with_fake_quantized=True), 3, reps, warmup)
    d_ms = _timed_cold(lambda i: hip_dequantize(*codes[i % 8], rows, cols, 32), 8, reps, warmup)
    n = xs[0].numel()
    q_bytes = n * (4 + 1 + 1 + 4) + n // 32
    d_bytes = n * (1 + 1 + 4) + n // 32
    return {"metric": "NF5 quantize (+FQ output) / dequantize GB/s @8192x4096 fp32, block 32",
            "cache": "cold: rotating inputs and freshly written outputs, past the 256 MiB last-level cache",
            "quantize_ms": round(q_ms, 5), "dequantize_ms": round(d_ms, 5),
            "quantize_gbs": round(q_bytes / (q_ms * 1e-3) / 1e9, 1),
            "dequantize_gbs": round(d_bytes / (d_ms * 1e-3) / 1e9, 1)}


def bench_configs(steps: int = 200, warmup: int = 20):
    """The smaller shapes of configs 1 and 2, timed like the headline (graph
    replays, device time per launch): FQ at 256^2 and 4096^2 (config 2), the
    headline FQ shape in bf16 (4 B per value of traffic), and quantize +
    dequantize of config 1's 1024^2 tensor (x = 0.02 N(0,1))."""
    import torch

    from axs.unified.hip_kernels import hip_dequantize, hip_fused_fake_quantize, hip_quantize

    out = {}
    g = torch.Generator(device="cuda").manual_seed(5)
    for shape, dt in (((256, 256), torch.float32), ((4096, 4096), torch.float32), (FQ_SHAPE, torch.bfloat16)):
        x = torch.randn(*shape, device="cuda", generator=g).to(dt)
        launch = lambda: hip_fused_fake_quantize(x, 32, "nearest")  # noqa: E731
        _, gpu_ms, _ = time_steps(launch, launch, steps, warmup)
        nbytes = 2 * x.element_size() * x.numel()
        tag = "" if dt == torch.float32 else "_bf16"
        rates = lambda ms: {"us_per_launch": round(ms * 1e3, 2),  # noqa: E731
                            "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                            "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        if x.numel() * x.element_size() >= (64 << 20):
            # HBM-cold: 5 rotating inputs (320 MiB) and fresh outputs; the
            # one-input replay (the last-level cache may hold it) beside it
            xs = [x] + [torch.randn(*shape, device="cuda", generator=g).to(dt) for _ in range(4)]
            cold_ms = _timed_cold(lambda i: hip_fused_fake_quantize(xs[i % 5], 32, "nearest"), 5, steps // 2,
                                  warmup)
            out[f"fq_{shape[0]}x{shape[1]}{tag}"] = {**rates(cold_ms), "cache": "cold", "warm": rates(gpu_ms)}
            del xs
        else:
            out[f"fq_{shape[0]}x{shape[1]}{tag}"] = rates(gpu_ms)
    x = torch.randn(1024, 1024, device="cuda", generator=g) * 0.02
    e, c, s_, _ = hip_quantize(x, 32)
    q = lambda: hip_quantize(x, 32)  # noqa: E731
    d = lambda: hip_dequantize(e, c, s_, 1024, 1024, 32)  # noqa: E731
    _, q_ms, _ = time_steps(q, q, steps, warmup)
    _, d_ms, _ = time_steps(d, d, steps, warmup)
    n = x.numel()
    out["config1_quantize_1024x1024"] = {"us_per_launch": round(q_ms * 1e3, 2),
                                         "gbs": round(n * 6.03125 / (q_ms * 1e-3) / 1e9, 1)}
    out["config1_dequantize_1024x1024"] = {"us_per_launch": round(d_ms * 1e3, 2),
                                           "gbs": round(n * 6.03125 / (d_ms * 1e-3) / 1e9, 1)}
    out["note"] = ("device time per launch from HIP-graph replays; shapes below ~4M values are "
                   "launch-latency-bound, not HBM-bound")
    return out


LIN_TRAIN_SHAPES = [(8192, 4096, 11008), (8192, 11008, 4096), (2048, 768, 3072), (2048, 3072, 768)]


def bench_fused(reps: int = 100, warmup: int = 10):
    """The fused linear (FQ in the tile loads) at outputs <= 128K elements,
    where accelerated_linear / triton_fused_linear dispatch to it: decode-like
    M against a 4096 x 4096 weight and a small square layer, device time per
    call from HIP-graph replays, beside the packing + fp16-GEMM path on the
    same inputs.  fused_us is hip_linear.fused_forward (one launch, or where
    the library advises it, split_x, two: FQ(X) once into the contraction's
    read order, then the contraction);
    one_launch_us the single fused launch.  They replay one weight (the
    last-level cache may hold it); for the 4096 x 4096 weights fused_cold_us
    rotates 5 (320 MiB, past the cache)."""
    import torch

    from axs import _lib
    from axs.unified import hip_linear

    def stream():   # taken at call time: inside a graph capture it is the capture stream
        return torch.cuda.current_stream().cuda_stream

    g = torch.Generator(device="cuda").manual_seed(9)
    out = {"metric": "fused FQ + linear (M*N <= 128K outputs), device us per call",
           "note": "fused: hip_linear.fused_forward, one launch (M <= 2: a weight row per wave, VALU products; "
                   "else FQ of each 32-wide K tile as it is loaded, fp32 MFMA) or, where split_x, two (FQ(X) "
                   "once in the MFMA read order, then the contraction); packed: FQ + fp16 packing of X and W, "
                   "then the fp16-MFMA GEMM; HIP-graph replays"}
    for M, K, N in ((1, 4096, 4096), (32, 4096, 4096), (128, 1024, 1024), (256, 512, 512)):
        X = torch.randn(M, K, device="cuda", generator=g)
        big = N * K * 4 >= (64 << 20)
        Ws = [torch.randn(N, K, device="cuda", generator=g) * K ** -0.5 for _ in range(5 if big else 1)]
        W = Ws[0]
        b = torch.zeros(N, device="cuda")
        y = torch.empty(M, N, device="cuda")

        def fused_call(w):
            # the public path (triton_fused_linear's): one launch, or the
            # two-launch entry where axs6_nf5_fused_linear_split_x advises it
            return hip_linear.fused_forward(X, w, b)

        def one_launch(w):
            _lib.call("axs6_nf5_fused_linear", X.data_ptr(), w.data_ptr(), b.data_ptr(), y.data_ptr(),
                      _lib.F32, M, N, K, 32, 1, stream())

        fused = _timed_cold(lambda i: fused_call(W), 1, reps, warmup)
        single = _timed_cold(lambda i: one_launch(W), 1, reps, warmup)
        Kp = hip_linear.padded_k(K)
        xq = torch.empty(M, Kp, dtype=torch.float16, device="cuda")
        wq = torch.empty(N, Kp, dtype=torch.float16, device="cuda")
        sx = torch.empty(M, dtype=torch.int32, device="cuda")
        sw = torch.empty(N, dtype=torch.int32, device="cuda")
        packed = _timed_cold(lambda i: _lib.call("axs6_nf5_linear_forward", X.data_ptr(), W.data_ptr(),
                                                 b.data_ptr(), y.data_ptr(), _lib.F32, M, N, K, 32, 1,
                                                 xq.data_ptr(), sx.data_ptr(), wq.data_ptr(), sw.data_ptr(),
                                                 stream()), 1, reps, warmup)
        row = {"fused_us": round(fused * 1e3, 1), "one_launch_us": round(single * 1e3, 1),
               "split_x": bool(_lib.lib().axs6_nf5_fused_linear_split_x(M, N, K, _lib.F32)),
               "packed_us": round(packed * 1e3, 1), "weight_gbs": round(N * K * 4 / (fused * 1e-3) / 1e9, 1)}
        if big:
            cold = _timed_cold(lambda i: fused_call(Ws[i % 5]), 5, reps, warmup)
            row["fused_cold_us"] = round(cold * 1e3, 1)
            row["weight_gbs_cold"] = round(N * K * 4 / (cold * 1e-3) / 1e9, 1)
        out[f"{M}x{K}x{N}"] = row
        del Ws, W
    return out


def _graph_ms(fn, steps: int, replays: int = 3) -> float:
    """Device ms per call of `fn` as replays of a HIP graph of `steps` calls
    (captured after one call on a side stream; one untimed replay first), so
    host launch time is not mixed in; HIP events on the launch stream."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(steps):
            fn()
    g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    del g
    return e0.elapsed_time(e1) / (replays * steps)


def bench_linear_train(reps: int = 5, warmup: int = 2):
    """quantized linear forward + backward (stochastic FQ of
    dY, dX, dW and db) at each [M, K, N]; FLOPs per step = 6*M*N*K.  The
    step's device time from replays of a HIP graph of steps through hip_linear
    (graph-recorded stochastic calls draw a fresh dither per replay from the
    device counter), so the small shapes' host launch time is not mixed in;
    the eager steps (HIP events around `reps` steps) reported beside it."""
    import torch

    from axs.unified import hip_linear

    rows = []
    for (M, K, N) in LIN_TRAIN_SHAPES:
        g = torch.Generator(device="cuda").manual_seed(7)
        X = torch.randn(M, K, device="cuda", generator=g)
        W = torch.randn(N, K, device="cuda", generator=g) * K ** -0.5
        b = torch.zeros(N, device="cuda")
        dY = torch.randn(M, N, device="cuda", generator=g)

        def fwd():
            return hip_linear.forward_train(X, W, b, 32, True)

        def step():
            _, saved = fwd()
            hip_linear.backward(dY, saved, 32, True, True, True, True)

        def timed(fn):
            for _ in range(warmup):
                fn()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                fn()
            e1.record()
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) / reps

        eager_step = timed(step)
        eager_fwd = timed(fwd)
        n_graph = 20 if M * N * K < (1 << 33) else 4
        ms_step = _graph_ms(step, n_graph)
        ms_fwd = _graph_ms(fwd, n_graph)
        flops = 6.0 * M * N * K
        rows.append({"shape_mkn": [M, K, N], "ms_per_step": round(ms_step, 4), "fwd_ms": round(ms_fwd, 4),
                     "bwd_ms": round(ms_step - ms_fwd, 4),
                     "tflops": round(flops / (ms_step * 1e-3) / 1e12, 1),
                     "frac_of_peak": round(flops / (ms_step * 1e-3) / 1e12 / BF16_DENSE_PEAK_TFLOPS, 4),
                     "timing": f"HIP-graph replays of {n_graph} steps",
                     "eager_ms_per_step": round(eager_step, 4), "eager_fwd_ms": round(eager_fwd, 4)})
        log(f"linear fwd+bwd {M}x{K}x{N}: {ms_step:.3f} ms/step graph, {eager_step:.3f} eager "
            f"({rows[-1]['tflops']} TFLOP/s)")
        del X, W, b, dY
    return {"metric": "AXS-6 linear fwd+bwd TFLOP/s (config 4, 6*M*N*K per step)", "shapes": rows}


def bench_minigpt(steps: int = 200, warmup: int = 5, ref_steps: int = 3):
    """MiniGPT (4 layers, d 256, FFN 1024, vocab 256, ctx 128,
    batch 64) with every nn.Linear converted to the AXS-6 linear, AdamW lr 3e-4,
    fp32 master weights, one fixed synthetic batch (tests/minigpt.py).  A step
    is forward + cross-entropy + backward + AdamW through the Python API.
    Reported: ms/step over the steps after `warmup` (torch's fused AdamW;
    multi_tensor_adamw_ms_per_step with its default multi-tensor form, whose
    extra launches dominate a host-bound eager step), the loss curve at a few
    points, the same with the step recorded in a HIP graph and replayed
    (graph_ms_per_step, fused AdamW; graph_multi_tensor_adamw_* with the
    capturable multi-tensor form, which adds two per-parameter broadcast
    divisions per step), the same for the unquantized fp32 model, and the CPU
    reference restatement's ms/step over `ref_steps` steps (host cores)."""
    import torch

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import minigpt

    x, y = minigpt.batch(1)
    # settle the GPU and host clocks on both models before anything is timed
    # (the first timed loop otherwise reads 10-20% slow, whichever model it is)
    for build in (lambda: minigpt.build_axs(0, "cuda"), lambda: minigpt.base_model(0).cuda()):
        minigpt.train(build(), x.cuda(), y.cuda(), 30)
    torch.cuda.synchronize()
    torch.manual_seed(5)
    model = minigpt.build_axs(0, "cuda")
    losses, ms = minigpt.train(model, x.cuda(), y.cuda(), steps, warmup=warmup, sync=torch.cuda.synchronize,
                               capturable=True, fused=True)
    torch.manual_seed(5)
    _, mt_ms = minigpt.train(minigpt.build_axs(0, "cuda"), x.cuda(), y.cuda(), steps, warmup=warmup,
                             sync=torch.cuda.synchronize)
    torch.manual_seed(5)
    g_losses, g_ms = minigpt.train_graphed(minigpt.build_axs(0, "cuda"), x.cuda(), y.cuda(), steps, warmup=3,
                                           fused=True)
    torch.manual_seed(5)
    _, gm_ms = minigpt.train_graphed(minigpt.build_axs(0, "cuda"), x.cuda(), y.cuda(), steps, warmup=3)
    fp32 = minigpt.base_model(0).cuda()
    fp_losses, fp_ms = minigpt.train(fp32, x.cuda(), y.cuda(), steps, warmup=warmup, sync=torch.cuda.synchronize,
                                     capturable=True, fused=True)
    _, fpm_ms = minigpt.train(minigpt.base_model(0).cuda(), x.cuda(), y.cuda(), steps, warmup=warmup,
                              sync=torch.cuda.synchronize)
    fg_losses, fg_ms = minigpt.train_graphed(minigpt.base_model(0).cuda(), x.cuda(), y.cuda(), steps, warmup=3,
                                             fused=True)
    _, fgm_ms = minigpt.train_graphed(minigpt.base_model(0).cuda(), x.cuda(), y.cuda(), steps, warmup=3)
    pipe = bench_pipeline(minigpt, x, y, steps=min(steps, 100), warmup=warmup)
    pts = [0, steps // 4, steps // 2, 3 * steps // 4, steps - 1]
    out = {
        "metric": "MiniGPT AXS-6 training ms/step (config 5)",
        "ms_per_step": round(ms, 3), "steps": steps, "warmup": warmup,
        "optimizer": "AdamW(fused=True) in every leg; *_multi_tensor_adamw_* with torch's default form",
        "multi_tensor_adamw_ms_per_step": round(mt_ms, 3),
        "loss": {str(i): round(losses[i], 4) for i in pts},
        "graph_ms_per_step": round(g_ms, 3),
        "graph_loss": {str(i): round(g_losses[i], 4) for i in pts},
        "graph_optimizer": "AdamW(fused=True)",
        "graph_multi_tensor_adamw_ms_per_step": round(gm_ms, 3),
        "fp32_model": {"ms_per_step": round(fp_ms, 3), "multi_tensor_adamw_ms_per_step": round(fpm_ms, 3),
                       "graph_ms_per_step": round(fg_ms, 3),
                       "graph_multi_tensor_adamw_ms_per_step": round(fgm_ms, 3),
                       "loss": {str(i): round(fp_losses[i], 4) for i in pts}},
        "pipeline": pipe,
    }
    if ref_steps:
        from oracle import eager_torch  # noqa: F401  (the CPU reference restatement)

        torch.manual_seed(6)
        ref = minigpt.build_reference(0)
        ref_losses, ref_ms = minigpt.train(ref, x, y, ref_steps + 1, warmup=1)
        out["cpu_reference"] = {"ms_per_step": round(ref_ms, 1), "threads": torch.get_num_threads(),
                                "steps_timed": ref_steps, "kind": "port",
                                "loss": {str(i): round(v, 4) for i, v in enumerate(ref_losses)}}
    return out


def bench_pipeline(minigpt, x, y, steps: int = 100, warmup: int = 5):
    """The MiniGPT step through AXSTrainingPipelineUnified (loss scaling,
    overflow check and clipping in one fused device pass, one host read per
    step) beside the same step through a restatement of the reference's
    pipeline (per-parameter unscale, two host-synchronising inf/NaN checks per
    parameter, clip_grad_norm_; tests/ref_pipeline.py), same model and batch."""
    import torch
    import torch.nn.functional as F

    from axs.unified import AXSTrainingPipelineUnified
    from ref_pipeline import RefPipeline

    xd, yd = x.cuda(), y.cuda()

    def loss_fn(out, inp):
        return F.cross_entropy(out.reshape(-1, out.shape[-1]), yd.reshape(-1))

    res = {}
    for name, cls in (("ms_per_step", AXSTrainingPipelineUnified), ("reference_style_ms_per_step", RefPipeline)):
        torch.manual_seed(5)
        model = minigpt.build_axs(0, "cuda")
        opt = torch.optim.AdamW(model.parameters(), lr=3e-4)
        p = cls(model, opt, max_grad_norm=1.0)
        for _ in range(warmup):
            p.training_step(xd, loss_fn)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            r = p.training_step(xd, loss_fn)
        torch.cuda.synchronize()
        res[name] = round((time.perf_counter() - t0) * 1e3 / steps, 3)
        res[name.replace("ms_per_step", "final_loss")] = round(r["loss"], 4)
    res["steps"] = steps
    res["param_tensors"] = sum(1 for _ in model.parameters())
    return res


def cpu_threads():
    """Host threads for the CPU baseline: every core this process may run on
    (len(os.sched_getaffinity(0))), capped by OMP_NUM_THREADS when the
    environment sets it (the GPU box sets it to its CPU share).  Sets torch's
    intra-op pool to that count and returns the figures to report."""
    import torch

    torch_default = torch.get_num_threads()
    affinity = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    threads = affinity
    if omp and omp.isdigit() and int(omp) > 0:
        threads = min(threads, int(omp))
    torch.set_num_threads(threads)
    return {"threads": torch.get_num_threads(), "affinity_cores": affinity, "omp_num_threads": omp,
            "torch_default_threads": torch_default, "cpu_model": cpu_model()}


def time_cpu(fn, warmup: int = 3, calls: int = 10, budget_s: float = 30.0):
    """warmup untimed calls, then `calls` timed ones (fewer if budget_s runs
    out first): (median, min, max, count) in seconds."""
    for _ in range(warmup):
        fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < calls and (not times or time.perf_counter() - t_start < budget_s):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), min(times), max(times), len(times)


def cpu_baseline_fq():
    """The reference's CPU eager fused_fake_quantize (oracle/eager_torch.py,
    restating quantize_unified.py:121-204) on the full 8192x4096 fp32 tensor:
    3 warm-ups, median of 10 calls, on every host core and on one."""
    import torch

    from oracle import eager_torch

    info = cpu_threads()
    g = torch.Generator().manual_seed(3)
    x = torch.randn(*FQ_SHAPE, generator=g)
    m = torch.rand(*FQ_SHAPE, generator=g) < 0.01
    x[m] *= 100.0
    nbytes = 8 * x.numel()
    med, lo, hi, n = time_cpu(lambda: eager_torch.fake_quantize(x, 32))
    torch.set_num_threads(1)
    med1, _, _, n1 = time_cpu(lambda: eager_torch.fake_quantize(x, 32), warmup=1, calls=3, budget_s=10.0)
    torch.set_num_threads(info["threads"])
    return {
        "value": round(nbytes / med / 1e9, 3),
        "unit": "GB/s",
        "cores": info["threads"],
        "kind": "port",
        "min_max_gbs": [round(nbytes / hi / 1e9, 3), round(nbytes / lo / 1e9, 3)],
        "one_thread_gbs": round(nbytes / med1 / 1e9, 3),
        "host": info,
        "sample": (f"torch-eager restatement of the reference's fused_fake_quantize "
                   f"(oracle/eager_torch.py) on the full 8192x4096 fp32 tensor: 3 warm-ups, median of "
                   f"{n} calls ({med * 1e3:.1f} ms/call, min {lo * 1e3:.1f}, max {hi * 1e3:.1f}) on "
                   f"{info['threads']} threads ({info['affinity_cores']} cores in the affinity mask, "
                   f"OMP_NUM_THREADS={info['omp_num_threads']}, torch default {info['torch_default_threads']}), "
                   f"{info['cpu_model']}; one thread: median of {n1} calls, {med1 * 1e3:.1f} ms/call"),
    }


def cpu_baseline_linear():
    """The reference's CPU eager linear forward at 4096^3 (FQ(W), FQ(X) with
    the eager fused_fake_quantize, fp32 F.linear -- oracle/eager_torch.py
    restating functional_unified.py:116-123) on the host cores: 3 warm-ups,
    median of 10 calls."""
    import torch

    from oracle import eager_torch

    info = cpu_threads()
    g = torch.Generator().manual_seed(7)
    x = torch.randn(4096, 4096, generator=g)
    w = torch.randn(4096, 4096, generator=g) * 4096 ** -0.5
    flops = 2 * 4096 ** 3
    med, lo, hi, n = time_cpu(lambda: eager_torch.linear_fwd(x, w, None))
    return {
        "value": round(flops / med / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": info["threads"],
        "kind": "port",
        "min_max_tflops": [round(flops / hi / 1e12, 4), round(flops / lo / 1e12, 4)],
        "host": info,
        "sample": (f"torch-eager restatement of the reference's CPU linear forward (FQ(W), FQ(X), fp32 F.linear; "
                   f"oracle/eager_torch.py) at 4096^3: 3 warm-ups, median of {n} calls ({med * 1e3:.1f} ms/call, "
                   f"min {lo * 1e3:.1f}, max {hi * 1e3:.1f}) on {info['threads']} threads "
                   f"({info['affinity_cores']} cores in the affinity mask), {info['cpu_model']}"),
    }


def pmc_pass() -> int:
    """A short run for rocprofv3 counter collection: 8 NF5 fake-quantize
    launches at 8192x4096 f32 over 4 rotating inputs, 3 linear forwards at 4096^3, 5 fused
    small-output linears at M=1, K=N=4096 and, as the calibration reference
    for HBM byte counters, 5 plain device copies of a known 128 MiB (torch's
    copy kernel: 128 MiB read + 128 MiB written)."""
    import torch

    from axs.unified import hip_linear
    from axs.unified.hip_kernels import hip_fused_fake_quantize

    g = torch.Generator(device="cuda").manual_seed(3)
    # HBM-cold like the bench's FQ leg: FQ_ROTATE inputs in turn, each output kept
    xs = [torch.randn(*FQ_SHAPE, device="cuda", generator=g) for _ in range(FQ_ROTATE)]
    outs = [hip_fused_fake_quantize(xs[i % FQ_ROTATE], 32, "nearest") for i in range(2 * FQ_ROTATE)]
    del outs, xs
    M, K, N = LIN_SHAPE
    X = torch.randn(M, K, device="cuda", generator=g)
    W = torch.randn(N, K, device="cuda", generator=g) * K ** -0.5
    for _ in range(3):
        hip_linear.linear_forward(X, W, None, 32, True)
    x1 = torch.randn(1, K, device="cuda", generator=g)
    for _ in range(5):
        hip_linear.fused_forward(x1, W, None)
    src = torch.randn(32 * 1024 * 1024, device="cuda", generator=g)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("pmc pass done", flush=True)
    return 0


def gemm_only(n: int, reps: int = 50) -> int:
    """Times the fp16 MFMA GEMM alone at n^3 (small-integer fp16 operands, so
    the fp32 result is exact and checked).  Prints one JSON line."""
    import torch

    from axs import _lib

    g = torch.Generator(device="cuda").manual_seed(0)
    A = torch.randint(-4, 5, (n, n), device="cuda", generator=g).half()
    B = torch.randint(-4, 5, (n, n), device="cuda", generator=g).half()
    C = torch.empty(n, n, device="cuda")
    st = _lib.stream_of(A)

    def run():
        _lib.call("axs6_gemm_f16_nt", A.data_ptr(), n, B.data_ptr(), n, n, n, n, None, None, None,
                  C.data_ptr(), n, _lib.F32, st)

    run()
    torch.cuda.synchronize()
    exact = bool(torch.equal(C, A.float() @ B.float().T))
    for _ in range(5):
        run()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        run()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / reps * 1e3
    print(json.dumps({"n": n, "us": round(us, 1),
                      "TFLOPs": round(2 * n ** 3 / us / 1e6, 1), "exact": exact}), flush=True)
    return 0 if exact else 1


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-linear", action="store_true")
    ap.add_argument("--no-minigpt", action="store_true")
    ap.add_argument("--gemm-only", type=int, default=0, metavar="N",
                    help="time the fp16 MFMA GEMM alone at N^3 (launch-shape sweeps)")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="short fixed workload for rocprofv3 counter runs (no JSON line)")
    a = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (got --gpus {a.gpus}, WORLD_SIZE {world}); the NF5 "
              "fake-quantize shards by rows with no exchange, so N GPUs run N copies of this "
              "workload.  Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    if a.pmc_pass:
        return pmc_pass()
    if a.gemm_only:
        return gemm_only(a.gemm_only)
    log(f"device: {torch.cuda.get_device_name()}  steps={a.steps} warmup={a.warmup}")

    fq = bench_fq(a.steps, a.warmup)
    gbs = fq["bytes"] / (fq["wall_ms"] * 1e-3) / 1e9
    achieved = fq["bytes"] / (fq["gpu_ms"] * 1e-3) / 1e9
    copy_gbs = fq["bytes"] / (fq["copy_gpu_ms"] * 1e-3) / 1e9
    warm_achieved = fq["bytes"] / (fq["warm"]["gpu_ms"] * 1e-3) / 1e9
    warm_copy_gbs = fq["bytes"] / (fq["warm"]["copy_gpu_ms"] * 1e-3) / 1e9
    log(f"fq 8192x4096: {fq['wall_ms']*1e3:.1f} us/step, {fq['gpu_ms']*1e3:.1f} us/launch (device), "
        f"{achieved:.0f} GB/s cold; eager API step {fq['eager_ms']*1e3:.1f} us; device copy of the same "
        f"bytes {copy_gbs:.0f} GB/s; warm (one buffer) {warm_achieved:.0f} GB/s")
    traffic = load_traffic("fq_8192x4096_traffic.json")
    out = {
        "metric": "NF5 fake-quant GB/s @8192x4096 fp32; AXS-6 linear TFLOP/s @4096^3 bf16",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(fq["wall_ms"], 5),
        "device_ms_per_launch": round(fq["gpu_ms"], 5),
        "eager_ms_per_step": round(fq["eager_ms"], 5),
        "launch": f"steps run as replays of a HIP graph of {GRAPH_STEPS} steps (every kernel runs every step); "
                  "eager_ms_per_step is the same step through the Python API and autograd",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: N(0,1) with 1% of elements x100, seeded",
        "config": {"workload": "NF5 fake-quantize fwd + STE bwd, 8192x4096 fp32, block 32",
                   "shape": list(FQ_SHAPE), "block_size": 32},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "copy_achieved": round(copy_gbs, 1),
                     "frac_of_copy": round(achieved / copy_gbs, 4),
                     "cache": f"cold: {FQ_ROTATE} rotating 128 MiB inputs and a fresh output buffer per launch "
                              "(past the 256 MiB last-level cache)",
                     "warm": {"note": "one input replayed every step (last-level cache partly serves it)",
                              "device_ms_per_launch": round(fq["warm"]["gpu_ms"], 5),
                              "achieved": round(warm_achieved, 1),
                              "frac": round(warm_achieved / HBM_PEAK_GBS, 4),
                              "copy_achieved": round(warm_copy_gbs, 1),
                              "frac_of_copy": round(warm_achieved / warm_copy_gbs, 4)}},
    }

    if not a.no_linear:
        try:
            lin = bench_linear(max(a.steps // 2, 10), max(a.warmup // 2, 3))
            tflops = lin["flops"] / (lin["wall_ms"] * 1e-3) / 1e12
            log(f"linear 4096^3 fwd: {lin['wall_ms']*1e3:.1f} us/step, {tflops:.0f} TFLOP/s")
            k = lin["kernels"]
            gemm_tf = lin["flops"] / (k["gemm_ms"] * 1e-3) / 1e12 if k.get("gemm_ms") else None
            # the whole forward (packing of X and W + GEMM) on the device, per step
            fwd_tf = lin["flops"] / (lin["gpu_ms"] * 1e-3) / 1e12
            out["linear"] = {
                "metric": "AXS-6 linear forward TFLOP/s @4096^3",
                "value": round(tflops, 1), "unit": "TFLOP/s",
                "ms_per_step": round(lin["wall_ms"], 5),
                "device_ms_per_step": round(lin["gpu_ms"], 5),
                "eager_ms_per_step": round(lin["eager_ms"], 5),
                "dtype": k.get("compute_dtype"),
                "kernels_ms": {kk: round(v, 5) for kk, v in k.items() if kk.endswith("_ms")},
                "roofline": {"bound": "mfma", "scope": "whole forward: FQ + packing of X and W, then the GEMM",
                             "achieved": round(fwd_tf, 1),
                             "peak": BF16_DENSE_PEAK_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(fwd_tf / BF16_DENSE_PEAK_TFLOPS, 4),
                             "gemm_only": {"achieved": round(gemm_tf, 1) if gemm_tf else None,
                                           "frac": round(gemm_tf / BF16_DENSE_PEAK_TFLOPS, 4) if gemm_tf else None,
                                           "traffic": load_traffic("linear_4096_traffic.json")},
                             "traffic": load_traffic("linear_4096_traffic.json", "forward_traffic_bytes")},
                "cold": {"note": "3 rotating X, W pairs (384 MiB) and a fresh Y per call, graph replays; "
                                 "the figures above replay one X, W pair, which the 256 MiB last-level "
                                 "cache partly holds",
                         "device_ms_per_step": round(lin["cold_ms"], 5),
                         "achieved": round(lin["flops"] / (lin["cold_ms"] * 1e-3) / 1e12, 1),
                         "frac": round(lin["flops"] / (lin["cold_ms"] * 1e-3) / 1e12 / BF16_DENSE_PEAK_TFLOPS, 4)},
            }
            lb = bench_linear(max(a.steps // 2, 10), max(a.warmup // 2, 3), dtype=torch.bfloat16)
            tb = lb["flops"] / (lb["wall_ms"] * 1e-3) / 1e12
            out["linear"]["bf16_io"] = {
                "note": "the same forward with bf16 X, W and Y (FQ of the bf16 values, fp16 MFMA, bf16 out)",
                "ms_per_step": round(lb["wall_ms"], 5), "device_ms_per_step": round(lb["gpu_ms"], 5),
                "value": round(tb, 1), "unit": "TFLOP/s", "end_to_end_frac": round(tb / BF16_DENSE_PEAK_TFLOPS, 4)}
            log(f"linear 4096^3 fwd, bf16 I/O: {lb['wall_ms']*1e3:.1f} us/step, {tb:.0f} TFLOP/s")
        except Exception as e:  # noqa: BLE001 - reported in the JSON line
            import traceback

            traceback.print_exc(file=sys.stderr)
            out.setdefault("linear", {})["error"] = f"{type(e).__name__}: {e}"

    def leg(dst: dict, key: str, fn, *args, **kw) -> bool:
        """Runs one secondary measurement into dst[key]; a Python exception in
        it is recorded there (and its traceback logged) instead of losing the
        headline line."""
        try:
            dst[key] = fn(*args, **kw)
            return True
        except Exception as e:  # noqa: BLE001 - reported in the JSON line
            import traceback

            traceback.print_exc(file=sys.stderr)
            dst[key] = {"error": f"{type(e).__name__}: {e}"}
            return False

    if leg(out, "wire", bench_wire):
        log(f"wire 8192x4096: pack {out['wire']['pack_gbs']} GB/s, unpack {out['wire']['unpack_gbs']} GB/s; "
            f"AXSBlock records {out['wire']['axs_blocks']}")
    if leg(out, "configs", bench_configs):
        log(f"configs: {out['configs']}")
    if leg(out, "codec", bench_codec):
        log(f"codec 8192x4096: quantize {out['codec']['quantize_gbs']} GB/s, "
            f"dequantize {out['codec']['dequantize_gbs']} GB/s")

    if not a.no_linear:
        if leg(out, "fused", bench_fused):
            log(f"fused small-output linear: {out['fused']}")
        log("linear fwd+bwd (config 4) ...")
        leg(out, "linear_train", bench_linear_train)

    if not a.no_minigpt:
        log("minigpt (config 5) ...")
        if leg(out, "minigpt", bench_minigpt, ref_steps=0 if a.no_cpu_baseline else 3):
            log(f"minigpt: {out['minigpt']['ms_per_step']} ms/step, loss {out['minigpt']['loss']}")

    if not a.no_cpu_baseline:
        log("cpu baseline ...")
        if leg(out, "cpu_baseline", cpu_baseline_fq):
            log(f"cpu baseline: {out['cpu_baseline']['value']} GB/s")
        if "linear" in out and "roofline" in out["linear"]:
            if leg(out["linear"], "cpu_baseline", cpu_baseline_linear):
                log(f"cpu baseline, linear: {out['linear']['cpu_baseline']['value']} TFLOP/s")
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
