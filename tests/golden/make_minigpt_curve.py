"""Write the 200-step MiniGPT loss curves of the CPU
restatement of the reference's eager NF5 path, the fixture the GPU product
path's curve is compared with (tests/test_gpu_minigpt.py).

    python tests/golden/make_minigpt_curve.py [--steps 200]

The model, initial weights (seed 0), batch (seed 1) and AdamW settings are
tests/minigpt.py's; the reference's operations are oracle/eager_torch.py's
(pinned to the reference by the golden vectors).  Two curves:
  * "nearest": dY taken as given (quantize_grad=False), deterministic;
  * "stochastic": dY fake-quantized with stochastic rounding, torch.rand_like
    drawn from torch's CPU generator seeded with 6 (the reference's own
    stream, which the GPU path does not share).
Data only (the curves and the settings) goes to minigpt_curve.npz beside
this script.  Runs on the CPU in a few minutes per curve.
"""
from __future__ import annotations

import argparse
import os
import sys
import time

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

import minigpt  # noqa: E402


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=200)
    a = ap.parse_args()
    x, y = minigpt.batch(1)
    out = {"steps": np.array(a.steps), "model_seed": np.array(0), "batch_seed": np.array(1)}
    for name, qgrad in (("nearest", False), ("stochastic", True)):
        torch.manual_seed(6)
        ref = minigpt.build_reference(0, quantize_grad=qgrad)
        t0 = time.time()
        losses, ms = minigpt.train(ref, x, y, a.steps)
        out[name] = np.array(losses, np.float64)
        print(f"{name}: {losses[0]:.4f} -> {losses[-1]:.4f} ({time.time() - t0:.0f} s, "
              f"{torch.get_num_threads()} threads)", flush=True)
    np.savez_compressed(os.path.join(HERE, "minigpt_curve.npz"), **out)
    print("wrote minigpt_curve.npz")


if __name__ == "__main__":
    main()
