"""Write the golden vectors that pin the CPU oracle to the reference.

Run once, in the build container where the reference is mounted:

    python tests/golden/make_golden.py /root/reference

It imports the reference's eager NF5 functions -- ``fused_fake_quantize``,
``quantize_unified`` and ``dequantize_unified`` from
``axs/unified/quantize_unified.py:121-308`` -- because the reference's own
tests hold no known-answer vectors for them and their order of operations and
edge semantics (NaN / inf / zero blocks, the exponent clamp of
``quantize_unified``, padding) are fixed by nothing else.  The codebook and
LUT are not taken from here: their closed forms pin them.

Outputs (data only: inputs and expected outputs) go next to this script:
  edge_cases.npz  -- hand-built edge blocks, nearest rounding, bs 8/16/32
  ragged.npz      -- odd shapes needing padding, fp32 / bf16 / fp16 inputs
  config1.npz     -- BASELINE config 1: randn(1024,1024, seed 0) * 0.02
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def edge_inputs() -> np.ndarray:
    """(rows, 32) float32 matrix; each row is one 32-wide block (and four
    8-wide / two 16-wide blocks) exercising one edge of the algorithm."""
    rows = []
    g = np.random.default_rng(1234)

    def gauss(scale=1.0):
        return (g.standard_normal(32) * scale).astype(np.float32)

    f32 = np.float32
    rows.append(np.zeros(32, f32))                                  # all zero
    r = np.zeros(32, f32); r[5] = -0.0; rows.append(r)              # -0.0
    r = np.full(32, -0.0, f32); rows.append(r)
    rows.append(np.full(32, 0.75, f32))                             # all equal
    rows.append(np.full(32, -3.0, f32))
    for e in (-149, -140, -130, -127, -126, -125, -60, -2, -1, 0, 1, 3, 5, 8, 64, 126, 127):
        r = gauss(0.25); r[7] = np.ldexp(f32(1.0), e) if e > -150 else 0; rows.append(r.astype(f32))
        r2 = np.zeros(32, f32); r2[0] = np.ldexp(1.0, e); r2[1] = -np.ldexp(0.7, e); rows.append(r2.astype(f32))
    # amax in (and just outside) the correctly-rounded log2 band below 2^k
    for k in (-130, -126, -124, -64, -20, -4, -3, -2, 3, 5, 9, 17, 33, 65, 100, 127, 128):
        top = np.array([np.ldexp(1.0, k)], np.float64).astype(np.float32).view(np.uint32)[0] \
            if k < 128 else np.uint32(0x7F800000)
        for d in (1, 2, 5, 11, 22, 44, 45, 60):
            b = np.uint32(top - d)
            v = np.array([b], np.uint32).view(np.float32)[0]
            if not np.isfinite(v) or v <= 0:
                continue
            r = (gauss(1.0) * f32(v) / f32(4.0)).astype(f32)
            r = np.clip(r, -v, v).astype(f32)
            r[3] = v
            rows.append(r)
    # subnormal / tiny blocks
    for m in (1, 2, 3, 7, 100, 4095, 2**22 - 1, 2**23 - 1):
        r = np.zeros(32, np.uint32); r[0] = m; r[9] = max(m // 3, 1) | 0x80000000
        rows.append(r.view(np.float32))
    # specials
    for special in (np.inf, -np.inf, np.nan):
        r = gauss(1.0); r[4] = special; rows.append(r)
        r = gauss(1.0); r[4] = special; r[10] = 0.0; r[11] = -0.0; rows.append(r)
    r = gauss(1.0); r[0] = np.inf; r[1] = -np.inf; rows.append(r)
    r = gauss(1.0); r[0] = np.inf; r[1] = np.nan; rows.append(r)
    fmax = np.finfo(np.float32).max
    r = gauss(1e37); r[2] = fmax; rows.append(r.astype(f32))
    r = gauss(1e37); r[2] = -fmax; r[3] = 0.0; rows.append(r.astype(f32))
    r = gauss(1.0) * f32(1e-40); rows.append(r.astype(f32))
    # LUT cell boundaries: n = i/1023 +- a few ulps in a block with amax = 1 - tiny
    for base in range(0, 1024, 37):
        r = np.zeros(32, np.float32)
        r[0] = np.float32(0.99999994)  # scale 1.0
        n = np.float32(base / 1023.0)
        vals = [n]
        for d in range(1, 8):
            vals.append(np.nextafter(vals[-1], np.float32(0)))
        up = [n]
        for d in range(1, 8):
            up.append(np.nextafter(up[-1], np.float32(2)))
        vv = np.array(vals + up[1:], np.float32)[:31]
        r[1:1 + len(vv)] = vv
        rows.append(r)
    for _ in range(16):
        rows.append(gauss(1.0))
        rows.append(gauss(1e-3))
    return np.stack(rows).astype(np.float32)


def ragged_inputs():
    g = np.random.default_rng(99)
    shapes = [(7, 13), (3, 100, 17), (4, 50), (1, 1), (100, 50), (5, 33), (2, 4, 8, 32), (9, 1000)]
    out = {}
    for i, s in enumerate(shapes):
        x = g.standard_normal(s).astype(np.float32)
        m = g.random(s) < 0.01
        x[m] *= 100.0
        out[f"x{i}"] = x
    return out


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from axs.unified.quantize_unified import (  # noqa: E402  (reference)
        dequantize_unified,
        fused_fake_quantize,
        quantize_unified,
    )

    # ---- edge suite -------------------------------------------------------
    x = edge_inputs()
    res = {"x": x}
    xt = torch.from_numpy(x)
    for bs in (8, 16, 32):
        res[f"fq_bs{bs}"] = fused_fake_quantize(xt, bs, "nearest").numpy()
        q = quantize_unified(xt, bs, "nearest")
        res[f"exp_bs{bs}"] = q.shared_exponents.numpy()
        res[f"code_bs{bs}"] = q.magnitudes.numpy()
        res[f"sign_bs{bs}"] = q.signs.numpy()
        res[f"deq_bs{bs}"] = dequantize_unified(q).numpy()
    np.savez_compressed(os.path.join(HERE, "edge_cases.npz"), **res)

    # ---- ragged shapes, three input dtypes -------------------------------
    rg = ragged_inputs()
    res = {}
    for name, xa in rg.items():
        res[name] = xa
        for bs in (8, 16, 32):
            res[f"{name}_fq_bs{bs}"] = fused_fake_quantize(torch.from_numpy(xa), bs, "nearest").numpy()
        for dt, tag in ((torch.bfloat16, "bf16"), (torch.float16, "f16")):
            xd = torch.from_numpy(xa).to(dt)
            yd = fused_fake_quantize(xd, 32, "nearest")
            assert yd.dtype == dt
            res[f"{name}_in_{tag}"] = xd.view(torch.int16).numpy()
            res[f"{name}_fq_{tag}"] = yd.view(torch.int16).numpy()
    np.savez_compressed(os.path.join(HERE, "ragged.npz"), **res)

    # ---- config 1 ----------------------------------------------------------
    gen = torch.Generator().manual_seed(0)
    x1 = torch.randn(1024, 1024, generator=gen) * 0.02
    fq = fused_fake_quantize(x1, 32, "nearest")
    q = quantize_unified(x1, 32, "nearest")
    deq = dequantize_unified(q)
    np.savez_compressed(
        os.path.join(HERE, "config1.npz"),
        input_sha=np.array(sha(x1.numpy())),
        exps=q.shared_exponents.numpy(),
        codes_head=q.magnitudes.numpy()[:32],
        signs_head=q.signs.numpy()[:32],
        fq_head=fq.numpy()[:32],
        codes_sha=np.array(sha(q.magnitudes.numpy())),
        signs_sha=np.array(sha(q.signs.numpy())),
        fq_sha=np.array(sha(fq.numpy())),
        deq_sha=np.array(sha(deq.numpy())),
    )
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
