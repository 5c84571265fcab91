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
  stochastic.npz  -- rounding="stochastic" of fused_fake_quantize and
                     quantize_unified with torch.rand_like replaced by a saved
                     array U (the draws, in the reference's padded
                     (rows, blocks, block) layout, are part of the fixture):
                     the edge suite, ragged rows, bf16 input

    python tests/golden/make_golden.py /root/reference [--only stochastic]
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


def draws(rng, shape) -> np.ndarray:
    """U[0,1) with torch.rand's 24-bit resolution, with the extreme and
    midpoint draws (0, 2^-24, 0.5 - 2^-24, 0.5, 0.5 + 2^-24, 1 - 2^-24)
    planted at every 7th position."""
    k = rng.integers(0, 1 << 24, size=shape, dtype=np.int64)
    special = np.array([0, 1, (1 << 23) - 1, 1 << 23, (1 << 23) + 1, (1 << 24) - 1], np.int64)
    flat = k.reshape(-1)
    flat[::7] = special[np.arange(flat[::7].size) % special.size]
    return (flat.reshape(shape).astype(np.float64) * 2.0 ** -24).astype(np.float32)


def dither_boundary_inputs(rng) -> tuple[np.ndarray, np.ndarray]:
    """Blocks whose dithered index (n + (U - 0.5)/1023) * 1023 lands within a
    few float32 ulps of an integer, for draws U picked so that float32
    restatements equal to it in exact arithmetic (n*1023 + (U - 0.5), ...)
    truncate to a different index: these pin the reference's order of
    operations.  Each row is one 32-block whose element 0 is 0.99999994
    (scale 1, so n = |x|); the rest are signed candidates n with their U.
    Returns x (rows, 32) and U (rows, 1, 32)."""
    f32 = np.float32
    n = (rng.random(40000) * 0.999).astype(f32)
    j = np.round(n.astype(np.float64) * 1023)
    k0 = np.round((0.5 + j - n.astype(np.float64) * 1023) * 2 ** 24).astype(np.int64)
    ks = np.clip(k0[:, None] + np.arange(-64, 65)[None, :], 0, (1 << 24) - 1)
    U = (ks.astype(np.float64) * 2.0 ** -24).astype(f32)
    nn = np.broadcast_to(n[:, None], U.shape)
    t_ref = (nn + (U - f32(0.5)) / f32(1023)) * f32(1023)
    t_alt = nn * f32(1023) + (U - f32(0.5))
    hit = np.argwhere(np.trunc(t_ref) != np.trunc(t_alt))
    rows = 64
    pick = hit[rng.choice(hit.shape[0], rows * 31, replace=False)]
    x = np.zeros((rows, 32), f32)
    u = draws(rng, (rows, 1, 32))
    x[:, 0] = f32(0.99999994)
    sign = np.where(rng.random(rows * 31) < 0.5, f32(-1), f32(1))
    x[:, 1:] = (n[pick[:, 0]] * sign).reshape(rows, 31)
    u[:, 0, 1:] = U[pick[:, 0], pick[:, 1]].reshape(rows, 31)
    return x, u


class fixed_rand:
    """Replaces torch.rand_like for one call with a saved array of the same shape."""

    def __init__(self, u: np.ndarray):
        self.u = torch.from_numpy(u)
        self.calls = 0

    def __enter__(self):
        self.orig = torch.rand_like

        def fake(t, *a, **k):
            assert tuple(t.shape) == tuple(self.u.shape), (tuple(t.shape), tuple(self.u.shape))
            self.calls += 1
            return self.u.clone().to(t.dtype)

        torch.rand_like = fake
        return self

    def __exit__(self, *exc):
        torch.rand_like = self.orig
        assert self.calls == 1, "the reference drew rand_like a different number of times"


def stochastic(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from axs.unified.quantize_unified import (  # noqa: E402  (reference)
        dequantize_unified,
        fused_fake_quantize,
        quantize_unified,
    )

    rng = np.random.default_rng(4321)
    res = {}
    g = np.random.default_rng(77)
    xr = (g.standard_normal((32, 1000)) * 10.0 ** g.uniform(-3, 3, (32, 1))).astype(np.float32)
    xr[g.random(xr.shape) < 0.01] *= 100.0
    cases = {"edge": (edge_inputs(), (8, 16, 32)), "ragged": (xr, (8, 32))}
    for name, (x, sizes) in cases.items():
        res[f"x_{name}"] = x
        R, C = x.shape
        for bs in sizes:
            nblk = (C + bs - 1) // bs
            u = draws(rng, (R, nblk, bs))      # the same draws for both functions
            res[f"u_{name}_bs{bs}"] = u
            with fixed_rand(u):
                res[f"fq_{name}_bs{bs}"] = fused_fake_quantize(torch.from_numpy(x), bs, "stochastic").numpy()
            with fixed_rand(u):
                q = quantize_unified(torch.from_numpy(x), bs, "stochastic")
            res[f"exp_{name}_bs{bs}"] = q.shared_exponents.numpy()
            res[f"code_{name}_bs{bs}"] = q.magnitudes.numpy()
            res[f"sign_{name}_bs{bs}"] = q.signs.numpy()
            res[f"deq_{name}_bs{bs}"] = dequantize_unified(q).numpy()
    # draws at the index boundaries (block 32)
    xd, ud = dither_boundary_inputs(rng)
    res["x_dither"], res["u_dither"] = xd, ud
    with fixed_rand(ud):
        res["fq_dither"] = fused_fake_quantize(torch.from_numpy(xd), 32, "stochastic").numpy()
    with fixed_rand(ud):
        q = quantize_unified(torch.from_numpy(xd), 32, "stochastic")
    res["exp_dither"] = q.shared_exponents.numpy()
    res["code_dither"] = q.magnitudes.numpy()
    # bf16 input: FQ in float32 of the bf16 values, result cast back to bf16
    xb = torch.from_numpy(xr).to(torch.bfloat16)
    u = draws(rng, (32, 32, 32))
    res["x_bf16"] = xb.view(torch.int16).numpy()
    res["u_bf16"] = u
    with fixed_rand(u):
        yb = fused_fake_quantize(xb, 32, "stochastic")
    assert yb.dtype == torch.bfloat16
    res["fq_bf16"] = yb.view(torch.int16).numpy()
    np.savez_compressed(os.path.join(HERE, "stochastic.npz"), **res)
    print("wrote stochastic.npz")


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
    args = [a for a in sys.argv[1:] if not a.startswith("--")]
    root = args[0] if args else "/root/reference"
    if "--only" in sys.argv:
        what = sys.argv[sys.argv.index("--only") + 1]
        assert what == "stochastic", what
        stochastic(root)
    else:
        main(root)
        stochastic(root)
