"""Pins the CPU oracle (oracle/nf5_oracle.c) before it is trusted as the
checker of the HIP kernels.

* tables: closed forms through torch's own erfinv / bucketize (the library
  calls of axs/unified/quantize_unified.py:50-97) and the SHA-256 values of
  the float32 bytes;
* exponent: floor(torch.log2(x)) -- the reference's call at
  quantize_unified.py:173-175 -- on every float32 in the rounding bands
  below each power of two, every subnormal and a stride through the rest
  (the full 2^31 sweep is the `slow` test);
* fused_fake_quantize / quantize_unified / dequantize_unified: golden
  vectors written from the reference (tests/golden/make_golden.py);
* invariants that a dropped term, a wrong sign or a wrong index would break.
"""
from __future__ import annotations

import hashlib
import math
import os

import numpy as np
import pytest
import torch

import oracle
from conftest import bits_equal, first_mismatch, load_golden

CODEBOOK_SHA = "1173960ec84b5b27bd114bb79830c21f0ba61bfced6efb0835ba794c4b5bb298"
LUT_SHA = "399b787320602da9cfb09d29335222c56cf39ee9ec1e59bfd2aa2d673591e271"


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# ---------------------------------------------------------------- tables --

def test_codebook_closed_form():
    cb, _, _ = oracle.tables()
    lv = torch.zeros(32, dtype=torch.float64)
    for i in range(32):
        lv[i] = math.sqrt(2.0) * torch.erfinv(torch.tensor((i + 0.5) / 32, dtype=torch.float64)).item()
    lv = (lv / lv[-1]).float().numpy()
    assert bits_equal(cb, lv)
    assert sha(cb) == CODEBOOK_SHA
    assert cb[-1] == 1.0 and np.all(np.diff(cb) > 0)


def test_lut_closed_form():
    cb, lut, rev = oracle.tables()
    cbd = torch.from_numpy(cb).double()
    bnd = torch.cat([torch.zeros(1, dtype=torch.float64), (cbd[:-1] + cbd[1:]) / 2,
                     torch.tensor([1.0 + 1e-6], dtype=torch.float64)])
    codes = (torch.bucketize(torch.linspace(0.0, 1.0, 1024, dtype=torch.float64), bnd) - 1).clamp(0, 31)
    assert bits_equal(lut, cbd[codes].float().numpy())
    assert np.array_equal(rev, codes.numpy().astype(np.uint8))
    assert sha(lut) == LUT_SHA
    # each code owns one contiguous run (first indices from the survey, A.2)
    first = [int(np.argmax(rev == c)) for c in range(32)]
    assert first == [0, 17, 34, 50, 67, 84, 101, 118, 135, 153, 171, 189, 207, 226, 246, 266, 286,
                     307, 329, 352, 376, 401, 428, 457, 488, 521, 559, 601, 651, 712, 794, 932]
    assert np.all(np.diff(rev.astype(int)) >= 0)


# -------------------------------------------------------------- exponent --

def _torch_floor_log2(x: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(x).clamp(min=1e-45)
    return torch.floor(torch.log2(t)).numpy()


def _band_region_floats(width: int = 128) -> np.ndarray:
    out = []
    for k in range(-148, 129):
        top = np.uint32((k + 127) << 23) if k >= -126 else np.uint32(1 << (k + 149))
        lo = max(int(top) - width, 1)
        hi = min(int(top) + width, 0x7F7FFFFF)
        out.append(np.arange(lo, hi + 1, dtype=np.uint32))
    return np.unique(np.concatenate(out)).view(np.float32)


def test_floor_log2_band_regions_vectorised():
    x = _band_region_floats()
    got = oracle.floor_log2(x)
    want = _torch_floor_log2(x)
    assert bits_equal(got, want), first_mismatch(got, want)


def test_floor_log2_band_regions_scalar_path():
    # 0-d tensors take torch's scalar (non-vectorised) log2 kernel
    x = _band_region_floats(48)[::3]
    got = oracle.floor_log2(x)
    want = np.array([math.floor(torch.log2(torch.tensor(float(v), dtype=torch.float32)).item())
                     for v in x], np.float32)
    assert bits_equal(got, want), first_mismatch(got, want)


def test_floor_log2_all_subnormals_and_stride():
    sub = np.arange(1, 1 << 23, dtype=np.uint32).view(np.float32)
    got = oracle.floor_log2(sub)
    assert bits_equal(got, _torch_floor_log2(sub))
    strided = np.arange(1, 0x7F7FFFFF, 4099, dtype=np.uint32).view(np.float32)
    got = oracle.floor_log2(strided)
    assert bits_equal(got, _torch_floor_log2(strided))
    specials = np.array([0.0, np.inf, np.nan, 1e-45, np.finfo(np.float32).max], np.float32)
    assert bits_equal(oracle.floor_log2(specials), _torch_floor_log2(specials))


@pytest.mark.slow
@pytest.mark.skipif(not os.environ.get("AXS6_SLOW"), reason="full 2^31 sweep: set AXS6_SLOW=1")
def test_floor_log2_every_positive_float():
    step = 1 << 24
    for start in range(1, 0x7F800000, step):
        x = np.arange(start, min(start + step, 0x7F800000), dtype=np.uint32).view(np.float32)
        got = oracle.floor_log2(x)
        want = _torch_floor_log2(x)
        assert bits_equal(got, want), (hex(start), first_mismatch(got, want))


def test_exp2_of_integers_is_exact():
    k = np.arange(-160, 140, dtype=np.float32)
    want = torch.exp2(torch.from_numpy(k)).numpy()
    got = np.ldexp(np.float32(1.0), k.astype(np.int32)).astype(np.float32)
    assert bits_equal(got, want)


# --------------------------------------------------- golden: edge cases --

@pytest.mark.parametrize("bs", [8, 16, 32])
def test_fake_quantize_edge_golden(bs):
    g = load_golden("edge_cases.npz")
    got = oracle.fake_quantize(g["x"], bs)
    assert bits_equal(got, g[f"fq_bs{bs}"]), first_mismatch(got, g[f"fq_bs{bs}"])


@pytest.mark.parametrize("bs", [8, 16, 32])
def test_quantize_edge_golden(bs):
    g = load_golden("edge_cases.npz")
    e, c, s = oracle.quantize(g["x"], bs)
    assert np.array_equal(e, g[f"exp_bs{bs}"]), first_mismatch(e, g[f"exp_bs{bs}"])
    assert np.array_equal(c, g[f"code_bs{bs}"])
    assert np.array_equal(s, g[f"sign_bs{bs}"])


@pytest.mark.parametrize("bs", [8, 16, 32])
def test_dequantize_edge_golden(bs):
    g = load_golden("edge_cases.npz")
    d = oracle.dequantize(g[f"exp_bs{bs}"], g[f"code_bs{bs}"], g[f"sign_bs{bs}"], g["x"].shape[1], bs)
    assert bits_equal(d, g[f"deq_bs{bs}"]), first_mismatch(d, g[f"deq_bs{bs}"])


def test_ragged_golden_all_dtypes():
    g = load_golden("ragged.npz")
    for i in range(8):
        x = g[f"x{i}"]
        for bs in (8, 16, 32):
            got = oracle.fake_quantize(x, bs)
            assert bits_equal(got, g[f"x{i}_fq_bs{bs}"]), (i, bs)
        for tag, dt in (("bf16", torch.bfloat16), ("f16", torch.float16)):
            xin = torch.from_numpy(g[f"x{i}_in_{tag}"]).view(dt).float().numpy()
            y = torch.from_numpy(oracle.fake_quantize(xin, 32)).to(dt).view(torch.int16).numpy()
            assert np.array_equal(y, g[f"x{i}_fq_{tag}"]), (i, tag)


def test_config1_golden():
    g = load_golden("config1.npz")
    gen = torch.Generator().manual_seed(0)
    x = (torch.randn(1024, 1024, generator=gen) * 0.02).numpy()
    if sha(x) != str(g["input_sha"]):
        pytest.skip("this host's torch.randn stream differs from the fixture's")
    e, c, s = oracle.quantize(x, 32)
    assert np.array_equal(e, g["exps"])
    assert np.array_equal(c[:32], g["codes_head"]) and sha(c) == str(g["codes_sha"])
    assert np.array_equal(s[:32], g["signs_head"]) and sha(s) == str(g["signs_sha"])
    fq = oracle.fake_quantize(x, 32)
    assert bits_equal(fq[:32], g["fq_head"]) and sha(fq) == str(g["fq_sha"])
    d = oracle.dequantize(e, c, s, 1024, 32)
    assert sha(d) == str(g["deq_sha"])


# ------------------------------------------------------------ invariants --

def test_invariants_random_blocks():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((512, 96)) * np.exp(rng.uniform(-20, 20, (512, 1)))).astype(np.float32)
    cb, lut, _ = oracle.tables()
    y = oracle.fake_quantize(x, 32)
    xb = x.reshape(512, 3, 32)
    yb = y.reshape(512, 3, 32)
    amax = np.abs(xb).max(-1, keepdims=True)
    scale = np.exp2(np.floor(np.log2(amax.astype(np.float64))) + 1)
    # signs preserved, magnitudes are codebook levels times the block scale
    nz = xb != 0
    assert np.all(np.sign(yb[nz]) == np.sign(xb[nz]))
    lv = np.abs(yb) / scale
    assert np.all(np.isin(lv.astype(np.float32), cb))
    # reconstruction error is bounded by one codebook gap times the scale
    gap = np.max(np.diff(np.concatenate([[0.0], cb.astype(np.float64)])))
    assert np.all(np.abs(yb - xb) <= gap * scale + 1e-30)
    # all-equal block is uniform, zero block is zero
    z = oracle.fake_quantize(np.zeros((2, 32), np.float32))
    assert np.all(z == 0)
    u = oracle.fake_quantize(np.full((1, 32), -0.3, np.float32))
    assert np.all(u == u[0, 0]) and u[0, 0] < 0


def test_exponent_matches_scale_of_fake_quantize():
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((256, 64)) * 10.0 ** rng.uniform(-30, 30, (256, 1))).astype(np.float32)
    e, c, s = oracle.quantize(x, 32)
    y = oracle.fake_quantize(x, 32)
    cb, _, _ = oracle.tables()
    # in the normal range FQ and quantize->dequantize agree on non-zero values
    d = oracle.dequantize(e, c, s, 64, 32)
    nz = x != 0
    assert bits_equal(d[nz], y[nz])


def test_uniform_stream_statistics():
    u = oracle.uniform(12345, 0, 1 << 20)
    assert u.min() >= 0.0 and u.max() < 1.0
    assert abs(u.mean() - 0.5) < 2e-3
    assert abs(u.var() - 1.0 / 12.0) < 2e-3
    hist = np.histogram(u, bins=64, range=(0, 1))[0]
    expected = u.size / 64
    chi2 = float(((hist - expected) ** 2 / expected).sum())
    assert chi2 < 120  # 63 dof; p << 1e-6 beyond this
    # offset continues the same stream
    assert bits_equal(oracle.uniform(12345, 1000, 16), u[1000:1016])


def test_stochastic_dither_is_unbiased():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((64, 256)).astype(np.float32)
    errs = []
    for s in range(24):
        y = oracle.fake_quantize(x, 32, oracle.uniform(1000 + s, 0, x.size))
        errs.append(float((x - y).mean()))
    assert abs(np.mean(errs)) < 0.01


def _unpad(u: np.ndarray, cols: int) -> np.ndarray:
    """The reference's draws in its padded (rows, blocks, block) layout ->
    the oracle's one draw per (row, col) element."""
    return np.ascontiguousarray(u.reshape(u.shape[0], -1)[:, :cols])


def test_stochastic_matches_reference_fixture():
    """rounding="stochastic" of the reference's fused_fake_quantize and
    quantize_unified with torch.rand_like replaced by saved draws
    (tests/golden/stochastic.npz): the oracle, given the same draws, gives
    the same bits, codes, exponents and signs."""
    g = load_golden("stochastic.npz")
    for name, sizes in (("edge", (8, 16, 32)), ("ragged", (8, 32))):
        x = g[f"x_{name}"]
        for bs in sizes:
            u = _unpad(g[f"u_{name}_bs{bs}"], x.shape[1])
            fq = oracle.fake_quantize(x, bs, u)
            want = g[f"fq_{name}_bs{bs}"]
            assert bits_equal(fq, want), f"{name} bs{bs}: {first_mismatch(fq, want)}"
            e, c, s = oracle.quantize(x, bs, u)
            assert np.array_equal(e, g[f"exp_{name}_bs{bs}"]), f"{name} bs{bs} exponents"
            assert np.array_equal(c.reshape(-1), g[f"code_{name}_bs{bs}"].reshape(-1)), f"{name} bs{bs} codes"
            assert np.array_equal(s.reshape(-1), g[f"sign_{name}_bs{bs}"].reshape(-1)), f"{name} bs{bs} signs"
            deq = oracle.dequantize(e, c, s, x.shape[1], bs)
            assert bits_equal(deq, g[f"deq_{name}_bs{bs}"]), f"{name} bs{bs} dequantize"
    # draws planted at the index boundaries
    x = g["x_dither"]
    u = _unpad(g["u_dither"], 32)
    fq = oracle.fake_quantize(x, 32, u)
    assert bits_equal(fq, g["fq_dither"]), first_mismatch(fq, g["fq_dither"])
    e, c, _ = oracle.quantize(x, 32, u)
    assert np.array_equal(e, g["exp_dither"]) and np.array_equal(c.reshape(-1), g["code_dither"].reshape(-1))
    # bf16 input: FQ of the bf16 values in float32, cast back to bf16
    xb = torch.from_numpy(g["x_bf16"]).view(torch.bfloat16)
    u = _unpad(g["u_bf16"], xb.shape[1])
    fq = torch.from_numpy(oracle.fake_quantize(xb.float().numpy(), 32, u)).to(torch.bfloat16)
    assert np.array_equal(fq.view(torch.int16).numpy(), g["fq_bf16"])


def _fq_stochastic_numpy(x: np.ndarray, u: np.ndarray, variant: str) -> np.ndarray:
    """fused_fake_quantize (block 32, rows of whole blocks, finite data) with
    the dither index computed in float32 numpy, per `variant`: "reference"
    the reference's order of operations (quantize_unified.py:186-189), the
    others plausible restatements that are equal in exact arithmetic."""
    f32 = np.float32
    _, lut, _ = oracle.tables()
    R, C = x.shape
    b = x.reshape(R, C // 32, 32)
    amax = np.abs(b).max(axis=2, keepdims=True)
    scale = np.ldexp(f32(1), (oracle.floor_log2(np.maximum(amax, f32(1e-45))) + 1).astype(np.int32)).astype(f32)
    scale = np.where(amax == 0, f32(1), scale)
    n = np.clip(np.abs(b) / scale, f32(0), f32(1)).astype(f32)
    uu = u.reshape(n.shape).astype(f32)
    if variant == "reference":
        t = (n + (uu - f32(0.5)) / f32(1023)) * f32(1023)
    elif variant == "expanded":          # n*1023 + (u - 0.5)
        t = n * f32(1023) + (uu - f32(0.5))
    elif variant == "no_centering":      # the dither drawn in [0, 1) steps
        t = (n + uu / f32(1023)) * f32(1023)
    else:                                # the dither added after the scaling to 1023
        t = (n * f32(1023) + uu) - f32(0.5)
    idx = np.clip(np.trunc(t).astype(np.int64), 0, 1023)
    return ((np.sign(b) * lut[idx]) * scale).astype(f32).reshape(R, C)


def test_stochastic_fixture_rejects_reordered_dither():
    """The fixture pins the operation order: the reference's order reproduces
    it, and each algebraically equal reordering of the dither fails it."""
    g = load_golden("stochastic.npz")
    x = g["x_dither"]
    u = _unpad(g["u_dither"], 32)
    want = g["fq_dither"]
    assert bits_equal(_fq_stochastic_numpy(x, u, "reference"), want)
    for variant in ("expanded", "no_centering", "after_scaling"):
        assert not bits_equal(_fq_stochastic_numpy(x, u, variant), want), variant
