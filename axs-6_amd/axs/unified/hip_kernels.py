"""Host wrappers of the gfx950 NF5 kernels (libaxs6.so).

These replace the reference's Triton entry points
``triton_fused_fake_quantize`` (``axs/unified/triton_kernels.py:295-370``)
and ``triton_fused_linear`` (``:385-482``) with the same argument meaning
and error behaviour:

* a CPU tensor raises ``RuntimeError`` mentioning CUDA (ROCm reports GPU
  tensors as ``is_cuda``), as ``triton_kernels.py:326-327,422-423`` do;
* an invalid ``block_size`` fails the ``assert`` (``:328-330``);
* output keeps the input's shape and dtype, computing in float32;
* padding of a ragged last dim is virtual (handled inside the kernels).

Nothing here computes on the CPU: if libaxs6.so is absent these raise.
"""
from __future__ import annotations

from typing import Literal

import torch

from axs import _lib
from axs.core import DEFAULT_BLOCK_SIZE, VALID_BLOCK_SIZES


def has_hip() -> bool:
    """True when libaxs6.so loads and a ROCm GPU is visible."""
    try:
        _lib.lib()
    except _lib.LibraryError:
        return False
    return torch.cuda.is_available()


def _require_device(t: torch.Tensor, fn: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{fn} requires a CUDA (ROCm/HIP) device tensor, got device {t.device}")


def _same_device(fn: str, first: torch.Tensor, *others: torch.Tensor | None) -> None:
    for t in others:
        if t is not None and t.device != first.device:
            raise RuntimeError(f"{fn}: tensors on {first.device} and {t.device}; all must be on one device")


def _check_rounding(rounding: str) -> bool:
    if rounding not in ("nearest", "stochastic"):
        raise ValueError(f"rounding must be 'nearest' or 'stochastic', got {rounding!r}")
    return rounding == "stochastic"


class _on_device:
    """Makes t's device current for the duration of a library call."""

    __slots__ = ("idx", "prev")

    def __init__(self, t: torch.Tensor):
        self.idx = t.device.index
        self.prev = None

    def __enter__(self):
        if self.idx is not None:
            cur = torch.cuda.current_device()
            if self.idx != cur:
                self.prev = cur
                torch.cuda.set_device(self.idx)

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)


def next_seed() -> int:
    """Seed for one stochastic call, drawn from torch's default CPU
    generator (so torch.manual_seed reproduces it) -- a host-side draw, with
    no device synchronisation (the reference's Triton path does a .item()
    on a device tensor for this, triton_kernels.py:351)."""
    return int(torch.randint(0, 2**62, (1,)).item())


# Per-device uint64 counters for stochastic calls recorded in a HIP graph.
# A recorded call keeps the seed drawn at capture time; the library adds the
# counter's value, read when the kernel runs, and one recorded increment per
# graph (after its first stochastic call) advances it -- so every replay draws
# fresh dither values.
_graph_counters: dict[int, torch.Tensor] = {}


def _graph_counter(device: torch.device) -> torch.Tensor:
    """The device's counter, shared with the linear's C++ backward (which
    keeps the registry: axs._C.graph_counter); created on first use, which
    raises while the current stream records a graph."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ctr = _graph_counters.get(idx)
    if ctr is None:
        ctr = _lib.ext().graph_counter(idx)
        _graph_counters[idx] = ctr
    return ctr


def advance_graph_counter(device: torch.device) -> None:
    """Records the device counter's advance after a graph-recorded stochastic
    call, once per capture (axs._C.graph_counter_advance)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    _lib.ext().graph_counter_advance(idx)


def prepare_graph_capture(device: torch.device | int | None = None) -> None:
    """Creates the device's dither counter outside capture (optional: the
    first eager stochastic call does it)."""
    d = torch.device("cuda", torch.cuda.current_device() if device is None else
                     (device if isinstance(device, int) else device.index))
    _graph_counter(d)


def stochastic_seed(device: torch.device, seed: int | None = None) -> tuple[int, int | None, torch.Tensor | None]:
    """(seed, seed_dev pointer or None, counter to advance after the call or None).

    Eagerly, a fresh host draw (or ``seed``) and no device term.  While the
    current stream is capturing a graph and no explicit ``seed`` is given, the
    draw is fixed at capture time and the per-device counter is added on the
    device; the caller calls advance_graph_counter after its launch."""
    s = next_seed() if seed is None else int(seed)
    if seed is None and torch.cuda.is_current_stream_capturing():
        ctr = _graph_counter(device)
        return s, ctr.data_ptr(), ctr
    if seed is None:
        _graph_counter(device)   # created eagerly, ready for a later capture
    return s, None, None


def as_rows(tensor: torch.Tensor) -> tuple[torch.Tensor, int, int]:
    """Contiguous view of ``tensor`` as (rows, cols) over its last dim, in a
    dtype the kernels take (f32 / bf16 / f16; anything else is computed in
    float32 like the reference's ``.float()``)."""
    x = tensor
    if x.dtype not in _lib.DTYPE_CODE:
        x = x.float()
    if not x.is_contiguous():
        x = x.contiguous()
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    return x, rows, cols


def hip_fused_fake_quantize(
    tensor: torch.Tensor,
    block_size: int = DEFAULT_BLOCK_SIZE,
    rounding: Literal["nearest", "stochastic"] = "nearest",
    *,
    n_blocks: int | None = None,
    seed: int | None = None,
) -> torch.Tensor:
    """NF5 fused fake-quantize on the GPU (one streaming HIP kernel).

    Bit-exact with the reference's eager ``fused_fake_quantize`` for
    ``rounding="nearest"``.  ``rounding="stochastic"`` dithers with the
    library's counter-based generator; ``seed`` fixes the draw (default: a
    fresh seed from torch's CPU generator).  ``n_blocks`` is accepted for
    signature compatibility with the reference's Triton wrapper; the launch
    shape is chosen by the library.
    """
    stochastic = fq_checks(tensor, block_size, rounding, "hip_fused_fake_quantize")
    return _lib.ext().fq(tensor, block_size, stochastic, None if seed is None else _as_int64(seed))


def fq_checks(tensor: torch.Tensor, block_size: int, rounding: str, fn: str) -> bool:
    """The fake-quantize entry points' argument checks, in the reference's
    order and exception types (triton_kernels.py:326-330): a host tensor
    raises RuntimeError naming CUDA, a block size outside (8, 16, 32)
    AssertionError, an unknown rounding mode ValueError.  Returns whether the
    rounding is stochastic."""
    _require_device(tensor, fn)
    assert block_size in VALID_BLOCK_SIZES, f"block_size must be one of {VALID_BLOCK_SIZES}"
    return _check_rounding(rounding)


def _as_int64(seed: int) -> int:
    """``seed`` modulo 2^64 as a signed 64-bit value (the same 64 bits)."""
    s = int(seed) & 0xFFFFFFFFFFFFFFFF
    return s - (1 << 64) if s >= (1 << 63) else s


def hip_quantize(
    tensor: torch.Tensor,
    block_size: int = DEFAULT_BLOCK_SIZE,
    rounding: Literal["nearest", "stochastic"] = "nearest",
    *,
    with_fake_quantized: bool = False,
    seed: int | None = None,
):
    """Runs the quantize kernel: returns (exponents u8 (R, nblk), codes u8
    (R, nblk, bs), signs bool (R, nblk, bs), fq or None)."""
    fn = "hip_quantize"
    _require_device(tensor, fn)
    assert block_size in VALID_BLOCK_SIZES, f"block_size must be one of {VALID_BLOCK_SIZES}"
    stochastic = _check_rounding(rounding)
    x, rows, cols = as_rows(tensor)
    nblk = (cols + block_size - 1) // block_size
    dev = x.device
    exps = torch.empty((rows, nblk), dtype=torch.uint8, device=dev)
    codes = torch.empty((rows, nblk, block_size), dtype=torch.uint8, device=dev)
    signs = torch.empty((rows, nblk, block_size), dtype=torch.uint8, device=dev)
    fq = torch.empty_like(x) if with_fake_quantized else None
    if rows and cols:
        s, sdev, ctr = stochastic_seed(x.device, seed) if stochastic else (0, None, None)
        with _on_device(x):
            _lib.call("axs6_nf5_quantize", x.data_ptr(), _lib.DTYPE_CODE[x.dtype], rows, cols,
                      block_size, int(stochastic), s, 0, exps.data_ptr(), codes.data_ptr(),
                      signs.data_ptr(), _lib.ptr(fq), sdev, _lib.stream_of(x))
            if ctr is not None:
                advance_graph_counter(x.device)
    if fq is not None:
        fq = fq.reshape(tensor.shape)
        if fq.dtype != tensor.dtype:
            fq = fq.to(tensor.dtype)
    return exps, codes, signs.view(torch.bool), fq


def components(exps: torch.Tensor, codes: torch.Tensor, signs: torch.Tensor | None, rows: int, nblk: int,
               block_size: int, fn: str):
    """The AXSTensor fields as contiguous uint8 tensors on the codes' device,
    checked to hold at least the rows * nblk exponents and rows * nblk *
    block_size codes (and signs) the kernels read: a short or host-side field
    raises here instead of being read out of bounds on the device."""
    _require_device(codes, fn)
    for name, t in (("shared_exponents", exps), ("signs", signs)):
        if t is not None and t.device != codes.device:
            raise RuntimeError(f"{fn}: {name} is on {t.device}, the codes on {codes.device}")
    need_e, need_c = rows * nblk, rows * nblk * block_size
    if exps.numel() < need_e or codes.numel() < need_c or (signs is not None and signs.numel() < need_c):
        raise ValueError(f"{fn}: fields too small for {rows} x {nblk} blocks of {block_size} "
                         f"(exponents {exps.numel()}, codes {codes.numel()}"
                         f"{'' if signs is None else f', signs {signs.numel()}'})")
    def u8(t):
        t = t.contiguous()
        return t.view(torch.uint8) if t.dtype in (torch.bool, torch.int8) else t.to(torch.uint8)

    return u8(exps), u8(codes), None if signs is None else u8(signs)


def hip_dequantize(exps: torch.Tensor, codes: torch.Tensor, signs: torch.Tensor | None,
                   rows: int, cols: int, block_size: int) -> torch.Tensor:
    assert block_size in VALID_BLOCK_SIZES, f"block_size must be one of {VALID_BLOCK_SIZES}"
    e, c, s = components(exps, codes, signs, rows, (cols + block_size - 1) // block_size, block_size,
                         "hip_dequantize")
    y = torch.empty((rows, cols), dtype=torch.float32, device=codes.device)
    if rows and cols:
        with _on_device(c):
            _lib.call("axs6_nf5_dequantize", e.data_ptr(), c.data_ptr(), _lib.ptr(s), y.data_ptr(),
                      rows, cols, block_size, _lib.stream_of(c))
    return y


def hip_fused_linear(
    input: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    block_size: int = DEFAULT_BLOCK_SIZE,
    quantize_input: bool = True,
) -> torch.Tensor:
    """``FQ(input) @ FQ(weight).T + bias`` on the fused HIP linear, for the
    argument conventions of the reference's ``triton_fused_linear``
    (``axs/unified/triton_kernels.py:385-482``): CUDA tensors only,
    ``block_size`` must be 32 (ValueError otherwise), output in the input's
    dtype."""
    if not input.is_cuda:
        raise RuntimeError("hip_fused_linear requires CUDA (ROCm/HIP) tensors")
    if block_size != 32:
        raise ValueError(f"hip_fused_linear requires block_size=32, got {block_size}. "
                         "Use accelerated_linear for other block sizes.")
    from axs.unified import hip_linear

    return hip_linear.linear_forward(input, weight, bias, block_size, quantize_input)
