"""Quantized linear and matmul on the HIP kernels of libaxs6.so.

``forward_train`` / ``backward`` implement the reference's
``_AXSLinearUnifiedFunction`` (``axs/unified/functional_unified.py:107-170``);
``linear_forward`` is ``accelerated_linear`` (``axs/unified/backend.py:540``)
and ``matmul`` is ``accelerated_matmul`` (``backend.py:621``).

The GEMMs run on fp16 MFMA with operands packed as power-of-two-scaled fp16
rows (see include/axs6.h); results are float32-accumulated and land within
rel-L2 ~3e-4 of the fp32 product of the fake-quantized operands.
K or N off a multiple of the block size go to the kernels as they are when
they are multiples of 4 (float32) or 8 (bfloat16, float16) -- the kernels
zero-pad the last NF5 block, as the reference pads it; other lengths are
zero-padded on the device to such a multiple first, which changes nothing.

The training forward and backward (shape handling, allocation, the dither
seed and the library calls) live in the torch extension ``axs._C``
(csrc/torch_ext.cpp); ``linear_autograd`` is the same pair as one C++
autograd node, which ``axs_linear_unified`` uses.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from axs import _lib
from axs.core import VALID_BLOCK_SIZES
from axs.unified.hip_kernels import _on_device, _require_device, _same_device

_SUPPORTED = (torch.float32, torch.bfloat16, torch.float16)


def _lib_sigs():
    return _lib.lib()


def padded_k(k: int) -> int:
    return int(_lib_sigs().axs6_linear_padded_k(k))


def _pad_last(t: torch.Tensor, mult: int) -> torch.Tensor:
    pad = (-t.shape[-1]) % mult
    return F.pad(t, (0, pad)) if pad else t


def _rows(t: torch.Tensor, cols: int) -> torch.Tensor:
    """t viewed as (rows, cols) over its last dim; unlike reshape(-1, cols)
    this also works when cols is 0 (an empty contraction or output)."""
    return t.reshape(math.prod(t.shape[:-1]), cols)


def _dense(t: torch.Tensor) -> torch.Tensor:
    """Contiguous with a 16-byte aligned data pointer (the packing kernels
    load 16-byte vectors); a view at an element offset is copied."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone(memory_format=torch.contiguous_format)


class Saved:
    """Packed operands of a forward, kept for its backward."""

    def __init__(self, xq, sx, wq, sw, M, N, K, n_true, k_true, dtype, x_shape, w_dtype, x_dtype=None):
        self.xq, self.sx, self.wq, self.sw = xq, sx, wq, sw
        self.M, self.N, self.K = M, N, K
        self.n_true, self.k_true = n_true, k_true
        self.dtype, self.x_shape, self.w_dtype = dtype, x_shape, w_dtype
        self.x_dtype = dtype if x_dtype is None else x_dtype   # dX comes back in this dtype

    def tensors(self):
        return (self.xq, self.sx, self.wq, self.sw)

    def meta(self):
        return (self.M, self.N, self.K, self.n_true, self.k_true, self.dtype, self.x_shape, self.w_dtype,
                self.x_dtype)

    @staticmethod
    def restore(tensors, meta) -> "Saved":
        return Saved(*tensors, *meta)


def _forward(input, weight, bias, block_size, quantize_input):
    """(Y, Saved) through the extension's forward (axs._C.linear_fwd: shape
    handling, allocation and the axs6_nf5_linear_forward call in C++)."""
    fn = "axs_linear"
    _require_device(input, fn)
    _require_device(weight, fn)
    assert block_size in VALID_BLOCK_SIZES, f"block_size must be one of {VALID_BLOCK_SIZES}"
    out, xq, sx, wq, sw, M, N, K, n_true, k_true, dtype = _lib.ext().linear_fwd(
        input, weight, bias, block_size, bool(quantize_input))
    return out, Saved(xq, sx, wq, sw, M, N, K, n_true, k_true, dtype, tuple(input.shape), weight.dtype,
                      input.dtype)


def forward_train(input, weight, bias, block_size=32, quantize_input=True):
    """(Y, Saved) -- Y = FQ(input) FQ(weight)^T + bias."""
    return _forward(input, weight, bias, block_size, quantize_input)


# Outputs up to this many elements take the single-launch fused kernel (the
# reference's _FUSED_SIZE_THRESHOLD, triton_kernels.py:382, applied the same
# way by its accelerated_linear, backend.py:577-590).
FUSED_SIZE_THRESHOLD = 128 * 1024


def _bias_vector(bias, N: int, fn: str):
    """The bias as F.linear broadcasts it over N output features (N values
    as (N,) or (1, N), or one value), float32 and contiguous; other shapes
    raise, as F.linear does -- the kernels read N values."""
    if bias is None:
        return None
    n = bias.numel()
    if n == 1 and N != 1:
        return bias.reshape(1).expand(N).to(torch.float32).contiguous()
    if n != N or not (bias.dim() == 1 or (bias.dim() == 2 and bias.shape[0] == 1)):
        raise RuntimeError(f"{fn}: bias of shape {tuple(bias.shape)} does not broadcast to the {N} output features")
    return bias.reshape(N).to(torch.float32).contiguous()


def _as_input_dtype(out: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Y in the input's floating dtype (float64 is computed in float32 and
    returned as float64, as the reference's F.linear on its FQ values)."""
    return out.to(dtype) if out.dtype != dtype and dtype.is_floating_point else out


def fused_forward(input, weight, bias=None, quantize_input=True):
    """``FQ(input) FQ(weight)^T + bias`` with block size 32 in one launch of
    the fused kernel (FQ in the tile loads, fp32 contraction): the
    reference's ``triton_fused_linear`` (``triton_kernels.py:385-482``).
    Returns the input's dtype (other floating dtypes are computed in float32)."""
    fn = "axs_fused_linear"
    _require_device(input, fn)
    _require_device(weight, fn)
    _same_device(fn, input, weight, bias)
    K = input.shape[-1]
    N, Kw = weight.shape
    if Kw != K:
        raise RuntimeError(f"{fn}: input has {K} features but weight expects {Kw}")
    b = _bias_vector(bias, N, fn)
    dtype = input.dtype if input.dtype in _SUPPORTED else torch.float32
    x2 = _dense(_pad_last(_rows(input, K).to(dtype), 32))
    w2 = _dense(_pad_last(weight.to(dtype), 32))
    M, Kb = x2.shape
    dev = x2.device
    y = torch.empty((M, N), dtype=dtype, device=dev)
    if M and N and not Kb:
        y.copy_(b.to(dtype).expand(M, N) if b is not None else torch.zeros((), dtype=dtype, device=dev).expand(M, N))
    elif M and N:
        code = _lib.DTYPE_CODE[dtype]
        qx = bool(quantize_input)
        with _on_device(x2):
            st = _lib.stream_of(x2)
            if _lib.lib().axs6_nf5_fused_linear_split_x(M, N, Kb, code):
                # FQ(X) written once in the contraction's read order, then the
                # contraction on it: the same values, where the single launch
                # would read and quantize all of X in every workgroup
                xa = torch.empty(_lib.lib().axs6_nf5_fused_linear_split_workspace(M, Kb) // 4,
                                 dtype=torch.float32, device=dev)
                _lib.call("axs6_nf5_fused_linear_split", x2.data_ptr(), w2.data_ptr(), _lib.ptr(b), y.data_ptr(),
                          xa.data_ptr(), code, M, N, Kb, 32, int(qx), st)
            else:
                _lib.call("axs6_nf5_fused_linear", x2.data_ptr(), w2.data_ptr(), _lib.ptr(b), y.data_ptr(),
                          code, M, N, Kb, 32, int(qx), st)
    return _as_input_dtype(y.reshape(*input.shape[:-1], N), input.dtype)


def linear_forward(input, weight, bias=None, block_size=32, quantize_input=True):
    """Y = FQ(input) FQ(weight)^T + bias (no autograd bookkeeping): the fused
    single-launch kernel for block size 32 and at most FUSED_SIZE_THRESHOLD
    outputs, else the packing kernels and the fp16-MFMA GEMM.  Y has the
    input's dtype."""
    if block_size == 32 and input.shape[-1] == weight.shape[-1]:
        rows = input.numel() // input.shape[-1] if input.shape[-1] else 0
        if rows * weight.shape[0] <= FUSED_SIZE_THRESHOLD:
            return fused_forward(input, weight, bias, quantize_input)
    out, _ = _forward(input, weight, bias, block_size, quantize_input)
    return out


def backward(grad_output, saved: Saved, block_size: int, quantize_grad: bool,
             need_x: bool, need_w: bool, need_b: bool, seed: int | None = None):
    """(dX, dW, db) of the quantized linear, each None when not needed, through
    the extension's backward (axs._C.linear_bwd).  ``seed`` fixes the
    stochastic rounding of dY (default: a fresh draw from torch's CPU
    generator; while a graph is recorded, plus the device's replay counter)."""
    return _lib.ext().linear_bwd(
        grad_output, saved.xq, saved.sx, saved.wq, saved.sw, saved.M, saved.N, saved.K, saved.n_true,
        saved.k_true, saved.dtype, list(saved.x_shape), saved.w_dtype, block_size, bool(quantize_grad),
        bool(need_x), bool(need_w), bool(need_b), seed, saved.x_dtype)


def linear_autograd(input, weight, bias, block_size=32, quantize_input=True, quantize_grad=True):
    """``axs_linear_unified`` as one C++ autograd node (axs._C.linear): the
    same forward and backward as forward_train / backward, with no Python on
    either side of the engine."""
    fn = "axs_linear"
    _require_device(input, fn)
    _require_device(weight, fn)
    assert block_size in VALID_BLOCK_SIZES, f"block_size must be one of {VALID_BLOCK_SIZES}"
    return _lib.ext().linear(input, weight, bias, block_size, bool(quantize_input), bool(quantize_grad))


def _matmul_2d(a2: torch.Tensor, bt: torch.Tensor, count: int, rows_b: int) -> torch.Tensor:
    """``count`` products a2[i] (M, K) @ bt[i]^T, bt[i] (N, K), with a2 and bt
    given as row stacks [count*M, K] and [count*N, K] (float32): one packing
    launch per operand for the whole stack, then one GEMM per product on the
    row ranges of the packed stacks.  Returns [count, M, N] float32."""
    K = a2.shape[1]
    M = a2.shape[0] // count if count else 0
    N = rows_b
    a2 = _dense(_pad_last(a2, 32))
    bt = _dense(_pad_last(bt, 32))
    Kb = a2.shape[1]
    Kp = padded_k(Kb)
    dev = a2.device
    out = torch.empty((count, M, N), dtype=torch.float32, device=dev)
    if not (count and M and N):
        return out
    if not Kb:
        return out.zero_()
    aq = torch.empty((count * M, Kp), dtype=torch.float16, device=dev)
    bq = torch.empty((count * N, Kp), dtype=torch.float16, device=dev)
    sa = torch.empty((count * M,), dtype=torch.int32, device=dev)
    sb = torch.empty((count * N,), dtype=torch.int32, device=dev)
    st = _lib.stream_of(a2)
    with _on_device(a2):
        _lib.call("axs6_nf5_pack_rows", a2.data_ptr(), _lib.F32, count * M, Kb, 32, 0, 0, 0, None,
                  aq.data_ptr(), Kp, Kp, sa.data_ptr(), None, st)
        _lib.call("axs6_nf5_pack_rows", bt.data_ptr(), _lib.F32, count * N, Kb, 32, 0, 0, 0, None,
                  bq.data_ptr(), Kp, Kp, sb.data_ptr(), None, st)
        for i in range(count):
            _lib.call("axs6_gemm_f16_nt", aq[i * M:].data_ptr(), Kp, bq[i * N:].data_ptr(), Kp, M, N, Kp,
                      sa[i * M:].data_ptr(), sb[i * N:].data_ptr(), None, out[i].data_ptr(), N, _lib.F32, st)
    return out


def matmul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """``torch.matmul(a, b)`` -> float32 on fp16 MFMA with per-row power-of-two
    scaled operands (no NF5 step): ``a (*, M, K) @ b (*, K, N)`` with the
    batch dims broadcast, and 1-D operands promoted and squeezed as
    torch.matmul does.  A 2-D ``b`` contracts all of a's rows in one GEMM."""
    fn = "axs_matmul"
    _require_device(a, fn)
    _require_device(b, fn)
    _same_device(fn, a, b)
    if a.dim() == 0 or b.dim() == 0:
        raise RuntimeError(f"{fn}: both arguments need at least 1 dimension, got {a.dim()}D and {b.dim()}D")
    a_vec, b_vec = a.dim() == 1, b.dim() == 1
    A = a.unsqueeze(0) if a_vec else a
    B = b.unsqueeze(-1) if b_vec else b
    K = A.shape[-1]
    if B.shape[-2] != K:
        raise RuntimeError(f"{fn}: shapes {tuple(a.shape)} and {tuple(b.shape)} do not contract")
    N = B.shape[-1]
    if B.dim() == 2:
        # every row of a against one right operand: a single GEMM over the rows
        out = _matmul_2d(_rows(A, K).float(), B.float().t(), 1, N)[0].reshape(*A.shape[:-1], N)
    else:
        batch = torch.broadcast_shapes(A.shape[:-2], B.shape[:-2])
        M = A.shape[-2]
        count = math.prod(batch)
        a3 = A.float().expand(*batch, M, K).reshape(count * M, K)
        bt = B.float().transpose(-1, -2).expand(*batch, N, K).reshape(count * N, K)
        out = _matmul_2d(a3, bt, count, N).reshape(*batch, M, N)
    if a_vec:
        out = out.squeeze(-2)
    if b_vec:
        out = out.squeeze(-1)
    return out


def last_forward_kernel_times(X, W, b, reps: int = 20) -> dict:
    """Per-kernel device times (ms) of the forward at this shape, measured
    with HIP events on torch's current stream: pack X, pack W, GEMM."""
    M, K = X.shape
    N = W.shape[0]
    Kp = padded_k(K)
    dev = X.device
    xq = torch.empty((M, Kp), dtype=torch.float16, device=dev)
    wq = torch.empty((N, Kp), dtype=torch.float16, device=dev)
    sx = torch.empty((M,), dtype=torch.int32, device=dev)
    sw = torch.empty((N,), dtype=torch.int32, device=dev)
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    st = _lib.stream_of(X)
    code = _lib.DTYPE_CODE[X.dtype]

    def pack_x():
        _lib.call("axs6_nf5_pack_rows", X.data_ptr(), code, M, K, 32, 1, 0, 0, None, xq.data_ptr(), Kp, Kp,
                  sx.data_ptr(), None, st)

    def pack_w():
        _lib.call("axs6_nf5_pack_rows", W.data_ptr(), code, N, K, 32, 1, 0, 0, None, wq.data_ptr(), Kp, Kp,
                  sw.data_ptr(), None, st)

    def gemm():
        _lib.call("axs6_gemm_f16_nt", xq.data_ptr(), Kp, wq.data_ptr(), Kp, M, N, Kp, sx.data_ptr(),
                  sw.data_ptr(), _lib.ptr(b), y.data_ptr(), N, _lib.F32, st)

    out = {"compute_dtype": "fp16 MFMA operands (power-of-two row scaled), fp32 accumulate"}
    for name, fn in (("pack_x_ms", pack_x), ("pack_w_ms", pack_w), ("gemm_ms", gemm)):
        out[name] = _event_time(fn, reps)
    # the forward packs X and W in one launch
    out["pack_xw_ms"] = _event_time(lambda: _lib.call(
        "axs6_nf5_linear_forward", X.data_ptr(), W.data_ptr(), _lib.ptr(b), y.data_ptr(), code, M, N, K, 32, 1,
        xq.data_ptr(), sx.data_ptr(), wq.data_ptr(), sw.data_ptr(), st), reps) - out["gemm_ms"]
    return out


def _event_time(fn, reps: int) -> float:
    for _ in range(3):
        fn()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def clear_weight_cache() -> None:
    """No cached weight encodings are kept between calls."""
    return None
