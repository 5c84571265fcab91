"""ctypes binding of libaxs6.so (C ABI declared in include/axs6.h), and the
loader of the torch extension ``axs._C`` built over the same C ABI.

The library is built in-tree by ``python axs-6_amd/build.py`` into
``axs-6_amd/axs/_lib/libaxs6.so`` (the extension into ``axs-6_amd/axs/_C.so``).
There is no fallback: if either is missing or fails to load, every entry
point that needs it raises.

torch is imported first so that the HIP runtime torch ships
(libamdhip64.so.7) is the one the library binds to; device pointers and
streams are then shared with torch.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libaxs6.so")

F32, BF16, F16 = 0, 1, 2
DTYPE_CODE = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_u8p = ctypes.POINTER(ctypes.c_uint8)
_f32p = ctypes.POINTER(ctypes.c_float)

# name -> argtypes; every entry point returns int (axs6_status)
_SIGNATURES: dict[str, list] = {
    "axs6_init": [],
    "axs6_get_tables": [_f32p, _f32p, _u8p, _u8p],
    "axs6_nf5_fake_quantize": [_vp, _vp, _i32, _i64, _i64, _i32, _i32, _u64, _u64, _vp, _vp],
    "axs6_nf5_quantize": [_vp, _i32, _i64, _i64, _i32, _i32, _u64, _u64, _vp, _vp, _vp, _vp, _vp, _vp],
    "axs6_nf5_dequantize": [_vp, _vp, _vp, _vp, _i64, _i64, _i32, _vp],
    "axs6_linear_padded_k": [_i64],
    "axs6_nf5_pack_rows": [_vp, _i32, _i64, _i64, _i32, _i32, _u64, _u64, _vp, _vp, _i64, _i64, _vp, _vp, _vp],
    "axs6_gemm_f16_nt": [_vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _i64, _i32, _vp],
    "axs6_nf5_row_stats_workspace": [_i64, _i64],
    "axs6_nf5_row_stats": [_vp, _i32, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp],
    "axs6_nf5_linear_forward": [_vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i32, _i32, _vp, _vp, _vp,
                                _vp, _vp],
    "axs6_nf5_linear_backward_workspace": [_i64, _i64, _i64, _i32, _i32, _i32],
    "axs6_nf5_fused_linear": [_vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i32, _i32, _vp],
    "axs6_nf5_fused_linear_split_x": [_i64, _i64, _i64, _i32],
    "axs6_nf5_fused_linear_split_workspace": [_i64, _i64],
    "axs6_nf5_fused_linear_split": [_vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i32, _i32, _vp],
    "axs6_nf5_wire_bytes": [_i64, _i64, _i32],
    "axs6_nf5_pack_wire": [_vp, _i32, _i64, _i64, _i32, _vp, _vp],
    "axs6_nf5_unpack_wire": [_vp, _i64, _i64, _i32, _vp, _vp],
    "axs6_nf5_wire_from_codes": [_vp, _vp, _vp, _i64, _i64, _i32, _vp, _vp],
    "axs6_nf5_wire_to_codes": [_vp, _i64, _i64, _i32, _vp, _vp, _vp, _vp],
    "axs6_nf5_block_bytes": [_i64, _i64, _i32],
    "axs6_nf5_pack_blocks": [_vp, _i32, _i64, _i64, _i32, _vp, _vp],
    "axs6_nf5_unpack_blocks": [_vp, _i64, _i64, _i32, _vp, _vp],
    "axs6_nf5_blocks_from_codes": [_vp, _vp, _vp, _i64, _i64, _i32, _vp, _vp],
    "axs6_nf5_blocks_to_codes": [_vp, _i64, _i64, _i32, _vp, _vp, _vp, _vp],
    "axs6_multi_tensor_workspace": [_vp, _i32],
    "axs6_multi_tensor_unscale_clip": [_vp, _vp, _vp, _i32, ctypes.c_float, ctypes.c_float, _i32, _vp, _i64, _vp, _vp],
    "axs6_nf5_linear_backward": [_vp, _i32, _i64, _i64, _i64, _i32, _i32, _u64, _u64, _vp, _vp, _vp, _vp,
                                 _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp, _vp],
    "axs6_nf5_linear_backward_noalloc": [_vp, _i32, _i64, _i64, _i64, _i32, _i32, _u64, _u64, _vp, _vp, _vp,
                                         _vp, _vp, _vp, _vp, _vp, _vp],
    "axs6_layer_norm_forward": [_vp, _i32, _i64, _i64, _vp, _vp, ctypes.c_float, _vp, _vp, _vp, _vp],
    "axs6_layer_norm_backward_workspace": [_i64, _i64],
    "axs6_layer_norm_backward": [_vp, _vp, _i32, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t,
                                 _vp],
}
# entry points that return a value rather than an axs6_status
_RESTYPES = {"axs6_linear_padded_k": _i64, "axs6_nf5_linear_backward_workspace": ctypes.c_size_t,
             "axs6_nf5_wire_bytes": _i64, "axs6_nf5_block_bytes": _i64, "axs6_multi_tensor_workspace": _i64,
             "axs6_nf5_row_stats_workspace": _i64, "axs6_nf5_fused_linear_split_x": ctypes.c_int32,
             "axs6_nf5_fused_linear_split_workspace": _i64, "axs6_layer_norm_backward_workspace": _i64}


class LibraryError(RuntimeError):
    """libaxs6.so is missing, failed to load, or a call returned an error."""


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise LibraryError(
                    f"libaxs6.so not found at {LIB_PATH}; build it with "
                    "`python axs-6_amd/build.py` (hipcc, gfx950)")
            try:
                L = ctypes.CDLL(LIB_PATH)
            except OSError as e:  # pragma: no cover - environment problem
                raise LibraryError(f"failed to load {LIB_PATH}: {e}") from e
            L.axs6_version.restype = ctypes.c_char_p
            L.axs6_version.argtypes = []
            L.axs6_last_error.restype = ctypes.c_char_p
            L.axs6_last_error.argtypes = []
            for name, argt in _SIGNATURES.items():
                fn = getattr(L, name, None)
                if fn is not None:
                    fn.argtypes = argt
                    fn.restype = _RESTYPES.get(name, ctypes.c_int)
            _lib = L
    return _lib


_ext = None
EXT_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_C.so")


def ext():
    """The torch extension ``axs._C`` (the linear's host logic and autograd
    node in C++), loaded after libaxs6.so so both share the one library."""
    global _ext
    if _ext is not None:
        return _ext
    lib()
    with _lock:
        if _ext is None:
            if not os.path.exists(EXT_PATH):
                raise LibraryError(
                    f"torch extension not found at {EXT_PATH}; build it with "
                    "`python axs-6_amd/build.py`")
            try:
                from axs import _C
            except ImportError as e:  # pragma: no cover - environment problem
                raise LibraryError(f"failed to load {EXT_PATH}: {e}") from e
            _ext = _C
    return _ext


def has(name: str) -> bool:
    return hasattr(lib(), name)


_fns: dict = {}


def call(name: str, *args) -> None:
    """Call an entry point and raise RuntimeError on a non-zero status."""
    fn = _fns.get(name)
    if fn is None:
        fn = _fns[name] = getattr(lib(), name)
    rc = fn(*args)
    if rc != 0:
        msg = lib().axs6_last_error().decode(errors="replace")
        raise LibraryError(f"{name} failed (status {rc}): {msg}")


def version() -> str:
    return lib().axs6_version().decode()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    """Raw hipStream_t of torch's current stream on t's device."""
    if _raw_stream is not None:
        return _raw_stream(t.device.index if t.device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def host_tables():
    """(codebook f32[32], lut f32[1024], reverse_lut u8[1024], log2_band u8[278])."""
    cb = (ctypes.c_float * 32)()
    lut = (ctypes.c_float * 1024)()
    rev = (ctypes.c_uint8 * 1024)()
    band = (ctypes.c_uint8 * 278)()
    call("axs6_get_tables", cb, lut, rev, band)
    return (torch.tensor(list(cb), dtype=torch.float32),
            torch.tensor(list(lut), dtype=torch.float32),
            torch.tensor(list(rev), dtype=torch.uint8),
            torch.tensor(list(band), dtype=torch.uint8))
