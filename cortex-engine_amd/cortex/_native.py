"""ctypes binding of libcortex_hip.so (the gfx950 kernels behind include/cortex_hip.h).

The library is loaded lazily on first use and never silently replaced: if it is
missing or fails to load, every kernel entry point raises ``NativeLibraryError``.
Tensors cross the boundary as raw device pointers plus int64 shapes/strides, and
work is enqueued on torch's *current* HIP stream of the tensor's device.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(os.environ.get("CORTEX_HIP_LIB", Path(__file__).resolve().parent / "libcortex_hip.so"))


class NativeLibraryError(RuntimeError):
    """The Cortex HIP library is missing, failed to load, or a kernel call failed."""


# dtype codes of include/cortex_hip.h; BF16_FRAG is a weight layout code (bf16 weights in MFMA
# fragment order, written by cortex_frag_weight), not a tensor dtype
F32, BF16, F16, I8, I32, I64, U8, BF16_FRAG = 0, 1, 2, 3, 4, 5, 6, 7
DTYPE_CODE = {
    torch.float32: F32,
    torch.bfloat16: BF16,
    torch.float16: F16,
    torch.int8: I8,
    torch.int32: I32,
    torch.int64: I64,
    torch.uint8: U8,
    torch.bool: U8,
}

_i64 = ctypes.c_int64
_int = ctypes.c_int
_ptr = ctypes.c_void_p
_f32 = ctypes.c_float

# name -> (restype, argtypes)
_SIGNATURES = {
    "cortex_version": (_int, []),
    "cortex_last_error": (ctypes.c_char_p, []),
    "cortex_pack_workspace_bytes": (_i64, [_i64, _i64]),
    "cortex_pack_plan": (_int, [_ptr, _i64, _i64, _i64, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _ptr, _ptr, _int, _ptr]),
    "cortex_pack_plan_widen": (
        _int, [_ptr, _i64, _i64, _i64, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _ptr, _ptr, _int, _int, _ptr, _ptr, _ptr,
               _ptr, _ptr]),
    "cortex_pack_noalloc_max_workspace_bytes": (_i64, []),
    "cortex_pack_plan_noalloc": (_int, [_ptr, _i64, _i64, _i64, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr]),
    "cortex_tokenize": (
        _int,
        [_int, _i64, _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _i64, _ptr, _i64, _ptr, _i64,
         _i64, _ptr, _ptr, _ptr, _i64, _i64, _ptr, _i64, _ptr, _ptr, _ptr, _ptr],
    ),
    "cortex_tokenize_ln": (
        _int,
        [_i64, _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _i64, _ptr, _i64, _ptr, _i64, _i64,
         _ptr, _ptr, _ptr, _ptr, _ptr, _f32, _ptr, _i64, _ptr, _ptr],
    ),
    "cortex_pack_rows": (
        _int, [_int, _i64, _ptr, _i64, _i64, _ptr, _ptr, _ptr, _i64, _i64, _ptr, _i64, _ptr, _ptr]),
    "cortex_quantize_int8": (_int, [_ptr, _i64, _i64, _i64, _ptr, _ptr, _ptr, _i64, _ptr]),
    "cortex_row_stats": (_int, [_i64, _i64, _int, _ptr, _i64, _int, _f32, _ptr, _ptr]),
    "cortex_layer_norm": (_int, [_i64, _i64, _int, _ptr, _i64, _ptr, _ptr, _int, _f32, _int, _ptr, _i64, _ptr]),
    "cortex_ln_rows": (
        _int, [_i64, _i64, _ptr, _i64, _ptr, _ptr, _f32, _ptr, _ptr, _f32, _ptr, _i64, _ptr, _i64, _ptr]),
    "cortex_convert": (_int, [_int, _ptr, _int, _ptr, _i64, _ptr]),
    "cortex_widen_int8": (_int, [_int, _ptr, _ptr, _ptr, _ptr, _ptr]),
    "cortex_ln_rows_widen": (
        _int, [_i64, _i64, _ptr, _i64, _ptr, _ptr, _f32, _ptr, _ptr, _f32, _ptr, _i64, _ptr, _i64, _int, _ptr, _ptr,
               _ptr, _ptr, _ptr]),
    "cortex_tokenize_ln_widen": (
        _int,
        [_i64, _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _i64, _ptr, _i64, _ptr, _i64, _i64,
         _ptr, _ptr, _ptr, _ptr, _ptr, _f32, _ptr, _i64, _ptr, _int, _ptr, _ptr, _ptr, _ptr, _ptr]),
    "cortex_norm_linear": (
        _int,
        [_i64, _i64, _i64, _int, _ptr, _i64, _int, _ptr, _ptr, _ptr, _int, _int, _int, _int, _ptr, _i64, _ptr,
         _int, _ptr, _int, _int, _ptr, _i64, _i64, _int, _ptr, _i64, _ptr],
    ),
    "cortex_attention": (
        _int,
        [_int, _i64, _i64, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr, _i64, _i64,
         _i64, _ptr, _ptr, _ptr, _i64, _ptr, _i64, _i64, _i64, _i64, _i64, _f32, _ptr, _i64, _i64, _i64, _ptr],
    ),
    "cortex_qkv_attention": (
        _int,
        [_i64, _i64, _i64, _i64, _ptr, _i64, _int, _ptr, _i64, _ptr, _ptr, _f32, _ptr, _i64, _ptr]),
    "cortex_linear_residual_ln": (
        _int,
        [_i64, _i64, _i64, _ptr, _i64, _int, _ptr, _i64, _ptr, _ptr, _ptr, _i64, _i64, _ptr, _i64, _ptr, _ptr, _f32, _ptr, _i64, _ptr]),
    "cortex_head_prep": (_int, [_ptr, _i64, _i64, _i64, _i64, _ptr, _ptr, _i64, _ptr, _ptr, _ptr, _ptr]),
    "cortex_behavior_head_workspace_bytes": (_i64, [_i64, _i64]),
    "cortex_behavior_head": (
        _int,
        [_ptr, _i64, _i64, _i64, _i64, _i64, _i64, _ptr, _ptr, _f32, _ptr, _ptr, _f32, _ptr, _ptr, _ptr, _i64,
         _ptr]),
    "cortex_norm_linear_fused": (
        _int,
        [_i64, _i64, _i64, _ptr, _i64, _int, _ptr, _ptr, _int, _f32, _int, _ptr, _i64, _ptr, _ptr, _int, _int, _ptr,
         _i64, _ptr]),
    "cortex_pooled_linear": (
        _int,
        [_ptr, _i64, _i64, _i64, _i64, _ptr, _ptr, _f32, _i64, _int, _ptr, _i64, _ptr, _ptr, _ptr, _ptr, _ptr]),
    "cortex_gather_event_pages": (_int, [_ptr, _i64, _i64, _ptr, _i64, _ptr, _i64, _i64, _ptr, _ptr]),
    "cortex_scatter_event_pages": (_int, [_ptr, _i64, _i64, _ptr, _i64, _ptr, _i64, _i64, _ptr, _ptr]),
    "cortex_linear_residual_ln_i8": (
        _int,
        [_i64, _i64, _i64, _ptr, _i64, _int, _ptr, _i64, _ptr, _ptr, _ptr, _i64, _i64, _ptr, _i64, _ptr, _ptr, _f32, _ptr, _i64, _f32, _ptr]),
    "cortex_linear_w8a8": (_int, [_i64, _i64, _i64, _ptr, _i64, _f32, _ptr, _i64, _ptr, _ptr, _int, _ptr, _i64, _i64,
                                  _ptr, _int, _f32, _i64, _ptr]),
    "cortex_qkv_attention_w8a8": (_int, [_i64, _i64, _i64, _i64, _ptr, _i64, _f32, _ptr, _i64, _ptr, _ptr, _f32, _ptr,
                                         _int, _f32, _i64, _ptr]),
    "cortex_linear_residual_ln_w8a8": (_int, [_i64, _i64, _i64, _ptr, _i64, _f32, _ptr, _i64, _ptr, _ptr, _ptr, _i64,
                                              _i64, _ptr, _i64, _ptr, _ptr, _f32, _ptr, _int, _f32, _i64, _ptr]),
    "cortex_ln_rows_i8": (_int, [_i64, _i64, _ptr, _i64, _ptr, _ptr, _f32, _ptr, _i64, _f32, _ptr]),
    "cortex_norm_rows": (_int, [_i64, _i64, _int, _ptr, _i64, _int, _ptr, _ptr, _int, _f32, _ptr, _i64, _ptr]),
    "cortex_transpose_bf16": (_int, [_i64, _i64, _ptr, _i64, _ptr, _i64, _ptr]),
    "cortex_fold_gain": (_int, [_i64, _i64, _ptr, _int, _int, _i64, _ptr, _int, _ptr, _i64, _ptr]),
    "cortex_frag_weight": (_int, [_i64, _i64, _ptr, _int, _i64, _ptr, _ptr]),
    "cortex_splitk_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "cortex_linear_residual_splitk": (
        _int, [_i64, _i64, _i64, _ptr, _i64, _ptr, _i64, _ptr, _ptr, _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _i64,
               _ptr]),
    "cortex_linear_residual_ln_splitk": (
        _int, [_i64, _i64, _i64, _ptr, _i64, _ptr, _i64, _ptr, _ptr, _ptr, _i64, _i64, _ptr, _i64, _ptr, _ptr, _f32,
               _ptr, _i64, _i64, _ptr, _i64, _ptr]),
    "cortex_page_table_create": (_int, [_i64, _ptr]),
    "cortex_page_table_destroy": (_int, [_ptr]),
    "cortex_page_table_write": (_int, [_ptr, _i64, _ptr, _ptr, _ptr, _ptr]),
    "cortex_page_table_lookup": (_int, [_ptr, _i64, _i64, _ptr, _ptr]),
    "cortex_page_table_plan": (_int, [_ptr, _i64, _ptr, _ptr, _i64, _i64, _ptr, _i64, _ptr, _ptr, _ptr, _ptr, _ptr]),
    "cortex_page_table_evict_session": (_int, [_ptr, _i64, _ptr]),
    "cortex_page_table_stats": (_int, [_ptr, _ptr, _ptr, _ptr]),
    "cortex_temporal_block_mask": (
        _int, [_ptr, _i64, _i64, _ptr, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _ptr, _i64, _ptr]),
}

EXPORTED = tuple(_SIGNATURES)

_lib: ctypes.CDLL | None = None
_load_error: str | None = None


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raise NativeLibraryError if unavailable."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    if _load_error is not None:
        raise NativeLibraryError(_load_error)
    if not LIB_PATH.exists():
        _load_error = (
            f"{LIB_PATH} not found: build it with `python -m cortex._build` (hipcc, gfx950) "
            "before using the Cortex HIP kernels"
        )
        raise NativeLibraryError(_load_error)
    try:
        lib = ctypes.CDLL(str(LIB_PATH))
    except OSError as exc:  # pragma: no cover - depends on the ROCm install
        _load_error = f"failed to load {LIB_PATH}: {exc}"
        raise NativeLibraryError(_load_error) from exc
    for name, (res, args) in _SIGNATURES.items():
        try:
            fn = getattr(lib, name)
        except AttributeError:
            _load_error = f"{LIB_PATH} does not export {name}: rebuild it with `python -m cortex._build`"
            raise NativeLibraryError(_load_error) from None
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def available() -> bool:
    try:
        load()
        return True
    except NativeLibraryError:
        return False


def call(name: str, *args) -> None:
    """Call an entry point and raise with the library's message on a non-zero status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.cortex_last_error().decode(errors="replace")
        raise NativeLibraryError(f"{name} failed ({rc}): {msg}")


def require_gpu(*tensors: torch.Tensor, what: str) -> torch.device:
    """All tensors on one ROCm device; the HIP path has no CPU execution."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"{what}: the Cortex MI355X kernels run on ROCm GPU tensors only (got a {t.device.type} "
                "tensor); move the inputs to the GPU, or call the *_reference function for the "
                "PyTorch formulation"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"{what}: tensors on different devices ({dev} vs {t.device})")
    assert dev is not None
    return dev


def stream_of(device: torch.device) -> int:
    """Handle of torch's current stream on ``device`` (what the kernels launch on)."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODE[dtype]
    except KeyError:
        raise NativeLibraryError(f"dtype {dtype} is not supported by the Cortex HIP kernels") from None
