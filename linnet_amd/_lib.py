"""ctypes binding of `liblinnet_quant_hip.so` (the C ABI in include/linnet_quant.h).

The pattern follows the reference's own binding of its native runtime
(`python/linnet/src/linnet/runtime.py:117-197`): load the library once,
declare every entry point's argument types, and turn a non-zero status into
an exception carrying `lnq_last_error()`.

There is no fallback: a missing or unloadable library raises.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

from .errors import LinnetError

LIBRARY = Path(__file__).resolve().parent / "_lib" / "liblinnet_quant_hip.so"
ABI_VERSION = 1

LNQ_OK, LNQ_ERROR, LNQ_UNAVAILABLE = 0, 1, 2
BF16, F16, F32 = 0, 1, 2
(KERNEL_AUTO, KERNEL_SKINNY, KERNEL_TILED, KERNEL_GEMV, KERNEL_TILED_128, KERNEL_TILED_256, KERNEL_PERSISTENT,
 KERNEL_SPLIT) = range(8)
PROLOGUE_RMSNORM, PROLOGUE_SILU_MUL = 1, 2
PACKING_GPTQ, PACKING_AWQ = 0, 1

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float

# Entry point -> argument types (the return type is always LnqStatus, int32).
SIGNATURES: dict[str, list[object]] = {
    "lnq_device_probe": [_i32, ctypes.POINTER(_i32), ctypes.POINTER(_i32)],
    "lnq_int4_linear": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32, _i32, _p],
    "lnq_int4_linear_plan": [_i64, _i64, _i64, _i64, _i32, _i32, ctypes.POINTER(_i32)],
    "lnq_int4_linear_ws": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32, _i32, _p, _i64, _p],
    "lnq_int4_linear_workspace": [_i64, _i64, _i64, _i64, _i32, _i32, ctypes.POINTER(_i32), ctypes.POINTER(_i64)],
    "lnq_x_tiles": [_p, _p, _i64, _i64, _p],
    "lnq_int4_linear_tiles": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32, _i32, _p, _i64, _p],
    "lnq_int4_linear_tiles_parts": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, ctypes.POINTER(_i32), _p],
    "lnq_int4_linear_executable": [_i64, _i64, _i64, _i32, _p],
    "lnq_int4_dequantize": [_p, _p, _p, _p, _i64, _i64, _i64, _i32, _p],
    "lnq_int4_quantize": [_p, _p, _p, _p, _i64, _i64, _i64, _p],
    "lnq_int4_pack": [_p, _p, _i64, _p],
    "lnq_int4_unpack": [_p, _p, _i64, _i32, _p],
    "lnq_int4_row_prepare": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _p],
    "lnq_take_inputs": [_p, _p, _p, _i64, _i64, _i32, _p],
    "lnq_int4_linear_ordered": [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32, _i32, _p],
    "lnq_int4_linear_prologue": [_p, _p, _p, _f32, _i32, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32, _i32, _p],
    "lnq_int4_repack": [_p, _p, _p, _i32, _i32, _i64, _i64, _i64, _p, _p, _p],
    "lnq_int8_quantize": [_p, _p, _p, _i64, _i64, _i64, _i32, _p],
    "lnq_w8a16": [_p, _p, _p, _p, _i64, _i64, _i64, _i32, _i64, _i64, _i32, _p],
    "lnq_dequantize8": [_p, _p, _p, _i64, _i64, _i32, _i64, _i64, _i32, _p],
    "lnq_rows8": [_p, _p, _p, _i64, _i64, _i32, _i32, _p],
    "lnq_mm8": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _i32, _p],
    "lnq_mm8_tiles": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _i32, _i32, _p],
    "lnq_mm8_plan": [_i64, _i64, _i64, _i32, ctypes.POINTER(_i32)],
    "lnq_fp8_groups": [_p, _p, _p, _i64, _i64, _i64, _i64, _i32, _p],
    "lnq_mm8_block": [_p, _p, _p, _i64, _p, _p, _i64, _i64, _i64, _i32, _p],
    "lnq_mxfp4_experts": [_p, _i64, _i64, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _p],
    "lnq_nf4_dequant": [_p, _p, _p, _i64, _i64, _i64, _i32, _p],
    "lnq_nf4_linear": [_p, _i64, _i64, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32, _p],
    "lnq_nf4_repack": [_p, _p, _p, _p, _i64, _f32, _p, _p, _i64, _i64, _i64, _p],
    "lnq_rmsnorm": [_p, _p, _p, _p, _i64, _i64, ctypes.c_float, _p],
    "lnq_rmsnorm_tiles": [_p, _p, _p, _p, _i64, _i64, ctypes.c_float, _p],
    "lnq_rmsnorm_parts": [_p, _p, _i32, _p, _p, _i32, _i64, _i64, ctypes.c_float, _p],
    "lnq_decode_attention": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p],
    "lnq_decode_attention_at": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _i64, _i64, _p],
    "lnq_decode_attention_tiles": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p,
                                   _i64, _i64, _p],
    "lnq_decode_attention_noalloc": [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p],
    "lnq_prefill_rope": [_p, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p],
    "lnq_silu_mul": [_p, _p, _p, _i64, _p],
    "lnq_silu_mul_rows": [_p, _p, _p, _i64, _i64, _i64, _i64, _p],
    "lnq_silu_mul_tiles": [_p, _p, _p, _i64, _i64, _i64, _i64, _p],
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """The loaded library, its entry points declared (loaded once per process)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIBRARY.exists():
            raise LinnetError(
                f"{LIBRARY.name} is not built: run `python -m linnet_amd._build` "
                "(or __graft_entry__.build()) on a machine with hipcc"
            )
        try:
            lib = ctypes.CDLL(str(LIBRARY))
        except OSError as error:
            raise LinnetError(f"cannot load {LIBRARY}: {error}") from error
        lib.lnq_abi_version.restype = ctypes.c_uint32
        lib.lnq_abi_version.argtypes = []
        lib.lnq_last_error.restype = ctypes.c_char_p
        lib.lnq_last_error.argtypes = []
        lib.lnq_decode_attention_workspace.restype = _i64
        lib.lnq_decode_attention_workspace.argtypes = [_i64, _i64, _i64, _i64]
        version = lib.lnq_abi_version()
        if version != ABI_VERSION:
            raise LinnetError(f"{LIBRARY.name} implements ABI {version}, this package needs {ABI_VERSION}")
        for name, argtypes in SIGNATURES.items():
            function = getattr(lib, name)
            function.restype = ctypes.c_int32
            function.argtypes = argtypes
        _lib = lib
        return lib


def last_error() -> str:
    return (load().lnq_last_error() or b"").decode("utf-8", "replace")


def call(name: str, *args: object) -> None:
    """Calls entry point `name`; raises LinnetError with the library's message on failure."""
    status = getattr(load(), name)(*args)
    if status != LNQ_OK:
        kind = "unavailable" if status == LNQ_UNAVAILABLE else "failed"
        raise LinnetError(f"{name} {kind}: {last_error()}")
