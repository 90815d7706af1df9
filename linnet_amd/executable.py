"""The int4 linear as an executable of the reference runtime's shape
(`include/linnet/runtime/runtime.h:44-94`), from Python: ctypes mirrors of
`LnTensor`, `LnContext` and `LnExecutable` (their layouts are the reference's,
declared in `include/linnet_quant.h`), and `Int4LinearExecutable`, which makes
one with `lnq_int4_linear_executable` and calls its `prepare` / `execute` /
`error` / `destroy` on torch tensors -- what a plan of the reference runtime
does with it (`ln_plan_add` / `ln_plan_run`, `runtime.h:112-131`)."""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .errors import LinnetError

LN_CPU, LN_CUDA, DL_ROCM = 1, 2, 10
_i64p = ctypes.POINTER(ctypes.c_int64)


class LnDevice(ctypes.Structure):
    _fields_ = [("type", ctypes.c_int32), ("id", ctypes.c_int32)]


class LnDataType(ctypes.Structure):
    _fields_ = [("code", ctypes.c_uint8), ("bits", ctypes.c_uint8), ("lanes", ctypes.c_uint16)]


class LnTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("device", LnDevice),
        ("ndim", ctypes.c_int32),
        ("dtype", LnDataType),
        ("shape", _i64p),
        ("strides", _i64p),
        ("byte_offset", ctypes.c_uint64),
    ]


class LnContext(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_uint32),
        ("device", LnDevice),
        ("stream", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("capturing", ctypes.c_int32),
    ]


_PREPARE = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.POINTER(LnContext))
_EXECUTE = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.POINTER(LnTensor), ctypes.c_size_t,
                            ctypes.POINTER(LnTensor), ctypes.c_size_t, ctypes.POINTER(LnContext))
_ERROR = ctypes.CFUNCTYPE(ctypes.c_char_p, ctypes.c_void_p)
_DESTROY = ctypes.CFUNCTYPE(None, ctypes.c_void_p)


class LnExecutable(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_uint32),
        ("state", ctypes.c_void_p),
        ("prepare", _PREPARE),
        ("execute", _EXECUTE),
        ("error", _ERROR),
        ("destroy", _DESTROY),
    ]


_DTYPES = {
    torch.bfloat16: (4, 16),
    torch.float16: (2, 16),
    torch.float32: (2, 32),
    torch.uint8: (1, 8),
    torch.int8: (0, 8),
}


def tensor(t: torch.Tensor, device_type: int | None = None) -> tuple[LnTensor, tuple]:
    """`t` described as an `LnTensor` (a GPU tensor as DLPack's ROCm device), and the
    ctypes arrays it points into (keep them alive while the descriptor is used)."""
    if t.dtype not in _DTYPES:
        raise LinnetError(f"no LnDataType for {t.dtype}")
    shape = (ctypes.c_int64 * t.dim())(*t.shape)
    strides = (ctypes.c_int64 * t.dim())(*t.stride())
    code, bits = _DTYPES[t.dtype]
    kind = device_type if device_type is not None else (DL_ROCM if t.is_cuda else LN_CPU)
    index = t.device.index if t.is_cuda else 0
    described = LnTensor(ctypes.c_void_p(t.data_ptr()), LnDevice(kind, index or 0), t.dim(), LnDataType(code, bits, 1),
                         shape, strides, 0)
    return described, (shape, strides)


class Int4LinearExecutable:
    """`lnq_int4_linear_executable(in, out, group, kernel)` driven from Python."""

    def __init__(self, in_features: int, out_features: int, group: int, kernel: int = _lib.KERNEL_AUTO) -> None:
        lib = _lib.load()
        self._exe = LnExecutable()
        status = lib.lnq_int4_linear_executable(in_features, out_features, group, kernel, ctypes.byref(self._exe))
        if status != _lib.LNQ_OK:
            raise LinnetError(f"lnq_int4_linear_executable failed: {_lib.last_error()}")
        self.out_features = out_features

    def _check(self, status: int, what: str) -> None:
        if status != _lib.LNQ_OK:
            message = (self._exe.error(self._exe.state) or b"").decode("utf-8", "replace")
            kind = "unavailable" if status == _lib.LNQ_UNAVAILABLE else "failed"
            raise LinnetError(f"int4 executable {what} {kind}: {message}")

    def context(self, device_type: int, device_id: int, stream: int | None) -> LnContext:
        return LnContext(_lib.ABI_VERSION, LnDevice(device_type, device_id), ctypes.c_void_p(stream or 0), None, 0, 0)

    def prepare(self, device_type: int = DL_ROCM, device_id: int = 0) -> None:
        ctx = self.context(device_type, device_id, None)
        self._check(self._exe.prepare(self._exe.state, ctypes.byref(ctx)), "prepare")

    def execute(self, inputs: list[torch.Tensor], outputs: list[torch.Tensor], stream: int | None = None,
                device_type: int | None = None) -> None:
        described = [tensor(t, device_type) for t in inputs]
        produced = [tensor(t, device_type) for t in outputs]
        ins = (LnTensor * len(inputs))(*[d for d, _ in described])
        outs = (LnTensor * len(outputs))(*[d for d, _ in produced])
        device = inputs[0].device if inputs else torch.device("cpu")
        kind = device_type if device_type is not None else (DL_ROCM if device.type == "cuda" else LN_CPU)
        if stream is None and device.type == "cuda":
            stream = torch.cuda.current_stream(device).cuda_stream
        ctx = self.context(kind, device.index or 0, stream)
        self._check(self._exe.execute(self._exe.state, ins, len(inputs), outs, len(outputs), ctypes.byref(ctx)),
                    "execute")

    def close(self) -> None:
        if self._exe.state:
            self._exe.destroy(self._exe.state)
            self._exe.state = None

    def __del__(self) -> None:
        self.close()


__all__ = ["Int4LinearExecutable", "LnContext", "LnDataType", "LnDevice", "LnExecutable", "LnTensor", "tensor"]
