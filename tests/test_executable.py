"""The executable-shaped C ABI (`lnq_int4_linear_executable`, the reference
runtime's `LnExecutable`, `include/linnet/runtime/runtime.h:44-94`) without a GPU:
the struct layouts match the reference's field for field, bad layer shapes are
refused at creation, `prepare` reports a CPU context as unavailable, and
`execute` refuses to run before `prepare` or with another ABI version -- all
before any device call."""

from __future__ import annotations

import ctypes

import pytest
import torch

from linnet_amd import LinnetError, _lib, executable


def test_struct_layouts_are_the_runtime_abi() -> None:
    # runtime.h:44-94 on LP64: offsets and sizes of the DLPack-style structs
    assert ctypes.sizeof(executable.LnDevice) == 8
    assert ctypes.sizeof(executable.LnDataType) == 4
    assert [executable.LnTensor.__dict__[f].offset for f in ("data", "device", "ndim", "dtype", "shape", "strides", "byte_offset")] == [0, 8, 16, 20, 24, 32, 40]
    assert ctypes.sizeof(executable.LnTensor) == 48
    assert [executable.LnContext.__dict__[f].offset for f in ("abi_version", "device", "stream", "workspace", "workspace_bytes", "capturing")] == [0, 4, 16, 24, 32, 40]
    assert [executable.LnExecutable.__dict__[f].offset for f in ("abi_version", "state", "prepare", "execute", "error", "destroy")] == [0, 8, 16, 24, 32, 40]


@pytest.mark.parametrize(("args", "message"), [
    ((4096, 14336, 100), "group"),
    ((100, 64, 32), "multiple of 128"),
    ((512, 0, 128), "bad shape"),
    ((512, 64, 32, _lib.KERNEL_TILED_256 + 3), "unknown kernel"),
])
def test_bad_layers_are_refused_at_creation(args, message: str) -> None:
    with pytest.raises(LinnetError, match=message):
        executable.Int4LinearExecutable(*args)


def test_prepare_on_a_cpu_context_is_unavailable() -> None:
    exe = executable.Int4LinearExecutable(512, 64, 128)
    with pytest.raises(LinnetError, match="unavailable: int4_linear: the HIP kernels run on a GPU"):
        exe.prepare(device_type=executable.LN_CPU)
    exe.close()
    exe.close()  # destroy runs once


def test_execute_refuses_before_prepare_and_another_abi() -> None:
    exe = executable.Int4LinearExecutable(512, 64, 128)
    x = torch.zeros(2, 512, dtype=torch.bfloat16)
    params = [torch.zeros(64, 4, 64, dtype=torch.uint8), torch.zeros(64, 4, dtype=torch.bfloat16),
              torch.zeros(64, 4, dtype=torch.uint8)]
    y = torch.empty(2, 64, dtype=torch.bfloat16)
    with pytest.raises(LinnetError, match="execute before prepare"):
        exe.execute([x, *params], [y], device_type=executable.DL_ROCM)
    ctx = executable.LnContext(_lib.ABI_VERSION + 7, executable.LnDevice(executable.DL_ROCM, 0), None, None, 0, 0)
    status = exe._exe.prepare(exe._exe.state, ctypes.byref(ctx))
    assert status == _lib.LNQ_ERROR
    assert b"context ABI" in exe._exe.error(exe._exe.state)
