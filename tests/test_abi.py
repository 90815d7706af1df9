"""The C ABI without a GPU: the library loads, exports every entry point
`include/linnet_quant.h` declares, and rejects bad arguments with a status and a
message before touching a device. The host wrappers refuse CPU tensors instead
of falling back to a CPU path."""

from __future__ import annotations

import ctypes
import re
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from linnet_amd import LinnetError, _lib
from linnet_amd.torch import generated, kernels, quantized

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "linnet_quant.h"


def declared() -> list[str]:
    text = HEADER.read_text()
    return re.findall(r"LNQ_API\s+[\w\s\*]+?\b(lnq_\w+)\s*\(", text)


def test_header_declares_the_abi() -> None:
    names = declared()
    expected = {"lnq_int4_linear", "lnq_int4_linear_plan", "lnq_int4_dequantize", "lnq_int4_quantize", "lnq_mm8",
                "lnq_mm8_tiles", "lnq_mm8_plan", "lnq_w8a16", "lnq_rows8", "lnq_mxfp4_experts"}
    assert expected <= set(names)
    assert len(names) == len(set(names))


def test_library_exports_every_declared_symbol() -> None:
    lib = _lib.load()
    for name in declared():
        assert hasattr(lib, name), name
    exported = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIBRARY)], capture_output=True, text=True, check=True).stdout
    for name in declared():
        assert re.search(rf"\bT {name}\b", exported), name
    assert set(_lib.SIGNATURES) | {"lnq_abi_version", "lnq_last_error", "lnq_decode_attention_workspace"} == set(declared())


def test_abi_version() -> None:
    assert _lib.load().lnq_abi_version() == _lib.ABI_VERSION == 1


def _status(name: str, *args: object) -> tuple[int, str]:
    status = getattr(_lib.load(), name)(*args)
    return status, _lib.last_error()


NULL = ctypes.c_void_p(0)
FAKE = ctypes.c_void_p(4096)  # never dereferenced: validation fails first


@pytest.mark.parametrize(
    ("args", "message"),
    [
        ((100, 64, 128, 7), "not a multiple of 128"),  # in_features
        ((128, 64, 48, 0), "group of 48"),
        ((128, 64, 128, 9), "dtype 9"),
    ],
)
def test_int4_linear_rejects_bad_arguments(args: tuple[int, int, int, int], message: str) -> None:
    depth, width, group, dtype = args
    dtype = dtype if dtype != 7 else _lib.BF16
    status, error = _status("lnq_int4_linear", FAKE, FAKE, FAKE, FAKE, NULL, FAKE, 1, depth, width, group, dtype, 0, NULL)
    assert status == _lib.LNQ_ERROR
    assert message in error


def test_unaligned_and_null_pointers_are_rejected() -> None:
    status, error = _status("lnq_int4_linear", ctypes.c_void_p(4098), FAKE, FAKE, FAKE, NULL, FAKE, 1, 128, 16, 128, _lib.BF16, 0, NULL)
    assert status == _lib.LNQ_ERROR and "aligned" in error
    status, error = _status("lnq_int4_linear", NULL, FAKE, FAKE, FAKE, NULL, FAKE, 1, 128, 16, 128, _lib.BF16, 0, NULL)
    assert status == _lib.LNQ_ERROR and "null" in error


def test_other_entry_points_validate() -> None:
    assert _status("lnq_int4_quantize", FAKE, FAKE, FAKE, FAKE, 4, 130, 64, NULL)[1].startswith("lnq_int4_quantize: groups of 64")
    assert "dtype 5" in _status("lnq_int4_dequantize", FAKE, FAKE, FAKE, FAKE, 4, 128, 128, 5, NULL)[1]
    assert "groups" in _status("lnq_int8_quantize", FAKE, FAKE, FAKE, 4, 100, 64, 0, NULL)[1]
    assert "in % 128" in _status("lnq_w8a16", FAKE, FAKE, FAKE, FAKE, 1, 16, 100, 0, 0, 1, _lib.BF16, NULL)[1]
    assert "64k" in _status("lnq_w8a16", FAKE, FAKE, FAKE, FAKE, 1, 16, 256, 0, 32, 1, _lib.BF16, NULL)[1]
    assert "in % 16" in _status("lnq_dequantize8", FAKE, FAKE, FAKE, 4, 100, 0, 0, 1, _lib.BF16, NULL)[1]
    assert "output is bf16 or f16" in _status("lnq_mm8", FAKE, FAKE, FAKE, FAKE, FAKE, 1, 16, 128, 1, _lib.F32, NULL)[1]
    assert "negative" in _status("lnq_int4_pack", FAKE, FAKE, -1, NULL)[1]
    big = 1 << 40
    assert "head_dim is 64 or 128" in _status("lnq_decode_attention", *[FAKE] * 9, big, 1, 32, 8, 96, 1025, 1024, 0, 0, NULL)[1]
    assert "outside the cache" in _status("lnq_decode_attention", *[FAKE] * 9, big, 1, 32, 8, 128, 1024, 1024, 0, 0, NULL)[1]
    assert "multiple" in _status("lnq_decode_attention", *[FAKE] * 9, big, 1, 30, 8, 128, 1025, 1024, 0, 0, NULL)[1]
    need = _lib.load().lnq_decode_attention_workspace(2, 8, 128, 1024)
    assert need == 2 * 8 * 17 * 8 * 130
    assert "workspace" in _status("lnq_decode_attention", *[FAKE] * 9, need - 1, 2, 32, 8, 128, 1028, 1024, 0, 0, NULL)[1]
    assert "multiple of 4" in _status("lnq_decode_attention", *[FAKE] * 9, big, 2, 32, 8, 128, 1025, 1024, 0, 0, NULL)[1]
    assert "strides" in _status("lnq_decode_attention", *[FAKE] * 9, big, 2, 32, 8, 128, 1028, 1024, 4000, 0, NULL)[1]
    # a row broadcast over rows (stride 0) is refused, not read as packed rows
    assert "strides" in _status("lnq_decode_attention", *[FAKE] * 9, big, 2, 32, 8, 128, 1028, 1024, 0, 1024, NULL)[1]
    assert "strides" in _status("lnq_decode_attention", *[FAKE] * 9, big, 2, 32, 8, 128, 1028, 1024, 4096, 0, NULL)[1]
    assert "bad shape" in _status("lnq_rmsnorm", FAKE, NULL, FAKE, FAKE, 1, 0, ctypes.c_float(1e-5), NULL)[1]
    assert "neither GPTQ" in _status("lnq_int4_repack", FAKE, FAKE, NULL, 2, 0, 64, 64, 1, FAKE, FAKE, NULL)[1]
    assert "multiples of 8" in _status("lnq_int4_repack", FAKE, FAKE, NULL, 0, 0, 60, 64, 1, FAKE, FAKE, NULL)[1]
    assert "equal groups" in _status("lnq_int4_repack", FAKE, FAKE, NULL, 0, 0, 64, 64, 3, FAKE, FAKE, NULL)[1]
    assert "only GPTQ" in _status("lnq_int4_repack", FAKE, FAKE, FAKE, 1, 0, 64, 64, 1, FAKE, FAKE, NULL)[1]
    assert "zero_offset" in _status("lnq_int4_repack", FAKE, FAKE, NULL, 0, 2, 64, 64, 1, FAKE, FAKE, NULL)[1]
    assert "bf16, f16 or f32" in _status("lnq_int4_row_prepare", FAKE, FAKE, FAKE, FAKE, FAKE, 4, 128, 128, 7, NULL)[1]
    assert "in % 32" in _status("lnq_int4_row_prepare", FAKE, FAKE, FAKE, FAKE, FAKE, 4, 48, 16, _lib.BF16, NULL)[1]
    assert "must be even" in _status("lnq_int4_row_prepare", FAKE, FAKE, FAKE, FAKE, FAKE, 4, 128, 96, _lib.BF16,
                                     NULL)[1]
    assert "taken" in _status("lnq_int4_linear_ordered", FAKE, FAKE, FAKE, FAKE, FAKE, NULL, FAKE, NULL, 4, 4096, 4096,
                              128, _lib.BF16, 0, NULL)[1]
    pro = lambda kind, norm, u, rows, dtype=_lib.BF16, staged=NULL: _status(  # noqa: E731
        "lnq_int4_linear_prologue", FAKE, u, norm, 1e-5, kind, FAKE, FAKE, FAKE, NULL, FAKE, staged, rows, 4096, 4096,
        128, dtype, 0, NULL)
    assert "prologue is" in pro(0, FAKE, NULL, 1)[1]
    assert "compute in bf16" in pro(_lib.PROLOGUE_RMSNORM, FAKE, NULL, 1, _lib.F16)[1]
    assert "needs norm_weight" in pro(_lib.PROLOGUE_RMSNORM, NULL, FAKE, 1)[1]
    assert "needs u" in pro(_lib.PROLOGUE_SILU_MUL, FAKE, NULL, 1)[1]
    assert "staged" in pro(_lib.PROLOGUE_SILU_MUL, NULL, FAKE, 4)[1]
    assert pro(_lib.PROLOGUE_RMSNORM, FAKE, NULL, 0)[0] == _lib.LNQ_OK
    rope = lambda positions, hd, cap, stride=4096: _status(  # noqa: E731
        "lnq_prefill_rope", FAKE, FAKE, FAKE, stride, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, positions, 32, 8, hd, cap,
        NULL)
    assert "head_dim is 64 or 128" in rope(10, 96, 16)[1]
    assert "positions <= cap" in rope(20, 128, 16)[1]
    assert "multiple of 8" in rope(10, 128, 16, stride=100)[1]
    # 32 heads of 128: a q row is 4096 elements, so a 1024-element stride overlaps rows.
    assert "shorter than a q row" in rope(10, 128, 16, stride=1024)[1]
    assert rope(0, 128, 16)[0] == _lib.LNQ_OK
    assert "bf16, f16 or f32" in _status("lnq_take_inputs", FAKE, FAKE, FAKE, 1, 8, 9, NULL)[1]
    assert "must not be x" in _status("lnq_take_inputs", FAKE, FAKE, FAKE, 1, 8, _lib.BF16, NULL)[1]
    assert "groups of 128" in _status("lnq_fp8_groups", FAKE, FAKE, FAKE, 2, 2, 256, 64, _lib.BF16, NULL)[1]
    assert "padded >= rows" in _status("lnq_fp8_groups", FAKE, FAKE, FAKE, 3, 2, 256, 128, _lib.BF16, NULL)[1]
    assert "in, out % 128" in _status("lnq_mm8_block", FAKE, FAKE, FAKE, 4, FAKE, FAKE, 4, 100, 256, _lib.BF16, NULL)[1]
    assert "stride" in _status("lnq_mm8_block", FAKE, FAKE, FAKE, 2, FAKE, FAKE, 4, 128, 256, _lib.BF16, NULL)[1]
    assert "multiple of 32" in _status("lnq_mxfp4_experts", FAKE, 0, 0, FAKE, FAKE, FAKE, FAKE, 1, 4, 32, 64, 100,
                                       _lib.BF16, NULL)[1]
    assert "bf16 or f16" in _status("lnq_mxfp4_experts", FAKE, 0, 0, FAKE, FAKE, FAKE, FAKE, 1, 4, 32, 64, 128,
                                    _lib.F32, NULL)[1]


def test_empty_calls_succeed_without_a_device() -> None:
    assert _status("lnq_int4_linear", FAKE, FAKE, FAKE, FAKE, NULL, FAKE, 0, 128, 16, 128, _lib.BF16, 0, NULL)[0] == _lib.LNQ_OK
    assert _status("lnq_int4_dequantize", NULL, NULL, NULL, NULL, 0, 128, 128, _lib.BF16, NULL)[0] == _lib.LNQ_OK
    assert _status("lnq_rows8", NULL, NULL, NULL, 0, 128, 1, _lib.BF16, NULL)[0] == _lib.LNQ_OK
    assert _status("lnq_silu_mul", NULL, NULL, NULL, 0, NULL)[0] == _lib.LNQ_OK
    assert _status("lnq_silu_mul_rows", NULL, NULL, NULL, 0, 8, 16, 16, NULL)[0] == _lib.LNQ_OK
    assert _status("lnq_fp8_groups", NULL, NULL, NULL, 0, 0, 256, 128, _lib.BF16, NULL)[0] == _lib.LNQ_OK
    assert _status("lnq_mm8_block", NULL, NULL, NULL, 0, NULL, NULL, 0, 128, 256, _lib.BF16, NULL)[0] == _lib.LNQ_OK
    assert _status("lnq_mxfp4_experts", NULL, 0, 0, NULL, NULL, NULL, NULL, 0, 4, 32, 64, 128, _lib.BF16, NULL)[0] == _lib.LNQ_OK
    assert "bad shape" in _status("lnq_silu_mul_rows", FAKE, FAKE, FAKE, 2, 8, 4, 16, NULL)[1]
    assert _status("lnq_rmsnorm", NULL, NULL, NULL, NULL, 0, 4096, ctypes.c_float(1e-5), NULL)[0] == _lib.LNQ_OK
    assert _status("lnq_int4_repack", NULL, NULL, NULL, 0, 1, 0, 64, 0, NULL, NULL, NULL)[0] == _lib.LNQ_OK
    assert _status("lnq_int4_row_prepare", NULL, NULL, NULL, NULL, NULL, 0, 128, 128, _lib.BF16, NULL)[0] == _lib.LNQ_OK
    assert _status("lnq_take_inputs", NULL, NULL, NULL, 0, 8, _lib.BF16, NULL)[0] == _lib.LNQ_OK
    assert _status("lnq_int4_linear_ordered", FAKE, FAKE, FAKE, FAKE, FAKE, NULL, FAKE, NULL, 0, 4096, 4096, 128,
                   _lib.BF16, 0, NULL)[0] == _lib.LNQ_OK


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU answer")
def test_device_probe_without_a_gpu() -> None:
    a, b = ctypes.c_int32(), ctypes.c_int32()
    status = _lib.load().lnq_device_probe(0, ctypes.byref(a), ctypes.byref(b))
    assert status == _lib.LNQ_UNAVAILABLE and "no HIP device" in _lib.last_error()


def test_call_raises_with_the_library_message() -> None:
    with pytest.raises(LinnetError, match="not a multiple of 128"):
        _lib.call("lnq_int4_linear", FAKE, FAKE, FAKE, FAKE, NULL, FAKE, 1, 100, 16, 100, _lib.BF16, 0, NULL)


# --------------------------------------------------------------- host wrappers


def test_cpu_tensors_raise_instead_of_falling_back() -> None:
    x = torch.zeros(1, 128, dtype=torch.bfloat16)
    packed = torch.zeros(16, 1, 64, dtype=torch.uint8)
    scale = torch.ones(16, 1, dtype=torch.bfloat16)
    zero = torch.zeros(16, 1, dtype=torch.uint8)
    with pytest.raises(LinnetError, match="GPU"):
        kernels.int4_linear(x, packed, scale, zero)
    with pytest.raises(LinnetError, match="GPU"):
        generated._int4_pack(packed, scale, zero)
    with pytest.raises(LinnetError, match="GPU"):
        quantized.int8_operands(torch.zeros(16, 128, dtype=torch.int8), torch.ones(16), 0)
    with pytest.raises(LinnetError, match="GPU"):
        quantized.fp8_operands(torch.zeros(16, 128, dtype=torch.uint8), torch.ones(16), 1)
    with pytest.raises(LinnetError, match="GPU"):
        kernels.fp8_rows(x)


def test_fused_group_gate_matches_the_reference() -> None:
    """`_int4_pack` takes groups 32, 64 and multiples of 128 (`torch_source.cpp:1489-1494`
    took 32, 64, 128, 256 for tinygemm)."""
    assert all(generated._fused_group(g) for g in (32, 64, 128, 256, 512))
    assert not any(generated._fused_group(g) for g in (2, 16, 48, 96))


def test_bench_refuses_more_than_one_gpu() -> None:
    done = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True, timeout=300)
    assert done.returncode == 2
    assert "one GPU" in done.stderr


def test_plan_queries_name_the_kernel_without_a_device() -> None:
    """The kernel choice a shape takes (256 compute units assumed with no device):
    config 2's decode rows on the GEMV, config 3's M = 2048 shapes on the tiled
    kernel with 256- or 128-column tiles, config 4 at 4096 rows on 256-column
    8-bit tiles; a forced kernel that does not take the shape is refused."""
    assert kernels.int4_linear_plan(1, 4096, 14336, 128) == "gemv"
    assert kernels.int4_linear_plan(16, 4096, 14336, 128) == "gemv"
    assert kernels.int4_linear_plan(2048, 4096, 14336, 128) == "persistent"
    assert kernels.int4_linear_plan(2048, 4096, 14336, 128, kernel="tiled") == "persistent"
    assert kernels.int4_linear_plan(2048, 4096, 14336, 32) == "tiled256"
    assert kernels.int4_linear_plan(2048, 4096, 4096, 128) == "tiled128"
    assert kernels.int4_linear_plan(2048, 14336, 4096, 128) == "tiled128"
    assert kernels.int4_linear_plan(8, 512, 64, 128) == "skinny"
    assert kernels.int4_linear_plan(8, 512, 64, 128, kernel="tiled256") == "tiled256"
    with pytest.raises(LinnetError, match="one-token kernel"):
        kernels.int4_linear_plan(1, 512, 64, 32, kernel="gemv")
    with pytest.raises(LinnetError, match="unknown kernel"):
        _lib.call("lnq_int4_linear_plan", 1, 512, 64, 128, _lib.BF16, 9, ctypes.byref(ctypes.c_int32()))
    # The split GEMV (a workspace of the caller's): the decode batch's down
    # projection and 17..64 rows over the widest outputs; without a workspace
    # (lnq_int4_linear and its plan) it is never chosen and refused when asked for.
    assert kernels.int4_linear_plan(32, 14336, 4096, 128) == "split"
    assert kernels.int4_linear_plan(16, 14336, 4096, 128) == "split"
    assert kernels.int4_linear_plan(64, 14336, 4096, 128) == "split"
    assert kernels.int4_linear_plan(8, 14336, 4096, 128) == "skinny"
    assert kernels.int4_linear_plan(32, 4096, 128256, 128) == "split"
    assert kernels.int4_linear_plan(32, 4096, 28672, 128) == "gemv"
    assert kernels.int4_linear_plan(4, 4096, 4096, 128, kernel="split") == "split"
    chosen, need = ctypes.c_int32(-1), ctypes.c_int64(-1)
    _lib.call("lnq_int4_linear_workspace", 32, 14336, 4096, 128, _lib.BF16, 0, ctypes.byref(chosen), ctypes.byref(need))
    assert (chosen.value, need.value) == (_lib.KERNEL_SPLIT, 4 * 32 * 4096 * 4)
    _lib.call("lnq_int4_linear_workspace", 48, 14336, 4096, 128, _lib.BF16, 0, ctypes.byref(chosen), ctypes.byref(need))
    assert (chosen.value, need.value) == (_lib.KERNEL_SPLIT, 4 * 32 * 4096 * 4)
    _lib.call("lnq_int4_linear_workspace", 1, 4096, 14336, 128, _lib.BF16, 0, ctypes.byref(chosen), ctypes.byref(need))
    assert (chosen.value, need.value) == (_lib.KERNEL_GEMV, 0)
    with pytest.raises(LinnetError, match="unknown kernel"):
        _lib.call("lnq_int4_linear_plan", 32, 14336, 4096, 128, _lib.BF16, _lib.KERNEL_SPLIT, ctypes.byref(chosen))
    with pytest.raises(LinnetError, match="split GEMV does not take"):
        kernels.int4_linear_plan(32, 4352, 4096, 128, kernel="split")  # 17 slices: no chunk of 8..16
    with pytest.raises(LinnetError, match="split GEMV does not take"):
        kernels.int4_linear_plan(65, 14336, 4096, 128, kernel="split")
    with pytest.raises(LinnetError, match="split GEMV does not take"):
        kernels.int4_linear_plan(32, 14336, 4094, 128, kernel="split")
    assert kernels.mm8_plan(4096, 28672, 8192) == kernels.MM8_PERSISTENT
    assert kernels.mm8_plan(4096, 28672, 8192, fp8=False) == 256
    assert kernels.mm8_plan(256, 28672, 8192) == kernels.MM8_STREAM
    assert kernels.mm8_plan(256, 28672, 8192, fp8=False) == 128
    assert kernels.mm8_plan(64, 28672, 8192) == 128
    assert kernels.mm8_plan(128, 28672, 8192) == 128  # the streaming form past 128 rows only
    assert kernels.mm8_plan(129, 28672, 8192) == kernels.MM8_STREAM
    assert kernels.mm8_plan(1024, 28672, 8192) == kernels.MM8_PERSISTENT  # 448 tiles of 256 x 256
    with pytest.raises(LinnetError, match="tile_n"):
        _lib.call("lnq_mm8_tiles", *[ctypes.c_void_p(256)] * 5, 4, 256, 128, 1, _lib.BF16, 64, None)


def test_nf4_entry_points_validate() -> None:
    """The NF4 entries refuse what their kernels do not take, before any device
    call: odd or non-dividing blocks, the GEMV's blocks that are no multiple of
    16, inputs past 32768, x's dtype, a half-given double quantization."""
    def linear(rows: int, out_f: int, in_f: int, block: int, dtype: int = _lib.BF16) -> str:
        return _status("lnq_nf4_linear", FAKE, in_f, rows, FAKE, FAKE, NULL, FAKE, out_f, out_f, in_f, block, dtype,
                       NULL)[1]

    assert "multiple of 16" in linear(1, 8, 128, 8)
    assert "multiple of 16" in linear(1, 8, 96, 64)
    assert "past the product's 32768" in linear(1, 8, 65536, 64)
    assert "bf16 or f16" in linear(1, 8, 128, 64, _lib.F32)
    assert "negative" in linear(-1, 8, 128, 64)
    assert "aligned" in _status("lnq_nf4_linear", ctypes.c_void_p(4098), 128, 1, FAKE, FAKE, NULL, FAKE, 8, 8, 128, 64,
                                _lib.BF16, NULL)[1]
    assert "even" in _status("lnq_nf4_dequant", FAKE, FAKE, FAKE, 4, 126, 63, _lib.BF16, NULL)[1]
    assert "dtype 5" in _status("lnq_nf4_dequant", FAKE, FAKE, FAKE, 4, 128, 64, 5, NULL)[1]
    assert "both" in _status("lnq_nf4_repack", FAKE, FAKE, FAKE, NULL, 256, ctypes.c_float(0.0), FAKE, FAKE, 4, 128,
                             64, NULL)[1]
    assert _status("lnq_nf4_linear", NULL, 128, 0, NULL, NULL, NULL, NULL, 8, 8, 128, 64, _lib.BF16, NULL)[0] == _lib.LNQ_OK
