"""The allocation-free decode attention (`lnq_decode_attention_noalloc`, its
workspace a static array of the library) against the entry point it varies
(`lnq_decode_attention`, workspace passed in), both called through the C ABI on
the same inputs: the outputs and the KV caches they write are equal bit for bit.
Two calls in a row, the second with a smaller step, since every call shares the
GPU's one array."""

from __future__ import annotations

import ctypes

import pytest
import torch

from linnet_amd import _lib

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _inputs(rows: int, heads: int, kvh: int, hd: int, cap: int, pos: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(rows, heads * hd, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(rows, kvh * hd, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(rows, kvh * hd, generator=g).to(torch.bfloat16).to(DEV)
    kt = torch.randn(rows, kvh, hd, cap, generator=g).to(torch.bfloat16).to(DEV)
    vc = torch.randn(rows, kvh, cap, hd, generator=g).to(torch.bfloat16).to(DEV)
    ang = pos / (500000.0 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))
    return q, k, v, torch.cos(ang).to(DEV), torch.sin(ang).to(DEV), kt, vc


def _p(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _both(rows: int, heads: int, kvh: int, hd: int, cap: int, pos: int, seed: int) -> None:
    print(f"noalloc attention rows={rows} heads={heads} kv_heads={kvh} hd={hd} cap={cap} pos={pos}", flush=True)
    q, k, v, cos, sin, kt, vc = _inputs(rows, heads, kvh, hd, cap, pos, seed)
    kt2, vc2 = kt.clone(), vc.clone()
    stream = ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)
    out = torch.empty_like(q)
    floats = _lib.load().lnq_decode_attention_workspace(rows, kvh, hd, pos)
    work = torch.empty(floats, dtype=torch.float32, device=DEV)
    _lib.call("lnq_decode_attention", _p(q), _p(k), _p(v), _p(cos), _p(sin), _p(kt), _p(vc), _p(out), _p(work),
              floats, rows, heads, kvh, hd, cap, pos, q.shape[1], k.shape[1], stream)
    out2 = torch.full_like(q, float("nan"))
    _lib.call("lnq_decode_attention_noalloc", _p(q), _p(k), _p(v), _p(cos), _p(sin), _p(kt2), _p(vc2), _p(out2),
              rows, heads, kvh, hd, cap, pos, q.shape[1], k.shape[1], stream)
    torch.cuda.synchronize()
    assert torch.equal(out2, out)
    assert torch.equal(kt2, kt) and torch.equal(vc2, vc)


def test_noalloc_attention_equals_the_workspace_entry_point() -> None:
    # config 5's step at 32 rows and a 1024-token context (4.5 M workspace floats),
    # then a smaller step (one row, head_dim 64) over the same scratch array
    _both(32, 32, 8, 128, 1028, 1024, seed=1)
    _both(1, 8, 2, 64, 68, 40, seed=2)


def test_noalloc_attention_refuses_a_step_past_its_scratch() -> None:
    stream = ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)
    fake = ctypes.c_void_p(256)
    status = _lib.load().lnq_decode_attention_noalloc(*[fake] * 8, 32, 32, 8, 128, 4096, 1984, 4096, 1024, stream)
    assert status == _lib.LNQ_ERROR and "more than" in _lib.last_error()
