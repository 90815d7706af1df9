"""The int4 decode step of bench.py's Llama-shaped stack, small:
every linear through the C ABI kernels against the same step with the reference's
fallback product (the weight dequantized to bf16, then `F.linear`,
`torch_source.cpp:1567-1568`), and its HIP-graph replays against eager steps.

The two paths differ only in the linear layers: the kernels multiply with the
exactly dequantized weight in f32 while the reference rounds the weight to bf16
first, so the logits agree to the bf16 rounding of a few layers (bound stated
below, max errors printed)."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))

import bench  # noqa: E402
from linnet_amd.torch import kernels  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
SMALL = dict(layers=2, hidden=512, heads=8, kv_heads=2, ffn=1536, vocab=1000, ctx=64)


def _reference_linear(x, w):
    return torch.nn.functional.linear(x, kernels.int4_weight(*w))


@pytest.mark.parametrize("batch", [1, 4])
def test_int4_decode_step_matches_the_dequantized_reference(batch: int) -> None:
    model = bench.Int4Llama(torch, kernels, DEV, batch=batch, seed=batch, **SMALL)
    x = (torch.randn(batch, SMALL["hidden"], generator=torch.Generator().manual_seed(7)) * 0.5).to(torch.bfloat16).to(DEV)
    got = model.step(x).float()
    model.linear = _reference_linear
    want = model.step(x).float()
    assert got.shape == (batch, SMALL["vocab"]) and torch.isfinite(got).all()
    err = (got - want).abs().max().item()
    scale = want.abs().max().item()
    print(f"logits max abs err {err:.3e}, rel to max|logit| {err / scale:.3e}")
    assert err <= 3e-2 * scale


def test_int4_decode_step_replays_as_a_graph() -> None:
    model = bench.Int4Llama(torch, kernels, DEV, batch=1, seed=3, **SMALL)
    x = (torch.randn(1, SMALL["hidden"], generator=torch.Generator().manual_seed(1)) * 0.5).to(torch.bfloat16).to(DEV)
    eager = model.step(x).clone()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = model.step(x)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        again = model.step(x)  # eager work between the replays
        torch.cuda.synchronize()
        assert torch.equal(again, eager)
