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


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("batch", [1, 4])
def test_int4_decode_step_matches_the_dequantized_reference(batch: int, fused: bool) -> None:
    """The step (decode kernels or torch glue between the int4 linears) against
    the torch-glue step with dequantized-bf16 linears."""
    from linnet_amd.torch import decode

    model = bench.Int4Llama(torch, kernels, DEV, batch=batch, seed=batch, fused=fused, **SMALL)
    x = (torch.randn(batch, SMALL["hidden"], generator=torch.Generator().manual_seed(7)) * 0.5).to(torch.bfloat16).to(DEV)
    calls = []
    attention = decode.decode_attention
    decode.decode_attention = lambda *a: calls.append(1) or attention(*a)
    try:
        got = model.step(x).float()
    finally:
        decode.decode_attention = attention
    assert len(calls) == (SMALL["layers"] if fused else 0)
    model.linear, model.fused = _reference_linear, False
    want = model.step(x).float()
    assert got.shape == (batch, SMALL["vocab"]) and torch.isfinite(got).all()
    err = (got - want).abs().max().item()
    scale = want.abs().max().item()
    print(f"logits max abs err {err:.3e}, rel to max|logit| {err / scale:.3e}")
    assert err <= 3e-2 * scale


@pytest.mark.parametrize("fused", [True, False])
def test_int4_decode_step_replays_as_a_graph(fused: bool) -> None:
    model = bench.Int4Llama(torch, kernels, DEV, batch=1, seed=3, fused=fused, **SMALL)
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


def test_decode_kernels_match_torch_ops() -> None:
    """Each decode kernel against the torch ops it replaces (f32 math, bf16 in and out)."""
    from linnet_amd.torch import decode

    g = torch.Generator().manual_seed(5)
    # hidden: two and four 16-byte chunks a thread (4096, 8192), a partial third
    # (5120), and the element-wise kernel (1000, not a multiple of 8)
    for hidden in (4096, 8192, 5120, 1000):
        x = torch.randn(3, hidden, generator=g).to(torch.bfloat16).to(DEV)
        d = torch.randn(3, hidden, generator=g).to(torch.bfloat16).to(DEV)
        w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(DEV)
        want_x = x + d
        xf = want_x.float()
        want_h = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-5) * w).to(torch.bfloat16)
        h = decode.rmsnorm(x, w, 1e-5, d)
        assert torch.equal(x, want_x)
        assert (h.float() - want_h.float()).abs().max().item() <= 1e-2 * want_h.float().abs().max().item()
        plain = x.clone()
        h2 = decode.rmsnorm(plain, w, 1e-5)
        assert torch.equal(plain, x)
        xf = x.float()
        want_h2 = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-5) * w).to(torch.bfloat16)
        assert (h2.float() - want_h2.float()).abs().max().item() <= 1e-2 * want_h2.float().abs().max().item()
    gg = torch.randn(5, 1000, generator=g).to(torch.bfloat16).to(DEV)
    uu = torch.randn(5, 1000, generator=g).to(torch.bfloat16).to(DEV)
    want_a = (torch.nn.functional.silu(gg.float()) * uu.float()).to(torch.bfloat16)
    assert (decode.silu_mul(gg, uu).float() - want_a.float()).abs().max().item() <= 1e-2
    # the two halves of a joined gate|up output (strided rows) give the same bits
    joined = torch.cat([gg, uu], dim=1)
    assert torch.equal(decode.silu_mul(joined[:, :1000], joined[:, 1000:]), decode.silu_mul(gg, uu))
    for rows, heads, kvh, hd, cap, pos in ((2, 8, 2, 128, 40, 37), (2, 8, 2, 128, 2048, 1999), (1, 8, 2, 128, 704, 700),
                                           (2, 8, 1, 128, 132, 130), (3, 6, 2, 64, 100, 64), (1, 4, 4, 64, 68, 3)):
        _attention_case(decode, g, rows, heads, kvh, hd, cap, pos)


def _attention_case(decode, g, rows: int, heads: int, kvh: int, hd: int, cap: int, pos: int) -> None:
    """One attention step against torch (bf16 caches, f32 math): group sizes 4, 8,
    3 and 1 (the LDS arrays sized 4, 8, 4, 1), head sizes 128 and 64, chunks from
    1 to 32 (the merge's eight-at-a-time loop and its tail)."""
    print(f"attention rows={rows} heads={heads} kv_heads={kvh} hd={hd} cap={cap} pos={pos}", flush=True)
    q = torch.randn(rows, heads * hd, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(rows, kvh * hd, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(rows, kvh * hd, generator=g).to(torch.bfloat16).to(DEV)
    kt = torch.randn(rows, kvh, hd, cap, generator=g).to(torch.bfloat16).to(DEV)
    vc = torch.randn(rows, kvh, cap, hd, generator=g).to(torch.bfloat16).to(DEV)
    ang = pos / (500000.0 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))
    cos, sin = torch.cos(ang).to(DEV), torch.sin(ang).to(DEV)
    kt_ref, vc_ref = kt.clone(), vc.clone()

    def rope(t):
        a, b = t[..., : hd // 2], t[..., hd // 2 :]
        return torch.cat([a * cos - b * sin, b * cos + a * sin], dim=-1)

    qr = rope(q.float().view(rows, heads, hd))
    kt_ref[:, :, :, pos] = rope(k.float().view(rows, kvh, hd))
    vc_ref[:, :, pos, :] = v.float().view(rows, kvh, hd)
    s = torch.matmul(qr.view(rows, kvh, heads // kvh, hd), kt_ref[..., : pos + 1].float()) * hd**-0.5
    want = torch.matmul(torch.softmax(s, dim=-1), vc_ref[:, :, : pos + 1].float()).reshape(rows, heads * hd)
    got = decode.decode_attention(q, k, v, cos, sin, kt, vc, pos)
    assert (got.float() - want).abs().max().item() <= 1e-2 * want.abs().max().item()
    # the new key and value in the caches as bf16 (the key rounded once from f32)
    assert (kt[:, :, :, pos].float() - kt_ref[:, :, :, pos].float()).abs().max().item() <= 1e-2
    assert torch.equal(vc, vc_ref)
