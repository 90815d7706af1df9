"""The int4 decode step of the Llama-shaped stack (`linnet_amd.llama`):
every linear through the C ABI kernels against the same step with the reference's
fallback product (the weight dequantized to bf16, then `F.linear`,
`torch_source.cpp:1567-1568`), and its HIP-graph replays against eager steps.

The two paths differ only in the linear layers: the kernels multiply with the
exactly dequantized weight in f32 while the reference rounds the weight to bf16
first, so the logits agree to the bf16 rounding of a few layers (bound stated
below, max errors printed)."""

from __future__ import annotations

import pytest
import torch

from linnet_amd.llama import Int4Llama
from linnet_amd.torch import kernels

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

    model = Int4Llama(torch, kernels, DEV, batch=batch, seed=batch, fused=fused, **SMALL)
    x = (torch.randn(batch, SMALL["hidden"], generator=torch.Generator().manual_seed(7)) * 0.5).to(torch.bfloat16).to(DEV)
    calls = []
    attention = decode.decode_attention
    decode.decode_attention = lambda *a, **kw: calls.append(1) or attention(*a, **kw)
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


def _exact_linear(x, w):
    """The product the kernels compute: the weight dequantized exactly in f32, f32
    sums, one rounding of the output to x's dtype."""
    packed, scale, zero = w
    return (x.float() @ kernels.int4_weight(packed, scale.float(), zero).T).to(x.dtype)


def _compare(what: str, got: torch.Tensor, want: torch.Tensor) -> tuple[float, float]:
    err = (got - want).abs().max().item()
    scale = want.abs().max().item()
    rel = (got - want).norm().item() / want.norm().item()
    agree = (got.argmax(-1) == want.argmax(-1)).float().mean().item()
    print(f"{what}: logits max abs err {err:.3e}, rel to max|logit| {err / scale:.3e}, relative L2 {rel:.3e}, "
          f"top-1 agreement {agree:.3f}", flush=True)
    return err / scale, agree


@pytest.mark.parametrize("batch", [1, 32])
def test_full_size_decode_step_matches_the_dequantized_reference(batch: int) -> None:
    """Config 5 at full size (32 layers, hidden 4096, 32/8 heads, FFN 14336, vocab
    128256, context 1024), layer by layer: each layer of the step (decode kernels,
    joined int4 projections) and the head take the same input as the torch-glue
    layer whose linears multiply (a) the exactly dequantized f32 weight -- the
    product the kernels compute -- and (b) the weight rounded to bf16, the
    reference's fallback (`torch_source.cpp:1567-1568`); the layer's attention and
    MLP branch outputs (each a chain of products with bf16 intermediates, every
    product held to 1e-2 on its own) must agree within 1e-2 of their largest
    element, the logits within 1e-2 (a) / 2e-2 (b) of max|logit|. The reference's
    output feeds the next layer, so an error is not compounded over 32 random
    layers: run end to end, the two steps' logits part by about 4% of their max
    (printed below) from summation-order differences alone."""
    print(f"full config-5 step batch={batch}", flush=True)
    model = Int4Llama(torch, kernels, DEV, batch=batch, seed=11, fused=True)
    x = (torch.randn(batch, 4096, generator=torch.Generator().manual_seed(2)) * 0.5).to(torch.bfloat16).to(DEV)
    errors = {(name, part): [] for name in ("exact", "bf16") for part in ("attn", "mlp")}
    cur = x
    for i in range(32):
        got = {}
        got["mlp"] = model.layer_fused(i, cur.clone(), None, got).float()
        for name, lin in (("exact", _exact_linear), ("bf16", _reference_linear)):
            want = {}
            model.layer_torch(i, cur, lin, want)
            for part in ("attn", "mlp"):
                w = want[part].float()
                errors[name, part].append((got[part].float() - w).abs().max().item() / w.abs().max().item())
        cur = model.layer_torch(i, cur, _exact_linear)
    for (name, part), errs in errors.items():
        print(f"batch {batch}: {part} branch error rel to its max vs {name}-weight layers: max {max(errs):.3e}, "
              f"mean {sum(errs) / len(errs):.3e}; " + " ".join(f"{e:.1e}" for e in errs), flush=True)
        assert max(errs) <= 1e-2
    logits = model.head_fused(cur.clone(), None).float()
    for name, lin, bound in (("exact", _exact_linear, 1e-2), ("bf16", _reference_linear, 2e-2)):
        rel, agree = _compare(f"batch {batch} head vs {name}-weight", logits, model.head_torch(cur, lin).float())
        assert rel <= bound and agree >= 0.95
    # End to end (reported only: chaotic over 32 random layers, see above).
    model.pos = 1024
    end = model.step(x).float()
    model.fused, model.linear = False, _reference_linear
    _compare(f"batch {batch} end to end vs bf16-weight step", end, model.step(x).float())
    del model


@pytest.mark.parametrize("fused", [True, False])
def test_int4_decode_step_replays_as_a_graph(fused: bool) -> None:
    model = Int4Llama(torch, kernels, DEV, batch=1, seed=3, fused=fused, **SMALL)
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


@pytest.mark.parametrize("shape", ["small", "config5"])
def test_folded_layers_match_the_fused_layers(shape: str) -> None:
    """A one-token step with the glue folded into the linear layers' kernels
    (`layer_folded`: RMSNorm and SiLU x up in the GEMVs' staging of x, the residual
    adds in their epilogues) against the step on the separate decode kernels
    (`layer_fused`), layer by layer from the same residual input: the layer's
    output residual agrees within 1e-2 of its largest value, the head's logits
    within 1e-2 of theirs with the same top token; the captured device-position
    step replays the eager folded step bit for bit."""
    dims = SMALL if shape == "small" else {}
    model = Int4Llama(torch, kernels, DEV, batch=1, seed=6, spare=4, **dims)
    hidden = dims.get("hidden", 4096)
    x = (torch.randn(1, hidden, generator=torch.Generator().manual_seed(8)) * 0.5).to(torch.bfloat16).to(DEV)
    worst = 0.0
    for i in range(len(model.layers)):
        folded = model.layer_folded(i, x)
        xc = x.clone()
        fused = (xc + model.layer_fused(i, xc, None)).to(torch.bfloat16)
        rel = (folded.float() - fused.float()).abs().max().item() / fused.float().abs().max().item()
        worst = max(worst, rel)
        assert rel <= 1e-2, (i, rel)
        x = folded
    rel, agree = _compare(f"{shape} head folded vs fused (worst layer {worst:.2e})", model.head_folded(x).float(),
                          model.head_fused(x.clone(), None).float())
    assert rel <= 1e-2 and agree == 1.0
    x = (torch.randn(1, hidden, generator=torch.Generator().manual_seed(9)) * 0.5).to(torch.bfloat16).to(DEV)
    pos = model.pos
    want = model.step(x)
    model.set_position(pos)
    model.step_at(x)
    model.set_position(pos)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = model.step_at(x)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    del model, graph


@pytest.mark.parametrize("batch", [1, 3])
def test_captured_step_advances_the_position(batch: int) -> None:
    """A step recorded with the position in device memory (`step_at`) moves one
    cache position a replay: three replays equal, bit for bit, three eager steps
    of an identical model at positions 64, 65, 66 (host position, per-position
    rotary values), each replay with eager work between, and every replay wrote
    its own k / v cache column."""
    x = (torch.randn(batch, SMALL["hidden"], generator=torch.Generator().manual_seed(5)) * 0.5).to(torch.bfloat16).to(DEV)
    live = Int4Llama(torch, kernels, DEV, batch=batch, seed=7, spare=8, **SMALL)
    twin = Int4Llama(torch, kernels, DEV, batch=batch, seed=7, spare=8, **SMALL)
    graph = torch.cuda.CUDAGraph()
    live.step_at(x)  # warm up at 64 (writes column 64, as the first eager step below does)
    live.set_position(64)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        out = live.step_at(x)
    torch.cuda.synchronize()
    assert int(live.pos_t.item()) == 64, "recording a step does not run it"
    for k in range(3):
        live.replay(graph)
        torch.cuda.synchronize()
        twin.set_position(64 + k)
        want = twin.step(x)
        torch.cuda.synchronize()
        assert int(live.pos_t.item()) == 65 + k
        assert torch.equal(out, want), f"replay {k}"
        for i in range(SMALL["layers"]):
            assert torch.equal(live.kt[i][..., 64 + k], twin.kt[i][..., 64 + k])
            assert torch.equal(live.vc[i][:, :, 64 + k], twin.vc[i][:, :, 64 + k])


def test_steps_past_the_cache_are_refused() -> None:
    """`step_at` and `replay` keep a host mirror of the device position and
    refuse a step at a position the cache does not hold."""
    from linnet_amd.errors import LinnetError

    x = (torch.randn(1, SMALL["hidden"], generator=torch.Generator().manual_seed(4)) * 0.5).to(torch.bfloat16).to(DEV)
    model = Int4Llama(torch, kernels, DEV, batch=1, seed=3, spare=0, **SMALL)
    model.set_position(model.cap - 2)
    model.step_at(x)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        model.step_at(x)
    assert model.device_pos == model.cap - 1, "recording a step does not move the mirror"
    model.replay(graph)
    torch.cuda.synchronize()
    assert model.device_pos == model.cap and int(model.pos_t.item()) == model.cap
    with pytest.raises(LinnetError, match="cache holds"):
        model.replay(graph)
    with pytest.raises(LinnetError, match="cache holds"):
        model.step_at(x)
    del model, graph


def test_device_position_outside_the_cache_writes_nothing() -> None:
    from linnet_amd.torch import decode

    g = torch.Generator(device=DEV).manual_seed(2)
    rows, heads, kvh, hd, cap = 2, 8, 2, 64, 16
    q = torch.randn(rows, heads * hd, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(rows, kvh * hd, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(rows, kvh * hd, generator=g, device=DEV).to(torch.bfloat16)
    kt = torch.randn(rows, kvh, hd, cap, generator=g, device=DEV).to(torch.bfloat16)
    vc = torch.randn(rows, kvh, cap, hd, generator=g, device=DEV).to(torch.bfloat16)
    cos, sin = decode.rope_tables(hd, cap, 500000.0, DEV)
    kt0, vc0 = kt.clone(), vc.clone()
    for bad in (cap, -1):
        out = decode.decode_attention(q, k, v, cos, sin, kt, vc, torch.tensor([bad], dtype=torch.int32, device=DEV))
        torch.cuda.synchronize()
        assert torch.equal(kt, kt0) and torch.equal(vc, vc0)
        assert bool((out == 0).all())
    # In range, the device position gives the host position's result.
    pos = 11
    want_kt, want_vc = kt.clone(), vc.clone()
    want = decode.decode_attention(q, k, v, cos[pos], sin[pos], want_kt, want_vc, pos)
    got = decode.decode_attention(q, k, v, cos, sin, kt, vc, torch.tensor([pos], dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    assert torch.equal(got, want) and torch.equal(kt, want_kt) and torch.equal(vc, want_vc)


def test_prefill_matches_token_by_token_reference_steps() -> None:
    """A 64-token prompt through `prefill` (the joined int4 projections at 64 rows,
    causal attention over the prompt) against the same tokens fed one at a time
    through the torch-glue step whose linears multiply the exactly dequantized f32
    weight, at positions 0..63 of an identical model: the last token's logits and
    every layer's k / v cache columns 0..63 agree within 3e-2 of their largest
    value (two chained layers of bf16 intermediates), and the next step starts at
    position 64."""
    prompt = (torch.randn(64, SMALL["hidden"], generator=torch.Generator().manual_seed(9)) * 0.5).to(torch.bfloat16).to(DEV)
    model = Int4Llama(torch, kernels, DEV, batch=1, seed=4, **SMALL)
    ref = Int4Llama(torch, kernels, DEV, batch=1, seed=4, fused=False, **SMALL)
    ref.linear = _exact_linear
    got = model.prefill(prompt).float()
    for t in range(64):
        ref.set_position(t)
        want = ref.step(prompt[t : t + 1]).float()
    torch.cuda.synchronize()
    assert model.pos == 64 and int(model.pos_t.item()) == 64
    rel, agree = _compare("prefill vs token-by-token reference", got, want)
    assert rel <= 3e-2
    for i in range(SMALL["layers"]):
        for name, a, b in (("k", model.kt[i][..., :64], ref.kt[i][..., :64]), ("v", model.vc[i][:, :, :64], ref.vc[i][:, :, :64])):
            err = (a.float() - b.float()).abs().max().item()
            print(f"layer {i} {name} cache max abs err {err:.3e} (max |{name}| {b.float().abs().max().item():.3e})")
            assert err <= 3e-2 * b.float().abs().max().item()


def _prompt_layer_reference(model: Int4Llama, i: int, x: torch.Tensor, linear) -> tuple[torch.Tensor, torch.Tensor]:
    """Layer i of a prompt as torch ops on the residual x [P, hidden] (bf16): RMSNorm,
    q / k / v apart through `linear`, the rotary embedding in f32 (angles p * theta^(-2j/hd)
    computed here), causal grouped-query attention in f32 with each kv head repeated
    over its query heads, o, the residual add, RMSNorm, SiLU(gate) * up, down.
    Writes no cache. Returns (attention output, MLP output)."""
    p, prompt, hd = model.layers[i], x.shape[0], model.hd
    inv = 1.0 / (500000.0 ** (torch.arange(0, hd, 2, device=DEV, dtype=torch.float32) / hd))
    ang = torch.arange(prompt, device=DEV, dtype=torch.float32)[:, None, None] * inv
    cos, sin = torch.cos(ang), torch.sin(ang)

    def rope(t):
        a, b = t[..., : hd // 2], t[..., hd // 2 :]
        return torch.cat([a * cos - b * sin, b * cos + a * sin], dim=-1)

    h = model._rms(x, p["n1"])
    q = rope(linear(h, p["q"]).float().view(prompt, model.heads, hd)).to(torch.bfloat16).float()
    k = rope(linear(h, p["k"]).float().view(prompt, model.kv_heads, hd)).to(torch.bfloat16).float()
    v = linear(h, p["v"]).float().view(prompt, model.kv_heads, hd)
    grp = model.heads // model.kv_heads
    qh = q.transpose(0, 1).contiguous()
    kh = k.transpose(0, 1).repeat_interleave(grp, dim=0).contiguous()
    vh = v.transpose(0, 1).repeat_interleave(grp, dim=0).contiguous()
    scores = torch.matmul(qh, kh.transpose(1, 2).contiguous()) * hd ** -0.5  # [heads, P, P]
    mask = torch.ones(prompt, prompt, dtype=torch.bool, device=DEV).triu(1)
    att = torch.matmul(torch.softmax(scores.masked_fill(mask, float("-inf")), dim=-1), vh)
    o = linear(att.transpose(0, 1).reshape(prompt, -1).to(torch.bfloat16), p["o"])
    h = model._rms(x + o, p["n2"])
    a = torch.nn.functional.silu(linear(h, p["gate"]).float()) * linear(h, p["up"]).float()
    return o, linear(a.to(torch.bfloat16), p["down"])


def test_full_size_prefill_matches_the_reference_layer_by_layer() -> None:
    """Config 5's 1024-token prompt, layer by layer: each layer of `prefill` (the
    joined int4 projections on the tiled GEMM at 1024 rows, PyTorch's fused
    causal attention) takes the same residual input as the torch-op prompt layer
    whose linears multiply the exactly dequantized f32 weight, and both branch
    outputs agree within 1e-2 of their largest value. Then the same prompt fed
    token by token through 1024 replays of the captured fused decode step
    (`step_at`) writes layer 0's k / v cache columns 0..1023 within 1e-2 of their
    largest value of what prefill wrote; the last logits after 32 chained random
    layers are compared and reported (not bounded: chaotic, as for the step)."""
    model = Int4Llama(torch, kernels, DEV, batch=1, seed=11)
    prompt = (torch.randn(1024, 4096, generator=torch.Generator().manual_seed(3)) * 0.5).to(torch.bfloat16).to(DEV)
    x, worst = prompt.clone(), {"attn": 0.0, "mlp": 0.0}
    for i in range(len(model.layers)):
        start = x.clone()
        o, mlp = model.prefill_layer(i, x, None)
        want_o, want_mlp = _prompt_layer_reference(model, i, start, _exact_linear)
        for name, got, want in (("attn", o, want_o), ("mlp", mlp, want_mlp)):
            rel = (got.float() - want.float()).abs().max().item() / want.float().abs().max().item()
            worst[name] = max(worst[name], rel)
            assert rel <= 1e-2, (i, name, rel)
        x += mlp
    print(f"attention: {'fused' if model._flash else 'f32 math'}; branch error rel to its max, worst layer: "
          f"attn {worst['attn']:.3e}, mlp {worst['mlp']:.3e}", flush=True)
    got = model.prefill(prompt).float()
    assert model.pos == 1024 and torch.isfinite(got).all()
    kt0, vc0 = model.kt[0][..., :1024].clone(), model.vc[0][:, :, :1024].clone()
    model.set_position(0)
    xin = prompt[:1].clone()
    model.step_at(xin)
    model.set_position(0)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = model.step_at(xin)
    print("1024 decode steps", flush=True)
    for t in range(1024):
        xin.copy_(prompt[t : t + 1])
        graph.replay()
    torch.cuda.synchronize()
    assert int(model.pos_t.item()) == 1024
    for name, a, b in (("k", kt0, model.kt[0][..., :1024]), ("v", vc0, model.vc[0][:, :, :1024])):
        err = (a.float() - b.float()).abs().max().item()
        print(f"layer 0 {name} cache max abs err {err:.3e} (max |{name}| {b.float().abs().max().item():.3e})")
        assert err <= 1e-2 * b.float().abs().max().item()
    _compare("prefill vs 1024 decode steps, end to end", got, out.float())
    del model, graph


@pytest.mark.parametrize("hd", [64, 128])
def test_prefill_rope_matches_torch_ops(hd: int) -> None:
    """`decode.prefill_rope` (one kernel) against the torch ops it replaces, bit for
    bit: q and k rotated in f32 from the tables and rounded to bf16, head-major
    q / k / v, k transposed into Kt and v into V at positions 0..P-1 (a ragged P of
    100 over a 136-position cache; q, k and v read as column slices of a joined
    output), the rest of the caches untouched."""
    from linnet_amd.torch import decode

    g = torch.Generator(device=DEV).manual_seed(hd)
    heads, kvh, prompt, cap = 8, 2, 100, 136
    joined = torch.randn(prompt, (heads + 2 * kvh) * hd, generator=g, device=DEV).to(torch.bfloat16)
    q, k, v = joined[:, : heads * hd], joined[:, heads * hd : (heads + kvh) * hd], joined[:, (heads + kvh) * hd :]
    cos, sin = decode.rope_tables(hd, cap, 500000.0, DEV)
    kt = torch.randn(kvh, hd, cap, generator=g, device=DEV).to(torch.bfloat16)
    vc = torch.randn(kvh, cap, hd, generator=g, device=DEV).to(torch.bfloat16)
    kt0, vc0 = kt.clone(), vc.clone()
    qh, kh, vh = decode.prefill_rope(q, k, v, cos, sin, kt, vc)
    c, sn = cos[:prompt, None, :], sin[:prompt, None, :]

    def rope(t):
        t = t.float()
        a, b = t[..., : hd // 2], t[..., hd // 2 :]
        return torch.cat([a * c - b * sn, b * c + a * sn], dim=-1).to(torch.bfloat16)

    want_q = rope(q.reshape(prompt, heads, hd))
    want_k = rope(k.reshape(prompt, kvh, hd))
    want_v = v.reshape(prompt, kvh, hd)
    assert torch.equal(qh[0], want_q.transpose(0, 1))
    assert torch.equal(kh[0], want_k.transpose(0, 1))
    assert torch.equal(vh[0], want_v.transpose(0, 1))
    assert torch.equal(kt[:, :, :prompt], want_k.permute(1, 2, 0)) and torch.equal(kt[:, :, prompt:], kt0[:, :, prompt:])
    assert torch.equal(vc[:, :prompt], want_v.transpose(0, 1)) and torch.equal(vc[:, prompt:], vc0[:, prompt:])


def test_decode_kernels_match_torch_ops() -> None:
    """Each decode kernel against the torch ops it replaces (f32 math, bf16 in and out)."""
    from linnet_amd.torch import decode

    g = torch.Generator().manual_seed(5)
    # hidden: two, four and seven 16-byte chunks a thread (4096, 8192, 14336), a
    # partial third (5120), and the element-wise kernel (1000, not a multiple of 8)
    for hidden in (4096, 8192, 14336, 5120, 1000):
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
                                           (2, 8, 1, 128, 132, 130), (3, 6, 2, 64, 100, 64), (1, 4, 4, 64, 68, 3),
                                           (32, 32, 8, 128, 1088, 1000), (32, 32, 8, 128, 1088, 512),
                                           (48, 16, 2, 128, 1088, 700), (24, 16, 4, 64, 1028, 1027)):
        _attention_case(decode, g, rows, heads, kvh, hd, cap, pos)


def _attention_case(decode, g, rows: int, heads: int, kvh: int, hd: int, cap: int, pos: int) -> None:
    """One attention step against torch (bf16 caches, f32 math): group sizes 4, 8,
    3 and 1 (the LDS arrays sized 4, 8, 4, 1), head sizes 128 and 64, chunks from
    1 to 32 (the merge's eight-at-a-time loop and its tail), and batches of 24 to
    48 rows (up to 4352 workgroups)."""
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


def test_decode_attention_copies_a_row_broadcast_over_rows() -> None:
    """q, k, v expanded from one row over two (row stride 0) are read as two equal
    rows, not as packed rows past the one that exists."""
    from linnet_amd.torch import decode

    g = torch.Generator().manual_seed(8)
    heads, kvh, hd, cap, pos = 8, 2, 128, 68, 40
    q1 = torch.randn(1, heads * hd, generator=g).to(torch.bfloat16).to(DEV)
    k1 = torch.randn(1, kvh * hd, generator=g).to(torch.bfloat16).to(DEV)
    v1 = torch.randn(1, kvh * hd, generator=g).to(torch.bfloat16).to(DEV)
    kt1 = torch.randn(1, kvh, hd, cap, generator=g).to(torch.bfloat16).to(DEV)
    vc1 = torch.randn(1, kvh, cap, hd, generator=g).to(torch.bfloat16).to(DEV)
    ang = pos / (500000.0 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))
    cos, sin = torch.cos(ang).to(DEV), torch.sin(ang).to(DEV)
    kt2, vc2 = kt1.expand(2, -1, -1, -1).contiguous(), vc1.expand(2, -1, -1, -1).contiguous()
    got = decode.decode_attention(q1.expand(2, -1), k1.expand(2, -1), v1.expand(2, -1), cos, sin, kt2, vc2, pos)
    one = decode.decode_attention(q1, k1, v1, cos, sin, kt1, vc1, pos)
    assert torch.equal(got[0], one[0]) and torch.equal(got[1], one[0])
