"""Decode-step glue of the int4 Llama-shaped workload, bf16:
the ops a decoder layer runs between its quantized linear layers, as three HIP
kernels (`csrc/decode.hip`) instead of ~40 small framework ops a layer. The
reference gets these from its generated module; they are not part of its
quantized-linear path. Every call enqueues on the current stream and returns.
"""

from __future__ import annotations

import torch

from .. import _lib
from ..errors import LinnetError
from .kernels import SplitParts, XTiles, _on_gpu, _ptr, _stream


def _bf16(what: str, *tensors: torch.Tensor) -> None:
    for t in tensors:
        if t.dtype != torch.bfloat16 or not t.is_contiguous():
            raise LinnetError(f"{what}: takes contiguous bf16 tensors, got {t.dtype}")


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5, delta: torch.Tensor | SplitParts | None = None,
            tiles: bool = False) -> torch.Tensor | XTiles:
    """`h = x * rsqrt(mean(x^2) + eps) * weight` per row of x [rows, hidden]; with
    `delta`, first `x += delta` in place (rounded to bf16), as the residual add
    before a norm. weight: f32 [hidden]. `tiles`: h is returned as x tiles (for
    `int4_linear_tiles`; hidden % 256 == 0), the same bits. `delta` may be a split
    product's partial sums (`int4_linear_tiles_parts`): they are added here, in
    chunk order and rounded once, as the product's own reduction would."""
    parts = delta if isinstance(delta, SplitParts) else None
    if parts is not None:
        delta = None
    device = _on_gpu("rmsnorm", x, weight, delta, None if parts is None else parts.data)
    _bf16("rmsnorm", x, *(() if delta is None else (delta,)))
    if weight.dtype != torch.float32 or weight.numel() != x.shape[-1]:
        raise LinnetError("rmsnorm: weight is f32 [hidden]")
    weight = weight.contiguous()  # a strided view (a column of stacked weights) is read packed
    if delta is not None and delta.shape != x.shape:
        raise LinnetError("rmsnorm: delta has x's shape")
    rows = x.numel() // x.shape[-1]
    if parts is not None:
        if parts.data.dim() != 3 or tuple(parts.data.shape[1:]) != (rows, x.shape[-1]) or not parts.data.is_contiguous():
            raise LinnetError("rmsnorm: split parts are a contiguous f32 [splits, rows, hidden]")
        out = XTiles.empty(rows, x.shape[-1], x.dtype, device) if tiles else torch.empty_like(x)
        with torch.cuda.device(device):
            _lib.call("lnq_rmsnorm_parts", _ptr(x), _ptr(parts.data), parts.data.shape[0], _ptr(weight),
                      _ptr(out.data if tiles else out), int(tiles), rows, x.shape[-1], float(eps), _stream(device))
        return out
    if tiles:
        xt = XTiles.empty(rows, x.shape[-1], x.dtype, device)
        with torch.cuda.device(device):
            _lib.call("lnq_rmsnorm_tiles", _ptr(x), _ptr(delta), _ptr(weight), _ptr(xt.data), rows, x.shape[-1],
                      float(eps), _stream(device))
        return xt
    h = torch.empty_like(x)
    with torch.cuda.device(device):
        _lib.call("lnq_rmsnorm", _ptr(x), _ptr(delta), _ptr(weight), _ptr(h), rows, x.shape[-1],
                  float(eps), _stream(device))
    return h


def prefill_rope(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                 kt_cache: torch.Tensor, v_cache: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """A prompt's rotary embedding and cache writes (`lnq_prefill_rope`): q [P,
    heads*hd], k and v [P, kv_heads*hd] (bf16; column slices of a joined q|k|v
    output are read in place); `cos`, `sin` f32 [cap, hd/2] (`rope_tables`);
    `kt_cache` [kv_heads, hd, cap] and `v_cache` [kv_heads, cap, hd] bf16 (one
    sequence's caches) receive positions 0..P-1. Returns q, k and v head-major,
    [1, heads, P, hd] and [1, kv_heads, P, hd], with q and k rotated and rounded
    to bf16."""
    device = _on_gpu("prefill_rope", q, k, v, cos, sin, kt_cache, v_cache)
    _bf16("prefill_rope", kt_cache, v_cache)
    if any(t.dtype != torch.bfloat16 for t in (q, k, v)):
        raise LinnetError("prefill_rope: q, k and v are bf16")
    if q.dim() != 2 or k.shape != v.shape or k.dim() != 2 or q.shape[0] != k.shape[0]:
        raise LinnetError("prefill_rope: q [P, heads*hd], k and v [P, kv_heads*hd]")
    kvh, hd, cap = kt_cache.shape
    prompt = q.shape[0]
    if tuple(v_cache.shape) != (kvh, cap, hd) or k.shape[1] != kvh * hd or q.shape[1] % hd != 0:
        raise LinnetError("prefill_rope: caches [kv_heads, hd, cap] and [kv_heads, cap, hd] matching k")
    if tuple(cos.shape) != (cap, hd // 2) or cos.shape != sin.shape or cos.dtype != torch.float32:
        raise LinnetError(f"prefill_rope: cos and sin are f32 [{cap}, {hd // 2}]")
    if not (kt_cache.is_contiguous() and v_cache.is_contiguous() and cos.is_contiguous() and sin.is_contiguous()):
        raise LinnetError("prefill_rope: contiguous caches and tables")
    stride = q.stride(0)
    if q.stride(1) != 1 or k.stride(1) != 1 or v.stride(1) != 1 or k.stride(0) != stride or v.stride(0) != stride:
        raise LinnetError("prefill_rope: q, k and v rows share one stride, each row contiguous")
    heads = q.shape[1] // hd
    q_out = torch.empty(1, heads, prompt, hd, dtype=q.dtype, device=device)
    k_out = torch.empty(1, kvh, prompt, hd, dtype=q.dtype, device=device)
    v_out = torch.empty(1, kvh, prompt, hd, dtype=q.dtype, device=device)
    with torch.cuda.device(device):
        _lib.call("lnq_prefill_rope", _ptr(q), _ptr(k), _ptr(v), stride, _ptr(cos), _ptr(sin), _ptr(q_out),
                  _ptr(k_out), _ptr(v_out), _ptr(kt_cache), _ptr(v_cache), prompt, heads, kvh, hd, cap, _stream(device))
    return q_out, k_out, v_out


def rope_tables(head_dim: int, positions: int, theta: float = 500000.0,
                device: torch.device | str = "cuda") -> tuple[torch.Tensor, torch.Tensor]:
    """`(cos, sin)` f32 [positions, head_dim/2]: row p holds cos / sin of p times the
    rotary frequencies theta^(-2i/head_dim) (no frequency scaling), the values
    `decode_attention` takes at one position, for every position of a cache."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device, dtype=torch.float32) / head_dim))
    ang = torch.arange(positions, device=device, dtype=torch.float32)[:, None] * inv[None, :]
    return torch.cos(ang).contiguous(), torch.sin(ang).contiguous()


def decode_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                     kt_cache: torch.Tensor, v_cache: torch.Tensor, pos: int | torch.Tensor,
                     tiles: bool = False) -> torch.Tensor | XTiles:
    """One decode step of grouped-query attention for q [rows, heads*hd], k, v
    [rows, kv_heads*hd] (bf16): rotary embedding (cos, sin f32 [hd/2] at `pos`) of
    q and k, k and v written (rounded) into the bf16 caches at `pos` (K transposed:
    kt_cache [rows, kv_heads, hd, cap]; v_cache [rows, kv_heads, cap, hd]), then
    softmax(q K^T / sqrt(hd)) V over positions 0..pos. Returns [rows, heads*hd] bf16.

    `pos` may be a one-element int32 tensor on the device instead: the kernels then
    read it there (a graph replaying the step follows the position as the device
    advances it), and cos / sin are the whole tables [cap, hd/2] of `rope_tables`.
    `tiles`: the output as x tiles (heads*hd % 256 == 0), the same bits."""
    device = _on_gpu("decode_attention", q, k, v, cos, sin, kt_cache, v_cache)
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise LinnetError("decode_attention: q, k and v are bf16")
    rows, kvh, hd, cap = kt_cache.shape
    if tuple(v_cache.shape) != (rows, kvh, cap, hd) or kt_cache.dtype != torch.bfloat16 or v_cache.dtype != torch.bfloat16:
        raise LinnetError("decode_attention: caches are bf16 [rows, kv_heads, hd, cap] and [rows, kv_heads, cap, hd]")
    if not (kt_cache.is_contiguous() and v_cache.is_contiguous() and cos.is_contiguous() and sin.is_contiguous()):
        raise LinnetError("decode_attention: contiguous caches and tables")
    heads = q.shape[-1] // hd
    if q.shape != (rows, heads * hd) or k.shape != (rows, kvh * hd) or v.shape != k.shape:
        raise LinnetError("decode_attention: q [rows, heads*hd], k and v [rows, kv_heads*hd]")
    # q, k and v may be column slices of one joined projection (rows strided, each
    # row contiguous; k and v with the same row stride). A row broadcast over rows
    # (stride 0, or any stride shorter than a row) is copied out first.
    short = rows > 1 and (q.stride(0) < q.shape[1] or k.stride(0) < k.shape[1] or v.stride(0) < v.shape[1])
    if short or q.stride(-1) != 1 or k.stride(-1) != 1 or v.stride(-1) != 1 or k.stride(0) != v.stride(0):
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    if isinstance(pos, torch.Tensor):
        if pos.dtype != torch.int32 or pos.numel() != 1 or pos.device != device:
            raise LinnetError("decode_attention: a device position is one int32 on q's device")
        if tuple(cos.shape) != (cap, hd // 2) or tuple(sin.shape) != (cap, hd // 2) or cos.dtype != torch.float32 \
                or sin.dtype != torch.float32:
            raise LinnetError(f"decode_attention: with a device position cos and sin are f32 [{cap}, {hd // 2}]")
        floats = _lib.load().lnq_decode_attention_workspace(rows, kvh, hd, cap - 1)
        work = torch.empty(max(floats, 1), dtype=torch.float32, device=device)
        if tiles:
            xt = XTiles.empty(rows, heads * hd, q.dtype, device)
            with torch.cuda.device(device):
                _lib.call("lnq_decode_attention_tiles", _ptr(q), _ptr(k), _ptr(v), _ptr(cos), _ptr(sin),
                          _ptr(kt_cache), _ptr(v_cache), _ptr(xt.data), _ptr(work), work.numel(), rows, heads, kvh,
                          hd, cap, 0, _ptr(pos), q.stride(0), k.stride(0), _stream(device))
            return xt
        out = torch.empty_like(q)
        with torch.cuda.device(device):
            _lib.call("lnq_decode_attention_at", _ptr(q), _ptr(k), _ptr(v), _ptr(cos), _ptr(sin), _ptr(kt_cache),
                      _ptr(v_cache), _ptr(out), _ptr(work), work.numel(), rows, heads, kvh, hd, cap, _ptr(pos),
                      q.stride(0), k.stride(0), _stream(device))
        return out
    if cos.numel() != hd // 2 or sin.numel() != hd // 2 or cos.dtype != torch.float32 or sin.dtype != torch.float32:
        raise LinnetError("decode_attention: cos and sin are f32 [hd/2]")
    floats = _lib.load().lnq_decode_attention_workspace(rows, kvh, hd, pos)
    work = torch.empty(max(floats, 1), dtype=torch.float32, device=device)
    if tiles:
        xt = XTiles.empty(rows, heads * hd, q.dtype, device)
        with torch.cuda.device(device):
            _lib.call("lnq_decode_attention_tiles", _ptr(q), _ptr(k), _ptr(v), _ptr(cos), _ptr(sin), _ptr(kt_cache),
                      _ptr(v_cache), _ptr(xt.data), _ptr(work), work.numel(), rows, heads, kvh, hd, cap, pos, None,
                      q.stride(0), k.stride(0), _stream(device))
        return xt
    out = torch.empty_like(q)
    with torch.cuda.device(device):
        _lib.call("lnq_decode_attention", _ptr(q), _ptr(k), _ptr(v), _ptr(cos), _ptr(sin), _ptr(kt_cache),
                  _ptr(v_cache), _ptr(out), _ptr(work), work.numel(), rows, heads, kvh, hd, cap, pos, q.stride(0),
                  k.stride(0), _stream(device))
    return out


def silu_mul(g: torch.Tensor, u: torch.Tensor, tiles: bool = False) -> torch.Tensor | XTiles:
    """`silu(g) * u` elementwise in f32, rounded once to bf16. g and u may be 2-D
    column slices (rows strided, each row contiguous), e.g. the two halves of a
    joined gate|up projection's output; the result is contiguous. `tiles`: the
    result as x tiles (2-D, width % 256 == 0), the same bits."""
    device = _on_gpu("silu_mul", g, u)
    if g.dtype != torch.bfloat16 or u.dtype != torch.bfloat16:
        raise LinnetError("silu_mul: g and u are bf16")
    if g.shape != u.shape:
        raise LinnetError("silu_mul: g and u have one shape")
    if tiles:
        if g.dim() != 2 or g.stride(1) != 1 or u.stride(1) != 1:
            g, u = g.contiguous(), u.contiguous()
        xt = XTiles.empty(g.shape[0], g.shape[1], g.dtype, device)
        with torch.cuda.device(device):
            _lib.call("lnq_silu_mul_tiles", _ptr(g), _ptr(u), _ptr(xt.data), g.shape[0], g.shape[1], g.stride(0),
                      u.stride(0), _stream(device))
        return xt
    if g.is_contiguous() and u.is_contiguous():
        a = torch.empty_like(g)
        with torch.cuda.device(device):
            _lib.call("lnq_silu_mul", _ptr(g), _ptr(u), _ptr(a), g.numel(), _stream(device))
        return a
    if g.dim() != 2 or g.stride(1) != 1 or u.stride(1) != 1:
        g, u = g.contiguous(), u.contiguous()
    rows, width = g.shape
    a = torch.empty(rows, width, dtype=g.dtype, device=device)
    with torch.cuda.device(device):
        _lib.call("lnq_silu_mul_rows", _ptr(g), _ptr(u), _ptr(a), rows, width, g.stride(0), u.stride(0),
                  _stream(device))
    return a
