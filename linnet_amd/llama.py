"""The int4 Llama-3.1-8B-shaped decoder of BASELINE config 5: every linear layer an
`Int4GroupLinear` (group 128, bf16 scales, u8 zeros) run by this package's HIP
kernels, the glue between them by the decode kernels of `torch/decode.py`.

It stands for the reference's `examples/01-llama` card with its `Linear` layers
swapped for `Int4GroupLinear<..., 128, bf16>` (`examples/01-llama/src/lib.linnet:79-82`,
`stdlib/nn/mlp.linnet:16-24`), run by the generated module's decode step
(`python/linnet/src/linnet/torch/compiled.py:430-503`). The weights are random
(N(0, 0.02), quantized on the GPU): there is no checkpoint to load.
"""

from __future__ import annotations


class Int4Llama:
    """A Llama-3.1-8B-shaped decoder whose linear layers are
    all int4 g128 through this package's `int4_linear` (the `Int4GroupLinear`
    swap of the reference's `examples/01-llama` card): random-init weights
    (N(0, 0.02)) quantized on the GPU, RMSNorm, rotary embedding (theta 500000,
    no frequency scaling), grouped-query attention over a KV cache of `ctx`
    random entries, SiLU MLP and an int4 lm_head. Attention runs in f32 on
    contiguous operands (K cache stored transposed). `step(x)` is one decode
    step of `batch` tokens at position `ctx`; `linear` may be swapped for a
    reference (dequantized weight and `F.linear`). `fused` runs the glue between
    the linear layers as this package's decode kernels (`torch/decode.py`: norm
    with the residual add, attention with the rotary embedding and cache write,
    SiLU x up); otherwise as torch ops (the reference for the tests)."""

    def __init__(self, torch, kernels, dev, layers=32, hidden=4096, heads=32, kv_heads=8, ffn=14336,
                 vocab=128256, ctx=1024, batch=1, seed=0, fused=True):
        self.torch, self.kernels, self.fused = torch, kernels, fused
        self.hidden, self.heads, self.kv_heads, self.hd = hidden, heads, kv_heads, hidden // heads
        g = torch.Generator(device=dev).manual_seed(seed)

        def lin(n, k):
            w = torch.randn(n, k, generator=g, device=dev) * 0.02
            packed, scale, zero = kernels.quantize_int4(w, 128)
            return packed, scale.to(torch.bfloat16), zero

        kvd = kv_heads * self.hd
        self.layers = [dict(q=lin(hidden, hidden), k=lin(kvd, hidden), v=lin(kvd, hidden), o=lin(hidden, hidden),
                            gate=lin(ffn, hidden), up=lin(ffn, hidden), down=lin(hidden, ffn),
                            n1=1 + 0.1 * torch.randn(hidden, generator=g, device=dev),
                            n2=1 + 0.1 * torch.randn(hidden, generator=g, device=dev)) for _ in range(layers)]
        # The decode kernels' step runs q, k and v as one joined projection (their
        # int4 rows stacked: one launch, one weight stream) and reads q, k and v as
        # column slices of its output; gate and up likewise.
        for p in self.layers:
            p["qkv"] = tuple(torch.cat([p["q"][i], p["k"][i], p["v"][i]], dim=0) for i in range(3))
            p["gate_up"] = tuple(torch.cat([p["gate"][i], p["up"][i]], dim=0) for i in range(3))
        self.norm = 1 + 0.1 * torch.randn(hidden, generator=g, device=dev)
        self.head = lin(vocab, hidden)
        # KV caches, bf16 (the model's dtype), capacity ctx + 1 rounded up to 4: Kt
        # [batch, kv_heads, hd, cap] (transposed), V [batch, kv_heads, cap, hd].
        # Position ctx is written by the step.
        cap = (ctx + 4) // 4 * 4
        self.kt = [torch.randn(batch, kv_heads, self.hd, cap, generator=g, device=dev).to(torch.bfloat16)
                   for _ in range(layers)]
        self.vc = [torch.randn(batch, kv_heads, cap, self.hd, generator=g, device=dev).to(torch.bfloat16)
                   for _ in range(layers)]
        self.pos = ctx
        inv = 1.0 / (500000.0 ** (torch.arange(0, self.hd, 2, device=dev, dtype=torch.float32) / self.hd))
        ang = ctx * inv
        self.cos, self.sin = torch.cos(ang), torch.sin(ang)
        self.linear = lambda x, w: kernels.int4_linear(x, *w)

    def _rms(self, x, w):
        torch = self.torch
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-5) * w).to(torch.bfloat16)

    def _rope(self, t):  # [B, H, hd] f32
        half = self.hd // 2
        a, b = t[..., :half], t[..., half:]
        return self.torch.cat([a * self.cos - b * self.sin, b * self.cos + a * self.sin], dim=-1)

    def layer_torch(self, i, x, linear=None, parts=None):
        """Layer i as torch ops on the residual stream x [batch, hidden] (bf16):
        returns the next residual. `linear` (default `self.linear`) multiplies;
        `parts`, if a dict, receives the attention and MLP branch outputs."""
        torch = self.torch
        linear = linear or self.linear
        p = self.layers[i]
        bsz = x.shape[0]
        grp = self.heads // self.kv_heads
        h = self._rms(x, p["n1"])
        q = self._rope(linear(h, p["q"]).float().view(bsz, self.heads, self.hd))
        k = self._rope(linear(h, p["k"]).float().view(bsz, self.kv_heads, self.hd))
        v = linear(h, p["v"]).float().view(bsz, self.kv_heads, self.hd)
        self.kt[i][:, :, :, self.pos] = k
        self.vc[i][:, :, self.pos, :] = v
        qg = q.view(bsz, self.kv_heads, grp, self.hd)
        live = self.pos + 1
        kt = self.kt[i][..., :live].float()
        scores = torch.matmul(qg, kt) * (self.hd ** -0.5)  # [B, kvh, grp, ctx + 1]
        att = torch.matmul(torch.softmax(scores, dim=-1), self.vc[i][:, :, :live].float())  # [B, kvh, grp, hd]
        o = linear(att.reshape(bsz, self.hidden).to(torch.bfloat16), p["o"])
        x = x + o
        h = self._rms(x, p["n2"])
        a = torch.nn.functional.silu(linear(h, p["gate"]).float()) * linear(h, p["up"]).float()
        mlp = linear(a.to(torch.bfloat16), p["down"])
        if parts is not None:
            parts["attn"], parts["mlp"] = o, mlp
        return x + mlp

    def head_torch(self, x, linear=None):
        return (linear or self.linear)(self._rms(x, self.norm), self.head)

    def layer_fused(self, i, x, delta, parts=None):
        """Layer i on the decode kernels and the joined int4 projections. `x` is the
        residual stream, updated in place; `delta` the previous layer's MLP output,
        not yet added (the norm adds it). Returns this layer's MLP output; `parts`,
        if a dict, receives the attention branch's output too."""
        from linnet_amd.torch import decode

        p = self.layers[i]
        h = decode.rmsnorm(x, p["n1"], 1e-5, delta)
        qkv = self.linear(h, p["qkv"])
        kvd = self.kv_heads * self.hd
        q, k, v = qkv[:, : self.hidden], qkv[:, self.hidden : self.hidden + kvd], qkv[:, self.hidden + kvd :]
        att = decode.decode_attention(q, k, v, self.cos, self.sin, self.kt[i], self.vc[i], self.pos)
        o = self.linear(att, p["o"])
        if parts is not None:
            parts["attn"] = o
        h = decode.rmsnorm(x, p["n2"], 1e-5, o)
        gu = self.linear(h, p["gate_up"])
        ffn = gu.shape[1] // 2
        return self.linear(decode.silu_mul(gu[:, :ffn], gu[:, ffn:]), p["down"])

    def head_fused(self, x, delta):
        from linnet_amd.torch import decode

        return self.linear(decode.rmsnorm(x, self.norm, 1e-5, delta), self.head)

    def step(self, x):
        if self.fused:
            x = x.clone()  # the residual stream is updated in place
            delta = None
            for i in range(len(self.layers)):
                delta = self.layer_fused(i, x, delta)
            return self.head_fused(x, delta)
        for i in range(len(self.layers)):
            x = self.layer_torch(i, x)
        return self.head_torch(x)
