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
    SiLU x up); otherwise as torch ops (the reference for the tests). With
    `fused` and `fold` (the default), a one-token step folds that glue into the
    linear layers' own kernels (`layer_folded`)."""

    def __init__(self, torch, kernels, dev, layers=32, hidden=4096, heads=32, kv_heads=8, ffn=14336,
                 vocab=128256, ctx=1024, batch=1, seed=0, fused=True, spare=0, tiles=True):
        self.torch, self.kernels, self.fused, self.tiles = torch, kernels, fused, tiles
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
        # int4 rows stacked at prepare: one launch, one weight stream) and reads q, k
        # and v as column slices of its output; gate and up likewise.
        from linnet_amd.torch import generated

        for p in self.layers:
            p["qkv"], p["qkv_rows"] = generated._int4_join(p["q"], p["k"], p["v"])
            p["gate_up"], p["gate_up_rows"] = generated._int4_join(p["gate"], p["up"])
        self.norm = 1 + 0.1 * torch.randn(hidden, generator=g, device=dev)
        self.head = lin(vocab, hidden)
        # KV caches, bf16 (the model's dtype), capacity ctx + 1 rounded up to 4: Kt
        # [batch, kv_heads, hd, cap] (transposed), V [batch, kv_heads, cap, hd].
        # Position ctx is written by the step; `spare` more positions stay free for
        # steps past it.
        cap = (ctx + 1 + spare + 3) // 4 * 4
        self.cap = cap
        self.kt = [torch.randn(batch, kv_heads, self.hd, cap, generator=g, device=dev).to(torch.bfloat16)
                   for _ in range(layers)]
        self.vc = [torch.randn(batch, kv_heads, cap, self.hd, generator=g, device=dev).to(torch.bfloat16)
                   for _ in range(layers)]
        self.pos = ctx
        inv = 1.0 / (500000.0 ** (torch.arange(0, self.hd, 2, device=dev, dtype=torch.float32) / self.hd))
        ang = ctx * inv
        self.cos, self.sin = torch.cos(ang), torch.sin(ang)
        # The position in device memory and the rotary tables of every cache
        # position, for steps whose position lives on the device (`step_at`).
        from linnet_amd.torch import decode

        self.pos_t = torch.tensor([ctx], dtype=torch.int32, device=dev)
        # Host mirror of pos_t: advanced by every step_at that runs (eagerly or
        # through `replay`), so that no step runs past the cache.
        self.device_pos = ctx
        self.cos_tab, self.sin_tab = decode.rope_tables(self.hd, cap, 500000.0, dev)
        # x tiles (the glue writes the few-row GEMVs' operand order) for 17..64 rows.
        self.linear = lambda x, w: (kernels.int4_linear_tiles(x, *w) if isinstance(x, kernels.XTiles)
                                    else kernels.int4_linear(x, *w))
        # One-token steps fold the glue into the linear layers (`layer_folded`).
        self.fold = True
        self._flash = None  # whether PyTorch's fused attention ran (None: not tried)

    def set_position(self, pos):
        """Moves the next step to cache position `pos` (host and device copies)."""
        torch = self.torch
        self.pos = pos
        inv = 1.0 / (500000.0 ** (torch.arange(0, self.hd, 2, device=self.pos_t.device, dtype=torch.float32) / self.hd))
        ang = pos * inv
        self.cos, self.sin = torch.cos(ang), torch.sin(ang)
        self.pos_t.fill_(pos)
        self.device_pos = pos

    def _check_room(self):
        if self.device_pos >= self.cap:
            from linnet_amd.errors import LinnetError

            raise LinnetError(f"decode step at cache position {self.device_pos}: the cache holds {self.cap} positions")

    def replay(self, graph):
        """Replays a graph that recorded one `step_at` (which moves the device
        position by one), refusing to run past the cache. A graph replayed
        directly (`graph.replay()`) bypasses this check: the attention kernel then
        reads and writes nothing past the cache, and the logits are wrong."""
        self._check_room()
        graph.replay()
        self.device_pos += 1

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

    def layer_fused(self, i, x, delta, parts=None, device_pos=False, partial=False):
        """Layer i on the decode kernels and the joined int4 projections. `x` is the
        residual stream, updated in place; `delta` the previous layer's MLP output,
        not yet added (the norm adds it). Returns this layer's MLP output; `parts`,
        if a dict, receives the attention branch's output too. `device_pos`: the
        position is read from `pos_t` on the device (with the rotary tables)."""
        from linnet_amd.torch import decode, generated

        p = self.layers[i]
        tiles = self._tiles(x)
        h = decode.rmsnorm(x, p["n1"], 1e-5, delta, tiles=tiles)
        q, k, v = generated._int4_split(self.linear(h, p["qkv"]), p["qkv_rows"])
        if device_pos:
            att = decode.decode_attention(q, k, v, self.cos_tab, self.sin_tab, self.kt[i], self.vc[i], self.pos_t,
                                          tiles=tiles)
        else:
            att = decode.decode_attention(q, k, v, self.cos, self.sin, self.kt[i], self.vc[i], self.pos, tiles=tiles)
        o = self.linear(att, p["o"])
        if parts is not None:
            parts["attn"] = o
        h = decode.rmsnorm(x, p["n2"], 1e-5, o, tiles=tiles)
        g, u = generated._int4_split(self.linear(h, p["gate_up"]), p["gate_up_rows"])
        a = decode.silu_mul(g, u, tiles=tiles)
        if partial and tiles and x.shape[0] <= 32 and a.width > 4096:
            # The split product's K-chunk sums, added by the next norm (`partial`:
            # the caller hands the result on as that norm's delta).
            return self.kernels.int4_linear_tiles_parts(a, *p["down"])
        return self.linear(a, p["down"])

    def _tiles(self, x):
        """Whether the glue hands the projections x tiles: 17..64 rows, where the
        32-row and split GEMVs take them."""
        return self.tiles and 17 <= x.shape[0] <= 64

    def layer_folded(self, i, x, parts=None, device_pos=False):
        """Layer i of a one-token step with the glue folded into the linear layers:
        the RMSNorms into the staging of x of the q|k|v and gate|up GEMVs, SiLU(gate)
        * up into the down projection's, each residual add into the epilogue of the
        o and down GEMVs (the residual row as their bias). Six launches a layer
        (four linears and the attention's two kernels) against nine for
        `layer_fused`, with its numbers up to the bf16 rounding of the normed
        activations (the GEMV stages x * w and scales its sums by the row's norm
        factor). x: the residual stream [1, hidden] with every earlier branch added;
        returns the next one (a new tensor)."""
        from linnet_amd.torch import decode, generated

        kernels, p = self.kernels, self.layers[i]
        qkv = kernels.int4_linear_rmsnorm(x, p["n1"], 1e-5, *p["qkv"])
        q, k, v = generated._int4_split(qkv, p["qkv_rows"])
        if device_pos:
            att = decode.decode_attention(q, k, v, self.cos_tab, self.sin_tab, self.kt[i], self.vc[i], self.pos_t)
        else:
            att = decode.decode_attention(q, k, v, self.cos, self.sin, self.kt[i], self.vc[i], self.pos)
        x = kernels.int4_linear(att, *p["o"], bias=x[0])
        if parts is not None:
            parts["resid"] = x
        g, u = generated._int4_split(kernels.int4_linear_rmsnorm(x, p["n2"], 1e-5, *p["gate_up"]), p["gate_up_rows"])
        return kernels.int4_linear_silu_mul(g, u, *p["down"], bias=x[0])

    def head_folded(self, x):
        return self.kernels.int4_linear_rmsnorm(x, self.norm, 1e-5, *self.head)

    def head_fused(self, x, delta):
        from linnet_amd.torch import decode

        return self.linear(decode.rmsnorm(x, self.norm, 1e-5, delta, tiles=self._tiles(x)), self.head)

    def _attend_prompt(self, qh, kh, vh):
        """Causal grouped-query attention of a prompt, q [1, heads, P, hd], k and v
        [1, kv_heads, P, hd] (bf16, rotated): PyTorch's fused attention (flash on
        this GPU when present), otherwise the same math in f32. Returns [P,
        heads*hd] bf16."""
        torch = self.torch
        fn = torch.nn.functional.scaled_dot_product_attention
        prompt = qh.shape[2]
        if self._flash is not False:
            try:
                from torch.nn.attention import SDPBackend, sdpa_kernel

                with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                    att = fn(qh, kh, vh, is_causal=True, enable_gqa=True)
                self._flash = True
                return att[0].transpose(0, 1).reshape(prompt, -1)
            except RuntimeError:
                self._flash = False
        grp = self.heads // self.kv_heads
        kf = kh.float().repeat_interleave(grp, dim=1)
        vf = vh.float().repeat_interleave(grp, dim=1)
        att = fn(qh.float(), kf, vf, is_causal=True)
        return att[0].transpose(0, 1).reshape(prompt, -1).to(torch.bfloat16)

    def prefill_layer(self, i, x, delta):
        """Layer i of a prompt (batch 1) on the residual stream x [P, hidden] (bf16,
        updated in place; `delta`, the previous layer's MLP output, is added first):
        the joined int4 projections at P rows, the rotary embedding at positions
        0..P-1 from the tables and k and v written into cache positions 0..P-1 (one
        kernel, `decode.prefill_rope`; k rounded to bf16, as the decode step stores
        it), causal attention over the prompt. Returns (attention output, MLP
        output); the latter is not added."""
        from linnet_amd.torch import decode, generated

        p = self.layers[i]
        tiles = self._tiles(x)
        h = decode.rmsnorm(x, p["n1"], 1e-5, delta, tiles=tiles)
        q, k, v = generated._int4_split(self.linear(h, p["qkv"]), p["qkv_rows"])
        qh, kh, vh = decode.prefill_rope(q, k, v, self.cos_tab, self.sin_tab, self.kt[i][0], self.vc[i][0])
        o = self.linear(self._attend_prompt(qh, kh, vh), p["o"])
        h = decode.rmsnorm(x, p["n2"], 1e-5, o)
        g, u = generated._int4_split(self.linear(h, p["gate_up"]), p["gate_up_rows"])
        return o, self.linear(decode.silu_mul(g, u), p["down"])

    def prefill(self, x):
        """The prompt x [P, hidden] (bf16, batch 1) through every layer
        (`prefill_layer`), then the lm_head on the last row only; moves the next
        step to position P. Returns the last row's logits [1, vocab]."""
        if self.kt[0].shape[0] != 1 or x.shape[0] > self.kt[0].shape[-1]:
            raise ValueError("prefill takes one sequence that fits the cache")
        x = x.clone()  # the residual stream is updated in place
        delta = None
        for i in range(len(self.layers)):
            _, delta = self.prefill_layer(i, x, delta)
        logits = self.head_fused(x[-1:].contiguous(), delta[-1:].contiguous())
        self.set_position(x.shape[0])
        return logits

    def _folds(self, x):
        return self.fused and self.fold and x.shape[0] == 1

    def step_at(self, x):
        """One fused decode step at the position held in `pos_t` on the device,
        which it then advances by one (a graph recording this step moves along the
        cache on each replay: replay it with `replay`). Returns the logits.
        Refuses a step past the cache; `pos` (the host-side position of `step`)
        is not moved."""
        torch = self.torch
        capturing = torch.cuda.is_current_stream_capturing()
        if not capturing:
            self._check_room()
        if self._folds(x):
            for i in range(len(self.layers)):
                x = self.layer_folded(i, x, device_pos=True)
            logits = self.head_folded(x)
        else:
            x = x.clone()
            delta = None
            for i in range(len(self.layers)):
                delta = self.layer_fused(i, x, delta, device_pos=True, partial=True)
            logits = self.head_fused(x, delta)
        self.pos_t.add_(1)
        if not capturing:
            self.device_pos += 1
        return logits

    def step(self, x):
        if self._folds(x):
            for i in range(len(self.layers)):
                x = self.layer_folded(i, x)
            return self.head_folded(x)
        if self.fused:
            x = x.clone()  # the residual stream is updated in place
            delta = None
            for i in range(len(self.layers)):
                delta = self.layer_fused(i, x, delta, partial=True)
            return self.head_fused(x, delta)
        for i in range(len(self.layers)):
            x = self.layer_torch(i, x)
        return self.head_torch(x)
