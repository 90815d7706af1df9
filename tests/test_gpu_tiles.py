"""x tiles on the GPU (`lnq_x_tiles`, `lnq_int4_linear_tiles`, `lnq_rmsnorm_tiles`,
`lnq_silu_mul_tiles`): the tiler against the host reordering, and every product and
producer on tiles against the same kernel on row-major x -- bit for bit, since
only the addresses x is loaded from differ. The row-major kernels themselves are
held to the oracle in test_gpu_int4.py and test_gpu_split.py."""

from __future__ import annotations

import pytest
import torch

from linnet_amd.errors import LinnetError
from linnet_amd.llama import Int4Llama
from linnet_amd.torch import decode, generated, kernels

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _layer(out: int, width: int, seed: int, dtype=torch.bfloat16):
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = torch.randn(out, width, generator=g, device=DEV) * 0.02
    packed, scale, zero = kernels.quantize_int4(w, 128)
    return packed, scale.to(dtype), zero


@pytest.mark.parametrize(("rows", "width"), [(1, 256), (17, 4096), (32, 14336), (45, 768), (64, 1024)])
def test_x_tiles_hold_x(rows: int, width: int) -> None:
    print(f"x tiles rows={rows} width={width}", flush=True)
    x = torch.randn(rows, width, device=DEV).to(torch.bfloat16)
    xt = kernels.x_tiles(x)
    assert torch.equal(xt.rows_major(), x)
    chunks = xt.data.view(-1, 32 * width)
    tail = torch.zeros(xt.data.numel() // width - rows, width, dtype=torch.bfloat16, device=DEV)
    full = kernels.XTiles(xt.data, xt.data.numel() // width, width).rows_major()
    assert torch.equal(full[rows:], tail)  # rows of the last chunk past `rows` are zero
    assert chunks.shape[0] == -(-rows // 32)


@pytest.mark.parametrize(
    ("rows", "width", "out", "kernel", "dtype", "with_bias"),
    [
        (32, 4096, 14336, "gemv", torch.bfloat16, False),  # the 32-row GEMV (gate|up-like)
        (24, 4096, 6144, "gemv", torch.bfloat16, True),  # q|k|v-like, 24 rows, the bias
        (56, 4096, 2048, "gemv", torch.float16, False),  # two chunks (32 + 24), f16
        (32, 14336, 4096, "split", torch.bfloat16, True),  # the down projection
        (48, 14336, 1024, "split", torch.bfloat16, False),  # two chunks of the split GEMV
        (32, 4096, 65536, "split", torch.bfloat16, False),  # 128-row blocks, 2 K chunks (lm_head-like)
    ],
)
def test_products_on_tiles_are_the_row_major_bits(rows, width, out, kernel, dtype, with_bias) -> None:
    print(f"tiles product rows={rows} in={width} out={out} {kernel} {dtype} bias={with_bias}", flush=True)
    packed, scale, zero = _layer(out, width, seed=out + rows, dtype=dtype)
    x = torch.randn(rows, width, device=DEV).to(dtype)
    bias = (torch.randn(out, device=DEV) * 0.5).to(dtype) if with_bias else None
    want = torch.cat([kernels.int4_linear(x[c:c + 32], packed, scale, zero, bias, kernel=kernel)
                      for c in range(0, rows, 32)])
    got = kernels.int4_linear_tiles(kernels.x_tiles(x), packed, scale, zero, bias, kernel=kernel)
    assert torch.equal(got, want)
    auto = kernels.int4_linear_tiles(kernels.x_tiles(x), packed, scale, zero, bias)
    assert torch.equal(auto, torch.cat([kernels.int4_linear(x[c:c + 32], packed, scale, zero, bias,
                                                            kernel="split" if width > 4096 else "gemv")
                                        for c in range(0, rows, 32)]))


@pytest.mark.parametrize("rows", [32, 20])
def test_split_parts_add_up_to_the_product_and_feed_the_norm(rows: int) -> None:
    """The split GEMV's partial sums (`int4_linear_tiles_parts`) added in chunk order
    and rounded once are the split product's bits, and RMSNorm taking them as its
    delta gives the bits it gives with that product as delta (row-major and tiles)."""
    print(f"split parts rows={rows}", flush=True)
    packed, scale, zero = _layer(4096, 14336, seed=rows)
    a = torch.randn(rows, 14336, device=DEV).to(torch.bfloat16)
    at = kernels.x_tiles(a)
    parts = kernels.int4_linear_tiles_parts(at, packed, scale, zero)
    assert parts.data.shape == (4, rows, 4096)
    product = kernels.int4_linear_tiles(at, packed, scale, zero)
    assert torch.equal(parts.total(), product)
    x = torch.randn(rows, 4096, device=DEV).to(torch.bfloat16)
    w = 1 + 0.1 * torch.randn(4096, device=DEV)
    for tiles in (False, True):
        x1, x2 = x.clone(), x.clone()
        want = decode.rmsnorm(x1, w, 1e-5, product, tiles=tiles)
        got = decode.rmsnorm(x2, w, 1e-5, parts, tiles=tiles)
        assert torch.equal(x1, x2)
        assert torch.equal(got.rows_major() if tiles else got, want.rows_major() if tiles else want)


def test_tiles_entry_refuses_what_it_does_not_take() -> None:
    packed, scale, zero = _layer(512, 8192, seed=3)
    xt = kernels.x_tiles(torch.randn(32, 8192, device=DEV).to(torch.bfloat16))
    with pytest.raises(LinnetError, match="in <= 4096"):
        kernels.int4_linear_tiles(xt, packed, scale, zero, kernel="gemv")
    with pytest.raises(LinnetError, match="kernel is auto, gemv or split"):
        kernels.int4_linear_tiles(xt, packed, scale, zero, kernel="skinny")
    big = kernels.x_tiles(torch.randn(65, 256, device=DEV).to(torch.bfloat16))
    p2, s2, z2 = _layer(64, 256, seed=4)
    with pytest.raises(LinnetError, match="up to 64 rows"):
        kernels.int4_linear_tiles(big, p2, s2, z2)


def test_glue_writes_the_tiles_of_its_row_major_output() -> None:
    rows, hidden, ffn = 32, 4096, 14336
    x = torch.randn(rows, hidden, device=DEV).to(torch.bfloat16)
    delta = torch.randn(rows, hidden, device=DEV).to(torch.bfloat16)
    w = 1 + 0.1 * torch.randn(hidden, device=DEV)
    x1, x2 = x.clone(), x.clone()
    h = decode.rmsnorm(x1, w, 1e-5, delta)
    ht = decode.rmsnorm(x2, w, 1e-5, delta, tiles=True)
    assert torch.equal(x1, x2)  # the residual add in place, the same bits
    assert torch.equal(ht.rows_major(), h)
    gu = torch.randn(rows, 2 * ffn, device=DEV).to(torch.bfloat16)
    g, u = gu[:, :ffn], gu[:, ffn:]
    assert torch.equal(decode.silu_mul(g, u, tiles=True).rows_major(), decode.silu_mul(g, u))


@pytest.mark.parametrize("device_pos", [False, True])
def test_decode_attention_writes_the_tiles_of_its_output(device_pos: bool) -> None:
    rows, heads, kvh, hd, cap, pos = 32, 32, 8, 128, 260, 200
    g = torch.Generator(device=DEV).manual_seed(7)
    qkv = torch.randn(rows, (heads + 2 * kvh) * hd, generator=g, device=DEV).to(torch.bfloat16)
    q, k, v = qkv[:, :heads * hd], qkv[:, heads * hd:(heads + kvh) * hd], qkv[:, (heads + kvh) * hd:]
    kt = torch.randn(rows, kvh, hd, cap, generator=g, device=DEV).to(torch.bfloat16)
    vc = torch.randn(rows, kvh, cap, hd, generator=g, device=DEV).to(torch.bfloat16)
    if device_pos:
        cos, sin = decode.rope_tables(hd, cap, 500000.0, DEV)
        p = torch.tensor([pos], dtype=torch.int32, device=DEV)
    else:
        inv = 1.0 / (500000.0 ** (torch.arange(0, hd, 2, device=DEV, dtype=torch.float32) / hd))
        cos, sin, p = torch.cos(pos * inv), torch.sin(pos * inv), pos
    want = decode.decode_attention(q, k, v, cos, sin, kt.clone(), vc.clone(), p)
    got = decode.decode_attention(q, k, v, cos, sin, kt.clone(), vc.clone(), p, tiles=True)
    assert torch.equal(got.rows_major(), want)


def test_batch32_step_on_tiles_gives_the_row_major_logits() -> None:
    """A two-layer config-5-shaped model at 32 rows: the step with the glue writing
    x tiles against the same step on row-major x (every projection the same
    kernel either way, so the same bits)."""
    model = Int4Llama(torch, kernels, DEV, layers=2, batch=32, seed=5, fused=True)
    x = (torch.randn(32, 4096, generator=torch.Generator().manual_seed(6)) * 0.5).to(torch.bfloat16).to(DEV)
    a = model.step(x)
    model.tiles = False
    plain = model.linear
    # Row-major x through the kernels the tiles path takes (the automatic choice on
    # row-major x picks the skinny kernel for some of these shapes).
    def row_major(h, w):
        kernel = "split" if h.shape[1] > 4096 else "gemv"
        return torch.cat([kernels.int4_linear(h[c:c + 32], *w, kernel=kernel) for c in range(0, h.shape[0], 32)])

    model.linear = row_major
    b = model.step(x)
    model.linear = plain
    print(f"tiles vs row-major logits: max diff {float((a.float() - b.float()).abs().max()):.3e}", flush=True)
    assert torch.equal(a, b)
