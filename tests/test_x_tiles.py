"""The x-tile layout (`lnq_x_tiles`, `include/linnet_quant.h`) on the host: the
index formula restated element by element against `XTiles.rows_major`'s
reordering, and the chunking of rows past 32."""

from __future__ import annotations

import pytest
import torch

from linnet_amd.torch.kernels import XTiles


def _index(m: int, k: int, width: int) -> int:
    """Value (m, k)'s place: chunk m // 32; operand 8 (m // 16 % 2) + 4 (k // 128 %
    2) + k // 32 % 4 of slice k // 256; lane 16 (k // 8 % 4) + m % 16; within the
    lane's 8 values, the pair order 0, 4, 1, 5, 2, 6, 3, 7 (element e at 2 (e % 4)
    + e // 4)."""
    chunk, mm = divmod(m, 32)
    s, kk = divmod(k, 256)
    op = 8 * (mm // 16) + 4 * (kk // 128) + (kk // 32) % 4
    lane = 16 * ((kk // 8) % 4) + mm % 16
    e = kk % 8
    return chunk * width * 32 + ((s * 16 + op) * 64 + lane) * 8 + [0, 2, 4, 6, 1, 3, 5, 7][e]


@pytest.mark.parametrize(("rows", "width"), [(1, 256), (17, 512), (32, 256), (45, 768)])
def test_rows_major_inverts_the_tile_index(rows: int, width: int) -> None:
    x = torch.arange(rows * width, dtype=torch.float32).reshape(rows, width)
    data = torch.full((-(-rows // 32) * 32 * width,), -1.0)
    for m in range(rows):
        for k in range(width):
            data[_index(m, k, width)] = x[m, k]
    assert torch.equal(XTiles(data, rows, width).rows_major(), x)
    # Every place is used once: the indices of a full chunk are a permutation.
    places = sorted(_index(m, k, width) for m in range(32) for k in range(width))
    assert places == list(range(32 * width))


def test_tiles_refuse_a_width_off_the_slice_size() -> None:
    from linnet_amd.errors import LinnetError

    with pytest.raises(LinnetError, match="multiple of 256"):
        XTiles.empty(4, 320, torch.bfloat16, torch.device("cpu"))
