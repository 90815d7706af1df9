"""GPTQ and AWQ checkpoint words for the repack tests (not a test module)."""

from __future__ import annotations

import numpy as np

# The two checkpoint formats' int32 words, built from their definitions:
# - GPTQ: `qweight[i // 8, o]` holds input i of output o at bits 4 (i % 8);
#   `qzeros[g, o // 8]` holds group g's zero point of output o at bits 4 (o % 8),
#   less `offset` (1 in GPTQ's first checkpoint format), wrapped to 4 bits.
# - AWQ (GEMM packing): `qweight[i, c]` and `qzeros[g, c]` hold output
#   8c + AWQ_SLOTS[k] at bits 4k, zero points as they are.
AWQ_SLOTS = (0, 2, 4, 6, 1, 3, 5, 7)


def _words(values: np.ndarray, slot_of: tuple[int, ...]) -> np.ndarray:
    """Eight 4-bit values along the last axis as one int32: value j at bits 4 slot_of[j]."""
    shifts = 4 * np.asarray(slot_of, dtype=np.uint32)
    return np.bitwise_or.reduce((values.astype(np.uint32) & 15) << shifts, axis=-1).view(np.int32)


def pack_gptq(q: np.ndarray, zero: np.ndarray, offset: int = 1) -> tuple[np.ndarray, np.ndarray]:
    """`q` [In, Out] codes and `zero` [Groups, Out] as GPTQ's (qweight, qzeros)."""
    inputs, outputs = q.shape
    down_rows = np.moveaxis(q.reshape(inputs // 8, 8, outputs), 1, -1)  # [In/8, Out, 8]
    along = (zero.astype(np.int64) - offset).reshape(zero.shape[0], outputs // 8, 8)
    return _words(down_rows, tuple(range(8))), _words(along, tuple(range(8)))


def pack_awq(q: np.ndarray, zero: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """`q` [In, Out] codes and `zero` [Groups, Out] as AWQ's (qweight, qzeros)."""
    slot_of = tuple(AWQ_SLOTS.index(j) for j in range(8))
    return (_words(q.reshape(q.shape[0], -1, 8), slot_of), _words(zero.reshape(zero.shape[0], -1, 8), slot_of))


def calibrated_layer(method: str, act_order: bool, seed: int = 3, in_features: int = 256,
                     out_features: int = 64, group: int = 64):
    """A random GPTQ/AWQ layer: its codes, zero points, scales and g_idx, its words,
    and the [In, Out] weight its format defines."""
    rng = np.random.default_rng(seed)
    groups = in_features // group
    q = rng.integers(0, 16, (in_features, out_features))
    zero = rng.integers(1, 16, (groups, out_features))
    scale = rng.uniform(0.01, 0.1, (groups, out_features)).astype(np.float16)
    group_of = np.arange(in_features) // group
    if act_order:
        group_of = group_of[rng.permutation(in_features)]
    weight = (q - zero[group_of]) * scale[group_of].astype(np.float32)
    qweight, qzeros = pack_gptq(q, zero) if method == "gptq" else pack_awq(q, zero)
    return dict(q=q, zero=zero, scale=scale, g_idx=group_of.astype(np.int32), qweight=qweight,
                qzeros=qzeros, weight=weight, group=group)
