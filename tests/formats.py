"""GPTQ and AWQ checkpoint words for the repack tests (not a test module)."""

from __future__ import annotations

import numpy as np

# GPTQ's and AWQ's int32 packings written from the formats' definitions, as the
# reference's tests write them (`test_quant_groups.py:198-221`), not from the
# importer: GPTQ `qweight[i // 8, o]` holds input i at bits 4 (i % 8) and
# `qzeros[g, o // 8]` group g's zero point, less one in the first format, at bits
# 4 (o % 8); AWQ `qweight[i, c]` and `qzeros[g, c]` hold output 8c + ORDER[k] at
# bits 4k, zero points as they are.
FORMAT_AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)


def pack_gptq(q: np.ndarray, zero: np.ndarray, offset: int = 1) -> tuple[np.ndarray, np.ndarray]:
    qweight = np.zeros((q.shape[0] // 8, q.shape[1]), np.uint32)
    qzeros = np.zeros((zero.shape[0], zero.shape[1] // 8), np.uint32)
    for k in range(8):
        qweight |= q[k::8].astype(np.uint32) << (4 * k)
        qzeros |= (zero[:, k::8] - offset).astype(np.uint32) << (4 * k)
    return qweight.view(np.int32), qzeros.view(np.int32)


def pack_awq(q: np.ndarray, zero: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    qweight = np.zeros((q.shape[0], q.shape[1] // 8), np.uint32)
    qzeros = np.zeros((zero.shape[0], zero.shape[1] // 8), np.uint32)
    for k, column in enumerate(FORMAT_AWQ_ORDER):
        qweight |= q[:, column::8].astype(np.uint32) << (4 * k)
        qzeros |= zero[:, column::8].astype(np.uint32) << (4 * k)
    return qweight.view(np.int32), qzeros.view(np.int32)


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
