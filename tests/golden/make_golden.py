"""Writes the small known-answer fixtures under tests/golden/ from the CPU oracle
(seeded inputs; regenerate with `python tests/golden/make_golden.py`).

The reference ships no golden vector files for this path -- its tests draw
seeded data and check invariants and tolerances -- so these fixtures are the
oracle's answers on fixed inputs, pinned by tests/test_oracle.py, and lock the
GPU kernels to them bit for bit.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import quant  # noqa: E402


def main() -> None:
    rng = np.random.default_rng(0)
    weight = (rng.standard_normal((32, 256)) * 0.02).astype(np.float32)
    weight[3, :128] = -0.01  # a constant group
    packed, scale, zero = quant.quantize_int4_groups(weight, 128)
    np.savez_compressed(HERE / "int4_quantize.npz", weight=weight, group=np.int64(128), packed=packed, scale=scale, zero=zero)

    x = rng.standard_normal((5, 300)).astype(np.float32)
    x[1] *= 30.0
    x[3] = 0.0
    x_bits = quant.to_bf16_bits(x).reshape(x.shape)
    xv = quant.from_bf16_bits(x_bits).reshape(x.shape)
    fq, fs = quant.rows8(xv, True)
    iq, is_ = quant.rows8(xv, False)
    np.savez_compressed(HERE / "rows8.npz", x_bits=x_bits, fp8_q=fq, fp8_scale=fs, int8_q=iq, int8_scale=is_)


if __name__ == "__main__":
    main()
