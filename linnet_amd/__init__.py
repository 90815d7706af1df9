"""linnet_amd: Linnet's weight-quantized linear path (`std.quant`) as hand-written
HIP kernels for AMD Instinct MI355X (gfx950), behind a C ABI
(`include/linnet_quant.h`, `linnet_amd/_lib/liblinnet_quant_hip.so`).

Modules mirror the reference's own (paths relative to
`python/linnet/src/linnet/`):

- `linnet_amd.quant`            <- `quant.py` (quantize / pack / dequantize)
- `linnet_amd.torch.kernels`    <- `torch/kernels.py` (int4_linear, gemv8, w8a16, ...)
- `linnet_amd.torch.quantized`  <- `torch/quantized.py` (8-bit operands / linear)
- `linnet_amd.torch.generated`  <- the generated `_int4_pack` / `_int4_linear` helpers
  (`src/backend/torch_source.cpp:1478-1571`)
- `linnet_amd.torch.native`     <- the interpreter's `NATIVE` entries (`torch/native.py`)
- `linnet_amd.torch.packed`     <- `torch/packed.py` (i4 / u4)
"""

from __future__ import annotations

from .errors import LinnetError

__all__ = ["LinnetError"]
__version__ = "0.1.0"
