"""CPU oracle for the weight-quantized linear path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what Linnet's reference implementation
computes for `std.quant`'s weight-quantized linear layers, so that the HIP
kernels of `linnet_amd` can be checked against it. It is imported only by
`tests/`, by `__graft_entry__.smoke()` and by the `cpu_baseline` leg of
`bench.py`, and only as the checker or the timed CPU baseline. No product
code path imports it; `linnet_amd` raises when its HIP library is missing
instead of falling back to anything here.

Modules:

- `oracle.quant`   -- group-wise int4 / int8 quantize, pack, unpack,
  dequantize; bf16 and fp8 bit encodings; per-token and per-group activation
  rounding; GPTQ / AWQ checkpoint repack; MXFP4 decoding (numpy, bit-exact
  restatements).
- `oracle.linear`  -- the reference's CPU linear paths (torch on the CPU, as
  the reference itself runs them) and fp64 products for tolerances (plain,
  8-bit rows, block-scaled FP8, MXFP4 experts).

Parity pins (what fixes each function independently of its own formula) are
listed in each function's docstring and exercised in `tests/test_oracle.py`.
Every function here is pinned; none is "parity unpinned".
"""
