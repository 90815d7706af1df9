"""PyTorch-facing side of linnet_amd: the reference's `linnet.torch` helpers for
`std.quant`'s layers, running the gfx950 HIP kernels."""
