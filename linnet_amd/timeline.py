"""Where the time of one one-token int4 GEMV goes: per-wave timestamps.

`python -m linnet_amd.timeline [--n N] [--k K]` runs the decode GEMV of
config 2 (K = 4096, N = 14336, group 128, bf16) from the diagnostic library
`liblinnet_quant_timeline.so` (the same kernels, the one-token kernel compiled
with `s_memrealtime` stamps at its phase boundaries; built beside the product
library by `linnet_amd._build`), as bench.py times it -- 11 rotating weight
copies, a graph of 2000 calls -- then one more call whose stamps it reads back.
It prints, in microseconds from the first wave's entry, the distribution over
all waves of each phase boundary, the workgroups' start and end, and the end per
XCD (workgroup b runs on XCD b % 8). The stamp stores add a little to each wave's
work, so the graph time per call is printed beside the product kernel's.
"""

from __future__ import annotations

import argparse
import ctypes
import statistics
import sys

import torch

from . import _build, _lib

POINTS = {
    0: "entry",
    1: "small loads issued",
    2: "past the start barrier",
    3: "weights issued",
    4: "x landed",
    5: "tile 0 folded",
    6: "tile 1 folded",
    7: "tile 2 folded",
    8: "tile 3 folded",
    9: "half tile folded",
    10: "before the final barrier",
    11: "after the final barrier",
    12: "end",
}


def _quantiles(values: list[float]) -> str:
    v = sorted(values)
    pick = lambda q: v[min(len(v) - 1, int(q * len(v)))]  # noqa: E731
    return f"min {v[0]:6.2f}  med {pick(0.5):6.2f}  p90 {pick(0.9):6.2f}  max {v[-1]:6.2f}"


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    parser.add_argument("--n", type=int, default=14336)
    parser.add_argument("--k", type=int, default=4096)
    parser.add_argument("--calls", type=int, default=2000)
    args = parser.parse_args(argv)
    if not torch.cuda.is_available():
        print("linnet_amd.timeline needs a GPU", file=sys.stderr)
        return 2
    from .torch import kernels

    stamped = ctypes.CDLL(str(_build.TIMELINE))
    for name, types in (("lnq_int4_linear", _lib.SIGNATURES["lnq_int4_linear"]), ("lnq_gemv_timeline_read", [ctypes.c_void_p])):
        getattr(stamped, name).argtypes = types
        getattr(stamped, name).restype = ctypes.c_int32
    dev = torch.device("cuda", 0)
    n, k = args.n, args.k
    g = torch.Generator(device=dev).manual_seed(0)
    w = torch.randn(n, k, generator=g, device=dev) * 0.02
    packed, scale, zero = kernels.quantize_int4(w, 128)
    del w
    layers = [(packed, scale.to(torch.bfloat16), zero)]
    layers += [tuple(t.clone() for t in layers[0]) for _ in range(10)]
    x = torch.randn(1, k, generator=g, device=dev).to(torch.bfloat16)
    y = torch.empty(1, n, dtype=torch.bfloat16, device=dev)

    def launch(lib: ctypes.CDLL, layer) -> None:
        p, s, z = (ctypes.c_void_p(t.data_ptr()) for t in layer)
        status = lib.lnq_int4_linear(ctypes.c_void_p(x.data_ptr()), p, s, z, None, ctypes.c_void_p(y.data_ptr()), 1, k, n,
                                     128, _lib.BF16, _lib.KERNEL_GEMV,
                                     ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
        if status != _lib.LNQ_OK:
            raise RuntimeError("lnq_int4_linear failed")

    def per_call(lib: ctypes.CDLL) -> float:
        for layer in layers:
            launch(lib, layer)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(args.calls):
                launch(lib, layers[i % len(layers)])
        graph.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        graph.replay()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / args.calls * 1e3

    product = per_call(_lib.load())
    with_stamps = per_call(stamped)
    ref = kernels.int4_linear(x, *layers[0])
    launch(stamped, layers[3])
    torch.cuda.synchronize()
    launch(stamped, layers[0])
    torch.cuda.synchronize()
    exact = torch.equal(y, ref)
    raw = (ctypes.c_ulonglong * (512 * 16 * 16))()
    if stamped.lnq_gemv_timeline_read(raw) != _lib.LNQ_OK:
        raise RuntimeError("lnq_gemv_timeline_read failed")
    rows = 8 * ((n + 2047) // 2048)
    blocks = min(512, (n + rows - 1) // rows)
    waves = k // 256
    at = lambda b, w, e: raw[(b * 16 + w) * 16 + e]  # noqa: E731
    t0 = min(at(b, w, 0) for b in range(blocks) for w in range(waves))
    us = lambda t: (t - t0) / 100.0  # noqa: E731 -- 100 MHz counter
    print(f"one-token GEMV K={k} N={n}: {blocks} workgroups x {waves} waves, {rows} rows each; result exact: {exact}")
    print(f"graph-replayed call: product kernel {product:.3f} us, stamped kernel {with_stamps:.3f} us")
    print("point (us from the first entry, over all waves)")
    present = [e for e in POINTS if all(at(b, w, e) >= t0 for b in range(blocks) for w in range(waves))]
    for e in present:
        print(f"  {e:2d} {POINTS[e]:26s} {_quantiles([us(at(b, w, e)) for b in range(blocks) for w in range(waves)])}")
    starts = [min(us(at(b, w, 0)) for w in range(waves)) for b in range(blocks)]
    ends = [max(us(at(b, w, 12)) for w in range(waves)) for b in range(blocks)]
    print(f"  workgroup start            {_quantiles(starts)}")
    print(f"  workgroup end              {_quantiles(ends)}")
    for xcd in range(8):
        e = [ends[b] for b in range(blocks) if b % 8 == xcd]
        if e:
            print(f"  XCD {xcd} workgroup end       med {statistics.median(e):6.2f}  max {max(e):6.2f}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
