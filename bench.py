"""Benchmark of the weight-quantized linear path on one MI355X.

Headline (BASELINE.json `metric`, config 2): the W4A16 group-128 decode GEMV,
M=1, K=4096, N=14336 (Llama-3-8B MLP up/gate), as GB/s of algorithmic bytes
(packed weight + bf16 scales + u8 zeros + x + y) against HBM peak. A "step" is
one `lnq_int4_linear` call over one batch (one token) with every operand
resident in HBM (the output too: a preallocated tensor written each call); the
steps rotate over enough distinct weight copies (> 256 MB, the Infinity Cache)
that each call streams its weight from HBM. The timed calls are made eagerly
behind untimed graph replays of the same calls queued on the stream, so the GPU
runs them back to back, and the timed region is bracketed by HIP events on that
stream (`gemv.M1_graph_replay_us`: the same calls timed as one graph replay).

Also reported (extra keys): M=4 and M=16 GEMV, the prefill dequant-GEMM
(config 3: M=2048 over three (K, N)) in TFLOP/s against bf16 MFMA peak beside
the reference's own prefill strategy (HIP dequantize + hipBLASLt), the 8-bit
paths (config 1: int8 per-row weight-only GEMV 4096x4096; config 4: FP8 weight
with per-token FP8 activations, K=8192 N=28672 at M=1/256/4096, against HBM
and fp8 MFMA peaks), the int4 Llama-shaped decode step (config 5), the GPTQ /
AWQ checkpoint repack kernel, gpt-oss-20B's MXFP4 expert projections at decode, a measured copy-bandwidth ceiling, and the
reference's CPU path timed on the host cores.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only gemv|gemm|8bit|llama|checkpoint|mxfp4|nf4|all]

The default K = 2000 GEMV calls (~16 ms) times the steady state of a decode
loop; 200 calls (~1.8 ms) read 10-15% slower, the clock still ramping.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, published
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, published
FP8_PEAK_TFLOPS = 5000.0  # MI355X dense fp8 MFMA, published
L3_BYTES = 256 << 20  # Infinity Cache


def gemv_bytes(m: int, k: int, n: int, group: int = 128) -> int:
    """Algorithmic bytes of one W4A16 call: N*K/2 packed + N*K/G*2 scales +
    N*K/G zeros + M*K*2 x + M*N*2 y."""
    return n * k // 2 + n * (k // group) * 2 + n * (k // group) + m * k * 2 + m * n * 2


def parse() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=2000)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--only", choices=("gemv", "gemm", "8bit", "llama", "checkpoint", "mxfp4", "nf4", "all"), default="all")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    return p.parse_args()


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the weight-quantized linear path runs on one MI355X "
              f"(sharding is described, not run); got --gpus {args.gpus}", file=sys.stderr)
        return 2
    import torch

    sys.path.insert(0, str(ROOT))
    from linnet_amd.torch import kernels

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    props = torch.cuda.get_device_properties(dev)
    stream = torch.cuda.current_stream(dev)

    def timed_graph(launches: list, steps: int, warmup: int, replay: list | None = None, eager: bool = True) -> float:
        """Seconds per call over exactly `steps` calls of the entry point,
        cycling through `launches`, timed between HIP events on the stream the
        kernels run on.

        `warmup` untimed eager calls, then the `steps` calls recorded into one
        HIP graph and replayed untimed until about 20 ms of GPU time have
        passed (the clock a decode loop runs at). The timed calls are then made
        eagerly, queued right behind more untimed replays: the host submits
        them (~13 us a call through Python) while the GPU still works through
        the replays, so the events see the `steps` calls back to back, as a
        decode loop's GPU does, with no graph launch inside the timed region
        (one replay of a graph adds ~8 us, 0.4 us a call when 20 calls are
        timed). The queued replays are sized from the measured submission time,
        and the run checks that the host finished submitting before the GPU
        reached the first timed call; it retries once with more queued work,
        and where the host still cannot get ahead (a profiler that traces every
        launch slows submission) returns the one-replay figure instead, counted
        in the line's `timing_fallbacks`, rather than time an idle GPU. A list
        passed as `replay` receives
        the seconds per call of the same calls timed as one graph replay (one
        replay queued ahead of it); `eager=False` returns that figure instead,
        for calls that wait on the device by design (a load-time check)."""
        t0 = time.perf_counter()
        for i in range(max(warmup, len(launches))):
            launches[i % len(launches)]()
        host_call = (time.perf_counter() - t0) / max(warmup, len(launches))
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(steps):
                launches[i % len(launches)]()
        graph.replay()
        torch.cuda.synchronize()
        queued, start, end = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        start.record(stream)
        graph.replay()
        end.record(stream)
        torch.cuda.synchronize()
        replay_ms = max(start.elapsed_time(end), 1e-3)
        for _ in range(min(400, int(20.0 / replay_ms))):
            graph.replay()
        torch.cuda.synchronize()
        def one_replay() -> float:
            graph.replay()
            start.record(stream)
            graph.replay()
            end.record(stream)
            torch.cuda.synchronize()
            return start.elapsed_time(end) / 1e3 / steps

        if replay is not None or not eager:
            sec = one_replay()
            if not eager:
                del graph
                return sec
            replay.append(sec)
        cap = max(1, int(400.0 / replay_ms))  # at most ~0.4 s of queued GPU work
        ahead = min(cap, 1 + int(2.0 * steps * host_call * 1e3 / replay_ms))
        for _ in range(2):
            t0 = time.perf_counter()
            queued.record(stream)
            for _ in range(ahead):
                graph.replay()
            start.record(stream)
            for i in range(steps):
                launches[i % len(launches)]()
            end.record(stream)
            submitted_ms = (time.perf_counter() - t0) * 1e3
            torch.cuda.synchronize()
            if submitted_ms < 0.9 * queued.elapsed_time(start):
                del graph
                return start.elapsed_time(end) / 1e3 / steps
            ahead = min(cap, 4 * ahead)
        fallbacks.append(steps)
        sec = one_replay()
        del graph
        return sec

    def int4_layers(n: int, k: int, copies: int, seed: int = 0):
        g = torch.Generator(device=dev).manual_seed(seed)
        w = torch.randn(n, k, generator=g, device=dev) * 0.02
        packed, scale, zero = kernels.quantize_int4(w, 128)
        del w
        layers = [(packed, scale.to(torch.bfloat16), zero)]
        for _ in range(copies - 1):
            layers.append(tuple(t.clone() for t in layers[0]))
        return layers

    result: dict[str, object] = {}
    extra: dict[str, object] = {}
    fallbacks: list = []  # timed calls the host could not queue ahead of the GPU

    # --- copy ceiling (1 GiB device-to-device copy).
    src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    copy_s = timed_graph([lambda: dst.copy_(src)], 20, 4)
    copy_gbps = 2 * src.numel() / copy_s / 1e9
    del src, dst
    extra["copy_gbps"] = round(copy_gbps, 1)

    k, n = 4096, 14336
    per_copy = gemv_bytes(1, k, n)
    copies = max(10, -(-(L3_BYTES + (64 << 20)) // per_copy))
    gemv: dict[str, object] = {}
    headline = None
    if args.only in ("gemv", "all"):
        layers = int4_layers(n, k, copies)
        g = torch.Generator(device=dev).manual_seed(1)
        for m in (1, 4, 16):
            x = torch.randn(m, k, generator=g, device=dev).to(torch.bfloat16)
            y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)  # resident output, written each call
            launches = [lambda l=l, x=x, y=y: kernels.int4_linear(x, *l, out=y) for l in layers]
            replay: list = []
            sec = timed_graph(launches, args.steps, args.warmup, replay if m == 1 else None)
            gbps = gemv_bytes(m, k, n) / sec / 1e9
            gemv[f"M{m}"] = {"us": round(sec * 1e6, 3), "gbps": round(gbps, 1), "frac_hbm_peak": round(gbps / HBM_PEAK_GBPS, 4)}
            if m == 1:
                headline = (sec, gbps)
                gemv["M1_graph_replay_us"] = round(replay[0] * 1e6, 3)
        # GPTQ's activation order at one token: the take_inputs gather fused
        # into the GEMV's x staging (lnq_int4_linear_ordered).
        order = torch.randperm(k, generator=g, device=dev).to(torch.int32)
        x = torch.randn(1, k, generator=g, device=dev).to(torch.bfloat16)
        y = torch.empty(1, n, dtype=torch.bfloat16, device=dev)
        launches = [lambda l=l: kernels.int4_linear(x, *l, out=y, order=order) for l in layers]
        sec = timed_graph(launches, args.steps, args.warmup)
        gbps = gemv_bytes(1, k, n) / sec / 1e9
        gemv["M1_act_order"] = {"us": round(sec * 1e6, 3), "gbps": round(gbps, 1),
                                "frac_hbm_peak": round(gbps / HBM_PEAK_GBPS, 4)}
        extra["gemv"] = gemv
        extra["gemv_weight_copies"] = copies
        del layers

    gemm: dict[str, object] = {}
    if args.only in ("gemm", "all"):
        m = 2048
        g = torch.Generator(device=dev).manual_seed(2)
        for kk, nn in ((4096, 4096), (4096, 14336), (14336, 4096)):
            copies_g = max(2, -(-L3_BYTES // (nn * kk // 2 + m * kk * 2)))
            layers = int4_layers(nn, kk, min(copies_g, 8), seed=3)
            x = torch.randn(m, kk, generator=g, device=dev).to(torch.bfloat16)
            ch = max(1, int(0.001 * kk) + (1 if 0.001 * kk % 1 else 0))
            cols = torch.randperm(kk, generator=torch.Generator().manual_seed(0))[:ch].to(dev)
            x[:, cols] *= 20
            flops = 2 * m * nn * kk
            fused = [lambda l=l: kernels.int4_linear(x, *l) for l in layers]
            sec = timed_graph(fused, max(8, args.steps // 10), 4)
            w_deq = [None]

            def dequant_blas(l=layers[0]):
                w = kernels.int4_weight(*l)
                return torch.nn.functional.linear(x, w)

            sec_ref = timed_graph([dequant_blas], max(8, args.steps // 10), 4)
            w = kernels.int4_weight(*layers[0])
            sec_blas = timed_graph([lambda: torch.nn.functional.linear(x, w)], max(8, args.steps // 10), 4)
            del w, w_deq, layers
            gemm[f"K{kk}_N{nn}"] = {
                "us": round(sec * 1e6, 2),
                "tflops": round(flops / sec / 1e12, 1),
                "frac_bf16_peak": round(flops / sec / 1e12 / BF16_PEAK_TFLOPS, 4),
                "dequant_hipblaslt_tflops": round(flops / sec_ref / 1e12, 1),
                "hipblaslt_bf16_only_tflops": round(flops / sec_blas / 1e12, 1),
            }
        extra["gemm_M2048"] = gemm
    torch.cuda.synchronize()

    if args.only in ("8bit", "all"):
        extra.update(eight_bit(torch, dev, timed_graph, args.steps))
    torch.cuda.synchronize()

    if args.only in ("llama", "all"):
        extra["llama_int4_decode"] = llama_decode(torch, kernels, dev)
    torch.cuda.synchronize()

    if args.only in ("mxfp4", "all"):
        extra["mxfp4_experts_gpt_oss_20b"] = mxfp4_decode(torch, kernels, dev, timed_graph, not args.no_cpu)
    torch.cuda.synchronize()

    if args.only in ("checkpoint", "all"):
        extra["int4_repack_K4096_N14336"] = checkpoint_repack(torch, kernels, dev, timed_graph, not args.no_cpu)
    torch.cuda.synchronize()

    if args.only in ("nf4", "all"):
        extra["nf4_K4096_N14336"] = nf4_decode(torch, kernels, dev, timed_graph, not args.no_cpu)
    torch.cuda.synchronize()

    # --- CPU baseline: the reference's CPU path (generated source: the weight
    # dequantized once at prepare, then bf16 F.linear per call), on host cores.
    cpu = None
    if not args.no_cpu and args.only in ("gemv", "all"):
        cpu = cpu_baseline(k, n, args.cpu_seconds)

    if headline is not None:
        sec, gbps = headline
        metric_value, unit, ms = gbps, "GB/s", sec * 1e3
        config = {"workload": "int4 g128 W4A16 decode GEMV (linear_int4_groups)", "M": 1, "K": k, "N": n,
                  "group": 128, "dtype": "bf16 activations, bf16 scales, u8 zeros", "baseline_config": 2}
        roofline = {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                    "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": traffic_from_profiles("int4_gemv_M1"),
                    "kernel": "int4_gemv_kernel<bf16,7,group128>", "bytes_per_launch": gemv_bytes(1, k, n)}
    elif gemm:
        key = next(iter(gemm))
        entry = gemm[key]
        metric_value, unit, ms = entry["tflops"], "TFLOP/s", entry["us"] / 1e3
        config = {"workload": f"int4 g128 prefill dequant-GEMM M=2048 {key}", "baseline_config": 3}
        roofline = {"bound": "mfma", "achieved": entry["tflops"], "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": entry["frac_bf16_peak"], "traffic": None}
    elif "fp8_C4_K8192_N28672" in extra:
        entry = extra["fp8_C4_K8192_N28672"]["M4096"]
        metric_value, unit, ms = entry["tflops"], "TFLOP/s", entry["us"] / 1e3
        config = {"workload": "FP8 weight x per-token FP8 rows, M=4096 K=8192 N=28672", "baseline_config": 4}
        roofline = {"bound": "mfma", "achieved": entry["tflops"], "peak": FP8_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": entry["frac_fp8_peak"], "traffic": None}
    elif "llama_int4_decode" in extra:  # --only llama: the batch-1 decode step (its roofline is the GEMV's)
        entry = extra["llama_int4_decode"]["B1"]
        metric_value, unit, ms = entry["tokens_per_s"], "tokens/s", entry["ms_per_step"]
        config = {"workload": "int4 g128 Llama-3.1-8B-shaped decode step, batch 1, context 1024", "baseline_config": 5}
        roofline = None
    elif "mxfp4_experts_gpt_oss_20b" in extra:  # --only mxfp4: the gate/up projection at batch 1
        entry = extra["mxfp4_experts_gpt_oss_20b"]["gate_up_B1"]
        metric_value, unit, ms = entry["gbps"], "GB/s", entry["us"] / 1e3
        config = {"workload": "MXFP4 experts (gpt-oss-20B gate/up, 32 experts, top 4), batch 1"}
        roofline = {"bound": "hbm", "achieved": entry["gbps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                    "frac": entry["frac_hbm_peak"], "traffic": None}
    elif "nf4_K4096_N14336" in extra and args.only == "nf4":  # --only nf4: the NF4 GEMV at one row
        entry = extra["nf4_K4096_N14336"]["M1"]
        metric_value, unit, ms = entry["gbps"], "GB/s", entry["us"] / 1e3
        config = {"workload": "NF4 (Nf4Linear, block 64) decode GEMV, M=1 K=4096 N=14336"}
        roofline = {"bound": "hbm", "achieved": entry["gbps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                    "frac": entry["frac_hbm_peak"], "traffic": None}
    else:  # --only checkpoint: the GPTQ repack of one layer
        entry = extra["int4_repack_K4096_N14336"]["gptq"]
        metric_value, unit, ms = entry["gbps"], "GB/s", entry["us"] / 1e3
        config = {"workload": "GPTQ int4 checkpoint repack, In=4096 Out=14336 group 128"}
        roofline = {"bound": "hbm", "achieved": entry["gbps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                    "frac": entry["frac_hbm_peak"], "traffic": None}
    result = {
        "metric": "W4A16 decode GEMV GB/s (% HBM peak); prefill qGEMM TFLOP/s (% MFMA peak)",
        "value": round(float(metric_value), 2),
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: weights N(0,0.02) quantized int4 g128 on the GPU, x N(0,1) bf16, seeded",
        "config": config,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "device": {"name": props.name, "arch": getattr(props, "gcnArchName", ""), "cus": props.multi_processor_count},
        **extra,
    }
    if fallbacks:  # lines timed as one graph replay (see timed_graph)
        result["timing_fallbacks"] = len(fallbacks)
    print(json.dumps(result))
    return 0


def _rows(kernels, x):
    """Per-token FP8 rows of x and their scales as `torch._scaled_mm` takes them."""
    qx, xs = kernels.fp8_rows(x)
    return qx, xs.reshape(-1, 1)


def eight_bit(torch, dev, timed_graph, steps: int) -> dict[str, object]:
    """Configs 1 and 4 through the `linnet.torch.quantized` operands/linear entry
    points (`quantized.py:113-194`), weights rotated past the Infinity Cache.
    Config 1: int8 per-row symmetric W [4096, 4096] ~ N(0, 0.02), one bf16 token
    (weight-only GEMV). Config 4: FP8 E4M3 W [28672, 8192] ~ N(0, 0.02) with
    the per-tensor scale max|W| / 448 broadcast per row, x ~ N(0, 1) bf16 with
    dynamic per-token FP8 quantization (`rounded`): M = 1 streams the weight
    (weight-only GEMV), M = 256 and 4096 run the per-token quantize + FP8 MFMA
    product. Bytes are algorithmic (weight + scales + x + y)."""
    from linnet_amd.torch import kernels, quantized

    out: dict[str, object] = {}
    g = torch.Generator(device=dev).manual_seed(0)
    k = n = 4096
    w = torch.randn(n, k, generator=g, device=dev) * 0.02
    q, s = kernels.quantize_int8(w, k, "f32")
    del w
    copies = -(-(L3_BYTES + (64 << 20)) // (n * k))
    ops = [quantized.int8_operands(q.clone(), s.clone(), 0) for _ in range(copies)]
    x = torch.randn(1, k, generator=g, device=dev).to(torch.bfloat16)
    sec = timed_graph([lambda o=o: quantized.int8_linear(x, o, None) for o in ops], steps, 4)
    nbytes = n * k + n * 4 + k * 2 + n * 2
    out["int8_gemv_C1"] = {"us": round(sec * 1e6, 3), "gbps": round(nbytes / sec / 1e9, 1),
                           "frac_hbm_peak": round(nbytes / sec / 1e9 / HBM_PEAK_GBPS, 4)}
    del ops, q, s

    n, k = 28672, 8192
    w = torch.randn(n, k, generator=g, device=dev) * 0.02
    per_tensor = w.abs().max() / 448
    wq = (w / per_tensor).to(torch.float8_e4m3fn)
    del w
    scale = per_tensor.reshape(1, 1).expand(n, 1).to(torch.bfloat16).contiguous()
    ops = [quantized.fp8_operands(wq, scale, 1), quantized.fp8_operands(wq.clone(), scale.clone(), 1)]
    fp8: dict[str, object] = {}
    for m in (1, 256, 4096):
        x = torch.randn(m, k, generator=g, device=dev).to(torch.bfloat16)
        calls = max(4, steps // 5) if m < 4096 else 10
        sec = timed_graph([lambda o=o, x=x: quantized.fp8_linear(x, o, None) for o in ops], calls, 2)
        nbytes = n * k + n * 2 + m * k * 2 + m * n * 2
        flops = 2 * m * n * k
        fp8[f"M{m}"] = {"us": round(sec * 1e6, 2), "gbps": round(nbytes / sec / 1e9, 1),
                        "frac_hbm_peak": round(nbytes / sec / 1e9 / HBM_PEAK_GBPS, 4),
                        "tflops": round(flops / sec / 1e12, 1),
                        "frac_fp8_peak": round(flops / sec / 1e12 / FP8_PEAK_TFLOPS, 4)}
        if m > 1:
            # The vendor library beside it: the reference's own fast path is the
            # per-token rounding then torch._scaled_mm (hipBLASLt's FP8 GEMM here;
            # `quantized.py:129`) -- timed on rows rounded once (the product
            # alone) and with the rounding in each call; null where torch's FP8
            # GEMM does not run.
            try:
                qx, sa = _rows(kernels, x)
                ws = [o[1] for o in ops]  # the FP8 views of the weight copies
                sb = ops[0][2]  # the scales, f32 [1, Out]
                mm = lambda qx, sa, w: torch._scaled_mm(qx, w.t(), scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16)  # noqa: E731
                t_mm = timed_graph([lambda w=w: mm(qx, sa, w) for w in ws], calls, 2)
                t_both = timed_graph([lambda w=w, x=x: mm(*_rows(kernels, x), w) for w in ws], calls, 2)
                fp8[f"M{m}"]["scaled_mm_tflops"] = round(flops / t_mm / 1e12, 1)
                fp8[f"M{m}"]["rows_scaled_mm_tflops"] = round(flops / t_both / 1e12, 1)
            except (RuntimeError, TypeError) as e:
                fp8[f"M{m}"]["scaled_mm_tflops"] = None
                fp8[f"M{m}"]["scaled_mm_error"] = str(e)[:200]
        del x
    out["fp8_C4_K8192_N28672"] = fp8
    del ops

    # The same shape as an Fp8BlockLinear (a scale per 128 x 128 weight block),
    # the rows rounded per 128 inputs (`fp8_groups`) past 32 rows and multiplied
    # by the block-scaled FP8 product (`quantized.py:154-166`).
    bscale = (torch.rand(n // 128, k // 128, generator=g, device=dev) + 0.5) * per_tensor.float()
    bops = [quantized.fp8_block_operands(wq, bscale, 1), quantized.fp8_block_operands(wq.clone(), bscale.clone(), 1)]
    block: dict[str, object] = {}
    for m in (256, 4096):
        x = torch.randn(m, k, generator=g, device=dev).to(torch.bfloat16)
        calls = max(4, steps // 5) if m < 4096 else 10
        sec = timed_graph([lambda o=o, x=x: quantized.fp8_block_linear(x, o, None) for o in bops], calls, 2)
        flops = 2 * m * n * k
        nbytes = n * k + (n // 128) * (k // 128) * 4 + m * k * 2 + m * n * 2
        block[f"M{m}"] = {"us": round(sec * 1e6, 2), "gbps": round(nbytes / sec / 1e9, 1),
                          "tflops": round(flops / sec / 1e12, 1),
                          "frac_fp8_peak": round(flops / sec / 1e12 / FP8_PEAK_TFLOPS, 4)}
        del x
    out["fp8_block_K8192_N28672"] = block
    del bops, wq
    return out


def llama_decode(torch, kernels, dev) -> dict[str, object]:
    """Config 5: the 1024-token prompt's prefill (time to first token) and one
    decode step of the int4 Llama-3.1-8B-shaped stack at a
    1024-token context, captured as one HIP graph and replayed; tokens/s =
    batch / step time. Batch 1 runs every linear on the one-token GEMV
    kernels; batch 32 runs q|k|v, o, gate|up and the head on the 32-row GEMV
    and down on the split GEMV, their inputs written as x tiles by the glue, and
    down's K-chunk partial sums added by the next layer's RMSNorm (which reads
    them as its residual delta) instead of a reduction kernel of their own; q|k|v
    and gate|up run as joined projections; between the linears, the decode
    kernels of `torch/decode.py` (4 a layer). `linears_ms` replays the step's 161
    int4 linear calls alone as the step makes them (x tiles, down's partial sums);
    `torch_glue_ms` is the same step with the glue as torch ops (~40 small kernels
    a layer) and the projections apart."""
    out: dict[str, object] = {"layers": 32, "hidden": 4096, "heads": "32/8", "ffn": 14336, "vocab": 128256,
                              "context": 1024, "weights": "int4 g128, bf16 scales, u8 zeros; random-init"}
    from linnet_amd.llama import Int4Llama

    model = Int4Llama(torch, kernels, dev)
    # The 1024-token prompt (batch 1): `prefill` runs every projection at 1024 rows
    # on the tiled GEMM, causal attention over the prompt, the head on the last row.
    # Time to first token = the prefill's time on the GPU (eager, inputs resident).
    prompt = (torch.randn(1024, 4096, device=dev) * 0.5).to(torch.bfloat16)
    model.prefill(prompt)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ttft = []
    for _ in range(5):
        start.record()
        first = model.prefill(prompt)
        end.record()
        torch.cuda.synchronize()
        ttft.append(start.elapsed_time(end))
    ttft_ms = sorted(ttft)[len(ttft) // 2]
    linear_params = sum(p[name][0].numel() * 2 for p in model.layers for name in ("qkv", "o", "gate_up", "down"))
    out["prefill_1024"] = {"ttft_ms": round(ttft_ms, 3), "tokens_per_s": round(1024e3 / ttft_ms, 1),
                           "linear_tflops": round(2 * linear_params * 1024 / ttft_ms / 1e9, 1),
                           "attention": "torch fused" if model._flash else "torch f32 math",
                           "finite": bool(torch.isfinite(first).all().item())}
    model.set_position(1024)
    del prompt, first
    for batch in (1, 32):
        if batch != 1:
            model.kt = [t[:1].expand(batch, -1, -1, -1).contiguous() for t in model.kt]
            model.vc = [t[:1].expand(batch, -1, -1, -1).contiguous() for t in model.vc]
        x = (torch.randn(batch, 4096, device=dev) * 0.5).to(torch.bfloat16)
        for _ in range(3):
            model.step(x)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            logits = model.step(x)
        graph.replay()
        torch.cuda.synchronize()
        reps = 20
        start.record()
        for _ in range(reps):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / reps
        # The same step's 161 int4 linear calls alone (inputs and outputs preallocated),
        # on x tiles where the step's glue hands its projections tiles (17..64 rows).
        calls = []

        def x_in(k, tiles):
            xin = (torch.randn(batch, k, device=dev) * 0.5).to(torch.bfloat16)
            return kernels.x_tiles(xin) if tiles else xin

        tiles = model._tiles(x)
        for p in model.layers:
            for name, k in (("qkv", 4096), ("o", 4096), ("gate_up", 4096), ("down", 14336)):
                yout = torch.empty(batch, p[name][0].shape[0], dtype=torch.bfloat16, device=dev)
                calls.append((x_in(k, tiles), p[name], yout))
        calls.append((x_in(4096, tiles), model.head, torch.empty(batch, 128256, dtype=torch.bfloat16, device=dev)))
        lin_graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(lin_graph):
            for xin, w, yout in calls:
                if isinstance(xin, kernels.XTiles):
                    kernels.int4_linear_tiles(xin, *w, out=yout)
                else:
                    kernels.int4_linear(xin, *w, out=yout)
        lin_graph.replay()
        torch.cuda.synchronize()
        start.record()
        for _ in range(reps):
            lin_graph.replay()
        end.record()
        torch.cuda.synchronize()
        lin_ms = start.elapsed_time(end) / reps
        nbytes = sum(w[0].numel() + w[1].numel() * 2 + w[2].numel() for _, w, _ in calls)
        model.fused = False
        model.step(x)  # eager first: library handles are created outside the capture
        torch.cuda.synchronize()
        glue_graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(glue_graph):
            model.step(x)
        glue_graph.replay()
        torch.cuda.synchronize()
        start.record()
        for _ in range(reps):
            glue_graph.replay()
        end.record()
        torch.cuda.synchronize()
        glue_ms = start.elapsed_time(end) / reps
        model.fused = True
        out[f"B{batch}"] = {"ms_per_step": round(ms, 3), "tokens_per_s": round(batch * 1e3 / ms, 1),
                            "linears_ms": round(lin_ms, 3), "linear_weight_gbps": round(nbytes / lin_ms / 1e6, 1),
                            "torch_glue_ms": round(glue_ms, 3),
                            "finite": bool(torch.isfinite(logits).all().item())}
        del graph, lin_graph, glue_graph, calls
    del model
    return out


def mxfp4_decode(torch, kernels, dev, timed_graph, with_cpu: bool) -> dict[str, object]:
    """gpt-oss-20B's MXFP4 expert projections at a decoding step
    (`std.quant::mxfp4_experts`, `torch/kernels.py:94-209`): 32 experts, top 4,
    gate/up 2880 -> 5760 and down 2880 -> 2880, batch 1 and 8. Random codes and
    scales (E8M0 118..135), random-init; each call picks the next 4 (or 32) of the
    experts over two copies of the expert weights (564 MB for gate/up > the
    Infinity Cache), so the chosen experts' bytes come from HBM. Bytes: the chosen
    experts' blocks and scales (distinct experts once each: the kernel reads a pair's
    expert in full, a repeated expert from L2 / the Infinity Cache), x and y."""
    count, top, width = 32, 4, 2880
    groups = width // 32
    g = torch.Generator(device=dev).manual_seed(0)
    found: dict[str, object] = {}
    for name, out in (("gate_up", 5760), ("down", 2880)):
        copies = [(torch.randint(0, 256, (count, out, groups, 16), generator=g, device=dev, dtype=torch.uint8),
                   torch.randint(118, 136, (count, out, groups), generator=g, device=dev, dtype=torch.uint8))
                  for _ in range(2)]
        for batch in (1, 8):
            x = torch.randn(batch, top, width, generator=g, device=dev).to(torch.bfloat16)
            sets = []
            for i in range(16):
                ids = (torch.arange(batch * top, device=dev) + i * batch * top) % count
                sets.append((copies[i % 2], ids.reshape(batch, top)))
            launches = [lambda c=c, e=e: kernels.mxfp4_experts(x, c[0], c[1], e) for c, e in sets]
            sec = timed_graph(launches, 400, 10)
            distinct = min(batch * top, count)
            nbytes = distinct * out * (groups * 16 + groups) + batch * top * (width * 2 + out * 2)
            entry = {"us": round(sec * 1e6, 2), "gbps": round(nbytes / sec / 1e9, 1),
                     "frac_hbm_peak": round(nbytes / sec / 1e9 / HBM_PEAK_GBPS, 4), "bytes_per_call": nbytes}
            if with_cpu and batch == 1:
                # The reference's fallback (generated `_mxfp4_experts` off its kernel,
                # `torch_source.cpp:1595-1601`): gather the chosen experts, widen in f32, einsum.
                table = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0,
                                      -4.0, -6.0])
                blocks, scales = copies[0][0].cpu(), copies[0][1].cpu()
                xc, ec = x.cpu(), sets[0][1].cpu()
                t0 = time.perf_counter()
                taken = blocks[ec]
                values = torch.stack([table[(taken & 15).long()], table[(taken >> 4).long()]], dim=-1)
                factor = torch.exp2(scales[ec].float() - 127)[..., None]
                weight = (values.reshape(*taken.shape[:-1], 32) * factor).reshape(*taken.shape[:-2], -1)
                torch.einsum("rki,rkoi->rko", xc.float(), weight).to(xc.dtype)
                cpu_s = time.perf_counter() - t0
                entry["cpu_reference_fallback_ms"] = round(cpu_s * 1e3, 1)
                entry["cpu_reference_fallback_gbps"] = round(nbytes / cpu_s / 1e9, 3)
                del blocks, scales, taken, values, weight
            found[f"{name}_B{batch}"] = entry
            del x
        del copies
    return found


def nf4_decode(torch, kernels, dev, timed_graph, with_cpu: bool) -> dict[str, object]:
    """`Nf4Linear` (block 64, bf16) on Llama-3.1-8B's 4096 -> 14336 at 1, 4 and 8
    rows: the NF4 GEMV (`lnq_nf4_linear`) and the reference's body (the weight
    widened by `lnq_nf4_dequant`, then bf16 `F.linear`, hipBLASLt), over 8 copies
    of random codes and absmax (265 MB > the Infinity Cache). Bytes: codes,
    absmax, x and y. The CPU leg times the reference's body on the host
    (codebook lookup, scale, bf16 `F.linear`) at one row."""
    n, k, block, copies = 14336, 4096, 64, 8
    g = torch.Generator(device=dev).manual_seed(0)
    layers = [(torch.randint(0, 256, (n, k // 2), generator=g, device=dev, dtype=torch.uint8),
               torch.rand(n, k // block, generator=g, device=dev) * 0.1 + 0.01) for _ in range(copies)]
    found: dict[str, object] = {}
    for m in (1, 4, 8):
        x = torch.randn(m, k, generator=g, device=dev).to(torch.bfloat16)
        gemv = [lambda c=c, a=a: kernels.nf4_linear(x, c, a, block) for c, a in layers]
        wide = [lambda c=c, a=a: torch.nn.functional.linear(x, kernels.nf4_dequantize(c, a, block, torch.bfloat16))
                for c, a in layers]
        nbytes = n * k // 2 + n * (k // block) * 4 + m * k * 2 + m * n * 2
        sec = timed_graph(gemv, 200, 10)
        sec_wide = timed_graph(wide, 80, 10)
        entry = {"us": round(sec * 1e6, 2), "gbps": round(nbytes / sec / 1e9, 1),
                 "frac_hbm_peak": round(nbytes / sec / 1e9 / HBM_PEAK_GBPS, 4), "bytes_per_call": nbytes,
                 "dequant_linear_us": round(sec_wide * 1e6, 2)}
        if with_cpu and m == 1:
            table = torch.tensor([-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
                                  -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
                                  0.07958029955625534, 0.16093020141124725, 0.2461123019456863, 0.33791524171829224,
                                  0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0])
            codes, absmax, xc = layers[0][0].cpu(), layers[0][1].cpu(), x.cpu()
            t0 = time.perf_counter()
            values = torch.stack([table[(codes & 15).long()], table[(codes >> 4).long()]], dim=-1).reshape(n, k)
            weight = (values.reshape(n, k // block, block) * absmax[:, :, None]).reshape(n, k).to(torch.bfloat16)
            torch.nn.functional.linear(xc, weight)
            cpu_s = time.perf_counter() - t0
            entry["cpu_reference_body_ms"] = round(cpu_s * 1e3, 1)
            entry["cpu_reference_body_gbps"] = round(nbytes / cpu_s / 1e9, 3)
            del codes, absmax, values, weight
        found[f"M{m}"] = entry
    del layers
    return found


def checkpoint_repack(torch, kernels, dev, timed_graph, with_cpu: bool) -> dict[str, object]:
    """The GPTQ / AWQ repack kernel (`lnq_int4_repack`) on one Llama-3.1-8B up
    projection (In 4096, Out 14336, group 128): GPTQ words, GPTQ in activation
    order, AWQ words. Bytes: the int32 words read and the packed bytes written
    (In*Out/2 each) plus the zero words read and zero bytes written. Ten copies of
    the words (290 MB > the Infinity Cache) rotate. Beside it, the reference's numpy
    repack (`quant.py:307-341`, restated in the oracle) on the same layer, once."""
    import numpy as np

    in_f, out_f, group = 4096, 14336, 128
    groups = in_f // group
    nbytes = 2 * (in_f * out_f // 2) + groups * out_f // 8 * 4 + groups * out_f
    rng = np.random.default_rng(0)
    g = torch.Generator(device=dev).manual_seed(0)
    found: dict[str, object] = {}
    for kind, method, act in (("gptq", "gptq", False), ("gptq_act_order", "gptq", True), ("awq", "awq", False)):
        shape = (in_f // 8, out_f) if method == "gptq" else (in_f, out_f // 8)
        words = [torch.randint(-2**31, 2**31 - 1, shape, generator=g, device=dev, dtype=torch.int32) for _ in range(10)]
        zeros = torch.randint(-2**31, 2**31 - 1, (groups, out_f // 8), generator=g, device=dev, dtype=torch.int32)
        order = torch.from_numpy(rng.permutation(in_f).astype(np.int32)).to(dev) if act else None
        offset = 1 if method == "gptq" else 0
        launches = [lambda w=w: kernels.int4_repack(w, zeros, method, group, offset, order) for w in words]
        # One graph replay: the act-order call checks its order on the host
        # (one device wait a call) when it is not being captured.
        sec = timed_graph(launches, 200, 10, eager=False)
        entry = {"us": round(sec * 1e6, 2), "gbps": round(nbytes / sec / 1e9, 1),
                 "frac_hbm_peak": round(nbytes / sec / 1e9 / HBM_PEAK_GBPS, 4)}
        if with_cpu:
            from oracle import quant

            host_w, host_z = words[0].cpu().numpy(), zeros.cpu().numpy()
            g_idx = None
            if act:
                g_idx = np.empty(in_f, np.int32)
                g_idx[order.cpu().numpy()] = np.arange(in_f) // group
            t0 = time.perf_counter()
            quant.repack_int4(host_w, host_z, method, group, offset, g_idx if method == "gptq" else None)
            cpu_s = time.perf_counter() - t0
            entry["cpu_numpy_ms"] = round(cpu_s * 1e3, 1)
            entry["cpu_numpy_gbps"] = round(nbytes / cpu_s / 1e9, 3)
        found[kind] = entry
        del words
    found["bytes_per_call"] = nbytes
    return found


def traffic_from_profiles(name: str) -> float | None:
    """HBM bytes per launch measured by rocprofv3 PMC runs and committed under
    profiles/traffic.json (None until such a measurement exists)."""
    path = ROOT / "profiles" / "traffic.json"
    try:
        table = json.loads(path.read_text())
        value = table.get(name, {}).get("hbm_bytes_per_launch")
        return None if value is None else float(value)
    except (OSError, ValueError):
        return None


def cpu_baseline(k: int, n: int, budget_s: float) -> dict[str, object]:
    """The reference's CPU path on the host cores, on the full layer: the weight
    dequantized once (prepare), then per call a bf16 `F.linear` of one token
    (`src/backend/torch_source.cpp:1501-1504, 1567-1568`). Median over as many
    calls as fit the budget (at least 3, after 1 warmup). The interpreter path
    (dequantize every call, `torch/native.py:417-423`) is timed once beside it."""
    import numpy as np
    import torch

    from oracle import linear, quant

    cores = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS"):
        cores = min(cores, int(os.environ["OMP_NUM_THREADS"]))
    torch.set_num_threads(cores)
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((n, k), dtype=np.float32) * 0.02).astype(np.float32)
    packed, scale, zero = quant.quantize_int4_groups(w, 128)
    del w
    p = torch.from_numpy(packed)
    s = torch.from_numpy(quant.to_bf16_bits(scale).view(np.int16)).view(torch.bfloat16)
    z = torch.from_numpy(zero)
    x = torch.randn(1, k, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    prepared = linear.int4_prepare_cpu(p, s, z)
    linear.int4_linear_generated_cpu(x, prepared, None)
    times = []
    start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - start < budget_s and len(times) < 20):
        t0 = time.perf_counter()
        linear.int4_linear_generated_cpu(x, prepared, None)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    t0 = time.perf_counter()
    linear.int4_groups_linear_interpreter(x, p, s, z, None)
    interp = time.perf_counter() - t0
    nbytes = gemv_bytes(1, k, n)
    del prepared, p, s, z
    return {
        "value": round(nbytes / med / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"full layer K={k} N={n} M=1, reference CPU generated-source path (bf16 F.linear over the "
                   f"prepared weight), median of {len(times)} calls = {med * 1e3:.2f} ms; interpreter path "
                   f"(dequantize per call) 1 call = {interp * 1e3:.1f} ms = {nbytes / interp / 1e9:.3f} GB/s"),
        "configs": eight_bit_cpu(budget_s),
    }


def eight_bit_cpu(budget_s: float) -> dict[str, object]:
    """The reference's CPU branch of the 8-bit linears (`torch/quantized.py:133-134,
    193`: the weight widened and scaled on every call, then a bf16 `F.linear`), at
    config 1 (int8 per-row, 4096 x 4096, one token) and config 4 (FP8 E4M3 per-row,
    K 8192 x N 28672, one token), on the host cores: median of the calls that fit
    `budget_s` (at least 3, after 1 warmup). GB/s counts the weight, its scales and
    the activations once, as the GPU figures do."""
    import numpy as np
    import torch

    from oracle import linear

    g = torch.Generator().manual_seed(0)
    found: dict[str, object] = {}
    for key, n, k, fp8 in (("C1_int8_M1", 4096, 4096, False), ("C4_fp8_M1", 28672, 8192, True)):
        w = torch.randn(n, k, generator=g) * 0.02
        if fp8:
            s = (w.abs().max() / 448).expand(n).contiguous()
            q = (w / s[:, None]).to(torch.float8_e4m3fn).view(torch.uint8)
            run = linear.fp8_linear_cpu
        else:
            s = w.abs().amax(1) / 127
            q = torch.round(w / s[:, None]).clamp(-127, 127).to(torch.int8)
            run = linear.int8_linear_cpu
        del w
        x = torch.randn(1, k, generator=g).to(torch.bfloat16)
        run(x, q, s, None)
        times: list[float] = []
        start = time.perf_counter()
        while len(times) < 3 or (time.perf_counter() - start < budget_s and len(times) < 20):
            t0 = time.perf_counter()
            run(x, q, s, None)
            times.append(time.perf_counter() - t0)
        med = float(np.median(times))
        nbytes = n * k + n * 4 + k * 2 + n * 2
        found[key] = {"ms": round(med * 1e3, 3), "gbps": round(nbytes / med / 1e9, 3), "calls": len(times),
                      "path": "per call: weight widened x scale -> bf16, F.linear"}
        del q, s
    return found


if __name__ == "__main__":
    sys.exit(main())
