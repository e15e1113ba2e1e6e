"""Benchmark of the MI355X quantized-linear hot path on BASELINE.json's headline metric.

Primary metric (``value``): W4A16 GEMV HBM throughput at M=1 on the Llama-3-8B decode linears.
One *step* = every W4A16 linear of one Llama-3-8B decode token: 32 layers x {qkv (K=4096, N=6144), o_proj (4096,
4096), gate+up (4096, 28672), down (14336, 4096)} = 128 GEMVs over 32 distinct weight sets (3.64 GB of packed weights,
far above the 256 MB Infinity Cache, so every weight byte comes from HBM).  Each linear runs through
KernelW4A16Linear, the module a model loader swaps in (its prepare() keeps the scales and zero-points blocked by 8
channels beside the portable_row tensors, which the 1..2-row GEMV reads); ``portable_row_raw_op`` times the same ring
through w4a16_linear on the portable_row tensors alone.  Inputs are resident in HBM before timing; the step is captured
once as a HIP graph and replayed (launch overhead excluded, as a decode server runs it).
value = algorithmic bytes per step / step time, bytes per linear = N*K/2 + 2*G*N + G*N/2 + 2*M*K + 2*M*N
(packed weights, fp16 scales, packed zeros, bf16 x and y; forge/kernels/bench.py:164-166).

Secondary (``w4_decode_sweep``, ``w4_prefill``): the same four shapes at M in {4, 16, 64} (configs[1], GB/s) and
M in {512, 2048, 8192} (configs[2], TFLOP/s against 2.5 PFLOP/s dense bf16).
Secondary (``w8a16_decode``): int8 weight-only linears on the same shapes at M in {1, 16} (GB/s).
Secondary (``w8a8_small_m``): FP8 at M in {16, 256} and INT8 at M in {1, 64} (HBM-bound, GB/s).
Secondary (``w8a8``): FP8 e4m3fn GEMM at M=4096, K=N=8192 and INT8 GEMM at M=4096 on the Llama-3-70B
shapes, in TFLOP/s against the dense fp8 / int8 MFMA peaks, on pre-quantised operands.

``roofline``: the dominant kernel (the gate+up GEMV, 61 MB per launch) timed with HIP events on its launch stream;
``traffic`` (HBM bytes per launch) comes from the FETCH_SIZE / WRITE_SIZE counter passes summarised in
profiles/w4_gemv_gate_up_pmc.json (made with ``--pmc-workload``), when that file is present.
``roofline.measured_peak``: a 1 GiB device copy (read + write counted); the W8A8 rows carry hipBLASLt's time on the
same operands (``vendor``).  Every timed row reports the mean with the median and IQR of the per-call times.
``cpu_baseline``: the reference's oracle arithmetic in torch on the host CPU (oracle/torch_ref.py, every thread given
to the process) on configs[0], plus one FP8 and one INT8 GEMM at M=4096.

Usage: ``python bench.py [--steps K] [--warmup W] [--gpus 1]``; prints one JSON line.
``python bench.py --pmc-workload [gemv|decode|w8a8|prefill]``: only a 256 MiB device copy (counter calibration) and the
named kernels, eager, for ``rocprofv3 --pmc`` passes (gemv: 64 gate+up GEMV launches; decode: the CDNA4-layout kernel
at M=16/64 on the four shapes; w8a8: the FP8 / INT8 GEMMs at M=4096; prefill: the ping-pong prefill kernel at
M=8192).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "forge-llm_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
FP8_PEAK_TFLOPS = 5000.0  # dense
BF16_PEAK_TFLOPS = 2500.0  # dense
INT8_PEAK_TOPS = 5000.0  # dense
SHAPES = {"qkv": (4096, 6144), "o_proj": (4096, 4096), "gate_up": (4096, 28672), "down": (14336, 4096)}  # (K, N)
LAYERS = 32
GROUP = 128
# the launch the C library's policy makes for gate+up at M=1: one row of x, one 16-byte chunk per lane, 8 output
# channels per wavefront (two K slices of 2048 columns, eight channel blocks per workgroup)
DOM_KERNEL = "w4_gemv_split_kernel<1,1,8,bf16> sz8"  # the gate+up GEMV the packed-linear module runs at M=1
METRIC = "W4A16 GEMV HBM GB/s (% peak) at M=1; W8A8 TFLOPS (% MFMA peak) at M=4096"


def w4_bytes(m: int, k: int, n: int, g: int = GROUP) -> int:
    G = -(-k // g)
    return n * k // 2 + 2 * G * n + G * n // 2 + 2 * m * k + 2 * m * n


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def make_layer_weights(torch, layouts, dev, k, n, gen):
    """Packed W4 weight in the configs' distributions, generated directly on the GPU: q ~ U{0..15} (uniform random
    words), scales ~ U[0.002, 0.02] fp16, zero-points ~ U{6..9}."""
    G = k // GROUP
    qweight = torch.randint(-2 ** 31, 2 ** 31 - 1, (n, k // 8), dtype=torch.int32, device=dev, generator=gen)
    scales = (torch.rand(G, n, device=dev, generator=gen) * 0.018 + 0.002).half()
    z = torch.randint(6, 10, (G, n), dtype=torch.uint8, device=dev, generator=gen)
    zeros = layouts.pack_nibbles_int32(z.view(G, n // 8, 8))
    return layouts.PackedW4(qweight, scales, zeros, layouts.PORTABLE_W4, n, k, GROUP)


class Timing(float):
    """Mean milliseconds per call (the float value) with the median and inter-quartile range of the per-call
    times next to it."""

    def __new__(cls, samples_ms: list[float]):
        xs = sorted(samples_ms)
        obj = super().__new__(cls, sum(xs) / len(xs))
        q = lambda f: xs[min(len(xs) - 1, max(0, round(f * (len(xs) - 1))))]  # noqa: E731
        obj.median, obj.iqr, obj.n = q(0.5), q(0.75) - q(0.25), len(xs)
        return obj

    def stats(self, scale: float = 1.0, nd: int = 4) -> dict:
        return {"median": round(self.median * scale, nd), "iqr": round(self.iqr * scale, nd), "samples": self.n}


def _timed_calls(torch, call, reps: int) -> Timing:
    """`reps` calls of `call()`, each between two HIP events on the current stream (the one the work is launched on)."""
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    evs[0].record()
    for i in range(reps):
        call()
        evs[i + 1].record()
    torch.cuda.synchronize()
    return Timing([evs[i].elapsed_time(evs[i + 1]) for i in range(reps)])


def time_graph(torch, fn, reps: int, warmup: int) -> Timing:
    """Capture fn() once as a HIP graph; replay `warmup` times, then `reps` times, each replay timed with HIP events."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    return _timed_calls(torch, g.replay, reps)


def time_eager(torch, fn, reps: int, warmup: int) -> Timing:
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    return _timed_calls(torch, fn, reps)


def bench_w4_sweep(torch, ops, ring, mods, dev, gen, timer, steps: int, warmup: int) -> tuple[dict, dict]:
    """configs[1] decode sweep at M in {4, 16, 64} (GB/s of algorithmic bytes, HIP-graph replays over the 32-layer
    ring) and configs[2] prefill at M in {512, 2048, 8192} (TFLOP/s against bf16 dense MFMA, one weight per shape).
    The decode rows ``M4 / M16 / M64`` go through KernelW4A16Linear, the module a served model runs (portable_row
    weights plus the CDNA4-layout copy its prepare() keeps for 3..64 rows); ``M*_portable_row`` are the raw op on the
    portable_row weights alone."""
    decode = {}

    def sweep(label: str, m: int, weights: list, call) -> None:
        row = {}
        xs = {k: torch.randn(m, k, device=dev, generator=gen).bfloat16() for k in {k for k, _ in SHAPES.values()}}
        for name, (k, n) in SHAPES.items():
            sel = [(xs[k], w) for nm, w in weights if nm == name]

            def run(sel=sel):
                for x, w in sel:
                    call(x, w)

            t = timer(torch, run, steps, warmup) / len(sel)
            gbs = w4_bytes(m, k, n) / (t * 1e-3) / 1e9
            row[name] = {"us": round(t * 1e3, 3), "GBps": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "kernel": ops.last_kernel()}
        decode[label] = row
        log(f"decode {label}: " + "  ".join(f"{nm} {v['us']:.2f} us {v['GBps']:.0f} GB/s" for nm, v in row.items()))

    portable = [(nm, p) for nm, _, p in ring]
    for m in (4, 16, 64):
        sweep(f"M{m}_portable_row", m, portable, lambda x, p: ops.w4a16_linear(x, p))
    # the modules a model loader swaps in: the same portable_row tensors, and the CDNA4-layout copy each keeps
    for m in (4, 16, 64):
        sweep(f"M{m}", m, [(nm, mod) for nm, _, mod in mods], lambda x, mod: mod(x))
    prefill = {}
    dense = {name: torch.randn(n, k, device=dev, generator=gen).bfloat16() for name, (k, n) in SHAPES.items()}
    for m in (512, 2048, 8192):
        row = {}
        for name, (k, n) in SHAPES.items():
            ws = [p for nm, _, p in ring if nm == name][:4]  # four distinct weights, graph-replayed in turn
            x = torch.randn(m, k, device=dev, generator=gen).bfloat16()

            def run(x=x, ws=ws):
                for p in ws:
                    ops.w4a16_linear(x, p)

            t = time_graph(torch, run, max(5, steps // 2), 2)
            kern = ops.last_kernel()
            ms = t / len(ws)
            tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
            # the reference's large-M route after its dequantised copy: hipBLASLt's bf16 GEMM via F.linear
            vend = time_graph(torch, lambda x=x, w=dense[name]: torch.nn.functional.linear(x, w),
                              max(5, steps // 2), 2)
            row[name] = {"ms": round(ms, 4), "tflops": round(tf, 1), "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                         "median_ms": round(t.median / len(ws), 4), "kernel": kern,
                         "vendor_bf16_gemm_ms": round(vend, 4)}
            del x
        prefill[f"M{m}"] = row
        log(f"prefill M={m}: " + "  ".join(f"{nm} {v['ms']:.3f} ms {v['tflops']:.0f} TF" for nm, v in row.items()))
    del dense
    return decode, prefill


def bench_w8a16(torch, layouts, ops, dev, gen, timer, steps: int, warmup: int) -> dict:
    """W8A16 (int8 weight-only, per-channel fp16 scales) decode on the four Llama-3-8B shapes at M in {1, 16, 64}: HBM
    GB/s of algorithmic bytes (N*K weights + 2*N scales + 2*M*K + 2*M*N), HIP-graph replays over a ring of distinct
    weights (at least 1.2 GB per shape); prefill at M in {2048, 8192}: TFLOP/s, replays over four of those weights."""
    out = {}
    for name, (k, n) in SHAPES.items():
        nring = max(4, (1200 << 20) // (n * k) + 1)
        ring = [layouts.PackedW8(torch.randint(-128, 128, (n, k), dtype=torch.int8, device=dev, generator=gen),
                                 (torch.rand(1, n, device=dev, generator=gen) * 0.018 + 0.002).half(),
                                 layouts.PORTABLE_W8, n, k, -1) for _ in range(nring)]
        row = {}
        for m in (1, 16, 64):
            x = torch.randn(m, k, device=dev, generator=gen).bfloat16()

            def run(x=x, ring=ring):
                for p in ring:
                    ops.w8a16_linear(x, p)

            t = timer(torch, run, steps, warmup) / len(ring)
            by = n * k + 2 * n + 2 * m * (k + n)
            row[f"M{m}"] = {"us": round(t * 1e3, 3), "GBps": round(by / (t * 1e-3) / 1e9, 1),
                            "frac": round(by / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "kernel": ops.last_kernel()}
        log(f"w8a16 {name:8s}: " + "  ".join(f"M={mm[1:]} {v['us']:.2f} us {v['GBps']:.0f} GB/s" for mm, v in row.items()))
        for m in (2048, 8192):  # prefill: the ping-pong / 64-channel kernels, TFLOP/s against bf16 dense MFMA
            x = torch.randn(m, k, device=dev, generator=gen).bfloat16()

            def run(x=x, ws=ring[:4]):
                for p in ws:
                    ops.w8a16_linear(x, p)

            t = time_graph(torch, run, max(5, steps // 2), 2) / 4
            tf = 2.0 * m * n * k / (t * 1e-3) / 1e12
            row[f"M{m}"] = {"ms": round(t, 4), "tflops": round(tf, 1), "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                            "kernel": ops.last_kernel()}
            log(f"w8a16 {name:8s}: M={m} {t:.3f} ms {tf:.0f} TF  {ops.last_kernel()}")
            del x
        out[name] = row
        del ring
    return out


RING_BYTES = 800 << 20  # >= 3x the 256 MB Infinity Cache: every weight byte of a replayed ring comes from HBM


def bench_w8a8_small(torch, ops, dev, reps: int) -> dict:
    """configs[3] fp8 at M in {16, 256} (K = N = 8192) and configs[4] int8 at M in {1, 64} on the three 70B shapes:
    HBM-bound, reported in GB/s of algorithmic bytes (weights N*K + activations M*K + scales + bf16 output) and in
    TFLOP/s; HIP-graph replays over a ring of distinct weights of at least 800 MB."""
    out = {}
    gen = torch.Generator(device=dev).manual_seed(11)
    k, n = 8192, 8192
    ring = [(torch.randn(n, k, device=dev, generator=gen) * 0.02).to(torch.float8_e4m3fn)
            for _ in range(-(-RING_BYTES // (n * k)))]
    sw = torch.rand(n, device=dev, generator=gen) * 0.01
    for m in (16, 256):
        xq = torch.randn(m, k, device=dev, generator=gen).to(torch.float8_e4m3fn)
        sx = torch.rand(m, device=dev, generator=gen) * 0.01

        def run(xq=xq, sx=sx):
            for w in ring:
                ops.fp8_linear(xq, w, sw, x_scale=sx, out_dtype=torch.bfloat16)

        t = time_graph(torch, run, reps, 3)
        ms = t / len(ring)
        by = n * k + m * k + 4 * (m + n) + 2 * m * n
        out[f"fp8_m{m}_k{k}_n{n}"] = {"us": round(ms * 1e3, 2), "GBps": round(by / (ms * 1e-3) / 1e9, 1),
                                      "tflops": round(2.0 * m * n * k / (ms * 1e-3) / 1e12, 1),
                                      "median_us": round(t.median / len(ring) * 1e3, 2),
                                      "kernel": ops.last_kernel()}
        log(f"fp8 M={m} K=N=8192: {ms * 1e3:.1f} us  {out[f'fp8_m{m}_k{k}_n{n}']['GBps']:.0f} GB/s")
    del ring
    for (k8, n8) in ((8192, 10240), (8192, 57344), (28672, 8192)):
        nring = max(2, -(-RING_BYTES // (n8 * k8)))
        ring = [torch.randint(-127, 128, (n8, k8), dtype=torch.int8, device=dev, generator=gen) for _ in range(nring)]
        swi = torch.rand(n8, device=dev, generator=gen) * 0.01
        for m in (1, 64):
            xi = torch.randint(-127, 128, (m, k8), dtype=torch.int8, device=dev, generator=gen)
            sxi = torch.rand(m, device=dev, generator=gen) * 0.01

            def run(xi=xi, sxi=sxi):
                for w in ring:
                    ops.int8_linear(xi, w, swi, x_scale=sxi, out_dtype=torch.bfloat16)

            t = time_graph(torch, run, reps, 3)
            ms = t / len(ring)
            by = n8 * k8 + m * k8 + 4 * (m + n8) + 2 * m * n8
            key = f"int8_m{m}_k{k8}_n{n8}"
            out[key] = {"us": round(ms * 1e3, 2), "GBps": round(by / (ms * 1e-3) / 1e9, 1),
                        "frac": round(by / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                        "median_us": round(t.median / len(ring) * 1e3, 2), "kernel": ops.last_kernel()}
            log(f"int8 M={m} K={k8} N={n8}: {ms * 1e3:.1f} us  {out[key]['GBps']:.0f} GB/s")
        del ring
    return out


def _vendor(torch, fn, reps: int) -> Timing | None:
    """A vendor-library call timed like ours, or None where this torch build lacks it for these operands."""
    try:
        fn()
        torch.cuda.synchronize()
    except (RuntimeError, TypeError, NotImplementedError) as e:
        log(f"vendor call unavailable: {type(e).__name__}: {str(e)[:120]}")
        return None
    return time_eager(torch, fn, reps, 2)


def bench_w8a8(torch, ops, dev, reps: int) -> dict:
    """configs[3] FP8 at M=4096 and configs[4] INT8 at M=4096 on pre-quantised operands, against the dense MFMA peaks
    and against hipBLASLt through torch on the same operands (``torch._scaled_mm`` rowwise, ``torch._int_mm``): the
    measured denominators next to the datasheet ones."""
    out = {}
    gen = torch.Generator(device=dev).manual_seed(7)
    m, k, n = 4096, 8192, 8192
    x = torch.randn(m, k, device=dev, generator=gen).bfloat16()
    w = torch.randn(n, k, device=dev, generator=gen) * 0.02
    xq, sx = ops.quantize_act_fp8(x)
    wq, sw = ops.quantize_weight_fp8(w, "per_channel")
    del w
    flops = 2.0 * m * n * k
    t = time_eager(torch, lambda: ops.fp8_linear(xq, wq, sw, x_scale=sx, out_dtype=torch.bfloat16), reps, 3)
    tf = flops / (t * 1e-3) / 1e12
    row = {"ms": round(t, 4), "tflops": round(tf, 1), "frac": round(tf / FP8_PEAK_TFLOPS, 4), **t.stats(),
           "kernel": ops.last_kernel()}
    wt = wq.t()
    vend = _vendor(torch, lambda: torch._scaled_mm(xq, wt, scale_a=sx.reshape(m, 1), scale_b=sw.reshape(1, n),
                                                   out_dtype=torch.bfloat16), reps)
    if vend is not None:
        vtf = flops / (vend * 1e-3) / 1e12
        row["vendor"] = {"op": "torch._scaled_mm rowwise (hipBLASLt)", "ms": round(vend, 4), "tflops": round(vtf, 1)}
        row["frac_of_vendor"] = round(tf / vtf, 4)
    out["fp8_m4096_k8192_n8192"] = row
    log(f"fp8 M=4096 K=N=8192: {t:.3f} ms  {tf:.0f} TFLOP/s" + (f" (vendor {vend:.3f} ms)" if vend else ""))
    del xq, wq, x, wt
    for (k8, n8) in ((8192, 10240), (8192, 57344), (28672, 8192)):
        xi = torch.randint(-127, 128, (m, k8), dtype=torch.int8, device=dev, generator=gen)
        wi = torch.randint(-127, 128, (n8, k8), dtype=torch.int8, device=dev, generator=gen)
        sxi = torch.rand(m, device=dev, generator=gen) * 0.01
        swi = torch.rand(n8, device=dev, generator=gen) * 0.01
        t = time_eager(torch, lambda: ops.int8_linear(xi, wi, swi, x_scale=sxi, out_dtype=torch.bfloat16), reps, 3)
        ops_n = 2.0 * m * n8 * k8
        tops = ops_n / (t * 1e-3) / 1e12
        row = {"ms": round(t, 4), "tops": round(tops, 1), "frac": round(tops / INT8_PEAK_TOPS, 4), **t.stats(),
               "kernel": ops.last_kernel()}
        wti = wi.t()
        vend = _vendor(torch, lambda: torch._int_mm(xi, wti), reps)
        if vend is not None:
            vt = ops_n / (vend * 1e-3) / 1e12
            row["vendor"] = {"op": "torch._int_mm, int32 out (hipBLASLt)", "ms": round(vend, 4), "tops": round(vt, 1)}
            row["frac_of_vendor"] = round(tops / vt, 4)
        out[f"int8_m4096_k{k8}_n{n8}"] = row
        log(f"int8 M=4096 K={k8} N={n8}: {t:.3f} ms  {tops:.0f} TOP/s" + (f" (vendor {vend:.3f} ms)" if vend else ""))
        del xi, wi, wti
    return out


def measure_copy_bandwidth(torch, dev, nbytes: int = 1 << 30, reps: int = 20) -> dict:
    """Device-to-device copy of `nbytes` (read + write counted), the reference's measured-bandwidth denominator
    (forge/kernels/bench.py:450-462)."""
    a = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).normal_()
    b = torch.empty_like(a)
    t = time_eager(torch, lambda: b.copy_(a), reps, 5)
    del a, b
    return {"op": "torch copy_ 1 GiB (read + write)", "GBps": round(2.0 * nbytes / (t.median * 1e-3) / 1e9, 1),
            "median_ms": round(t.median, 4)}


def pmc_workload(torch, layouts, ops, dev, gen, which: str = "gemv") -> None:
    """Counter-pass workloads (no timing), each after a 256 MiB device-to-device copy run three times (known bytes:
    calibrates FETCH_SIZE / WRITE_SIZE):
    gemv   -- the gate+up GEMV (K=4096, N=28672, M=1) through KernelW4A16Linear over a ring of 32 weights, twice
              (64 launches of the 8-channel-block GEMV);
    decode -- the CDNA4-layout W4 kernel at M=16 and M=64 on the four Llama-3-8B shapes, over a ring of 6 weights per
              shape, twice (12 launches per shape and M);
    decode_portable -- the same on the portable_row tensors (the raw op's kernels: skinny / LDS ring + reduce);
    w8a8   -- the FP8 GEMM at M=4096, K=N=8192 and the INT8 GEMM at M=4096, K=8192, N=10240, 5 launches each;
    prefill -- the W4A16 ping-pong prefill kernel at M=8192 on gate+up and down and the W8A16 one on gate+up, 5
              launches each."""
    src = torch.empty(64 << 20, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    if which == "gemv":
        k, n = SHAPES["gate_up"]
        x = torch.randn(1, k, device=dev, generator=gen).bfloat16()
        ring = [ops.KernelW4A16Linear.from_packed(make_layer_weights(torch, layouts, dev, k, n, gen))
                for _ in range(LAYERS)]
        torch.cuda.synchronize()
        for _ in range(2):
            for mod in ring:
                mod(x)
        torch.cuda.synchronize()
        log(f"pmc gemv: {ops.last_kernel()}")
        log("pmc workload done: 3 x 256 MiB copy, 64 gate_up GEMV launches (packed-linear modules)")
    elif which == "decode":
        for name, (k, n) in SHAPES.items():
            ring = [layouts.repack(make_layer_weights(torch, layouts, dev, k, n, gen), layouts.CDNA4_W4)
                    for _ in range(6)]
            for m in (16, 64):
                x = torch.randn(m, k, device=dev, generator=gen).bfloat16()
                torch.cuda.synchronize()
                for _ in range(2):
                    for p in ring:
                        ops.w4a16_linear(x, p)
                torch.cuda.synchronize()
            del ring
        log("pmc workload done: 3 x 256 MiB copy, CDNA4-layout W4 at M=16/64 x 4 shapes x 12 launches")
    elif which == "decode_portable":
        for name, (k, n) in SHAPES.items():
            ring = [make_layer_weights(torch, layouts, dev, k, n, gen) for _ in range(6)]
            for m in (16, 64):
                x = torch.randn(m, k, device=dev, generator=gen).bfloat16()
                torch.cuda.synchronize()
                for _ in range(2):
                    for p in ring:
                        ops.w4a16_linear(x, p)
                torch.cuda.synchronize()
                log(f"pmc decode_portable {name} M={m}: {ops.last_kernel()}")
            del ring
        log("pmc workload done: 3 x 256 MiB copy, portable_row W4 at M=16/64 x 4 shapes x 12 launches")
    elif which == "prefill":
        m = 8192
        for name, bits in (("gate_up", 4), ("down", 4), ("gate_up", 8)):
            k, n = SHAPES[name]
            x = torch.randn(m, k, device=dev, generator=gen).bfloat16()
            if bits == 4:
                p = make_layer_weights(torch, layouts, dev, k, n, gen)
                fn = ops.w4a16_linear
            else:
                p = layouts.PackedW8(torch.randint(-128, 128, (n, k), dtype=torch.int8, device=dev, generator=gen),
                                     (torch.rand(1, n, device=dev, generator=gen) * 0.018 + 0.002).half(),
                                     layouts.PORTABLE_W8, n, k, -1)
                fn = ops.w8a16_linear
            torch.cuda.synchronize()
            for _ in range(5):
                fn(x, p)
            torch.cuda.synchronize()
            log(f"pmc prefill {name} W{bits}: {ops.last_kernel()}")
            del x, p
        log("pmc workload done: 3 x 256 MiB copy, prefill M=8192 W4 gate_up / down, W8 gate_up x 5 launches")
    elif which == "w8a8":
        m = 4096
        x = torch.randn(m, 8192, device=dev, generator=gen).bfloat16()
        xq, sx = ops.quantize_act_fp8(x)
        wq, sw = ops.quantize_weight_fp8(torch.randn(8192, 8192, device=dev, generator=gen) * 0.02, "per_channel")
        xi = torch.randint(-127, 128, (m, 8192), dtype=torch.int8, device=dev, generator=gen)
        wi = torch.randint(-127, 128, (10240, 8192), dtype=torch.int8, device=dev, generator=gen)
        sxi = torch.rand(m, device=dev, generator=gen) * 0.01
        swi = torch.rand(10240, device=dev, generator=gen) * 0.01
        torch.cuda.synchronize()
        for _ in range(5):
            ops.fp8_linear(xq, wq, sw, x_scale=sx, out_dtype=torch.bfloat16)
        torch.cuda.synchronize()
        for _ in range(5):
            ops.int8_linear(xi, wi, swi, x_scale=sxi, out_dtype=torch.bfloat16)
        torch.cuda.synchronize()
        log("pmc workload done: 3 x 256 MiB copy, 5 FP8 + 5 INT8 GEMMs at M=4096")
    else:
        raise SystemExit(f"unknown counter workload {which!r}")


def load_traffic() -> dict | None:
    """HBM bytes per gate+up launch from the committed counter summary (None when absent or measured on another
    kernel than the one the policy runs now)."""
    path = os.path.join(ROOT, "profiles", "w4_gemv_gate_up_pmc.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        tr = json.load(f)
    return tr if tr.get("kernel", "").startswith(DOM_KERNEL + " ") else None


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def _cpu_times(fn, reps: int) -> Timing:
    fn()  # warm-up
    out = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        out.append((time.perf_counter() - t0) * 1e3)
    return Timing(out)


def cpu_baseline(reps: int = 7) -> dict:
    """The reference's oracle arithmetic restated in torch (oracle/torch_ref.py) on the host CPU, on every thread this
    process is given (OMP_NUM_THREADS, else os.cpu_count()): configs[0] (W4A16 GEMV, M=1, K=N=4096, group 128, the
    configs' distributions) in GB/s of the same algorithmic bytes as ``value``, one warm-up then the median of
    `reps`; and one stated repeat each of configs[3] FP8 and configs[4] INT8 at M=4096 (TFLOP/s)."""
    import torch

    from forge_amd import layouts
    from oracle import torch_ref as tr

    threads = int(os.environ.get("OMP_NUM_THREADS") or 0) or os.cpu_count() or 1
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    k = n = 4096
    G = k // GROUP
    qweight = torch.randint(-2 ** 31, 2 ** 31 - 1, (n, k // 8), dtype=torch.int32, generator=g)
    scales = (torch.rand(G, n, generator=g) * 0.018 + 0.002).half()
    zeros = layouts.pack_nibbles_int32(torch.randint(6, 10, (G, n), dtype=torch.uint8, generator=g).view(G, n // 8, 8))
    x = torch.randn(1, k, generator=g).bfloat16()
    t = _cpu_times(lambda: tr.w4a16_gemm(x, qweight, scales, zeros, GROUP).bfloat16(), reps)
    by = w4_bytes(1, k, n)
    out = {"value": round(by / (t.median * 1e-3) / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
           "kind": "port",
           "sample": f"configs[0]: W4A16 M=1 K=N=4096 g128 ({by / 1e6:.2f} MB), torch-CPU restatement of "
                     f"w4a16_gemm_ref (oracle/torch_ref.py), 1 warm-up + median of {reps}",
           "median_ms": round(t.median, 3), "iqr_ms": round(t.iqr, 3), "threads": torch.get_num_threads(),
           "os_cpu_count": os.cpu_count(), "cpu_model": _cpu_model()}
    m = 4096
    xq = torch.randn(m, 8192, generator=g).to(torch.float8_e4m3fn)
    wq = (torch.randn(8192, 8192, generator=g) * 0.02).to(torch.float8_e4m3fn)
    sx, sw = torch.rand(m, generator=g) * 0.01, torch.rand(8192, generator=g) * 0.01
    t0 = time.perf_counter()
    tr.fp8_gemm(xq, sx, wq, sw).bfloat16()
    el = time.perf_counter() - t0
    out["fp8_m4096_k8192_n8192"] = {"s": round(el, 3), "tflops": round(2.0 * m * 8192 * 8192 / el / 1e12, 4),
                                    "repeats": 1}
    del xq, wq
    xi = torch.randint(-127, 128, (m, 8192), dtype=torch.int8, generator=g)
    wi = torch.randint(-127, 128, (10240, 8192), dtype=torch.int8, generator=g)
    si, swi = torch.rand(m, generator=g) * 0.01, torch.rand(10240, generator=g) * 0.01
    t0 = time.perf_counter()
    tr.int8_gemm(xi, si, wi, swi).bfloat16()
    el = time.perf_counter() - t0
    out["int8_m4096_k8192_n10240"] = {"s": round(el, 3), "tops": round(2.0 * m * 8192 * 10240 / el / 1e12, 4),
                                      "repeats": 1, "note": "exact int32 through a float64 matmul, as the oracle"}
    return out


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-w8a8", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-sweep", action="store_true", help="skip the W4A16 M=4..64 decode and prefill sweeps")
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of a captured HIP graph")
    ap.add_argument("--pmc-workload", nargs="?", const="gemv", default=None,
                    choices=("gemv", "decode", "decode_portable", "w8a8", "prefill"),
                    help="run only a counter-pass workload (no timing): gemv (default), decode or w8a8")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the hot path is a single-GPU kernel; multi-GPU sharding is "
              "design-only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    from forge_amd import layouts
    from forge_amd import ops_gemm as ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log(f"device: {torch.cuda.get_device_name(dev)}")
    gen = torch.Generator(device=dev).manual_seed(1234)
    if args.pmc_workload:
        pmc_workload(torch, layouts, ops, dev, gen, args.pmc_workload)
        return
    ring = []  # (name, x, packed)
    xs = {k: torch.randn(1, k, device=dev, generator=gen).bfloat16() for k in {k for k, _ in SHAPES.values()}}
    for layer in range(LAYERS):
        for name, (k, n) in SHAPES.items():
            ring.append((name, xs[k], make_layer_weights(torch, layouts, dev, k, n, gen)))
    # the modules a model loader swaps in over the same portable_row tensors: prepare() keeps the 8-channel scale
    # blocks (1..2 rows) and the CDNA4-layout copy (3..64 rows) beside them
    mods = [(name, x, ops.KernelW4A16Linear.from_packed(p)) for name, x, p in ring]
    torch.cuda.synchronize()
    step_bytes = sum(w4_bytes(1, p.k, p.n) for _, _, p in ring)
    log(f"ring: {len(ring)} linears, {sum(p.nbytes for _, _, p in ring) / 1e9:.2f} GB packed weights")

    def step():
        for _, x, mod in mods:
            mod(x)

    def step_portable():
        for _, x, p in ring:
            ops.w4a16_linear(x, p)

    timer = time_eager if args.eager else time_graph
    ms = timer(torch, step, args.steps, args.warmup)
    value = step_bytes / (ms * 1e-3) / 1e9
    log(f"step: {ms:.4f} ms (median {ms.median:.4f}, IQR {ms.iqr:.4f}), {value:.1f} GB/s "
        f"({value / HBM_PEAK_GBS:.1%} of 8 TB/s)")
    ms_port = timer(torch, step_portable, args.steps, args.warmup)
    log(f"step on the portable_row tensors alone (raw op): {ms_port:.4f} ms, "
        f"{step_bytes / (ms_port * 1e-3) / 1e9:.1f} GB/s")

    def shape_rows(items, call) -> dict:
        rows = {}
        for name, (k, n) in SHAPES.items():
            sel = [(x, w) for nm, x, w in items if nm == name]

            def run(sel=sel):
                for x, w in sel:
                    call(x, w)

            tt = timer(torch, run, args.steps, args.warmup)
            t = tt / len(sel)
            gbs = w4_bytes(1, k, n) / (t * 1e-3) / 1e9
            rows[name] = {"K": k, "N": n, "us": round(t * 1e3, 3), "GBps": round(gbs, 1),
                          "frac": round(gbs / HBM_PEAK_GBS, 4), "median_us": round(tt.median / len(sel) * 1e3, 3),
                          "iqr_us": round(tt.iqr / len(sel) * 1e3, 3), "kernel": ops.last_kernel()}
            log(f"  {name:8s} K={k:5d} N={n:5d}: {t * 1e3:8.3f} us  {gbs:7.1f} GB/s  {ops.last_kernel()}")
        return rows

    per_shape = shape_rows(mods, lambda x, mod: mod(x))
    per_shape_portable = shape_rows(ring, lambda x, p: ops.w4a16_linear(x, p))
    copy_bw = measure_copy_bandwidth(torch, dev)
    log(f"copy bandwidth: {copy_bw['GBps']:.0f} GB/s")
    dom = per_shape["gate_up"]
    tr = load_traffic()
    roofline = {"bound": "hbm", "achieved": dom["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(dom["GBps"] / HBM_PEAK_GBS, 4), "traffic": None if tr is None else tr["traffic_bytes"],
                "measured_peak": copy_bw["GBps"], "frac_of_measured": round(dom["GBps"] / copy_bw["GBps"], 4),
                "measured_peak_source": copy_bw["op"],
                "kernel": f"{DOM_KERNEL} (gate_up K=4096 N=28672, M=1)",
                "bytes_per_launch": w4_bytes(1, 4096, 28672), "avg_launch_us": dom["us"],
                "traffic_source": None if tr is None else "profiles/w4_gemv_gate_up_pmc.json"}

    out = {"metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "bf16",
           "data": "synthetic (random int4 codes, fp16 scales U[0.002,0.02], zero-points U{6..9}, bf16 N(0,1) x)",
           "config": {"workload": "llama3-8b decode W4A16 linears, M=1, 32 layers x (qkv, o_proj, gate_up, down)",
                      "M": 1, "group_size": GROUP, "layers": LAYERS,
                      "shapes_KN": {k: list(v) for k, v in SHAPES.items()}, "parallelism": "single GPU",
                      "timing": "eager" if args.eager else "hip graph replay"},
           "frac_of_peak": round(value / HBM_PEAK_GBS, 4),
           "frac_of_measured_copy": round(value / copy_bw["GBps"], 4),
           "step_ms": ms.stats(), "per_shape": per_shape, "roofline": roofline,
           "portable_row_raw_op": {"ms_per_step": round(ms_port, 4),
                                   "GBps": round(step_bytes / (ms_port * 1e-3) / 1e9, 1), "per_shape": per_shape_portable,
                                   "note": "the same ring through w4a16_linear on the portable_row tensors alone (no "
                                           "prepared copies)"}}
    if not args.no_sweep:
        out["w4_decode_sweep"], out["w4_prefill"] = bench_w4_sweep(torch, ops, ring, mods, dev, gen, timer, args.steps,
                                                                   args.warmup)
    del ring, mods
    torch.cuda.empty_cache()
    if not args.no_sweep:
        out["w8a16_decode"] = bench_w8a16(torch, layouts, ops, dev, gen, timer, args.steps, args.warmup)
        torch.cuda.empty_cache()
    if not args.no_w8a8:
        out["w8a8"] = bench_w8a8(torch, ops, dev, max(5, args.steps))
        if not args.no_sweep:
            out["w8a8_small_m"] = bench_w8a8_small(torch, ops, dev, max(5, args.steps))
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
