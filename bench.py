"""Benchmark of the MI355X quantized-linear hot path on BASELINE.json's headline metric.

Primary metric (``value``): W4A16 GEMV HBM throughput at M=1 on the Llama-3-8B decode linears.
One *step* = every W4A16 linear of one Llama-3-8B decode token: 32 layers x {qkv (K=4096, N=6144), o_proj (4096,
4096), gate+up (4096, 28672), down (14336, 4096)} = 128 GEMVs over 32 distinct weight sets (3.64 GB of packed weights,
far above the 256 MB Infinity Cache, so every weight byte comes from HBM).  Inputs are resident in HBM before timing;
the step is captured once as a HIP graph and replayed (launch overhead excluded, as a decode server runs it).
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
``cpu_baseline``: the C oracle (oracle/c/oracle.c, scalar, one thread) on a bounded sample of the same workload.

Usage: ``python bench.py [--steps K] [--warmup W] [--gpus 1]``; prints one JSON line.
``python bench.py --pmc-workload``: only a 256 MiB device copy (counter calibration) and 64 gate+up GEMV launches,
eager, for ``rocprofv3 --pmc`` passes.
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
# the launch the C library's policy makes for gate+up at M=1: one row of x, one 16-byte chunk per lane, 16 output
# channels per wavefront (two K slices of 2048 columns, four channel blocks per workgroup)
DOM_KERNEL = "w4_gemv_split_kernel<1,1,16,bf16>"
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


def time_graph(torch, fn, reps: int, warmup: int) -> float:
    """Capture fn() once as a HIP graph; replay `warmup` times, then `reps` times between HIP events (ms/replay)."""
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
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    st.record()
    for _ in range(reps):
        g.replay()
    en.record()
    torch.cuda.synchronize()
    return st.elapsed_time(en) / reps


def time_eager(torch, fn, reps: int, warmup: int) -> float:
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    st.record()
    for _ in range(reps):
        fn()
    en.record()
    torch.cuda.synchronize()
    return st.elapsed_time(en) / reps


def bench_w4_sweep(torch, ops, ring, dev, gen, timer, steps: int, warmup: int) -> tuple[dict, dict]:
    """configs[1] decode sweep at M in {4, 16, 64} (GB/s of algorithmic bytes, HIP-graph replays over the 32-layer
    ring) and configs[2] prefill at M in {512, 2048, 8192} (TFLOP/s against bf16 dense MFMA, one weight per shape)."""
    decode = {}
    for m in (4, 16, 64):
        row = {}
        xs = {k: torch.randn(m, k, device=dev, generator=gen).bfloat16() for k in {k for k, _ in SHAPES.values()}}
        for name, (k, n) in SHAPES.items():
            sel = [(xs[k], p) for nm, _, p in ring if nm == name]

            def run(sel=sel):
                for x, p in sel:
                    ops.w4a16_linear(x, p)

            t = timer(torch, run, steps, warmup) / len(sel)
            gbs = w4_bytes(m, k, n) / (t * 1e-3) / 1e9
            row[name] = {"us": round(t * 1e3, 3), "GBps": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
        decode[f"M{m}"] = row
        log(f"decode M={m}: " + "  ".join(f"{nm} {v['us']:.2f} us {v['GBps']:.0f} GB/s" for nm, v in row.items()))
    prefill = {}
    for m in (512, 2048, 8192):
        row = {}
        for name, (k, n) in SHAPES.items():
            p = next(p for nm, _, p in ring if nm == name)
            x = torch.randn(m, k, device=dev, generator=gen).bfloat16()
            fn = lambda x=x, p=p: ops.w4a16_linear(x, p)  # noqa: E731
            ms = time_eager(torch, fn, max(5, steps // 2), 2)
            tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
            row[name] = {"ms": round(ms, 4), "tflops": round(tf, 1), "frac": round(tf / BF16_PEAK_TFLOPS, 4)}
            del x
        prefill[f"M{m}"] = row
        log(f"prefill M={m}: " + "  ".join(f"{nm} {v['ms']:.3f} ms {v['tflops']:.0f} TF" for nm, v in row.items()))
    return decode, prefill


def bench_w8a16(torch, layouts, ops, dev, gen, timer, steps: int, warmup: int) -> dict:
    """W8A16 (int8 weight-only, per-channel fp16 scales) decode on the four Llama-3-8B shapes at M in {1, 16}: HBM
    GB/s of algorithmic bytes (N*K weights + 2*N scales + 2*M*K + 2*M*N), HIP-graph replays over a ring of distinct
    weights (at least 1.2 GB per shape)."""
    out = {}
    for name, (k, n) in SHAPES.items():
        nring = max(4, (1200 << 20) // (n * k) + 1)
        ring = [layouts.PackedW8(torch.randint(-128, 128, (n, k), dtype=torch.int8, device=dev, generator=gen),
                                 (torch.rand(1, n, device=dev, generator=gen) * 0.018 + 0.002).half(),
                                 layouts.PORTABLE_W8, n, k, -1) for _ in range(nring)]
        row = {}
        for m in (1, 16):
            x = torch.randn(m, k, device=dev, generator=gen).bfloat16()

            def run(x=x, ring=ring):
                for p in ring:
                    ops.w8a16_linear(x, p)

            t = timer(torch, run, steps, warmup) / len(ring)
            by = n * k + 2 * n + 2 * m * (k + n)
            row[f"M{m}"] = {"us": round(t * 1e3, 3), "GBps": round(by / (t * 1e-3) / 1e9, 1),
                            "frac": round(by / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        out[name] = row
        log(f"w8a16 {name:8s}: " + "  ".join(f"M={mm[1:]} {v['us']:.2f} us {v['GBps']:.0f} GB/s" for mm, v in row.items()))
        del ring
    return out


def bench_w8a8_small(torch, ops, dev, reps: int) -> dict:
    """configs[3] fp8 at M in {16, 256} (K = N = 8192) and configs[4] int8 at M in {1, 64} on the three 70B shapes:
    HBM-bound, reported in GB/s of algorithmic bytes (weights N*K + activations M*K + scales + bf16 output) and in
    TFLOP/s."""
    out = {}
    gen = torch.Generator(device=dev).manual_seed(11)
    k, n = 8192, 8192
    ring = [(torch.randn(n, k, device=dev, generator=gen) * 0.02).to(torch.float8_e4m3fn) for _ in range(6)]
    sw = torch.rand(n, device=dev, generator=gen) * 0.01
    for m in (16, 256):
        xq = torch.randn(m, k, device=dev, generator=gen).to(torch.float8_e4m3fn)
        sx = torch.rand(m, device=dev, generator=gen) * 0.01

        def run(xq=xq, sx=sx):
            for w in ring:
                ops.fp8_linear(xq, w, sw, x_scale=sx, out_dtype=torch.bfloat16)

        ms = time_eager(torch, run, reps, 3) / len(ring)
        by = n * k + m * k + 4 * (m + n) + 2 * m * n
        out[f"fp8_m{m}_k{k}_n{n}"] = {"us": round(ms * 1e3, 2), "GBps": round(by / (ms * 1e-3) / 1e9, 1),
                                      "tflops": round(2.0 * m * n * k / (ms * 1e-3) / 1e12, 1)}
        log(f"fp8 M={m} K=N=8192: {ms * 1e3:.1f} us  {out[f'fp8_m{m}_k{k}_n{n}']['GBps']:.0f} GB/s")
    del ring
    for (k8, n8) in ((8192, 10240), (8192, 57344), (28672, 8192)):
        nring = max(2, min(6, (1536 << 20) // (n8 * k8)))
        ring = [torch.randint(-127, 128, (n8, k8), dtype=torch.int8, device=dev, generator=gen) for _ in range(nring)]
        swi = torch.rand(n8, device=dev, generator=gen) * 0.01
        for m in (1, 64):
            xi = torch.randint(-127, 128, (m, k8), dtype=torch.int8, device=dev, generator=gen)
            sxi = torch.rand(m, device=dev, generator=gen) * 0.01

            def run(xi=xi, sxi=sxi):
                for w in ring:
                    ops.int8_linear(xi, w, swi, x_scale=sxi, out_dtype=torch.bfloat16)

            ms = time_eager(torch, run, reps, 3) / len(ring)
            by = n8 * k8 + m * k8 + 4 * (m + n8) + 2 * m * n8
            key = f"int8_m{m}_k{k8}_n{n8}"
            out[key] = {"us": round(ms * 1e3, 2), "GBps": round(by / (ms * 1e-3) / 1e9, 1),
                        "frac": round(by / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
            log(f"int8 M={m} K={k8} N={n8}: {ms * 1e3:.1f} us  {out[key]['GBps']:.0f} GB/s")
        del ring
    return out


def bench_w8a8(torch, ops, dev, reps: int) -> dict:
    out = {}
    gen = torch.Generator(device=dev).manual_seed(7)
    m, k, n = 4096, 8192, 8192
    x = torch.randn(m, k, device=dev, generator=gen).bfloat16()
    w = torch.randn(n, k, device=dev, generator=gen) * 0.02
    xq, sx = ops.quantize_act_fp8(x)
    wq, sw = ops.quantize_weight_fp8(w, "per_channel")
    del w
    fn = lambda: ops.fp8_linear(xq, wq, sw, x_scale=sx, out_dtype=torch.bfloat16)  # noqa: E731
    ms = time_eager(torch, fn, reps, 3)
    tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    out["fp8_m4096_k8192_n8192"] = {"ms": round(ms, 4), "tflops": round(tf, 1), "frac": round(tf / FP8_PEAK_TFLOPS, 4)}
    log(f"fp8 M=4096 K=N=8192: {ms:.3f} ms  {tf:.0f} TFLOP/s")
    del xq, wq, x
    for (k8, n8) in ((8192, 10240), (8192, 57344), (28672, 8192)):
        xi = torch.randint(-127, 128, (m, k8), dtype=torch.int8, device=dev, generator=gen)
        wi = torch.randint(-127, 128, (n8, k8), dtype=torch.int8, device=dev, generator=gen)
        sxi = torch.rand(m, device=dev, generator=gen) * 0.01
        swi = torch.rand(n8, device=dev, generator=gen) * 0.01
        fn = lambda: ops.int8_linear(xi, wi, swi, x_scale=sxi, out_dtype=torch.bfloat16)  # noqa: E731
        ms = time_eager(torch, fn, reps, 3)
        tops = 2.0 * m * n8 * k8 / (ms * 1e-3) / 1e12
        out[f"int8_m4096_k{k8}_n{n8}"] = {"ms": round(ms, 4), "tops": round(tops, 1),
                                          "frac": round(tops / INT8_PEAK_TOPS, 4)}
        log(f"int8 M=4096 K={k8} N={n8}: {ms:.3f} ms  {tops:.0f} TOP/s")
        del xi, wi
    return out


def pmc_workload(torch, layouts, ops, dev, gen) -> None:
    """Counter-pass workload: a 256 MiB device-to-device copy (known bytes: calibrates FETCH_SIZE / WRITE_SIZE) three
    times, then the gate+up GEMV (K=4096, N=28672, M=1) over a ring of 32 weights, twice (64 launches)."""
    src = torch.empty(64 << 20, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    k, n = SHAPES["gate_up"]
    x = torch.randn(1, k, device=dev, generator=gen).bfloat16()
    ring = [make_layer_weights(torch, layouts, dev, k, n, gen) for _ in range(LAYERS)]
    torch.cuda.synchronize()
    for _ in range(2):
        for p in ring:
            ops.w4a16_linear(x, p)
    torch.cuda.synchronize()
    log("pmc workload done: 3 x 256 MiB copy, 64 gate_up GEMV launches")


def load_traffic() -> dict | None:
    """HBM bytes per gate+up launch from the committed counter summary (None when absent or measured on another
    kernel than the one the policy runs now)."""
    path = os.path.join(ROOT, "profiles", "w4_gemv_gate_up_pmc.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        tr = json.load(f)
    return tr if tr.get("kernel", "").split(" ")[0] == DOM_KERNEL.split("<")[0] else None


def cpu_baseline(seconds: float = 12.0) -> dict:
    """The scalar C oracle (one thread) on one decode layer's four W4A16 linears at M=1, repeated to ~`seconds`."""
    import numpy as np

    from oracle import c_oracle
    from oracle import w4 as ow

    rng = np.random.default_rng(0)
    layer = []
    for name, (k, n) in SHAPES.items():
        G = k // GROUP
        p = {"qweight": rng.integers(-2 ** 31, 2 ** 31 - 1, size=(n, k // 8), dtype=np.int64).astype(np.int32),
             "scales": (rng.random((G, n)) * 0.018 + 0.002).astype(np.float16).astype(np.float32),
             "zeros": ow.pack_nibbles_int32(rng.integers(6, 10, size=(G, n // 8, 8), dtype=np.uint8)),
             "g_idx": None, "n": n, "k": k, "group_size": GROUP}
        layer.append((p, rng.standard_normal((1, k)).astype(np.float32), w4_bytes(1, k, n)))
    c_oracle.w4a16_gemm(layer[1][1], layer[1][0])  # load the library
    done_bytes, reps, t0 = 0, 0, time.perf_counter()
    while True:
        for p, x, b in layer:
            c_oracle.w4a16_gemm(x, p)
            done_bytes += b
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"value": round(done_bytes / el / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{reps} pass(es) over one Llama-3-8B layer's 4 W4A16 linears at M=1 "
                      f"(qkv, o_proj, gate_up, down; {sum(b for _, _, b in layer) / 1e6:.1f} MB per pass), "
                      f"scalar C oracle oracle/c/oracle.c, {el:.1f} s"}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-w8a8", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-sweep", action="store_true", help="skip the W4A16 M=4..64 decode and prefill sweeps")
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of a captured HIP graph")
    ap.add_argument("--pmc-workload", action="store_true", help="run only the counter-pass workload (no timing)")
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
        pmc_workload(torch, layouts, ops, dev, gen)
        return
    ring = []  # (name, x, packed)
    xs = {k: torch.randn(1, k, device=dev, generator=gen).bfloat16() for k in {k for k, _ in SHAPES.values()}}
    for layer in range(LAYERS):
        for name, (k, n) in SHAPES.items():
            ring.append((name, xs[k], make_layer_weights(torch, layouts, dev, k, n, gen)))
    torch.cuda.synchronize()
    step_bytes = sum(w4_bytes(1, p.k, p.n) for _, _, p in ring)
    log(f"ring: {len(ring)} linears, {sum(p.nbytes for _, _, p in ring) / 1e9:.2f} GB packed weights")

    def step():
        for _, x, p in ring:
            ops.w4a16_linear(x, p)

    timer = time_eager if args.eager else time_graph
    ms = timer(torch, step, args.steps, args.warmup)
    value = step_bytes / (ms * 1e-3) / 1e9
    log(f"step: {ms:.4f} ms, {value:.1f} GB/s ({value / HBM_PEAK_GBS:.1%} of 8 TB/s)")

    per_shape = {}
    for name, (k, n) in SHAPES.items():
        sel = [(x, p) for nm, x, p in ring if nm == name]

        def run(sel=sel):
            for x, p in sel:
                ops.w4a16_linear(x, p)

        t = timer(torch, run, args.steps, args.warmup) / len(sel)
        gbs = w4_bytes(1, k, n) / (t * 1e-3) / 1e9
        per_shape[name] = {"K": k, "N": n, "us": round(t * 1e3, 3), "GBps": round(gbs, 1),
                           "frac": round(gbs / HBM_PEAK_GBS, 4)}
        log(f"  {name:8s} K={k:5d} N={n:5d}: {t * 1e3:8.3f} us  {gbs:7.1f} GB/s")
    dom = per_shape["gate_up"]
    tr = load_traffic()
    roofline = {"bound": "hbm", "achieved": dom["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(dom["GBps"] / HBM_PEAK_GBS, 4), "traffic": None if tr is None else tr["traffic_bytes"],
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
           "frac_of_peak": round(value / HBM_PEAK_GBS, 4), "per_shape": per_shape, "roofline": roofline}
    if not args.no_sweep:
        out["w4_decode_sweep"], out["w4_prefill"] = bench_w4_sweep(torch, ops, ring, dev, gen, timer, args.steps,
                                                                   args.warmup)
    del ring
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
