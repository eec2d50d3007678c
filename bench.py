"""Benchmark of the GEMM-with-fused-epilogue path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--copy-probe]
    python bench.py --ref-table

A step is one call of hk.templates.gemm on BASELINE.json's config 2 -- the workload its
metric is quoted on: x bf16[4096, 4096] ~N(0,1), w bf16[4096 (K), 12288 (N)] ~N(0, 0.02)
(handed to the GEMM once, untimed, as w.t().contiguous(): F.linear's (N, K)), b
bf16[12288] ~N(0, 0.1); y = gelu_tanh(x @ w + b), fp32 accumulate. Synthetic data,
resident in HBM before the timed region.

Prints ONE JSON line: the metric and its value (whole-job TFLOP/s), the roofline of the
dominant kernel (achieved TFLOP/s from HIP events around each launch, against the
2.5 PFLOP/s bf16 dense peak, and against this GPU's own ceilings measured in the same run:
a register-only MFMA loop on constant operands, and the same loop on random operands --
the rate the board's power limit allows on data that toggles like real tensors), the CPU
baseline (the oracle, torch fp32 on the host
cores, on a bounded sample), and, under "also", the other BASELINE configs measured the
same way: the fused gate_up + silu_and_mul GEMM, the decode GEMMs (HBM GB/s of W, with
weight copies rotated past the 256 MB Infinity Cache; kernel time from a replayed graph,
since a ~20 us launch is shorter than the host's per-call overhead) and the fp8 scaled
GEMM. Before the warmup steps, each workload runs untimed for a quarter of a second: the
GPU's clocks settle only after tens of milliseconds of load.

`--ref-table` instead times the 48 calls of the reference's published template table (see
ref_table) and prints one JSON line with this build's time beside the reference's for each.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "hk-dsl_amd"))
sys.path.insert(0, ROOT)

METRIC = "TFLOP/s & % MFMA peak (prefill M), HBM GB/s & % peak (decode M≤16)"
PEAK_BF16, PEAK_FP8, PEAK_HBM = 2500.0, 5000.0, 8000.0


def _ramp(fn, seconds=0.25):
    """Untimed calls until `seconds` of device work have run: the GPU's clocks take tens of
    milliseconds of load to settle (a 20 ms burst from idle runs ~15% slower than the same
    burst after it), which a few warmup steps do not cover."""
    import torch

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()


RAMP_S = 0.25


def _events_time(fn, steps, warmup, ramp=True):
    """Average device time of one call (HIP events on the current stream, which the
    kernels launch on) and the wall time of `steps` calls bracketed by synchronize."""
    import torch

    if ramp and RAMP_S > 0:
        _ramp(fn, RAMP_S)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = [s.elapsed_time(e) * 1e-3 for s, e in zip(starts, ends)]
    return statistics.mean(per), statistics.median(per), wall


def _wall_time(fn, steps, warmup):
    """Wall time of `steps` calls bracketed by synchronize, after the ramp and `warmup`
    untimed calls: the whole-job figure, with nothing but the calls in the timed region
    (the per-launch events of _events_time add a few µs a step)."""
    import torch

    if RAMP_S > 0:
        _ramp(fn, RAMP_S)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def _graph_time(calls, reps=7):
    """Device time of one call of `calls`, captured in one HIP graph and replayed (median of
    `reps` replays): the kernel time of launches shorter than the host's call overhead."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for c in calls:
            c()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for c in calls:
            c()
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        g.replay()
        t1.record()
        torch.cuda.synchronize()
        ts.append(t0.elapsed_time(t1) * 1e-3 / len(calls))
    return statistics.median(ts)


def _inputs(m, k, n, seed, dev):
    import torch

    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = (torch.randn(k, n, generator=g) * 0.02).to(torch.bfloat16)
    b = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16)
    return x.to(dev), w.t().contiguous().to(dev), b.to(dev)


def _cpu_median(fn, runs=5):
    fn()  # warm-up
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def cpu_baseline(x, wt, b):
    """The oracle on the host (torch fp32 closed forms, all host threads), each BASELINE
    config on the same seeded inputs as its GPU arm, the median of 5 timed runs after a
    warm-up. The top-level figure is config 2's, the bench's workload; "configs" holds
    each config's own. Config 3 at M = 8192 runs on a bounded row sample (1024 rows of x:
    a GEMM's rate is flat in M at these sizes), named in its "sample"."""
    import torch

    from oracle import gemm_oracle as O

    torch.set_num_threads(os.cpu_count() or 1)
    threads = torch.get_num_threads()
    xc, wc, bc = x.cpu().float(), wt.cpu().float().t().contiguous(), b.cpu().float()
    m, k = xc.shape
    n = wc.shape[1]
    t2 = _cpu_median(lambda: O.linear_bias_gelu(xc, wc, bc))
    cfgs = {}

    def put(name, flops, t, sample, byts=None):
        r = {"TFLOP/s": round(flops / t / 1e12, 4), "s_per_run": round(t, 5), "sample": sample}
        if byts is not None:
            r["GB/s"] = round(byts / t / 1e9, 2)
        cfgs[name] = r

    put("cfg2_bias_gelu", 2.0 * m * n * k, t2, f"full {m}x{k}x{n}")
    # config 1: linear_bias_gelu 256 x 1024 x 1024
    x1, w1, b1 = (t.cpu().float() for t in _inputs(256, 1024, 1024, 1, "cpu"))
    w1 = w1.t().contiguous()
    put("cfg1_bias_gelu", 2.0 * 256 * 1024 * 1024,
        _cpu_median(lambda: O.linear_bias_gelu(x1, w1, b1)), "full 256x1024x1024")
    # config 3: gate_up + silu_and_mul, w (4096, 24576)
    x3, w3, _ = (t.cpu().float() for t in _inputs(2048, 4096, 24576, 3, "cpu"))
    w3 = w3.t().contiguous()

    def c3(xs):
        h = xs @ w3
        return O.silu_and_mul(h[:, :12288], h[:, 12288:])
    put("cfg3_gate_up_silu_mul_M2048", 2.0 * 2048 * 24576 * 4096, _cpu_median(lambda: c3(x3)),
        "full M=2048")
    put("cfg3_gate_up_silu_mul_M8192", 2.0 * 1024 * 24576 * 4096, _cpu_median(lambda: c3(x3[:1024])),
        "1024 of the 8192 rows (the rate of the full call, flops counted for the rows run)")
    del x3, w3
    # config 4: decode y = x @ W^T (+ bias), W (12288, 4096)
    w4 = _inputs(1, 4096, 12288, 40, "cpu")[1].float()
    b4 = _inputs(1, 4096, 12288, 4, "cpu")[2].float()
    for m4 in (1, 4, 16):
        x4 = _inputs(m4, 4096, 12288, 4, "cpu")[0].float()
        byts = 12288 * 4096 * 2 + m4 * 4096 * 2 + m4 * 12288 * 2
        put(f"cfg4_decode_M{m4}_bias", 2.0 * m4 * 12288 * 4096,
            _cpu_median(lambda: O.apply_epilogue("bias", O.gemm_fp32(x4, w4), bias=b4)),
            f"full M={m4} (GB/s counts W, x and y at bf16 size, as the GPU arm)", byts)
    del w4
    # config 5: fp8 scaled + dequant + bias, 8192 x 4096 x 4096 (fp8 values exact in fp32)
    g = torch.Generator().manual_seed(5)
    x5 = torch.randn(8192, 4096, generator=g).to(torch.float8_e4m3fn)
    w5 = torch.randn(4096, 4096, generator=g).to(torch.float8_e4m3fn).t().contiguous()
    sa = (torch.rand(8192, 1, generator=g) * 1.5 + 0.5) / 448
    sb = (torch.rand(4096, generator=g) * 1.5 + 0.5) / 448
    bias = (torch.randn(4096, generator=g) * 0.1).to(torch.bfloat16)
    put("cfg5_fp8_scaled_dequant_bias", 2.0 * 8192 * 4096 * 4096,
        _cpu_median(lambda: O.scaled_mm(x5, w5, sa, sb, bias)), "full 8192x4096x4096")
    return {"value": round(2 * m * n * k / t2 / 1e12, 3), "unit": "TFLOP/s",
            "cores": threads, "kind": "port",
            "sample": f"oracle linear_bias_gelu at the full config-2 size {m}x{k}x{n} (fp32), "
                      f"median of 5 runs after a warm-up, {t2:.2f} s each; "
                      f"torch.get_num_threads() = {threads}, os.cpu_count() = {os.cpu_count()}",
            "configs": cfgs}


#: The reference's published device times of hk.templates.gemm on MI355X, µs: (layer,
#: N, K, M, epilogue, time) -- the "template" column of docs/templates/gemm.md:273-324
#: (Qwen3-8B's and Llama-3-8B's linear layers; bias + GELU(tanh) and a residual add; a
#: replayed graph of the calls). Data only, compared against in ref_table.
REF_TABLE = [
    ('qwen3-8b o_proj', 4096, 4096, 16, 'bias_gelu', 9.1),
    ('qwen3-8b o_proj', 4096, 4096, 128, 'bias_gelu', 14.5),
    ('qwen3-8b o_proj', 4096, 4096, 1024, 'bias_gelu', 37.3),
    ('qwen3-8b o_proj', 4096, 4096, 4096, 'bias_gelu', 99.1),
    ('qwen3-8b down', 4096, 12288, 16, 'bias_gelu', 19.3),
    ('qwen3-8b down', 4096, 12288, 128, 'bias_gelu', 27.7),
    ('qwen3-8b down', 4096, 12288, 1024, 'bias_gelu', 88.7),
    ('qwen3-8b down', 4096, 12288, 4096, 'bias_gelu', 266.2),
    ('llama3-8b down', 4096, 14336, 16, 'bias_gelu', 21.4),
    ('llama3-8b down', 4096, 14336, 128, 'bias_gelu', 29.9),
    ('llama3-8b down', 4096, 14336, 1024, 'bias_gelu', 99.3),
    ('llama3-8b down', 4096, 14336, 4096, 'bias_gelu', 311.5),
    ('qwen3-8b qkv', 6144, 4096, 16, 'bias_gelu', 12.3),
    ('qwen3-8b qkv', 6144, 4096, 128, 'bias_gelu', 18.2),
    ('qwen3-8b qkv', 6144, 4096, 1024, 'bias_gelu', 57.2),
    ('qwen3-8b qkv', 6144, 4096, 4096, 'bias_gelu', 155.0),
    ('qwen3-8b gate_up', 24576, 4096, 16, 'bias_gelu', 36.7),
    ('qwen3-8b gate_up', 24576, 4096, 128, 'bias_gelu', 35.2),
    ('qwen3-8b gate_up', 24576, 4096, 1024, 'bias_gelu', 175.1),
    ('qwen3-8b gate_up', 24576, 4096, 4096, 'bias_gelu', 595.0),
    ('llama3-8b gate_up', 28672, 4096, 16, 'bias_gelu', 34.5),
    ('llama3-8b gate_up', 28672, 4096, 128, 'bias_gelu', 40.6),
    ('llama3-8b gate_up', 28672, 4096, 1024, 'bias_gelu', 197.6),
    ('llama3-8b gate_up', 28672, 4096, 4096, 'bias_gelu', 697.6),
    ('qwen3-8b o_proj', 4096, 4096, 16, 'residual', 9.1),
    ('qwen3-8b o_proj', 4096, 4096, 128, 'residual', 14.6),
    ('qwen3-8b o_proj', 4096, 4096, 1024, 'residual', 39.5),
    ('qwen3-8b o_proj', 4096, 4096, 4096, 'residual', 98.4),
    ('qwen3-8b down', 4096, 12288, 16, 'residual', 19.2),
    ('qwen3-8b down', 4096, 12288, 128, 'residual', 27.9),
    ('qwen3-8b down', 4096, 12288, 1024, 'residual', 90.3),
    ('qwen3-8b down', 4096, 12288, 4096, 'residual', 264.5),
    ('llama3-8b down', 4096, 14336, 16, 'residual', 21.4),
    ('llama3-8b down', 4096, 14336, 128, 'residual', 30.1),
    ('llama3-8b down', 4096, 14336, 1024, 'residual', 100.3),
    ('llama3-8b down', 4096, 14336, 4096, 'residual', 315.6),
    ('qwen3-8b qkv', 6144, 4096, 16, 'residual', 12.3),
    ('qwen3-8b qkv', 6144, 4096, 128, 'residual', 18.3),
    ('qwen3-8b qkv', 6144, 4096, 1024, 'residual', 57.6),
    ('qwen3-8b qkv', 6144, 4096, 4096, 'residual', 155.1),
    ('qwen3-8b gate_up', 24576, 4096, 16, 'residual', 36.0),
    ('qwen3-8b gate_up', 24576, 4096, 128, 'residual', 35.3),
    ('qwen3-8b gate_up', 24576, 4096, 1024, 'residual', 178.7),
    ('qwen3-8b gate_up', 24576, 4096, 4096, 'residual', 597.9),
    ('llama3-8b gate_up', 28672, 4096, 16, 'residual', 34.1),
    ('llama3-8b gate_up', 28672, 4096, 128, 'residual', 40.4),
    ('llama3-8b gate_up', 28672, 4096, 1024, 'residual', 200.0),
    ('llama3-8b gate_up', 28672, 4096, 4096, 'residual', 703.0),
]


def ref_table():
    """hk.templates.gemm on each REF_TABLE call, as the reference timed it (a graph of 16
    calls replayed, the median of 15 replays a call, after RAMP_S of untimed replays): with
    one weight copy ("hot", as a
    replay of the same calls reads it) and with four copies rotated past the 256 MB
    Infinity Cache ("cold"). Each call is checked against the fp32 result first."""
    import torch

    import hk

    T = hk.templates.gemm
    dev = "cuda:0"
    g = torch.Generator().manual_seed(0)

    def graph_us(calls):
        st = torch.cuda.Stream()
        st.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(st):
            for c in calls[:3]:
                c()
        torch.cuda.current_stream().wait_stream(st)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for c in calls:
                c()
        for _ in range(3):
            gr.replay()
        torch.cuda.synchronize()
        # the clocks settle only after tens of milliseconds of load, as for the main bench
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < RAMP_S:
            gr.replay()
            torch.cuda.synchronize()
        ts = []
        for _ in range(15):
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            gr.replay()
            e.record()
            e.synchronize()
            ts.append(s.elapsed_time(e) * 1e3 / len(calls))
        return statistics.median(ts)

    rows, weights = [], {}
    for layer, n, k, m, ep, ref_us in REF_TABLE:
        if (n, k) not in weights:
            weights.clear()
            torch.cuda.empty_cache()
            weights[(n, k)] = [(torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16).to(dev)
                               for _ in range(4)]
        ws = weights[(n, k)]
        x = torch.randn(m, k, generator=g).to(torch.bfloat16).to(dev)
        b = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16).to(dev)
        r = torch.randn(m, n, generator=g).to(torch.bfloat16).to(dev)
        y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)

        def call(w, ep=ep, x=x, b=b, r=r, y=y):
            if ep == "bias_gelu":
                T(x, w, epilogue=T.bias_gelu, bias=b, out=y)
            else:
                T(x, w, epilogue=T.residual, residual=r, out=y)

        call(ws[0])
        acc = x.float() @ ws[0].float().t()
        want = (torch.nn.functional.gelu(acc + b.float(), approximate="tanh") if ep == "bias_gelu"
                else acc + r.float())
        torch.testing.assert_close(y.float(), want, rtol=1e-2, atol=4e-2)
        hot = graph_us([lambda: call(ws[0]) for _ in range(16)])
        cold = graph_us([lambda i=i: call(ws[i % 4]) for i in range(16)])
        rows.append({"layer": layer, "N": n, "K": k, "M": m, "epilogue": ep,
                     "reference_us": ref_us, "hot_us": round(hot, 2), "cold_us": round(cold, 2),
                     "reference_over_hot": round(ref_us / hot, 3)})
    under = sum(1 for x in rows if x["hot_us"] <= x["reference_us"])
    within10 = sum(1 for x in rows if x["reference_over_hot"] >= 0.9)
    print(json.dumps({"ref_table": "docs/templates/gemm.md:273-324 (reference, template column)",
                      "calls": len(rows), "at_or_under_reference": under,
                      "within_10pct": within10, "rows": rows}))


ARMS = ["cfg2_bias_gelu", "cfg2_plain", "cfg2_hipblaslt", "cfg2_bias_gelu_zero_x",
        "cfg5_deq_bias", "cfg5_deq_bias_zero_x", "cfg5_torch_scaled_mm", "cfg2_plain_4wave"]


def arms():
    """The workload of the clock-and-cycles profile: config 2 (bias + GELU, plain, hipBLASLt's
    plain GEMM through torch.matmul, bias + GELU on an all-zero x), config 5 (dequant +
    bias, the same on an all-zero x, torch._scaled_mm) and config 2's plain GEMM on the
    4-wave kernel (one wave a SIMD, 128 x 128 a wave), each 0.4 s of untimed calls, a
    50 ms pause, 30 calls, a 50 ms pause -- so a trace splits into the arms by its gaps. Run
    under rocprofv3 twice: --kernel-trace, and --pmc GRBM_GUI_ACTIVE ...; then
    `bench.py --arms-summary TRACE_DIR PMC_DIR` prints the table."""
    import torch

    import hk

    T = hk.templates.gemm
    dev = "cuda:0"
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(4096, 4096, device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn(12288, 4096, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    b = (torch.randn(12288, device=dev, generator=g) * 0.1).to(torch.bfloat16)
    y = torch.empty(4096, 12288, device=dev, dtype=torch.bfloat16)
    zx = torch.zeros_like(x)
    x8 = torch.randn(8192, 4096, device=dev, generator=g).to(torch.float8_e4m3fn)
    w8 = torch.randn(4096, 4096, device=dev, generator=g).to(torch.float8_e4m3fn)
    z8 = torch.zeros_like(x8)
    sa = (torch.rand(8192, 1, device=dev, generator=g) * 1.5 + 0.5) / 448
    sb = (torch.rand(4096, device=dev, generator=g) * 1.5 + 0.5) / 448
    b5 = (torch.randn(4096, device=dev, generator=g) * 0.1).to(torch.bfloat16)
    y5 = torch.empty(8192, 4096, device=dev, dtype=torch.bfloat16)
    sm = hk.ops.scaled_mm
    fns = [lambda: T(x, w, epilogue=T.bias_gelu, bias=b, out=y),
           lambda: T(x, w, out=y),
           lambda: torch.matmul(x, w.t(), out=y),
           lambda: T(zx, w, epilogue=T.bias_gelu, bias=b, out=y),
           lambda: sm(x8, w8, sa, sb, bias=b5, out=y5),
           lambda: sm(z8, w8, sa, sb, bias=b5, out=y5),
           lambda: torch._scaled_mm(x8, w8.t(), scale_a=sa, scale_b=sb.reshape(1, -1),
                                    out_dtype=torch.bfloat16),
           lambda: T(x, w, out=y, schedule="t256w4")]
    for name, fn in zip(ARMS, fns):
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < 0.4:
            fn()
        torch.cuda.synchronize()
        time.sleep(0.05)
        for _ in range(30):
            fn()
        torch.cuda.synchronize()
        time.sleep(0.05)
        print(name, flush=True)


def arms_summary(trace_dir, pmc_dir):
    """The clock-and-cycles table from the two rocprofv3 runs of `arms`: per arm, the
    median kernel time of its 30 timed calls (kernel trace), the median GRBM_GUI_ACTIVE of
    the same calls divided by the 8 XCDs (the counter sums them) -- cycles a launch --,
    their ratio (the clock the launch ran at), and the fraction of the datasheet peak at
    that clock and at 2.4 GHz (the cycles alone)."""
    import collections
    import csv

    def gemm(name):
        return "quad" in name or "Cijk" in name or "tile4" in name

    def by_gap(items, st, en):
        out, last = [], None
        for it in items:
            if last is None or st(it) - last > 20e6:
                out.append([])
            out[-1].append(it)
            last = en(it)
        return out[1::2]  # each arm: its untimed calls, then (after the pause) the 30 timed

    rows = sorted((r for r in csv.DictReader(open(os.path.join(trace_dir, "run_kernel_trace.csv")))
                   if gemm(r["Kernel_Name"])), key=lambda r: int(r["Start_Timestamp"]))
    tarms = by_gap(rows, lambda r: int(r["Start_Timestamp"]), lambda r: int(r["End_Timestamp"]))
    disp = collections.OrderedDict()
    for r in csv.DictReader(open(os.path.join(pmc_dir, "run_counter_collection.csv"))):
        if gemm(r["Kernel_Name"]):
            e = disp.setdefault(int(r["Dispatch_Id"]), {"st": int(r["Start_Timestamp"]),
                                                         "en": int(r["End_Timestamp"]),
                                                         "c": collections.Counter()})
            e["c"][r["Counter_Name"]] += float(r["Counter_Value"])
    carms = by_gap(sorted(disp.values(), key=lambda e: e["st"]), lambda e: e["st"], lambda e: e["en"])
    flops = {"cfg2": 2.0 * 4096 * 4096 * 12288, "cfg5": 2.0 * 8192 * 4096 * 4096}
    peak = {"cfg2": PEAK_BF16 * 1e12, "cfg5": PEAK_FP8 * 1e12}
    print("| arm | kernel | median µs | cycles a launch | clock GHz | frac of peak | frac at 2.4 GHz |")
    print("|---|---|---:|---:|---:|---:|---:|")
    for name, ta, ca in zip(ARMS, tarms, carms):
        us = statistics.median((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in ta[-30:])
        cyc = statistics.median(c["c"]["GRBM_GUI_ACTIVE"] for c in ca[-30:]) / 8
        kn = ta[-1]["Kernel_Name"]
        kn = kn[:kn.find("(")] if "(" in kn else kn[:48]
        f, pk = flops[name[:4]], peak[name[:4]]
        print(f"| {name} | `{kn}` | {us:.1f} | {cyc / 1e3:.0f} K | {cyc / us / 1e3:.2f} | "
              f"{f / (us * 1e-6) / pk:.3f} | {f / (cyc / 2.4e9) / pk:.3f} |")
    # every other counter of the run: median over the timed calls, millions, summed over the chip
    names = sorted({k for a in carms for c in a for k in c["c"]} - {"GRBM_GUI_ACTIVE"})
    if names:
        print()
        print("| arm | " + " | ".join(names) + " |")
        print("|---|" + "---:|" * len(names))
        for name, ca in zip(ARMS, carms):
            vals = [statistics.median(c["c"][k] for c in ca[-30:]) / 1e6 for k in names]
            print(f"| {name} | " + " | ".join(f"{v:.2f}" for v in vals) + " |")


def main():
    global RAMP_S
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--quick", action="store_true", help="config 2 only, no CPU baseline")
    ap.add_argument("--ramp", type=float, default=RAMP_S,
                    help="seconds of untimed work before the warmup steps (0 under a profiler)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a 1 GiB device copy (the scale of rocprof's FETCH/WRITE_SIZE)")
    ap.add_argument("--ref-table", action="store_true",
                    help="time the reference's published template table instead (one JSON line)")
    ap.add_argument("--arms", action="store_true",
                    help="run the clock-and-cycles profile's workload instead (see arms)")
    ap.add_argument("--arms-summary", nargs=2, metavar=("TRACE_DIR", "PMC_DIR"),
                    help="print the clock-and-cycles table from two rocprofv3 runs of --arms")
    args = ap.parse_args()
    RAMP_S = args.ramp
    if args.arms_summary:
        arms_summary(*args.arms_summary)
        return
    if args.arms:
        arms()
        return
    if args.ref_table:
        ref_table()
        return
    if args.gpus != 1:
        print(f"bench.py: this path runs on one GPU; --gpus {args.gpus} is not measured "
              f"(the GEMM shards over M or N with no exchange, or over K with one all-reduce "
              f"before the epilogue)", file=sys.stderr)
        sys.exit(2)

    import torch

    import hk
    from hk import _native as nat

    dev = "cuda:0"
    T = hk.templates.gemm
    m, k, n = 4096, 4096, 12288
    x, wt, b = _inputs(m, k, n, 0, dev)
    out = torch.empty(m, n, device=dev, dtype=torch.bfloat16)
    step = lambda: T(x, wt, epilogue=T.bias_gelu, bias=b, out=out)  # noqa: E731
    # parity first: the measured arm is checked against the fp32 reference
    ref = torch.nn.functional.gelu(x.float() @ wt.float().t() + b.float(), approximate="tanh")
    step()
    torch.testing.assert_close(out.float(), ref, rtol=1e-2, atol=1e-2)
    del ref
    flops = 2.0 * m * n * k
    peaks = measured_peaks()
    wall = _wall_time(step, args.steps, args.warmup)
    value = flops * args.steps / wall / 1e12
    # the dominant kernel's launch time: HIP events around each launch, on the stream the
    # kernel is launched on, over a second pass of the same steps (clocks already settled)
    mean_s, med_s, _ = _events_time(step, args.steps, 0, ramp=False)
    achieved = flops / mean_s / 1e12
    plan = T.plan(m, n, k)
    sched = plan[0].sched.get("schedule")
    variant = plan[0].sched.get("variant", 0) or 0
    # the ring schedule runs this form (bf16, a bias and an activation) on the quadrant
    # kernel unless the half-stage ring is asked for
    ring = ("hkx::ring_kernel<bf16, kStore16, GELU_TANH, kEpBias>" if variant & nat.RING_HALFSTAGE
            else "hkx::quad_kernel<GELU_TANH, kEpBias>")
    kname = {"ring": ring,
             "pp": "hkx::pp_kernel<bf16, kStore16, GELU_TANH, mfma16>",
             "w4": "hkx::tile4_kernel<256, 256, bf16, kStore16, GELU_TANH>"}.get(sched, str(sched))
    res = {
        "metric": METRIC, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded ~N(0,1) x, ~N(0,0.02) w, ~N(0,0.1) b; resident in HBM)",
        "config": {"workload": "config 2: bias+gelu_tanh, x bf16[4096,4096] @ w bf16[4096,12288] + b",
                   "M": m, "N": n, "K": k, "epilogue": "bias_gelu (fused in registers)",
                   "route": plan[0].route, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16, 4), "traffic": None,
                     "peak_measured": peaks["mfma_bf16_tflops"],
                     "frac_measured": round(achieved / peaks["mfma_bf16_tflops"], 4),
                     "peak_measured_random_operands": peaks["mfma_bf16_random_operands_tflops"],
                     "frac_measured_random_operands": round(achieved / peaks["mfma_bf16_random_operands_tflops"], 4),
                     "kernel": kname,
                     "avg_launch_us": round(mean_s * 1e6, 2), "median_launch_us": round(med_s * 1e6, 2),
                     "algorithmic_flops_per_launch": flops},
    }
    # HBM bytes a launch of this kernel moves, from the rocprofv3 FETCH_SIZE / WRITE_SIZE
    # runs summarised under profiles/ (null if they were taken on another kernel)
    # (FETCH_SIZE + WRITE_SIZE: the L2's misses, of which the 256 MB Infinity Cache serves
    # part, so an upper bound on HBM bytes; taken in the profiled runs named in that file)
    tr = os.path.join(ROOT, "profiles", "traffic_quad_bias_gelu_cfg2.json")
    if os.path.isfile(tr):
        with open(tr) as f:
            rec = json.load(f)
        if rec.get("kernel") == kname:
            res["roofline"]["traffic"] = rec.get("l2_miss_bytes_per_launch")
            res["roofline"]["traffic_source"] = (
                "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (L2-miss bytes, scaled by a 1 GiB "
                "copy; an upper bound on HBM bytes: the Infinity Cache serves part of them), "
                "from the runs in profiles/traffic_quad_bias_gelu_cfg2.json")
    res["measured_peaks"] = peaks
    if not args.quick:
        res["also"] = other_configs(args.steps, args.warmup, peaks)
        del x, wt, b, out
        torch.cuda.empty_cache()
        res["cpu_baseline"] = cpu_baseline(*_inputs(m, k, n, 0, "cpu"))
    else:
        res["cpu_baseline"] = None
    if args.copy_probe:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        res["copy_probe_bytes"] = src.numel() * 4
    print(json.dumps(res), flush=True)


def measured_peaks():
    """This GPU's own ceilings, measured in this run with the build's probe (hk.peaks):
    the dense MFMA rate of a register-only loop (bf16, fp8) and the HBM read rate over four
    1 GiB buffers read in rotation (past the 256 MB Infinity Cache). Each is the best of 5."""
    from hk import peaks

    hbm, hbm_by = peaks.hbm_read_gbs(detail=True)
    return {"mfma_bf16_tflops": round(peaks.mfma_tflops(False), 1),
            "mfma_fp8_tflops": round(peaks.mfma_tflops(True), 1),
            "mfma_bf16_random_operands_tflops": round(peaks.mfma_random_tflops(False), 1),
            "mfma_fp8_random_operands_tflops": round(peaks.mfma_random_tflops(True), 1),
            "hbm_read_gbs": round(hbm, 1),
            "hbm_read_gbs_by_kernel": {k: round(v, 1) for k, v in hbm_by.items()},
            "how": "hk.peaks: register-only MFMA loops on every CU, 32x32 on constant operands, "
                   "and on random ones (the power-limited rate on data that toggles like real "
                   "tensors) the better of the 32x32 and 16x16 instructions; HBM: four 1 GiB "
                   "buffers read in rotation past the 256 MB Infinity Cache, the best of three "
                   "read kernels"}


def other_configs(steps, warmup, peaks):
    """Configs 3-5: configs 3 and 5 timed as config 2 is (HIP events per launch, mean, for
    the kernel; and K calls back to back, as config 2's value), config 4 from replayed
    graphs (its launches are shorter than the host's call overhead)."""
    import torch

    import hk

    T = hk.templates.gemm
    dev = "cuda:0"
    out = {}
    # config 2 on the same box: the plain GEMM (no epilogue) on the same kernel, and
    # hipBLASLt's plain GEMM (torch.matmul) on the same operands -- what the bias + GELU
    # epilogue costs, and where the vendor library stands
    x, wt, b = _inputs(4096, 4096, 12288, 0, dev)
    y = torch.empty(4096, 12288, device=dev, dtype=torch.bfloat16)
    fl = 2.0 * 4096 * 12288 * 4096
    cmp = {}
    for name, fn in (("quad_plain", lambda: T(x, wt, out=y)),
                     ("quad_bias_gelu", lambda: T(x, wt, epilogue=T.bias_gelu, bias=b, out=y)),
                     ("hipblaslt_plain_torch_matmul", lambda: torch.matmul(x, wt.t(), out=y))):
        t, _, _ = _events_time(fn, steps, warmup)
        cmp[name] = {"us": round(t * 1e6, 2), "TFLOP/s": round(fl / t / 1e12, 1)}
    out["cfg2_same_box"] = cmp
    del x, wt, b, y
    # config 3: fused gate_up + silu_and_mul
    for m in (2048, 8192):
        x, wt, _ = _inputs(m, 4096, 24576, 3, dev)
        y = torch.empty(m, 12288, device=dev, dtype=torch.bfloat16)
        f3 = lambda: T(x, wt, epilogue=T.silu_and_mul, out=y)  # noqa: E731
        t, _, _ = _events_time(f3, steps, warmup)
        tw = _wall_time(f3, steps, 0) / steps  # back to back, as config 2's value
        fl = 2.0 * m * 24576 * 4096
        out[f"cfg3_gate_up_silu_mul_M{m}"] = {"TFLOP/s": round(fl / t / 1e12, 1),
                                              "TFLOP/s_back_to_back": round(fl / tw / 1e12, 1),
                                              "frac_bf16_peak": round(fl / t / 1e12 / PEAK_BF16, 4),
                                              "frac_measured": round(fl / t / 1e12 / peaks["mfma_bf16_tflops"], 4),
                                              "frac_measured_random_operands": round(
                                                  fl / t / 1e12 / peaks["mfma_bf16_random_operands_tflops"], 4),
                                              "us": round(t * 1e6, 1)}
        del x, wt, y
    # config 4: decode, 4 weight copies (403 MB) rotated past the 256 MB MALL; kernel time
    # from a replayed graph of 32 calls
    ws = [_inputs(1, 4096, 12288, 40 + i, dev)[1] for i in range(4)]
    bias = _inputs(1, 4096, 12288, 4, dev)[2]
    for m in (1, 4, 16):
        x = _inputs(m, 4096, 12288, 4, dev)[0]
        for epi in ("plain", "bias"):
            y = torch.empty(m, 12288, device=dev, dtype=torch.bfloat16)
            if epi == "bias":
                calls = [lambda w=ws[i % 4]: T(x, w, epilogue=T.bias, bias=bias, out=y) for i in range(32)]
            else:
                calls = [lambda w=ws[i % 4]: T(x, w, out=y) for i in range(32)]
            # ~20 us launches: timed as a graph of 32 calls, the host's call overhead out,
            # after the same untimed ramp as the other arms
            if RAMP_S > 0:
                _ramp(calls[0], RAMP_S)
            t = _graph_time(calls)
            byts = 12288 * 4096 * 2 + m * 4096 * 2 + m * 12288 * 2 + (12288 * 2 if epi == "bias" else 0)
            out[f"cfg4_decode_M{m}_{epi}"] = {"GB/s": round(byts / t / 1e9, 1),
                                              "frac_hbm_peak": round(byts / t / 1e9 / PEAK_HBM, 4),
                                              "frac_measured": round(byts / t / 1e9 / peaks["hbm_read_gbs"], 4),
                                              "us": round(t * 1e6, 2)}
    del ws
    # config 5: fp8 e4m3 scaled GEMM + dequant + bias
    g = torch.Generator().manual_seed(5)
    x8 = torch.randn(8192, 4096, generator=g).to(torch.float8_e4m3fn).to(dev)
    w8 = torch.randn(4096, 4096, generator=g).to(torch.float8_e4m3fn).t().contiguous().to(dev)
    sa = ((torch.rand(8192, 1, generator=g) * 1.5 + 0.5) / 448).to(dev)
    sb = ((torch.rand(4096, generator=g) * 1.5 + 0.5) / 448).to(dev)
    bias = (torch.randn(4096, generator=g) * 0.1).to(torch.bfloat16).to(dev)
    y = torch.empty(8192, 4096, device=dev, dtype=torch.bfloat16)
    f5 = lambda: hk.ops.scaled_mm(x8, w8, sa, sb, bias=bias, out=y)  # noqa: E731
    t, _, _ = _events_time(f5, steps, warmup)
    tw = _wall_time(f5, steps, 0) / steps  # back to back, as config 2's value
    fl = 2.0 * 8192 * 4096 * 4096
    out["cfg5_fp8_scaled_dequant_bias"] = {"TFLOP/s": round(fl / t / 1e12, 1),
                                           "TFLOP/s_back_to_back": round(fl / tw / 1e12, 1),
                                           "us_back_to_back": round(tw * 1e6, 1),
                                           "frac_fp8_peak": round(fl / t / 1e12 / PEAK_FP8, 4),
                                           "frac_measured": round(fl / t / 1e12 / peaks["mfma_fp8_tflops"], 4),
                                           "frac_measured_random_operands": round(
                                               fl / t / 1e12 / peaks["mfma_fp8_random_operands_tflops"], 4),
                                           "us": round(t * 1e6, 1)}
    # the vendor path on the same operands: torch._scaled_mm (hipBLASLt), which takes the
    # scales but not the bias in this form
    try:
        wcol = w8.t()  # (K, N) column-major, as _scaled_mm wants its second operand
        t, _, _ = _events_time(lambda: torch._scaled_mm(x8, wcol, scale_a=sa, scale_b=sb.reshape(1, -1),
                                                         out_dtype=torch.bfloat16), steps, warmup)
        out["cfg5_fp8_scaled_dequant_bias"]["torch_scaled_mm_no_bias_us"] = round(t * 1e6, 1)
    except Exception as ex:  # noqa: BLE001 - a vendor-side refusal is reported, not fatal
        out["cfg5_fp8_scaled_dequant_bias"]["torch_scaled_mm_no_bias_us"] = f"unavailable: {str(ex)[:120]}"
    return out


if __name__ == "__main__":
    main()
