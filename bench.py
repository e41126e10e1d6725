"""Benchmark of the quantized-matmul hot path on one MI355X.

Headline (BASELINE.json metric, configs[1]): one decode step's Q8_0 matvec
set of a dense 9B-class layer (q, k, v, o 4096->4096; gate, up 4096->12288;
down 12288->4096) plus the lm_head matvec 4096->151936, batch 1, FP32
activations, launched in the reference's call pattern (q|k|v and gate|up
each one projections launch, o and down accumulating into the residual).
value = algorithmic bytes (weights + inputs + outputs) / step time, GB/s,
with all inputs resident in HBM.  Distinct weight copies are rotated so the
256 MB Infinity Cache cannot serve them.  The other configurations are
reported under "configs" (matvec GB/s, GEMM TFLOP/s, MoE).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-configs] [--no-cpu] [--roofline-only]
    python bench.py --trace-summary <rocprofv3 kernel_trace.csv>
"""
from __future__ import annotations

import argparse
import csv
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
# The prefill GEMMs run FP32 arithmetic as three bf16 matrix instructions per
# product (exact split of the FP32 activations), so their ceiling is the
# dense bf16 matrix-core peak over three: FP32-equivalent TFLOP/s.
BF16_MFMA_PEAK_TFLOPS = 2500.0
X3_PEAK_TFLOPS = BF16_MFMA_PEAK_TFLOPS / 3
MALL_BYTES = 256 << 20


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-configs", action="store_true", help="headline only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the lm_head kernel (--steps launches) and a same-size copy, for counter runs")
    ap.add_argument("--only", default="",
                    help="comma list of configs (cfg0,cfg2,cfg3,cfg4,engine) to run alone, for counter runs")
    ap.add_argument("--trace-summary", default="",
                    help="summarise a rocprofv3 kernel trace (--kernel-trace --output-format csv) of this "
                         "program by kernel and grid, with the roofline kernel's back-to-back block; no GPU")
    return ap.parse_args()


def mv_bytes(m) -> int:
    return m.nbytes + 4 * m.cols + 4 * m.rows


def copies_for(total_bytes: int) -> int:
    """Distinct copies so that a full rotation is >= 4x the Infinity Cache."""
    return max(2, -(-4 * MALL_BYTES // total_bytes))


def capture(torch, fn):
    """Capture fn's launches (all on the current stream) into a HIP graph."""
    fn()  # eager warm-up outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


LAYER_LAUNCHES = ("attention projections q|k|v (one q3x_hip_mv_multi), o (mv_add), "
                  "ffn projections gate|up (one q3x_hip_mv_multi), down (mv_add), then lm_head (mv)")


class LayerStep:
    """One decode step's matvecs in the reference's call pattern (engine.cu
    attention :1682-1700 and ffn :1701-1707 over the projection helpers
    :1607-1619, then the lm_head mv :1990): q/k/v share the normed input, o and
    down add into the residual, gate/up share the FFN input."""

    def __init__(self, torch, q3x, wl, mats):
        self.q3x = q3x
        self.by = {m.name: m for m in mats}
        h = 4096
        self.x_attn = wl.activations(1, 1, h, salt=1)[0].contiguous()
        self.x_o = wl.activations(1, 1, h, salt=2)[0].contiguous()
        self.x_ffn = wl.activations(1, 1, h, salt=3)[0].contiguous()
        self.h = wl.activations(1, 1, 12288, salt=4)[0].contiguous()
        self.x_final = wl.activations(1, 1, h, salt=5)[0].contiguous()
        self.resid0 = wl.activations(1, 1, h, salt=6)[0].contiguous()
        self.resid = self.resid0.clone()
        self.out = {m.name: torch.empty(m.rows, dtype=torch.float32, device="cuda") for m in mats
                    if m.name not in ("o", "down")}

    def run_layer(self, s):
        q3x, o = self.q3x, self.out
        q3x.mv_multi([s["q"].linear, s["k"].linear, s["v"].linear], self.x_attn, [o["q"], o["k"], o["v"]])
        q3x.mv_add(s["o"].linear, self.x_o, self.resid)
        q3x.mv_multi([s["gate"].linear, s["up"].linear], self.x_ffn, [o["gate"], o["up"]])
        q3x.mv_add(s["down"].linear, self.h, self.resid)

    def run_lm(self, lm):
        self.q3x.mv(lm.linear, self.x_final, self.out["lm_head"])

    def reset(self):
        self.resid.copy_(self.resid0)

    def step_bytes(self):
        """Algorithmic HBM bytes of one step: every weight byte once, each
        launch's input once, each output written (and read once more where it
        accumulates)."""
        b = self.by
        weights = sum(m.nbytes for m in b.values())
        inputs = 4 * (4096 * 4 + 12288)                       # q|k|v, o, gate|up, lm_head inputs + down's h
        outputs = 4 * (b["q"].rows + b["k"].rows + b["v"].rows + b["gate"].rows + b["up"].rows
                       + b["lm_head"].rows) + 2 * 4 * (b["o"].rows + b["down"].rows)
        return weights + inputs + outputs


def lm_head_launch_ms(torch, step, lm_set, reps):
    """Average duration of the lm_head kernel: `reps` back-to-back launches
    (rotating weight copies) between two HIP events on the launch stream."""
    for i in range(3):
        step.run_lm(lm_set[i % len(lm_set)])
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(reps):
        step.run_lm(lm_set[i % len(lm_set)])
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def launch_breakdown(torch, q3x, step, layer_sets):
    """Each launch of the layer on its own: 4n launches of one kind (rotating
    the n weight copies) captured in one graph and replayed, so the host's
    per-call cost (ctypes and Python, ~8 us, more than a small launch's GPU
    time) does not set the rate: microseconds and algorithmic GB/s."""
    n = len(layer_sets)
    o = step.out

    def mb(*names, inputs=4096, acc=False):
        b = sum(layer_sets[0][k].nbytes + 4 * layer_sets[0][k].rows * (2 if acc else 1) for k in names)
        return b + 4 * inputs

    kinds = {
        "q|k|v": (lambda i: q3x.mv_multi([layer_sets[i % n][k].linear for k in ("q", "k", "v")], step.x_attn,
                                         [o["q"], o["k"], o["v"]]), mb("q", "k", "v")),
        "o (+=)": (lambda i: q3x.mv_add(layer_sets[i % n]["o"].linear, step.x_o, step.resid), mb("o", acc=True)),
        "gate|up": (lambda i: q3x.mv_multi([layer_sets[i % n][k].linear for k in ("gate", "up")], step.x_ffn,
                                           [o["gate"], o["up"]]), mb("gate", "up")),
        "down (+=)": (lambda i: q3x.mv_add(layer_sets[i % n]["down"].linear, step.h, step.resid),
                      mb("down", inputs=12288, acc=True)),
    }
    out = {}
    for name, (fn, nbytes) in kinds.items():
        # Median of five timings (each 5 replays): one slow window (a clock
        # or power transition) does not stand for the launch.
        ms = statistics.median(time_graph(torch, fn, 4 * n, 5) for _ in range(5))
        out[name] = {"us": round(ms * 1e3, 2), "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    step.reset()
    return out


def headline(torch, q3x, wl, steps, warmup):
    mats = wl.dense_matrices(1)
    layer = [m for m in mats if m.name != "lm_head"]
    lm = [m for m in mats if m.name == "lm_head"][0]
    layer_bytes = sum(m.nbytes for m in layer)
    n_layer = copies_for(layer_bytes)
    n_lm = copies_for(lm.nbytes)
    layer_sets = [{m.name: m for m in layer}] + [
        {m.name: wl.Matrix(m.name, m.type, m.rows, m.cols, m.weight.clone()) for m in layer}
        for _ in range(n_layer - 1)]
    lm_set = [lm] + [wl.Matrix(lm.name, lm.type, lm.rows, lm.cols, lm.weight.clone()) for _ in range(n_lm - 1)]
    step = LayerStep(torch, q3x, wl, mats)

    # A step is five launches on one stream (back-to-back kernels on a
    # stream start without a gap on this runtime, while consecutive graph
    # launches leave ~8 us between graphs).
    def run_step(r):
        step.run_layer(layer_sets[r])
        step.run_lm(lm_set[r % n_lm])

    # The lm_head kernel's duration before the steps (the box as it comes)
    # and after them (under the sustained load the steps put on HBM), both
    # over the same 20 back-to-back launches: the drift of the dominant
    # kernel within the run.
    lm_before_ms = lm_head_launch_ms(torch, step, lm_set, 20)
    for i in range(warmup):
        run_step(i % n_layer)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        run_step(i % n_layer)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms = elapsed * 1e3 / steps
    lm_ms = lm_head_launch_ms(torch, step, lm_set, 20)
    lm_alg = mv_bytes(lm)
    step_bytes = step.step_bytes()
    per_launch = launch_breakdown(torch, q3x, step, layer_sets)
    per_launch["lm_head"] = {"us": round(lm_ms * 1e3, 2), "GBps": round(lm_alg / (lm_ms * 1e-3) / 1e9, 1)}
    # The layer's four launches without lm_head (rotating the copies, in one
    # graph as above): the rate of the smaller matvecs, which the 662 MB
    # lm_head otherwise carries in the step's figure.
    set_bytes = step_bytes - lm_alg
    set_ms = statistics.median(time_graph(torch, lambda i: step.run_layer(layer_sets[i % n_layer]), 4 * n_layer, 5)
                               for _ in range(5))
    step.reset()
    # The same launches as plain reads of the same weight bytes (q|k|v,
    # o, gate|up, down): what the box reaches at these sizes with no work.
    by = {m.name: m.nbytes for m in layer}
    read_us = plain_read_us(torch, q3x, [by["q"] + by["k"] + by["v"], by["o"], by["gate"] + by["up"], by["down"]],
                            n_layer, graph=True)
    layer_set = {"us": round(set_ms * 1e3, 2), "bytes": set_bytes,
                 "GBps": round(set_bytes / (set_ms * 1e-3) / 1e9, 1),
                 "frac_of_hbm_peak": round(set_bytes / (set_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                 "plain_read_us": round(read_us, 2),
                 "note": "plain_read_us: the four launches' weight bytes read by q3x_hip_read_probe "
                         "(no work on the data), replayed the same way"}
    return {
        "layer_set": layer_set,
        "per_launch": per_launch,
        "value": step_bytes / (ms * 1e-3) / 1e9,
        "ms_per_step": ms,
        "step_bytes": step_bytes,
        "copies": {"layer_set": n_layer, "lm_head": n_lm},
        "lm_head": {"bytes": lm_alg, "ms": lm_ms, "GBps": lm_alg / (lm_ms * 1e-3) / 1e9,
                    "before_ms": lm_before_ms},
        "mats": mats,
    }


def measured_traffic():
    """HBM bytes per lm_head launch from the committed rocprofv3 counter
    summary (FETCH_SIZE + WRITE_SIZE, calibrated on a copy kernel), or None."""
    path = os.path.join(ROOT, "profiles", "pmc_traffic_lm_head_q8_0.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def roofline_only(torch, q3x, wl, reps):
    """Short program for counter runs: the lm_head kernel `reps` times on two
    weight copies, then a plain device copy of the same size (the calibration
    kernel for FETCH_SIZE / WRITE_SIZE)."""
    mats = wl.dense_matrices(1)
    lm = [m for m in mats if m.name == "lm_head"][0]
    lm_set = [lm, wl.Matrix(lm.name, lm.type, lm.rows, lm.cols, lm.weight.clone())]
    step = LayerStep(torch, q3x, wl, mats)
    ms = lm_head_launch_ms(torch, step, lm_set, reps)
    src = torch.empty(lm.nbytes // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"lm_head_ms": ms, "lm_head_bytes": mv_bytes(lm), "copy_bytes_each_way": src.numel() * 4,
                      "GBps": mv_bytes(lm) / (ms * 1e-3) / 1e9}), flush=True)


def time_graph(torch, fn, calls, replays, warmup=2):
    """Mean ms per call of fn(i), i = 0..calls-1 captured in one graph."""
    g = capture(torch, lambda: [fn(i) for i in range(calls)])
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (replays * calls)


def plain_read_us(torch, q3x, sizes, copies, graph):
    """Microseconds per round of plain streaming reads (q3x_hip_read_probe:
    every byte once, no work on the data) of buffers of the given byte
    sizes, one launch per size, over `copies` rotating sets -- the read rate
    this box reaches at the matvecs' sizes.  graph: replayed from a graph
    like the matvec it stands beside, else back to back on the stream."""
    sizes = [(b + 15) // 16 * 16 for b in sizes]
    bufs = [[torch.empty(b, dtype=torch.uint8, device="cuda") for b in sizes] for _ in range(copies)]
    sink = torch.zeros(4, dtype=torch.uint8, device="cuda")

    def run(i):
        for b in bufs[i % copies]:
            q3x.read_probe(b, sink)
    if graph:
        ms = statistics.median(time_graph(torch, run, 4 * copies, 5) for _ in range(3))
    else:
        for i in range(2 * copies):
            run(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(8 * copies):
            run(i)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / (8 * copies)
    del bufs
    return ms * 1e3


def cpu_median(fn, seconds, max_reps=25):
    """Median seconds of fn() over repeats filling about `seconds` (>= 3
    repeats after one warm-up)."""
    fn()
    times = []
    while len(times) < 3 or (sum(times) < seconds and len(times) < max_reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


class CpuReference:
    """The reference CPU path, single thread, on host copies of a config's
    weights: the reference's own try_mv (arch/cpu.cpp:192-226, scalar on
    x86) from oracle/_ref, or this repository's bit-identical restatement
    when the reference build is absent.  Prefill is the reference's
    token-by-token loop (engine.cpp:580-583), timed on a token subset and
    scaled linearly (every token does the same work)."""

    def __init__(self):
        import oracle
        self.oracle = oracle
        self.ref = oracle.ref()
        self.kind = "reference" if self.ref is not None else "port"

    def mv(self, w, type_, rows, cols, x, y):
        if self.ref is not None:
            self.ref.q3xr_try_mv(w.ctypes.data, type_, rows, cols, x.ctypes.data, y.ctypes.data)
        else:
            self.oracle.lib().q3xo_mv_rows(w.ctypes.data, type_, 0, rows, cols, x.ctypes.data, y.ctypes.data)

    def entry(self, value, unit, sample):
        return {"value": value, "unit": unit, "cores": 1, "kind": self.kind,
                "sample": f"{sample}; single thread; host nproc={os.cpu_count()}"}


def cpu_matvecs(cpu, mats, seconds):
    """Seconds of one pass of the reference mv over `mats` (one token)."""
    import numpy as np
    hosts = [(m, np.ascontiguousarray(m.weight.cpu().numpy())) for m in mats]
    x = np.random.default_rng(1).normal(0, 1, max(m.cols for m in mats)).astype(np.float32)
    ys = [np.empty(m.rows, np.float32) for m in mats]

    def one_pass():
        for (m, w), y in zip(hosts, ys):
            cpu.mv(w, m.type, m.rows, m.cols, x, y)
    return cpu_median(one_pass, seconds)


def gemm_entry(torch, q3x, mats, X, H, Ys, count, ms_plain, flops, replays):
    """A GEMM config's line: q3x_hip_gemm_ws with the workspace its plan asks
    for (K split over workgroups where few tiles meet a long K) when any
    matrix splits, q3x_hip_gemm beside it; otherwise q3x_hip_gemm alone.
    replays: (calls per graph, replays) as the plain timing used."""
    plain = {"TFLOPs": flops / (ms_plain * 1e-3) / 1e12, "ms": ms_plain,
             "frac_x3_peak": flops / (ms_plain * 1e-3) / 1e12 / X3_PEAK_TFLOPS}
    need = max(q3x.gemm_workspace_bytes(mm.linear, count) for mm in mats)
    if need == 0:
        return plain
    ws = torch.empty(need // 4, dtype=torch.float32, device="cuda")

    def run(i):
        for mm in mats:
            q3x.batch_mv_ws(mm.linear, H if mm.name == "down" else X, Ys[mm.name], count, ws)
    ms = time_graph(torch, run, *replays)
    del ws
    return {"TFLOPs": flops / (ms * 1e-3) / 1e12, "ms": ms, "frac_x3_peak": flops / (ms * 1e-3) / 1e12 / X3_PEAK_TFLOPS,
            "workspace_bytes": need, "split_k": {mm.name: q3x.gemm_workspace_bytes(mm.linear, count) > 0 for mm in mats},
            "no_workspace": plain,
            "note": "q3x_hip_gemm_ws with the workspace its plan asks for (the matrices marked split_k run K over "
                    "several workgroups and a fixup launch); no_workspace: q3x_hip_gemm"}


def extra_configs(torch, q3x, wl, only=None, cpu=False):
    out = {}
    want = (lambda c: only is None or c in only)
    ref_cpu = CpuReference() if cpu else None
    if want("cfg0"):
        # config 0: one Q8_0 4096x4096 matvec, copies rotated
        m = wl.dense_matrices(0)[0]
        n = copies_for(m.nbytes)
        ws = [m.weight] + [m.weight.clone() for _ in range(n - 1)]
        x = wl.activations(0, 1, 4096)[0].contiguous()
        y = torch.empty(4096, dtype=torch.float32, device="cuda")
        ms = time_graph(torch, lambda i: q3x.mv(q3x.Linear(ws[i % n], 4096, 4096, m.type), x, y), 4 * n, 20)
        out["cfg0_q8_mv_4096"] = {"GBps": mv_bytes(m) / (ms * 1e-3) / 1e9, "us": ms * 1e3, "copies": n,
                                  "plain_read_us": plain_read_us(torch, q3x, [m.nbytes], n, graph=True)}
        if ref_cpu:
            t, reps = cpu_matvecs(ref_cpu, [m], 1.0)
            out["cfg0_q8_mv_4096"]["cpu_baseline"] = ref_cpu.entry(
                mv_bytes(m) / t / 1e9, "GB/s", f"the 4096x4096 matvec, median of {reps} calls ({t * 1e3:.1f} ms each)")
        del ws
    if want("cfg2"):
        # config 2: Q8_0 prefill GEMM, N in {512, 4096}
        mats = wl.dense_matrices(2)
        for count in (512, 4096):
            X = wl.activations(2, count, 4096)
            H = wl.activations(2, count, 12288, salt=1)
            Ys = {mm.name: torch.empty((count, mm.rows), dtype=torch.float32, device="cuda") for mm in mats}

            def run(i):
                for mm in mats:
                    q3x.batch_mv(mm.linear, H if mm.name == "down" else X, Ys[mm.name], count)
            # Several calls to a graph replay where a call is short, so that the
            # replay's own launch is a small share of the timed span.
            shape = (1, 4) if count == 4096 else (4, 3)
            ms = time_graph(torch, run, *shape)
            flops = sum(2.0 * count * mm.rows * mm.cols for mm in mats)
            out[f"cfg2_q8_gemm_N{count}"] = gemm_entry(torch, q3x, mats, X, H, Ys, count, ms, flops, shape)
            del X, H, Ys
        if ref_cpu:
            # one token through gate, up and down, the reference's prefill unit
            t, reps = cpu_matvecs(ref_cpu, mats, 2.0)
            per_token = sum(2.0 * mm.rows * mm.cols for mm in mats)
            for count in (512, 4096):
                out[f"cfg2_q8_gemm_N{count}"]["cpu_baseline"] = ref_cpu.entry(
                    per_token / t / 1e12, "TFLOP/s",
                    f"the reference's prefill, one mv per token and matrix (engine.cpp:580-583): {reps} tokens "
                    f"through gate/up/down ({t * 1e3:.0f} ms per token, median), scaled to N={count}: "
                    f"{count * t:.1f} s")
        del mats
    if want("cfg3"):
        # config 3: Q4_0 27B FFN at N = 1 (matvec) and N = 512 (GEMM)
        mats = wl.dense_matrices(3)
        total = sum(mm.nbytes for mm in mats)
        n = copies_for(total)
        sets = [mats] + [[wl.Matrix(mm.name, mm.type, mm.rows, mm.cols, mm.weight.clone()) for mm in mats]
                         for _ in range(n - 1)]
        x = wl.activations(3, 1, 17408)[0].contiguous()
        ys = {mm.name: torch.empty(mm.rows, dtype=torch.float32, device="cuda") for mm in mats}

        def run_mv(i):
            s = {mm.name: mm for mm in sets[i % n]}
            q3x.mv_multi([s["gate"].linear, s["up"].linear], x, [ys["gate"], ys["up"]])
            q3x.mv(s["down"].linear, x, ys["down"])
        # As the headline step: the launches back to back on one stream (the
        # host issues a call in ~16 us, under the ~37 us the GPU takes, so
        # the GPU sets the rate), timed with HIP events; the same calls
        # replayed from a graph, which adds a node boundary per launch, are
        # reported beside it.
        ms_graph = time_graph(torch, run_mv, 2 * n, 10)
        for i in range(2 * n):
            run_mv(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(8 * n):
            run_mv(i)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / (8 * n)
        alg = sum(mv_bytes(mm) for mm in mats) - 4 * 5120  # gate|up read x once
        by = {mm.name: mm.nbytes for mm in mats}
        read_us = plain_read_us(torch, q3x, [by["gate"] + by["up"], by["down"]], n, graph=False)
        out["cfg3_q4_mv_27b_ffn"] = {"GBps": alg / (ms * 1e-3) / 1e9, "us": ms * 1e3, "copies": n,
                                     "us_graph": ms_graph * 1e3,
                                     "GBps_graph": alg / (ms_graph * 1e-3) / 1e9,
                                     "plain_read_us": read_us,
                                     "note": "plain_read_us: gate|up and down weight bytes read by "
                                             "q3x_hip_read_probe (no work on the data), back to back as above"}
        del sets
        X = wl.activations(3, 512, 5120)
        H = wl.activations(3, 512, 17408, salt=1)
        Ys = {mm.name: torch.empty((512, mm.rows), dtype=torch.float32, device="cuda") for mm in mats}

        def run_gemm(i):
            for mm in mats:
                q3x.batch_mv(mm.linear, H if mm.name == "down" else X, Ys[mm.name], 512)
        ms = time_graph(torch, run_gemm, 4, 3)
        flops = sum(2.0 * 512 * mm.rows * mm.cols for mm in mats)
        out["cfg3_q4_gemm_N512"] = gemm_entry(torch, q3x, mats, X, H, Ys, 512, ms, flops, (4, 3))
        if ref_cpu:
            t, reps = cpu_matvecs(ref_cpu, mats, 2.0)
            out["cfg3_q4_mv_27b_ffn"]["cpu_baseline"] = ref_cpu.entry(
                alg / t / 1e9, "GB/s", f"gate, up and down matvecs, median of {reps} passes ({t * 1e3:.0f} ms each)")
            per_token = sum(2.0 * mm.rows * mm.cols for mm in mats)
            out["cfg3_q4_gemm_N512"]["cpu_baseline"] = ref_cpu.entry(
                per_token / t / 1e12, "TFLOP/s",
                f"the reference's prefill, one mv per token and matrix (engine.cpp:580-583): {reps} tokens "
                f"({t * 1e3:.0f} ms per token, median), scaled to N=512: {512 * t:.1f} s")
        del mats, X, H, Ys
    if want("cfg4"):
        # config 4: Q4_0 routed MoE (router + experts), decode and 2048-token prefill
        moe = wl.moe_weights(4)
        cfg = wl.CONFIGS[4]
        k = cfg["top_k"]
        for T in (1, 2048):
            logits = wl.router_logits(4, T, moe.experts)
            X = wl.activations(4, T, moe.H)
            ids = torch.empty((T, k), dtype=torch.int32, device="cuda")
            wts = torch.empty((T, k), dtype=torch.float32, device="cuda")
            Y = torch.empty((T, moe.H), dtype=torch.float32, device="cuda")
            wsb = torch.empty(q3x.moe_workspace_bytes(T, moe.experts, k, moe.H, moe.I), dtype=torch.uint8,
                              device="cuda")

            def run_moe(i):
                q3x.moe_routed_logits(moe.gate_up_linear, moe.down_linear, X, T, logits, k, ids, wts, Y,
                                      workspace=wsb)
            ms = time_graph(torch, run_moe, 20 if T == 1 else 4, 10 if T == 1 else 3)
            router_ms = time_graph(torch, lambda i: q3x.router_top_k(logits, T, moe.experts, k, ids, wts), 20, 5)
            if T == 1:
                per_expert = (moe.gate_up.numel() + moe.down.numel()) // moe.experts
                alg = k * per_expert
                # Decode from HBM: 64 distinct tokens in turn, so consecutive
                # calls read other experts and a rotation (64 x 14 MB) is far
                # past the 256 MB Infinity Cache.
                R = 64
                logits_r = wl.router_logits(4, R, moe.experts)
                X_r = wl.activations(4, R, moe.H, salt=3)
                ids_r = torch.empty((R, k), dtype=torch.int32, device="cuda")
                wts_r = torch.empty((R, k), dtype=torch.float32, device="cuda")

                def run_moe_rot(i):
                    j = i % R
                    q3x.moe_routed_logits(moe.gate_up_linear, moe.down_linear, X_r[j:j + 1], 1, logits_r[j:j + 1],
                                          k, ids_r[j], wts_r[j], Y, workspace=wsb)

                def run_two_calls(i):
                    j = i % R
                    q3x.router_top_k(logits_r[j:j + 1], 1, moe.experts, k, ids_r[j], wts_r[j])
                    q3x.moe_routed(moe.gate_up_linear, moe.down_linear, X_r[j:j + 1], 1, ids_r[j], wts_r[j], k, Y,
                                   workspace=wsb)
                ms_rot = time_graph(torch, run_moe_rot, R, 10)
                ms_two = time_graph(torch, run_two_calls, R, 10)
                distinct = int(torch.unique(ids_r).numel())
                out["cfg4_q4_moe_decode"] = {
                    "GBps": alg / (ms_rot * 1e-3) / 1e9, "us": ms_rot * 1e3, "bytes": alg,
                    "router_us": router_ms * 1e3, "us_same_token": ms * 1e3, "us_two_calls": ms_two * 1e3,
                    "note": f"q3x_hip_moe_routed_logits (router inside the gate_up launch, then down: 2 launches) "
                            f"per call, 64 distinct tokens in turn ({distinct} of 256 experts read per rotation); "
                            "us_same_token repeats one token, whose 14 MB the Infinity Cache then serves; "
                            "us_two_calls: q3x_hip_router_topk then q3x_hip_moe_routed (3 launches)"}
                if ref_cpu:
                    import numpy as np
                    gu_h = np.ascontiguousarray(moe.gate_up.cpu().numpy())
                    dn_h = np.ascontiguousarray(moe.down.cpu().numpy())
                    lg_h = np.ascontiguousarray(logits_r.cpu().numpy())
                    X_h = np.ascontiguousarray(X_r.cpu().numpy())
                    sel = np.empty(k, np.int32)
                    prob = np.empty(moe.experts, np.float32)
                    y_h = np.empty(moe.H, np.float32)
                    state = {"j": 0}

                    def cpu_token():
                        j = state["j"] % R
                        state["j"] += 1
                        self_ref = ref_cpu.ref
                        if self_ref is not None:
                            self_ref.q3xr_router_top_k(lg_h[j].ctypes.data, moe.experts, k, sel.ctypes.data,
                                                       prob.ctypes.data)
                            w_sel = np.ascontiguousarray(prob[sel])
                            self_ref.q3xr_moe_routed(moe.type, gu_h.ctypes.data, dn_h.ctypes.data, moe.experts,
                                                     moe.H, moe.I, X_h[j].ctypes.data, sel.ctypes.data,
                                                     w_sel.ctypes.data, k, y_h.ctypes.data)
                        else:
                            ids_o, w_o, _ = ref_cpu.oracle.router_top_k(lg_h[j], k)
                            ref_cpu.oracle.moe_routed(gu_h, dn_h, moe.type, moe.experts, moe.H, moe.I, X_h[j],
                                                      ids_o, w_o, threads=1)
                    t_tok, reps = cpu_median(cpu_token, 2.0, 64)
                    out["cfg4_q4_moe_decode"]["cpu_baseline"] = ref_cpu.entry(
                        alg / t_tok / 1e9, "GB/s",
                        f"router_top_k + the routed loop of moe() (engine.cpp:377-420) per token, median of {reps} "
                        f"of the same 64 tokens ({t_tok * 1e3:.1f} ms each)")
                    flops_tok = 2.0 * k * 3 * moe.I * moe.H
                    cpu4_prefill = ref_cpu.entry(
                        flops_tok / t_tok / 1e12, "TFLOP/s",
                        f"the reference's prefill is the same per-token loop (engine.cpp:580-583): "
                        f"{t_tok * 1e3:.1f} ms per token (median of {reps}), scaled to T=2048: {2048 * t_tok:.1f} s")
                del logits_r, X_r, ids_r, wts_r
            else:
                flops = 2.0 * T * k * (2 * moe.I * moe.H + moe.H * moe.I)
                out["cfg4_q4_moe_prefill_T2048"] = {"TFLOPs": flops / (ms * 1e-3) / 1e12, "ms": ms,
                                                    "router_ms": router_ms,
                                                    "frac_x3_peak": flops / (ms * 1e-3) / 1e12 / X3_PEAK_TFLOPS}
                if ref_cpu:
                    out["cfg4_q4_moe_prefill_T2048"]["cpu_baseline"] = cpu4_prefill
            del logits, X, ids, wts, Y, wsb
        # The whole MoE layer (engine.cpp:406-430): BF16 router, top-k,
        # routed experts and the sigmoid-gated shared expert, one call.
        layer = wl.moe_layer_weights(4)
        E, H, I, SI = layer.experts, layer.H, layer.I, layer.shared_I
        shared_bytes = layer.shared_gate.numel() + layer.shared_up.numel() + layer.shared_down.numel()
        for T in (1, 2048):
            X = wl.activations(4, T, H, salt=9)
            Y = torch.empty((T, H), dtype=torch.float32, device="cuda")
            wsl = torch.empty(q3x.moe_layer_workspace_bytes(layer, T), dtype=torch.uint8, device="cuda")
            ms = time_graph(torch, lambda i: q3x.moe_layer(layer, X, T, Y, workspace=wsl), 20 if T == 1 else 4,
                            10 if T == 1 else 3)
            if T == 1:
                per_expert = (moe.gate_up.numel() + moe.down.numel()) // moe.experts
                alg = 2 * (E + 1) * H + k * per_expert + shared_bytes
                out["cfg4_q4_moe_layer_decode"] = {
                    "GBps": alg / (ms * 1e-3) / 1e9, "us": ms * 1e3, "bytes": alg,
                    "note": "router GEMV (BF16 256x2048) + shared-expert gate, then top-8 inside the 8 routed + "
                            "shared experts' gate/up launch, then their down launch: 3 launches"}
            else:
                flops = 2.0 * T * ((E + 1) * H + k * 3 * I * H + 3 * SI * H)
                out["cfg4_q4_moe_layer_prefill_T2048"] = {
                    "TFLOPs": flops / (ms * 1e-3) / 1e12, "ms": ms,
                    "frac_x3_peak": flops / (ms * 1e-3) / 1e12 / X3_PEAK_TFLOPS}
            del X, Y, wsl
        del layer
    if want("engine"):
        out.update(engine_runs(torch, q3x, wl))
    return out


def engine_runs(torch, q3x, wl, prompt=4096, decode=32):
    """The decode engine on full-size models with synthetic weights, in the
    shape of the reference's own benchmark (`--bench 4096 32`: prefill a
    4096-token prompt, then decode 32 tokens one call each, as in
    eval/q8-9b.md:80).  Weights are drawn and quantised on the GPU; the
    tokens are random ids."""
    import numpy as np
    out = {}
    for model_id, name in ((9000, "9b_q8_0"), (36035, "35b_a3b_q4_0"), (38027, "27b_q4_0")):
        config, buf = wl.synthetic_model_weights(model_id, wl.SEED_BASE + model_id)
        engine = q3x.Engine(config, buf, context=prompt + decode + 8)
        tokens = np.random.default_rng(model_id).integers(0, config.V, prompt + decode).astype(np.int32)
        engine.forward(tokens[:8])
        engine.reset()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        engine.forward(tokens[:prompt])
        t_prefill = time.perf_counter() - t0
        t0 = time.perf_counter()
        for i in range(prompt, prompt + decode):
            engine.forward(tokens[i:i + 1])
        t_decode = time.perf_counter() - t0
        out[f"engine_{name}_prefill{prompt}_decode{decode}"] = {
            "prefill_tok_s": prompt / t_prefill, "decode_tok_s": decode / t_decode,
            "decode_ms_per_token": t_decode / decode * 1e3, "model_bytes": buf.numel(),
            "note": "whole-model forward (engine), synthetic full-size weights; decode at 4K context, "
                    "logits every token; host wall clock around each forward call"}
        engine.close()
        del buf, engine
        torch.cuda.empty_cache()
    return out


def cpu_baseline(mats, seconds):
    """The reference CPU path (single thread) over the same matvec set."""
    import numpy as np
    import oracle
    ref = oracle.ref()
    hosts = [(m, np.ascontiguousarray(m.weight.cpu().numpy())) for m in mats]
    x = np.random.default_rng(1).normal(0, 1, 12288).astype(np.float32)
    kind = "reference" if ref is not None else "port"

    def one_pass():
        t0 = time.perf_counter()
        for m, w in hosts:
            y = np.empty(m.rows, np.float32)
            if ref is not None:
                ref.q3xr_try_mv(w.ctypes.data, m.type, m.rows, m.cols, x.ctypes.data, y.ctypes.data)
            else:
                oracle.lib().q3xo_mv_rows(w.ctypes.data, m.type, 0, m.rows, m.cols, x.ctypes.data, y.ctypes.data)
        return time.perf_counter() - t0

    times = [one_pass()]
    while sum(times) < seconds and len(times) < 25:
        times.append(one_pass())
    t = statistics.median(times)
    total = sum(mv_bytes(m) for m in mats)
    return {"value": total / t / 1e9, "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": f"the full config-1 matvec set ({total} B) per pass, median of {len(times)} passes "
                      f"({t * 1e3:.0f} ms each), single thread; host nproc={os.cpu_count()}"}


def kernel_name(name):
    """A demangled kernel name without its argument list (the last
    parenthesised group; "(anonymous namespace)" inside the name stays)."""
    name = name.strip()
    if not name.endswith(")"):
        return name
    depth = 0
    for i in range(len(name) - 1, -1, -1):
        depth += {")": 1, "(": -1}.get(name[i], 0)
        if depth == 0:
            return name[:i].strip()
    return name


def trace_summary(path, top=40):
    """Kernel durations from a rocprofv3 kernel trace of this program
    (--kernel-trace --output-format csv), grouped by kernel and launch shape
    (workgroups x workgroup size), so launches of one template at different
    shapes (lm_head and config 0) stay apart.  The roofline kernel's
    measurement -- the longest run of back-to-back dispatches of one kernel
    and shape (the 20 launches timed after the steps) -- is reported with the
    lm_head algorithmic bytes and the fraction of the HBM peak they imply, and
    that shape's dispatches are listed over the whole run (first and last
    five) to show the drift under sustained load."""
    with open(path, newline="") as f:
        rows = list(csv.DictReader(f))
    if not rows:
        print("empty trace")
        return

    def field(r, *names):
        for n in names:
            if n in r and r[n] != "":
                return r[n]
        raise KeyError(names)

    disp = []
    for r in rows:
        name = field(r, "Kernel_Name", "Kernel-Name", "KernelName")
        wg = int(field(r, "Workgroup_Size_X", "Workgroup_Size", "WorkgroupSizeX"))
        grid = int(field(r, "Grid_Size_X", "Grid_Size", "GridSizeX"))
        t0, t1 = int(field(r, "Start_Timestamp", "BeginNs")), int(field(r, "End_Timestamp", "EndNs"))
        disp.append((t0, t1, kernel_name(name), grid // max(wg, 1), wg))
    disp.sort()
    groups = {}
    for t0, t1, name, wgs, wg in disp:
        groups.setdefault((name, wgs, wg), []).append((t1 - t0) / 1e3)
    print(f"trace: {path}\n{len(disp)} dispatches\n")
    total = sum(sum(d) for d in groups.values())
    by_name = {}
    for (name, _, _), d in groups.items():
        by_name.setdefault(name, []).extend(d)
    print(f"By kernel (all shapes; share of all kernel time, {total / 1e3:.1f} ms):")
    print(f"{'calls':>6} {'mean_us':>9} {'total_ms':>9} {'share':>6}  kernel")
    for name, d in sorted(by_name.items(), key=lambda kv: -sum(kv[1]))[:top]:
        print(f"{len(d):6d} {statistics.mean(d):9.2f} {sum(d) / 1e3:9.2f} {sum(d) / total:6.3f}  {name[:150]}")
    print(f"\nBy kernel and shape:")
    print(f"{'calls':>6} {'mean_us':>9} {'median_us':>9} {'min_us':>8} {'max_us':>8}  workgroups x size  kernel")
    for (name, wgs, wg), d in sorted(groups.items(), key=lambda kv: -sum(kv[1]))[:top]:
        print(f"{len(d):6d} {statistics.mean(d):9.2f} {statistics.median(d):9.2f} {min(d):8.2f} {max(d):8.2f}  "
              f"{wgs:6d} x {wg:<5d}  {name[:150]}")
    # Engine decode steps: the dispatches up to and including advance_kernel
    # (the step's last kernel), among them no prefill kernel; steps of one
    # model have the same kernel count.
    steps, cur = [], []
    for t0, t1, name, wgs, wg in disp:
        cur.append((t0, t1, name))
        if name.endswith("advance_kernel"):
            steps.append(cur)
            cur = []
    prefill = ("gemm_x3_kernel", "delta_chunk", "delta_scan", "delta_conv", "attention_prefill", "rms_kernel")
    by_len = {}
    for s in steps:
        if not any(p in name for _, _, name in s for p in prefill):
            by_len.setdefault(len(s), []).append(s)
    for n, ss in sorted(by_len.items()):
        if len(ss) < 16:
            continue
        span = statistics.median([(s[-1][1] - s[0][0]) / 1e3 for s in ss])
        print(f"\nDecode steps of {n} kernels ({len(ss)} steps): median span {span:.1f} us; per kernel, "
              "median us per step:")
        per = {}
        for s in ss:
            acc = {}
            for t0, t1, name in s:
                acc.setdefault(name, [0.0, 0])
                acc[name][0] += (t1 - t0) / 1e3
                acc[name][1] += 1
            for name, (us, cnt) in acc.items():
                per.setdefault(name, []).append((us, cnt))
        for name, v in sorted(per.items(), key=lambda kv: -statistics.median(u for u, _ in kv[1]))[:12]:
            print(f"  x{v[0][1]:3d} {statistics.median(u for u, _ in v):8.1f}  {name[:120]}")
    # The headline's lm_head launches (q3x_hip_mv of a Q8_0 matrix: the
    # dense-row pipe kernel) are the shape of that kernel whose dispatches
    # come in back-to-back blocks of 10 or more (the blocks timed before the
    # steps and after them, the second being the roofline measurement) and
    # last longest; config 0's launches of the same kernel come in graph
    # replays of another shape.
    def blocks_of(key):
        out, run = [], []
        for t0, t1, *k in disp + [(0, 0, None, 0, 0)]:
            if tuple(k) == key:
                run.append((t1 - t0) / 1e3)
                continue
            if len(run) >= 10:
                out.append(run)
            run = []
        return out

    cand = [k for k, v in groups.items() if "mv_pipe_kernel<1u" in k[0] and "DenseRows<false>" in k[0]
            and statistics.mean(v) > 50 and blocks_of(k)]
    if not cand:
        return
    key = max(cand, key=lambda k: statistics.mean(groups[k]))
    lm_bytes = 151936 * (4096 // 32) * 34 + 4 * 4096 + 4 * 151936
    same = groups[key]
    print(f"\nlm_head: {key[0][:120]} ({key[1]} x {key[2]}), {len(same)} dispatches, algorithmic bytes {lm_bytes}")
    blocks = blocks_of(key)
    labels = ["before the steps", "after the steps (roofline)"]
    for i, b in enumerate(blocks):
        # The timed launches are a block's last 20 (its first are the
        # untimed warm-up launches and, after the steps, the last step's).
        timed = b[-20:]
        mean = statistics.mean(timed)
        label = labels[i] if len(blocks) == 2 else f"block {i}"
        print(f"  back-to-back block {i} ({label}): {len(b)} dispatches; its last {len(timed)} (the timed ones) "
              f"mean {mean:.2f} us, median {statistics.median(timed):.2f} us -> "
              f"{lm_bytes / (mean * 1e-6) / 1e9:.1f} GB/s = {lm_bytes / (mean * 1e-6) / 1e9 / HBM_PEAK_GBS:.4f} "
              f"of {HBM_PEAK_GBS:.0f} GB/s")
    print(f"  all its dispatches in order: first five {', '.join(f'{v:.1f}' for v in same[:5])}; "
          f"last five {', '.join(f'{v:.1f}' for v in same[-5:])} (us)")


def main():
    args = parse()
    if args.trace_summary:
        trace_summary(args.trace_summary)
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the matvec/GEMM shard by output rows with an all-gather, not measured here.", file=sys.stderr)
        sys.exit(2)
    import torch
    import qwen3x_amd as q3x
    from qwen3x_amd import workloads as wl

    torch.cuda.set_device(0)
    if args.roofline_only:
        roofline_only(torch, q3x, wl, args.steps)
        return
    if args.only:
        print(json.dumps(extra_configs(torch, q3x, wl, set(args.only.split(",")), cpu=not args.no_cpu)), flush=True)
        return
    head = headline(torch, q3x, wl, args.steps, args.warmup)
    lm = head["lm_head"]
    traffic = measured_traffic()
    result = {
        "metric": "Q8/Q4 matvec HBM GB/s (% of peak) at N=1; prefill GEMM FP32 TFLOP/s",
        "value": round(head["value"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,0.02) weights quantised to Q8_0; N(0,1) activations)",
        "config": {"workload": "config 1: Q8_0 decode matvec set of one 9B-class layer "
                               "(q/k/v/o 4096->4096, gate/up 4096->12288, down 12288->4096) + lm_head "
                               "4096->151936, batch 1", "launches": LAYER_LAUNCHES, "step_bytes": head["step_bytes"],
                   "weight_copies_rotated": head["copies"], "frac_of_hbm_peak": round(head["value"] / HBM_PEAK_GBS, 4),
                   "seeds": {"base": wl.SEED_BASE, "rule": "config c: weights (SEED_BASE + c) * 1000 + matrix "
                             "index, activations (SEED_BASE + c) * 1000 + 500 + salt, router logits "
                             "(SEED_BASE + c) * 1000 + 700 + tokens (torch.Generator on cuda:0)"},
                   "layer_set": head["layer_set"], "per_launch": head["per_launch"]},
        "roofline": {"bound": "hbm", "achieved": round(lm["GBps"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(lm["GBps"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "mv_pipe_kernel<Q8_0, 64 lanes/row, 1 row/step, 2x16 waves/CU> on lm_head 151936x4096",
                     "algorithmic_bytes_per_launch": lm["bytes"], "avg_launch_ms": round(lm["ms"], 5),
                     "drift": {"before_steps_ms": round(lm["before_ms"], 5), "after_steps_ms": round(lm["ms"], 5),
                               "note": "20 back-to-back lm_head launches timed by HIP events before the warm-up "
                                       "steps and after the timed steps; avg_launch_ms is the second"},
                     "trace": "profiles/bench_default_trace.txt",
                     "traffic_source": "profiles/pmc_traffic_lm_head_q8_0.txt" if traffic else None},
    }
    if not args.no_configs:
        result["configs"] = extra_configs(torch, q3x, wl, cpu=not args.no_cpu)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(head["mats"], args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
