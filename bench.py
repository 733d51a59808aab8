#!/usr/bin/env python3
"""Benchmark of the fp32 elementwise / broadcast / reduction path on one MI355X.

Default workload (one "step" = one pass of the hot path over one batch):
broadcast binary ops on x[32,1024,4096] fp32 ~ N(0,1) with bias[4096] ~
U(-0.1,0.1) and scale[32,1,4096] ~ U(0.5,1.5), forward and backward:
    y1 = x + bias                     (broadcast binary)
    y2 = x * scale                    (broadcast binary)
    dbias  = sum_{B,T} G              (broadcast-gradient reduction)
    dscale = sum_T G * x              (fused product reduction)
    dx     = G * scale                (broadcast binary)
with upstream gradient G ~ N(0,1).  Every op runs through the backend's C ABI
(the entry points the Tensor layer calls) with inputs resident in HBM.

`value` is the step's algorithmic HBM bytes (each distinct input byte read
once, each output byte written once, broadcast operands at their stored size)
divided by the measured time, in GB/s (1e9 B/s).  One JSON line is printed.
Its `suite` key holds every op of the other configurations (C1, C3, C4, C5
and the optimizer kernels), each timed steady state, with the HBM traffic per
launch that the committed rocprof summaries measured, and per configuration a
roofline record for its dominant op.  `--suite` also prints one JSON line per
op; `--suite-op CONFIG/OP --profile-launches K` runs only that op, K times,
for the counter passes that write those summaries.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E peak, 8 TB/s
METRIC = "achieved HBM GB/s (% of MI355X peak) for fp32 elementwise/broadcast/reduce ops"

B, T, C = 32, 1024, 4096
SEEDS = {"x": 11, "bias": 12, "scale": 13, "G": 14}


def parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--suite", action="store_true",
                   help="also print one JSON line per suite op")
    p.add_argument("--suite-only", default=None,
                   help="comma-separated suite sections to run (C1,C3,C4,C5,optim)")
    p.add_argument("--no-suite", action="store_true", help="leave the suite out of the line")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--profile-loop", type=int, default=0,
                   help="run only N steps of the workload (for rocprofv3) and exit")
    p.add_argument("--suite-op", default=None,
                   help="CONFIG/OP: run only this suite op (for rocprofv3) and exit")
    p.add_argument("--profile-launches", type=int, default=4,
                   help="launches of the --suite-op op")
    p.add_argument("--list-suite-ops", action="store_true",
                   help="print the suite's configurations and ops as JSON and exit")
    return p.parse_args()


class Workload:
    """Device buffers and launchers of the broadcast workload."""

    def __init__(self, hip, batch=B):
        self.hip = hip
        self.batch = batch
        n = batch * T * C
        self.n = n
        f = 4
        self.x = hip.DeviceBuffer(n * f)
        self.G = hip.DeviceBuffer(n * f)
        self.bias = hip.DeviceBuffer(C * f)
        self.scale = hip.DeviceBuffer(batch * C * f)
        self.y1 = hip.DeviceBuffer(n * f)
        self.y2 = hip.DeviceBuffer(n * f)
        self.dx = hip.DeviceBuffer(n * f)
        self.dbias = hip.DeviceBuffer(C * f)
        self.dscale = hip.DeviceBuffer(batch * C * f)
        hip.call("spar_hip_random_normal", self.x.ptr, n, hip.FLOAT32, SEEDS["x"], 0.0, 1.0, 0)
        hip.call("spar_hip_random_normal", self.G.ptr, n, hip.FLOAT32, SEEDS["G"], 0.0, 1.0, 0)
        hip.call("spar_hip_random_uniform", self.bias.ptr, C, hip.FLOAT32, SEEDS["bias"], -0.1, 0.1, 0)
        hip.call("spar_hip_random_uniform", self.scale.ptr, batch * C, hip.FLOAT32, SEEDS["scale"],
                 0.5, 1.5, 0)
        u = hip.u64_array
        self.shape3 = u([batch, T, C])
        self.x_strides = u([T * C, C, 1])
        self.bias_strides = u([0, 0, 1])
        self.scale_strides = u([C, 0, 1])
        self.bias_shape = u([C])
        self.scale_shape = u([batch, 1, C])
        self.zero8 = u([0] * 8)
        hip.synchronize()

    # algorithmic bytes of each op: every distinct input byte read once, every
    # output byte written once, broadcast operands at their stored size
    def op_bytes(self):
        n, f = self.n, 4
        return {
            "x+bias": 2 * n * f + C * f,
            "x*scale": 2 * n * f + self.batch * C * f,
            "dbias=sum_BT(G)": n * f + C * f,
            "dscale=sum_T(G*x)": 2 * n * f + self.batch * C * f,
            "dx=G*scale": 2 * n * f + self.batch * C * f,
        }

    def ops(self):
        hip = self.hip
        call = hip.call
        F = hip.FLOAT32
        return [
            ("x+bias", "broadcast_binary", lambda: call(
                "spar_hip_launch_strided_binary", self.y1.ptr, self.x.ptr, self.x_strides, 0,
                self.bias.ptr, self.bias_strides, 0, 3, self.shape3, F, hip.ADD, 0)),
            ("x*scale", "broadcast_binary", lambda: call(
                "spar_hip_launch_strided_binary", self.y2.ptr, self.x.ptr, self.x_strides, 0,
                self.scale.ptr, self.scale_strides, 0, 3, self.shape3, F, hip.MULTIPLY, 0)),
            ("dbias=sum_BT(G)", "column_reduction", lambda: call(
                "spar_hip_launch_broadcast_reduce", self.dbias.ptr, self.G.ptr, 3, self.shape3, 1,
                self.bias_shape, self.zero8, self.n, F, 0)),
            ("dscale=sum_T(G*x)", "column_reduction", lambda: call(
                "spar_hip_launch_multiply_reduce", self.dscale.ptr, self.G.ptr, self.x.ptr, 3,
                self.shape3, 3, self.scale_shape, self.n, F, 0)),
            ("dx=G*scale", "broadcast_binary", lambda: call(
                "spar_hip_launch_strided_binary", self.dx.ptr, self.G.ptr, self.x_strides, 0,
                self.scale.ptr, self.scale_strides, 0, 3, self.shape3, F, hip.MULTIPLY, 0)),
        ]

    def step(self):
        for _, _, launch in self.ops():
            launch()


def time_ops(hip, ops, reps=20, warmup=3):
    """Per-launch time (ms) of each op: `reps` back-to-back launches of the op
    bracketed by one pair of HIP events on the backend's stream, divided by
    `reps`, so no event sits between two launches.  Every op streams at least
    512 MiB, twice the Infinity Cache, so repeated launches read from HBM."""
    for _ in range(warmup):
        for _, _, launch in ops:
            launch()
    hip.synchronize()
    times = {}
    start, stop = hip.Event(), hip.Event()
    for name, _, launch in ops:
        start.record()
        for _ in range(reps):
            launch()
        stop.record()
        times[name] = start.elapsed_ms(stop) / reps
    return times


def cpu_baseline(hip, work: Workload, sample_batch=16, repeats=3):
    """The oracle (a 1-thread C restatement of Spar's CPU loops) on the first
    `sample_batch` batch rows of the same device inputs."""
    import oracle.ops as O

    rows = sample_batch * T * C
    x = work.x.to_numpy(np.float32, (B, T, C))[:sample_batch].copy()
    G = work.G.to_numpy(np.float32, (B, T, C))[:sample_batch].copy()
    bias = work.bias.to_numpy(np.float32, (C,))
    scale = work.scale.to_numpy(np.float32, (B, 1, C))[:sample_batch].copy()
    sample = Workload.__new__(Workload)
    sample.n, sample.batch = rows, sample_batch
    nbytes = Workload.op_bytes(sample)
    ops = [
        ("x+bias", lambda: O.binary(x, bias, "add")),
        ("x*scale", lambda: O.binary(x, scale, "multiply")),
        ("dbias=sum_BT(G)", lambda: O.reduce_gradient(G, (C,))),
        ("dscale=sum_T(G*x)", lambda: O.reduce_gradient(O.binary(G, x, "multiply"), (sample_batch, 1, C))),
        ("dx=G*scale", lambda: O.binary(G, scale, "multiply")),
    ]
    per_rep = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        for _, fn in ops:
            fn()
        per_rep.append(time.perf_counter() - t0)
    seconds = statistics.median(per_rep)
    total = sum(nbytes.values())
    model = cpu_model()
    return {
        "value": round(total / seconds / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "cpu_model": model,
        "sample": (f"the five ops of the step on the first {sample_batch} of {B} batch rows "
                   f"(x[{sample_batch},{T},{C}], half the step's bytes, scaled by its own bytes), "
                   f"the oracle's C loops (-O2 -ffp-contract=off) on 1 core of {model} "
                   f"({os.cpu_count()} logical CPUs visible), median of {repeats} runs of "
                   f"{sum(per_rep) / repeats:.2f} s"),
        "seconds_per_step_sample": round(seconds, 4),
    }


def cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it, with its family, model and
    stepping numbers (a virtual machine may report only a vendor name)."""
    fields = {}
    try:
        with open("/proc/cpuinfo") as info:
            for line in info:
                if not line.strip():
                    break  # the first processor's block is enough
                key, _, value = line.partition(":")
                fields[key.strip()] = value.strip()
    except OSError:
        pass
    name = fields.get("model name") or platform.processor() or "unknown CPU"
    numbers = [f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields]
    return f"{name} ({', '.join(numbers)})" if numbers else name


def calibration_copy(hip, work):
    """One plain contiguous copy of x (512 MiB read, 512 MiB written), whose
    counters calibrate bytes per counter unit in the traffic summaries."""
    hip.call("spar_hip_launch_strided_copy", work.y1.ptr, work.x.ptr, 1, hip.u64_array([work.n]),
             hip.u64_array([1]), 0, work.n, 4, 0)
    hip.synchronize()


def main():
    args = parse()
    if args.list_suite_ops:
        print(json.dumps(SUITE_OPS))
        return
    if args.gpus != 1:
        print(f"bench.py runs on exactly one GPU (asked for {args.gpus}); this backend's "
              "benchmark is a single-device measurement", file=sys.stderr)
        sys.exit(2)
    from spar_amd import hip

    hip.load()
    if hip.device_count() < 1:
        print("no HIP device visible", file=sys.stderr)
        sys.exit(1)

    if args.suite_op:
        config, _, op = args.suite_op.partition("/")
        if op not in SUITE_OPS.get(config, []):
            print(f"unknown suite op {args.suite_op!r}", file=sys.stderr)
            sys.exit(2)
        suite = Suite(hip, profile=(config, op, args.profile_launches))
        suite.run([config])
        op_bytes = suite.profile_bytes
        del suite
        calibration_copy(hip, Workload(hip))
        print(json.dumps({"suite_op": args.suite_op, "launches": args.profile_launches,
                          "bytes": op_bytes, "copy_bytes": B * T * C * 4}))
        return

    work = Workload(hip)
    if args.profile_loop:
        for _ in range(args.profile_loop):
            work.step()
        calibration_copy(hip, work)
        print(json.dumps({"profile_loop_steps": args.profile_loop, "copy_bytes": work.n * 4}))
        return
    nbytes = work.op_bytes()
    step_bytes = sum(nbytes.values())
    for _ in range(args.warmup):
        work.step()
    hip.synchronize()

    start, stop = hip.Event(), hip.Event()
    hip.synchronize()
    wall0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        work.step()
    stop.record()
    hip.synchronize()
    wall = time.perf_counter() - wall0
    elapsed_ms = start.elapsed_ms(stop)
    ms_per_step = elapsed_ms / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    # per-kernel event timing (same stream as the launches)
    ops = work.ops()
    times = time_ops(hip, ops)
    per_op = {}
    kernel_time = {}
    kernel_bytes = {}
    for name, kernel, _ in ops:
        mean_ms = times[name]
        gbps = nbytes[name] / (mean_ms * 1e-3) / 1e9
        per_op[name] = {"kernel": kernel, "ms": round(mean_ms, 5), "GB/s": round(gbps, 1),
                        "frac": round(gbps / HBM_PEAK_GBPS, 4), "bytes": nbytes[name]}
        kernel_time[kernel] = kernel_time.get(kernel, 0.0) + mean_ms
        kernel_bytes[kernel] = kernel_bytes.get(kernel, 0) + nbytes[name]
    dominant = max(kernel_time, key=kernel_time.get)
    launches = sum(1 for _, k, _ in ops if k == dominant)
    achieved = kernel_bytes[dominant] / (kernel_time[dominant] * 1e-3) / 1e9
    # HBM bytes per launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE
    # (python3 -m spar_amd.rocprof_summary run ...), null until profiled.
    from spar_amd.rocprof_summary import TRAFFIC_FILE, read_traffic

    traffic = read_traffic(ROOT / "profiles" / TRAFFIC_FILE).get(dominant)
    roofline = {
        "bound": "hbm",
        "kernel": dominant,
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBPS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBPS, 4),
        "traffic": traffic,
        "bytes_per_launch": kernel_bytes[dominant] // launches,
        "avg_launch_ms": round(kernel_time[dominant] / launches, 5),
    }

    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (device SplitMix64 generator, seeds %s)" % SEEDS,
        "config": {
            "workload": "broadcast binary fp32: x[32,1024,4096]+bias[4096], x*scale[32,1,4096]; "
                        "backward dbias=sum_BT(G), dscale=sum_T(G*x), dx=G*scale",
            "elements": work.n,
            "step_bytes": step_bytes,
            "parallelism": "single device",
        },
        "frac_of_peak": round(value / HBM_PEAK_GBPS, 4),
        "elements_per_s": round(5 * work.n / (ms_per_step * 1e-3), 1),
        "wall_s": round(wall, 4),
        "per_op": per_op,
        "roofline": roofline,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(hip, work)
    suite = None
    if not args.no_suite:
        del work
        suite = Suite(hip)
        suite.run(None if args.suite_only is None else args.suite_only.split(","))
        result["suite"] = suite.summary()
    print(json.dumps(result), flush=True)
    if args.suite and suite is not None:
        for line in suite.lines:
            print(json.dumps(line), flush=True)


# ----------------------------------------------------------------- suite

MALL_BYTES = 256 << 20  # MI355X Infinity Cache

# The suite's configurations, their workloads and their ops, in run order.
SUITE_WORKLOADS = {
    "C1": "contiguous fp32 elementwise on [4096, 4096] a, b ~ N(0,1)",
    "C3": "axis reductions on [8192, 8192] ~ N(0,1); full reductions of 2^28 ~ U(-1,1)",
    "C4": "row softmax / log-softmax (and cross entropy) on logits [8192, 32768] ~ N(0, 2)",
    "C5": "LayerNorm chain through the Tensor API on [4096, 8192] views: a transposed "
          "[8192, 4096] base and a block of a [4608, 9216] base",
    "optim": "AdamW, gradient-norm summary and scaling over 124,439,808 fp32 parameters",
}
SUITE_OPS = {
    "C1": ["a+b", "a*b", "gelu(a)", "exp(a)"],
    "C3": [f"{op} axis {axis}" for axis in (1, 0) for op in ("sum", "mean", "max", "argmax")]
          + [f"full {op} 2^28" for op in ("sum", "mean", "max")],
    "C4": ["softmax forward", "softmax backward", "log_softmax forward", "log_softmax backward",
           "cross_entropy forward (fused)", "cross_entropy backward (fused)",
           "cross_entropy forward (composed, vs fused bytes)",
           "cross_entropy backward (composed, vs fused bytes)"],
    "C5": [f"{op} {view}" for view in ("transposed", "sliced")
           for op in ("mu=mean(x,1)", "xc=x-mu", "square(xc)", "var=mean(sq,1)", "xhat=xc/sd",
                      "xhat*gamma", "+beta", "y*G", "sum(y*G)")]
          + [f"{op} {view} (vs fused minimum)" for view in ("transposed", "sliced")
             for op in ("forward chain", "backward chain", "fused layer_norm forward",
                        "fused layer_norm backward")],
    "optim": ["adamw step (fp32, double math)", "gradient norm summary",
              "scale gradients in place"],
}
# Ops measured against a minimum other than their own bytes (the fused
# minimum of the C5 chain, the fused cross entropy's bytes): reported, but
# never a configuration's roofline op.
SUITE_REFERENCE_ONLY = ("composed", "chain", "fused layer_norm")


def rotation(set_bytes):
    """Buffer sets to rotate so that the other sets touched between two uses
    of one set total at least three times the Infinity Cache."""
    return max(3, -(-3 * MALL_BYTES // max(set_bytes, 1)) + 1)


class Suite:
    """Times every op of the benchmark configurations other than the default
    workload, two ways:

    * steady state ("ms", "GB/s", "frac"): back-to-back launches rotating over
      input/output sets that together exceed the Infinity Cache several times,
      so every launch reads from HBM and pays for the write-back of the dirty
      lines its predecessors left; HIP events bracket the whole run, which is
      divided by the number of launches;
    * cold ("cold_ms", "cold_GB/s"): one launch after a 512 MiB cached read
      (spar_hip_touch) that evicts the Infinity Cache and writes back its dirty
      lines, bracketed by its own events (median of `reps`).  It includes the
      launch's dispatch latency, and it excludes the write-back of what the
      launch itself leaves dirty in the cache, which flatters ordinary stores
      against non-temporal ones.

    Ops that need a fresh graph per launch (the backward chains) are timed
    cold only.

    With `profile=(config, op, launches)` only that op runs, `launches`
    times, each launch preceded by a marker dispatch (a 16-byte
    spar_hip_touch) and the last one followed by another, so a counter pass
    can attribute the dispatches between markers to the op (a prepare step,
    such as building a fresh graph, runs before its marker)."""

    def __init__(self, hip, reps=20, warmup=3, profile=None):
        self.hip = hip
        self.reps = reps
        self.warmup = warmup
        self.profile = profile
        self.lines = []
        self.results = {}
        self.profile_bytes = None
        self.flush = hip.DeviceBuffer(512 << 20)
        hip.call("spar_hip_zero", self.flush.ptr, self.flush.nbytes, 0)
        self.sink = hip.DeviceBuffer(16)
        self.start, self.stop = hip.Event(), hip.Event()

    def wanted(self, config, name):
        return self.profile is None or (config, name) == self.profile[:2]

    def measure(self, config, name, nbytes, launches, elements, prepare=None):
        assert name in SUITE_OPS[config], (config, name)
        if not self.wanted(config, name):
            return
        hip = self.hip
        if callable(launches):
            launches = [launches]
        if self.profile is not None:
            self.profile_bytes = nbytes
            hip.synchronize()
            for k in range(self.profile[2]):
                if prepare is not None:
                    prepare()
                hip.call("spar_hip_touch", self.sink.ptr, 16, 0, 0)  # marker: a launch starts
                launches[k % len(launches)]()
            hip.call("spar_hip_touch", self.sink.ptr, 16, 0, 0)  # marker: the last one ended
            hip.synchronize()
            return
        for _ in range(self.warmup):
            for launch in launches:
                if prepare is not None:
                    prepare()
                launch()
        hip.synchronize()
        samples = []
        for _ in range(self.reps):
            if prepare is not None:
                prepare()
            hip.call("spar_hip_touch", self.flush.ptr, self.flush.nbytes, self.sink.ptr, 0)
            self.start.record()
            launches[0]()
            self.stop.record()
            samples.append(self.start.elapsed_ms(self.stop))
        cold = statistics.median(samples)
        line = {"suite": config, "op": name}
        if prepare is None and len(launches) > 1:
            count = max(self.reps, 2 * len(launches))
            hip.synchronize()
            self.start.record()
            for k in range(count):
                launches[k % len(launches)]()
            self.stop.record()
            ms = self.start.elapsed_ms(self.stop) / count
            line["timing"] = f"steady, {len(launches)} rotated sets"
        else:
            ms = cold
            line["timing"] = "cold"
        gbps = nbytes / (ms * 1e-3) / 1e9
        line.update({"ms": round(ms, 5), "GB/s": round(gbps, 1),
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "bytes": nbytes,
                     "elements_per_s": round(elements / (ms * 1e-3), 1),
                     "cold_ms": round(cold, 5),
                     "cold_GB/s": round(nbytes / (cold * 1e-3) / 1e9, 1)})
        self.lines.append(line)
        self.results.setdefault(config, {})[name] = line

    def summary(self):
        """Per configuration: every op's steady-state figures with its HBM
        traffic per launch from the committed counter summary (null where
        none was measured), and the roofline record of its dominant op (the
        longest op measured against its own bytes)."""
        from spar_amd.rocprof_summary import read_op_traffic, suite_traffic_file

        out = {}
        for config, ops in self.results.items():
            traffic = read_op_traffic(ROOT / "profiles" / suite_traffic_file(config))
            entry = {"workload": SUITE_WORKLOADS[config], "ops": {}}
            for name, line in ops.items():
                entry["ops"][name] = {key: line[key] for key in ("ms", "GB/s", "frac", "bytes",
                                                                 "timing")}
                entry["ops"][name]["traffic"] = traffic.get(name)
            own = {name: line for name, line in ops.items()
                   if not any(tag in name for tag in SUITE_REFERENCE_ONLY)}
            if own:
                name = max(own, key=lambda op: own[op]["ms"])
                line = own[name]
                entry["roofline"] = {"op": name, "bound": "hbm", "achieved": line["GB/s"],
                                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": line["frac"],
                                     "bytes_per_launch": line["bytes"],
                                     "avg_launch_ms": line["ms"], "traffic": traffic.get(name)}
            out[config] = entry
        return out

    def run(self, only=None):
        for name, section in self.sections().items():
            if (only is None or name in only) and (self.profile is None
                                                    or self.profile[0] == name):
                section()

    def sections(self):
        hip = self.hip
        F = hip.FLOAT32
        u = hip.u64_array
        measure = self.measure

        def normal(n, seed, std=1.0):
            buf = hip.DeviceBuffer(n * 4)
            hip.call("spar_hip_random_normal", buf.ptr, n, F, seed, 0.0, std, 0)
            return buf

        def uniform(n, seed, low, high):
            buf = hip.DeviceBuffer(n * 4)
            hip.call("spar_hip_random_uniform", buf.ptr, n, F, seed, low, high, 0)
            return buf

        def c1():
            # C1: contiguous elementwise on [4096, 4096]; set 0 carries the
            # benchmark seeds, the other sets only rotate the cache.
            n = 4096 * 4096
            sets = [(normal(n, 1 + 100 * k), normal(n, 2 + 100 * k), hip.DeviceBuffer(n * 4))
                    for k in range(rotation(12 * n))]
            for name, op in (("a+b", hip.ADD), ("a*b", hip.MULTIPLY)):
                measure("C1", name, 12 * n, [lambda a=a, b=b, out=out, op=op: hip.call(
                    "spar_hip_launch_binary", out.ptr, a.ptr, b.ptr, n, F, op, 0) for a, b, out in sets], n)
            measure("C1", "gelu(a)", 8 * n, [lambda a=a, out=out: hip.call(
                "spar_hip_launch_unary", out.ptr, a.ptr, n, F, hip.GELU, 0) for a, _, out in sets], n)
            # exp(clip(a, -10, 10)): the clip is the identity on these draws (checked here)
            peak = hip.DeviceBuffer(8)
            for a, _, out in sets:
                hip.call("spar_hip_launch_unary", out.ptr, a.ptr, n, F, hip.NEGATE, 0)
                for source in (a, out):  # max(a) and max(-a)
                    hip.call("spar_hip_launch_reduction", peak.ptr, source.ptr, n, F, hip.MAX, 0)
                    assert peak.to_numpy(np.float32, (1,))[0] <= 10.0, "C1 draw exceeds the clip range"
            measure("C1", "exp(a)", 8 * n, [lambda a=a, out=out: hip.call(
                "spar_hip_launch_unary", out.ptr, a.ptr, n, F, hip.EXP, 0) for a, _, out in sets], n)
            del sets

        def c3():
            # C3: axis reductions on [8192, 8192] and a full reduction of 2^28
            R = 8192
            n = R * R
            sets = [(normal(n, 3 + 100 * k), hip.DeviceBuffer(R * 8)) for k in range(rotation(4 * n))]
            codes = {"sum": hip.SUM, "mean": hip.MEAN, "max": hip.MAX, "argmax": hip.ARGMAX}
            for axis in (1, 0):
                for name, code in codes.items():
                    out_bytes = R * (8 if name == "argmax" else 4)
                    measure("C3", f"{name} axis {axis}", 4 * n + out_bytes, [
                        lambda x=x, out=out, code=code, axis=axis: hip.call(
                            "spar_hip_launch_axis_reduction", out.ptr, x.ptr, 2, u([R, R]), u([R, 1]), 0,
                            1 << axis, F, code, 0) for x, out in sets], n)
            del sets
            n = 1 << 28
            sets = [(uniform(n, 4 + 100 * k, -1.0, 1.0), hip.DeviceBuffer(8))
                    for k in range(rotation(4 * n))]
            for name in ("sum", "mean", "max"):
                measure("C3", f"full {name} 2^28", 4 * n + 4, [lambda v=v, out=out, name=name: hip.call(
                    "spar_hip_launch_reduction", out.ptr, v.ptr, n, F, codes[name], 0)
                    for v, out in sets], n)
            del sets

        def c4():
            # C4: row softmax / log-softmax on [8192, 32768]
            rows, V = 8192, 32768
            n = rows * V
            count = rotation(16 * n)

            class Set:
                def __init__(self, k):
                    self.logits = normal(n, 5 + 100 * k, np.sqrt(2.0))
                    self.grad = normal(n, 6 + 100 * k)
                    self.probs = hip.DeviceBuffer(n * 4)
                    self.dx = hip.DeviceBuffer(n * 4)
                    self.undefined = hip.DeviceBuffer(rows * 4)

            sets = [Set(k) for k in range(count)]
            for log in (0, 1):
                label = "log_softmax" if log else "softmax"
                measure("C4", f"{label} forward", 8 * n + 4 * rows, [lambda s=s, log=log: hip.call(
                    "spar_hip_launch_probability_forward", s.probs.ptr, s.undefined.ptr, s.logits.ptr,
                    rows, V, 1, F, log, 0) for s in sets], n)
                measure("C4", f"{label} backward", 12 * n + 4 * rows, [lambda s=s, log=log: hip.call(
                    "spar_hip_launch_probability_backward", s.dx.ptr, s.grad.ptr, s.probs.ptr,
                    s.undefined.ptr, rows, V, 1, F, log, 0) for s in sets], n)
            # C4 as a loss: cross entropy over the same logits, fused (one read of the
            # logits forward; one read and one write backward) and composed as the
            # reference runs it (log_softmax, NLL gather; zero fill, NLL scatter,
            # log_softmax backward), with the same targets.
            targets = hip.DeviceBuffer(rows * 8)
            hip.call("spar_hip_copy_host_to_device", targets.ptr,
                     np.random.default_rng(9).integers(0, V, rows).astype(np.int64).ctypes.data,
                     rows * 8, 0)
            losses, row_max, row_log_sum = (hip.DeviceBuffer(rows * 4) for _ in range(3))
            invalid = hip.DeviceBuffer(4)
            loss_grad = uniform(rows, 10, 0.5, 1.5)
            small = rows * (8 + 4 * 4)  # targets read; loss, max, log-sum, flag written
            measure("C4", "cross_entropy forward (fused)", 4 * n + small, [lambda s=s: hip.call(
                "spar_hip_launch_cross_entropy_forward", losses.ptr, row_max.ptr, row_log_sum.ptr,
                s.undefined.ptr, invalid.ptr, s.logits.ptr, targets.ptr, rows, V, 0, F, hip.INT64, 0, 0)
                for s in sets], n)
            # the backward of each set uses that set's forward statistics
            for s in sets:
                s.row_max, s.row_log_sum = hip.DeviceBuffer(rows * 4), hip.DeviceBuffer(rows * 4)
                hip.call("spar_hip_launch_cross_entropy_forward", losses.ptr, s.row_max.ptr,
                         s.row_log_sum.ptr, s.undefined.ptr, invalid.ptr, s.logits.ptr, targets.ptr, rows,
                         V, 0, F, hip.INT64, 0, 0)
            measure("C4", "cross_entropy backward (fused)", 8 * n + rows * 24, [lambda s=s: hip.call(
                "spar_hip_launch_cross_entropy_backward", s.dx.ptr, loss_grad.ptr, s.logits.ptr,
                s.row_max.ptr, s.row_log_sum.ptr, s.undefined.ptr, targets.ptr, rows, V, 0, F,
                hip.INT64, 0, 0) for s in sets], n)

            def composed_forward(s):
                hip.call("spar_hip_launch_probability_forward", s.probs.ptr, s.undefined.ptr,
                         s.logits.ptr, rows, V, 1, F, 1, 0)
                hip.call("spar_hip_launch_nll_forward", losses.ptr, s.probs.ptr, targets.ptr, rows, V, 0,
                         F, hip.INT64, 0, 0)

            def composed_backward(s):
                hip.call("spar_hip_zero", s.grad.ptr, n * 4, 0)
                hip.call("spar_hip_launch_nll_backward", s.grad.ptr, loss_grad.ptr, targets.ptr, rows, V,
                         0, F, hip.INT64, 0, 0)
                hip.call("spar_hip_launch_probability_backward", s.dx.ptr, s.grad.ptr, s.probs.ptr,
                         s.undefined.ptr, rows, V, 1, F, 1, 0)

            # reported against the fused kernels' bytes, so the ratio is the speed-up
            measure("C4", "cross_entropy forward (composed, vs fused bytes)", 4 * n + small,
                    [lambda s=s: composed_forward(s) for s in sets], n)
            measure("C4", "cross_entropy backward (composed, vs fused bytes)", 8 * n + rows * 24,
                    [lambda s=s: composed_backward(s) for s in sets], n)
            del sets, targets, losses, row_max, row_log_sum, invalid, loss_grad

        def c5():
            # C5: the LayerNorm chain on a transposed view (a [8192,4096] base viewed
            # as [4096,8192]) and on a [4096,8192] block at a nonzero offset of a
            # [4608,9216] base, through the Tensor API: each op's time includes its
            # host-side dispatch and allocation as well as its kernels.  Then
            # loss = sum(y * G) and loss.backward() into base, gamma and beta.  Each
            # rotated set has its own base, G and chain intermediates.
            from spar_amd import spar

            device = spar.Device.hip(0)
            f32 = spar.DType.float32
            rows, cols = 4096, 8192
            n = rows * cols
            T = 4 * n  # bytes of one full-tensor read or write
            rng = spar.Random(7)
            gamma = spar.random_uniform([cols], f32, rng, 0.5, 1.5, device)
            beta = spar.random_uniform([cols], f32, rng, -0.1, 0.1, device)
            count = rotation(3 * T)
            Gs = [spar.random_normal([rows, cols], f32, rng, 0.0, 1.0, device) for _ in range(count)]
            shapes = {"transposed": [8192, 4096], "sliced": [4608, 9216]}
            bases = {label: [spar.random_normal(shape, f32, rng, 0.0, 1.0, device) for _ in range(count)]
                     for label, shape in shapes.items()}
            for leaf in (gamma, beta, *bases["transposed"], *bases["sliced"]):
                leaf.set_requires_grad(True)

            def view_of(label, k=0):
                base = bases[label][k]
                return base.transpose(0, 1) if label == "transposed" else base.narrow(0, 256, rows).narrow(1, 512, cols)

            def forward(x, G):
                mu = spar.mean(x, [1], True)
                xc = spar.subtract(x, mu)
                var = spar.mean(spar.square(xc), [1], True)
                xhat = spar.divide(xc, spar.sqrt(spar.add_scalar(var, 1e-5)))
                y = spar.add(spar.multiply(xhat, gamma), beta)
                return spar.sum(spar.multiply(y, G), None, False)

            for label in bases:
                chains = []
                for k in range(count):
                    c = {"x": view_of(label, k), "G": Gs[k]}
                    c["mu"] = spar.mean(c["x"], [1], True)
                    c["xc"] = spar.subtract(c["x"], c["mu"])
                    c["sq"] = spar.square(c["xc"])
                    c["var"] = spar.mean(c["sq"], [1], True)
                    c["sd"] = spar.sqrt(spar.add_scalar(c["var"], 1e-5))
                    c["xhat"] = spar.divide(c["xc"], c["sd"])
                    c["yg"] = spar.multiply(c["xhat"], gamma)
                    c["y"] = spar.add(c["yg"], beta)
                    c["yG"] = spar.multiply(c["y"], c["G"])
                    chains.append(c)

                def each(fn):
                    return [lambda c=c: fn(c) for c in chains]

                measure("C5", f"mu=mean(x,1) {label}", T + 4 * rows,
                        each(lambda c: spar.mean(c["x"], [1], True)), n)
                measure("C5", f"xc=x-mu {label}", 2 * T + 4 * rows,
                        each(lambda c: spar.subtract(c["x"], c["mu"])), n)
                measure("C5", f"square(xc) {label}", 2 * T, each(lambda c: spar.square(c["xc"])), n)
                measure("C5", f"var=mean(sq,1) {label}", T + 4 * rows,
                        each(lambda c: spar.mean(c["sq"], [1], True)), n)
                measure("C5", f"xhat=xc/sd {label}", 2 * T + 4 * rows,
                        each(lambda c: spar.divide(c["xc"], c["sd"])), n)
                measure("C5", f"xhat*gamma {label}", 2 * T + 4 * cols,
                        each(lambda c: spar.multiply(c["xhat"], gamma)), n)
                measure("C5", f"+beta {label}", 2 * T + 4 * cols, each(lambda c: spar.add(c["yg"], beta)), n)
                measure("C5", f"y*G {label}", 3 * T, each(lambda c: spar.multiply(c["y"], c["G"])), n)
                measure("C5", f"sum(y*G) {label}", T + 4, each(lambda c: spar.sum(c["yG"], None, False)), n)
                del chains
                # Whole forward, then backward.  Both are reported against the fused
                # minimum: forward reads x and G once (the loss is a scalar);
                # backward reads x and G and writes dx (gamma, beta grads are small).
                measure("C5", f"forward chain {label} (vs fused minimum)", 2 * T,
                        [lambda k=k: forward(view_of(label, k), Gs[k]) for k in range(count)], n)
                losses = []

                def prepare():
                    for leaf in (gamma, beta, bases[label][0]):
                        leaf.zero_grad()
                    losses[:] = [forward(view_of(label), Gs[0])]

                measure("C5", f"backward chain {label} (vs fused minimum)", 3 * T,
                        lambda: losses[0].backward(), n, prepare=prepare)

                # The same LayerNorm fused (spar.layer_norm); a non-contiguous view is
                # first made contiguous, inside the timed op.
                measure("C5", f"fused layer_norm forward {label} (vs fused minimum)", 2 * T,
                        [lambda k=k: spar.layer_norm(view_of(label, k), gamma, beta, 1e-5)
                         for k in range(count)], n)

                def prepare_fused():
                    for leaf in (gamma, beta, bases[label][0]):
                        leaf.zero_grad()
                    y = spar.layer_norm(view_of(label), gamma, beta, 1e-5)
                    losses[:] = [spar.sum(spar.multiply(y, Gs[0]), None, False)]

                measure("C5", f"fused layer_norm backward {label} (vs fused minimum)", 3 * T,
                        lambda: losses[0].backward(), n, prepare=prepare_fused)
                del losses

        def optim():
            # Optimizer: one AdamW step, the gradient-norm summary and the clip scaling
            # over GPT-2 small's 124,439,808 fp32 parameters held as one flat buffer.
            n = 124_439_808
            count = rotation(16 * n)
            sets = [(normal(n, 81 + 100 * k), normal(n, 82 + 100 * k, 1e-2),
                     normal(n, 83 + 100 * k, 1e-3), uniform(n, 84 + 100 * k, 0.0, 1e-5),
                     hip.DeviceBuffer(64)) for k in range(count)]
            c1, c2 = 1.0 - 0.9 ** 1000, 1.0 - 0.95 ** 1000
            measure("optim", "adamw step (fp32, double math)", 28 * n, [
                lambda p=p, g=g, m=m, v=v: hip.call(
                    "spar_hip_launch_adamw", p.ptr, g.ptr, m.ptr, v.ptr, n, F, 3e-4, 0.9, 0.95, 1e-8, 0.1,
                    c1, c2, 0) for p, g, m, v, _ in sets], n)
            measure("optim", "gradient norm summary", 4 * n, [lambda g=g, summary=summary: hip.call(
                "spar_hip_launch_gradient_norm_summary", summary.ptr, g.ptr, n, F, 0)
                for _, g, _, _, summary in sets], n)
            measure("optim", "scale gradients in place", 8 * n, [lambda g=g: hip.call(
                "spar_hip_launch_scale_in_place", g.ptr, n, F, 1.0, 0) for _, g, _, _, _ in sets], n)
            del sets

        return {"C1": c1, "C3": c3, "C4": c4, "C5": c5, "optim": optim}


if __name__ == "__main__":
    main()
