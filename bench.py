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
Its `suite` key holds every op of the other configurations (C1, the same ops
on [8192, 8192] as C1L, C3, C4, C5 and the optimizer kernels), each timed
steady state, as a compact [ms, fraction of peak, L2-fabric traffic MB, CPU
GB/s] array: the traffic per launch that the committed rocprof summaries
measured, and Spar's CPU path (the oracle's 1-thread C loops) timed on a
bounded sample of the same inputs in the same run.  Each configuration also
carries a roofline record for its dominant op and its CPU baseline.
`--suite` also prints one JSON line per op with the cold timings;
`--suite-op CONFIG/OP --profile-launches K` runs only that op, K times, for
the counter passes that write those summaries.
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
                   help="comma-separated suite sections to run (C1,C1L,C3,C4,C5,optim)")
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


def cpu_baseline(hip, work: Workload, sample_batch=8, repeats=3):
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
        "sample": (f"the step's 5 ops on batch rows 0-{sample_batch - 1} of {B} "
                   f"(x[{sample_batch},{T},{C}]), GB/s from the sample's own bytes; oracle C "
                   f"loops (-O2 -ffp-contract=off), 1 thread, {os.cpu_count()} logical CPUs "
                   f"visible, median of {repeats}"),
        "s": round(seconds, 4),
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
        per_op[name] = [round(mean_ms, 5), round(gbps / HBM_PEAK_GBPS, 4)]
        kernel_time[kernel] = kernel_time.get(kernel, 0.0) + mean_ms
        kernel_bytes[kernel] = kernel_bytes.get(kernel, 0) + nbytes[name]
    dominant = max(kernel_time, key=kernel_time.get)
    launches = sum(1 for _, k, _ in ops if k == dominant)
    achieved = kernel_bytes[dominant] / (kernel_time[dominant] * 1e-3) / 1e9
    # HBM bytes per launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE
    # (python3 rocprof_summary.py run ...), null until profiled.
    from rocprof_summary import TRAFFIC_FILE, read_traffic

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
        "per_op": per_op,  # op: [ms per launch, fraction of 8 TB/s]
        "roofline": roofline,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(hip, work)
    suite = None
    if not args.no_suite:
        del work
        suite = Suite(hip, cpu=not args.no_cpu_baseline)
        suite.run(None if args.suite_only is None else args.suite_only.split(","))
        result["suite_format"] = ("op: [ms per launch, fraction of 8 TB/s, L2-fabric MB per "
                                  "launch, CPU path GB/s]; rooflines hbm-bound, peak 8000 GB/s")
        result["suite"] = suite.summary()
    print(json.dumps(result), flush=True)
    if args.suite and suite is not None:
        for line in suite.lines:
            print(json.dumps(line), flush=True)


# ----------------------------------------------------------------- suite

MALL_BYTES = 256 << 20  # MI355X Infinity Cache

# The suite's configurations, their workloads and their ops, in run order.
SUITE_WORKLOADS = {
    "C1": "a, b [4096,4096] ~ N(0,1)",
    "C1L": "a, b [8192,8192] ~ N(0,1)",
    "C3": "X [8192,8192] ~ N(0,1); v [2^28] ~ U(-1,1)",
    "C4": "logits [8192,32768] ~ N(0,2); composed CE (cross entropy) against fused CE bytes",
    "C5": "LayerNorm (LN) through the Tensor API on [4096,8192] views of a [8192,4096] base "
          "(transposed) and a [4608,9216] base (sliced); LN ops against the fused minimum "
          "(fwd: x in, y out; bwd: x, G in, dx out); the LN backwards timed cold",
    "optim": "124,439,808 fp32 parameters; AdamW with double inner math",
}
SUITE_OPS = {
    "C1": ["a+b", "a*b", "gelu(a)", "exp(a)"],
    "C1L": ["a+b", "a*b", "gelu(a)", "exp(a)"],
    "C3": [f"{op} axis {axis}" for axis in (1, 0) for op in ("sum", "mean", "max", "argmax")]
          + [f"full {op} 2^28" for op in ("sum", "mean", "max")],
    "C4": ["softmax forward", "softmax backward", "log_softmax forward", "log_softmax backward",
           "CE forward fused", "CE backward fused", "CE forward composed",
           "CE backward composed"],
    "C5": [f"{op} {view}" for view in ("transposed", "sliced")
           for op in ("mu=mean(x,1)", "xc=x-mu", "square(xc)", "var=mean(sq,1)", "xhat=xc/sd",
                      "xhat*gamma", "+beta", "y*G", "sum(y*G)")]
          + [f"{op} {view}" for view in ("transposed", "sliced")
             for op in ("LN forward chain", "LN backward chain", "fused LN forward",
                        "fused LN backward")],
    "optim": ["adamw step", "grad norm summary", "scale in place"],
}
# Ops measured against a minimum other than their own bytes (the fused
# minimum of the C5 chain, the fused cross entropy's bytes): reported, but
# never a configuration's roofline op.
SUITE_REFERENCE_ONLY = ("composed", "chain", "fused LN")


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

    Ops that need a fresh graph per launch (the backwards) are timed in
    steady state over graphs built beforehand on the rotated sets, each
    launch clearing its leaves' gradients on the host first (no device work)
    so that it writes fresh gradients as a cold launch does.

    With `profile=(config, op, launches)` only that op runs, `launches`
    times, each launch between an opening and a closing marker dispatch (a
    16-byte spar_hip_touch), so a counter pass attributes to the op exactly
    the dispatches inside each marker pair; a prepare step, such as building
    a fresh graph, runs between a closing marker and the next opening one."""

    def __init__(self, hip, reps=20, warmup=3, profile=None, cpu=False):
        self.hip = hip
        self.reps = reps
        self.warmup = warmup
        self.profile = profile
        self.with_cpu = cpu and profile is None
        self.lines = []
        self.results = {}
        self.cpu = {}
        self.profile_bytes = None
        self.flush = hip.DeviceBuffer(512 << 20)
        hip.call("spar_hip_zero", self.flush.ptr, self.flush.nbytes, 0)
        self.sink = hip.DeviceBuffer(16)
        self.start, self.stop = hip.Event(), hip.Event()

    def wanted(self, config, name):
        return self.profile is None or (config, name) == self.profile[:2]

    def measure(self, config, name, nbytes, launches, elements, prepare=None, build_runs=None):
        """`prepare`, when given, runs before each cold launch (outside its
        events): work the launch needs first, such as building a fresh graph.
        `build_runs(count)`, when given, returns `count` launches that are
        ready to run back to back (their graphs built beforehand, over the
        rotated sets), so that such an op is also timed in steady state."""
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
                    prepare()  # outside any window: its dispatches are not the op's
                hip.call("spar_hip_touch", self.sink.ptr, 16, 0, 0)  # marker: the launch opens
                launches[k % len(launches)]()
                hip.call("spar_hip_touch", self.sink.ptr, 16, 0, 0)  # marker: the launch closes
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
            line["sets"] = len(launches)
        elif build_runs is not None:
            runs, sets = build_runs(self.reps)
            hip.synchronize()
            self.start.record()
            for run in runs:
                run()
            self.stop.record()
            ms = self.start.elapsed_ms(self.stop) / len(runs)
            del runs
            line["timing"] = f"steady, {sets} rotated sets, graphs built beforehand"
            line["sets"] = sets
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

    def cpu_baseline(self, config, sample, ops, repeats=3):
        """Spar's CPU path, as the oracle restates it (1-thread C loops built
        -O2 -ffp-contract=off over logical indices), on a bounded sample of
        this configuration's inputs copied from the device: `ops` is a list
        of (op name, the sample's algorithmic bytes, callable).  Each op is
        timed per run; the median over `repeats` runs gives each op's GB/s
        and, over all ops, the configuration's."""
        if not self.with_cpu:
            return
        per_op = {name: [] for name, _, _ in ops}
        for _ in range(repeats):
            for name, _, fn in ops:
                t0 = time.perf_counter()
                fn()
                per_op[name].append(time.perf_counter() - t0)
        seconds = {name: statistics.median(times) for name, times in per_op.items()}
        total_s = sum(seconds.values())
        total_bytes = sum(nbytes for _, nbytes, _ in ops)
        self.cpu[config] = {
            "GB/s": round(total_bytes / total_s / 1e9, 3), "s": round(total_s, 3),
            "sample": sample,
            "ops": {name: round(nbytes / seconds[name] / 1e9, 3) for name, nbytes, _ in ops}}

    def summary(self):
        """Per configuration, compactly: each op as [ms per launch, fraction
        of 8 TB/s, L2-fabric MB per launch from the committed counter summary
        (null where none was measured), the CPU path's GB/s on its sample
        (null where it has none)]; the roofline record of the configuration's
        dominant op (the longest op measured against its own bytes); and the
        CPU baseline."""
        from rocprof_summary import read_op_traffic, suite_traffic_file

        out = {}
        for config, ops in self.results.items():
            traffic = read_op_traffic(ROOT / "profiles" / suite_traffic_file(config))
            cpu = self.cpu.get(config, {})
            cpu_ops = cpu.get("ops", {})
            entry = {"workload": SUITE_WORKLOADS[config], "ops": {}}
            for name, line in ops.items():
                moved = traffic.get(name)
                entry["ops"][name] = [line["ms"], line["frac"],
                                      None if moved is None else round(moved / 1e6, 1),
                                      cpu_ops.get(name)]
                if line["timing"] != "cold":
                    entry["sets"] = line["sets"]
            own = {name: line for name, line in ops.items()
                   if not any(tag in name for tag in SUITE_REFERENCE_ONLY)}
            if own:
                name = max(own, key=lambda op: own[op]["ms"])
                line = own[name]
                entry["roofline"] = {"op": name, "achieved": line["GB/s"], "frac": line["frac"],
                                     "bytes_per_launch": line["bytes"], "traffic": traffic.get(name)}
            if cpu:
                entry["cpu_baseline"] = {key: cpu[key] for key in ("GB/s", "s", "sample")}
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

        def elementwise(config, side, cpu_rows):
            # Contiguous elementwise on [side, side]; set 0 carries the
            # benchmark seeds, the other sets only rotate the cache.
            n = side * side
            sets = [(normal(n, 1 + 100 * k), normal(n, 2 + 100 * k), hip.DeviceBuffer(n * 4))
                    for k in range(rotation(12 * n))]
            for name, op in (("a+b", hip.ADD), ("a*b", hip.MULTIPLY)):
                measure(config, name, 12 * n, [lambda a=a, b=b, out=out, op=op: hip.call(
                    "spar_hip_launch_binary", out.ptr, a.ptr, b.ptr, n, F, op, 0) for a, b, out in sets], n)
            measure(config, "gelu(a)", 8 * n, [lambda a=a, out=out: hip.call(
                "spar_hip_launch_unary", out.ptr, a.ptr, n, F, hip.GELU, 0) for a, _, out in sets], n)
            # exp(clip(a, -10, 10)): the clip is the identity on these draws (checked here)
            peak = hip.DeviceBuffer(8)
            for a, _, out in sets:
                hip.call("spar_hip_launch_unary", out.ptr, a.ptr, n, F, hip.NEGATE, 0)
                for source in (a, out):  # max(a) and max(-a)
                    hip.call("spar_hip_launch_reduction", peak.ptr, source.ptr, n, F, hip.MAX, 0)
                    assert peak.to_numpy(np.float32, (1,))[0] <= 10.0, "draw exceeds the clip range"
            measure(config, "exp(a)", 8 * n, [lambda a=a, out=out: hip.call(
                "spar_hip_launch_unary", out.ptr, a.ptr, n, F, hip.EXP, 0) for a, _, out in sets], n)
            if self.with_cpu:
                import oracle.ops as O

                a = sets[0][0].to_numpy(np.float32, (side, side))[:cpu_rows].copy()
                b = sets[0][1].to_numpy(np.float32, (side, side))[:cpu_rows].copy()
                m = a.size
                self.cpu_baseline(config, f"rows 0-{cpu_rows - 1} of {side}", [
                    ("a+b", 12 * m, lambda: O.binary(a, b, "add")),
                    ("a*b", 12 * m, lambda: O.binary(a, b, "multiply")),
                    ("gelu(a)", 8 * m, lambda: O.unary(a, "gelu")),
                    ("exp(a)", 8 * m, lambda: O.unary(a, "exp"))])
            del sets

        def c1():
            elementwise("C1", 4096, 4096)

        def c1l():
            elementwise("C1L", 8192, 1024)

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
            cpu_ops = []
            if self.with_cpu:
                import oracle.ops as O

                # axis reductions of rows 0-1023: over axis 1, 1024 rows of 8192; over
                # axis 0, the block's 8192 columns of 1024
                block = sets[0][0].to_numpy(np.float32, (R, R))[:1024].copy()
                m = block.size
                for axis in (1, 0):
                    cpu_ops += [
                        (f"sum axis {axis}", 4 * m, lambda axis=axis: O.axis_sum(block, [axis])),
                        (f"mean axis {axis}", 4 * m,
                         lambda axis=axis: O.scalar(O.axis_sum(block, [axis]), "divide", block.shape[axis])),
                        (f"max axis {axis}", 4 * m, lambda axis=axis: O.axis_max(block, [axis])),
                        (f"argmax axis {axis}", 4 * m, lambda axis=axis: O.axis_max(block, [axis]))]
            del sets
            n = 1 << 28
            sets = [(uniform(n, 4 + 100 * k, -1.0, 1.0), hip.DeviceBuffer(8))
                    for k in range(rotation(4 * n))]
            for name in ("sum", "mean", "max"):
                measure("C3", f"full {name} 2^28", 4 * n + 4, [lambda v=v, out=out, name=name: hip.call(
                    "spar_hip_launch_reduction", out.ptr, v.ptr, n, F, codes[name], 0)
                    for v, out in sets], n)
            if self.with_cpu:
                head = sets[0][0].to_numpy(np.float32, (n,))[:1 << 24].copy()
                cpu_ops += [(f"full {name} 2^28", 4 * head.size,
                             lambda name=name: O.full_reduce(head, name)) for name in ("sum", "mean", "max")]
                self.cpu_baseline("C3", "axis ops: rows 0-1023 of 8192; full ops: the first 2^24 "
                                  "elements", cpu_ops)
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
            if self.with_cpu:
                import oracle.ops as O

                k = 128  # rows 0-127
                logits = sets[0].logits.to_numpy(np.float32, (rows, V))[:k].copy()
                grad = sets[0].grad.to_numpy(np.float32, (rows, V))[:k].copy()
                probs, undefined = O.softmax_axis(logits, 1)
                log_probs, log_undefined = O.log_softmax(logits, 1)
                m = logits.size
                self.cpu_baseline("C4", f"softmax family on rows 0-{k - 1} of {rows}", [
                    ("softmax forward", 8 * m + 4 * k, lambda: O.softmax_axis(logits, 1)),
                    ("softmax backward", 12 * m + 4 * k,
                     lambda: O.softmax_axis_backward(grad, probs, undefined, 1)),
                    ("log_softmax forward", 8 * m + 4 * k, lambda: O.log_softmax(logits, 1)),
                    ("log_softmax backward", 12 * m + 4 * k,
                     lambda: O.log_softmax_backward(grad, log_probs, log_undefined, 1))])
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
            measure("C4", "CE forward fused", 4 * n + small, [lambda s=s: hip.call(
                "spar_hip_launch_cross_entropy_forward", losses.ptr, row_max.ptr, row_log_sum.ptr,
                s.undefined.ptr, invalid.ptr, s.logits.ptr, targets.ptr, rows, V, 0, F, hip.INT64, 0, 0)
                for s in sets], n)
            # the backward of each set uses that set's forward statistics
            for s in sets:
                s.row_max, s.row_log_sum = hip.DeviceBuffer(rows * 4), hip.DeviceBuffer(rows * 4)
                hip.call("spar_hip_launch_cross_entropy_forward", losses.ptr, s.row_max.ptr,
                         s.row_log_sum.ptr, s.undefined.ptr, invalid.ptr, s.logits.ptr, targets.ptr, rows,
                         V, 0, F, hip.INT64, 0, 0)
            measure("C4", "CE backward fused", 8 * n + rows * 24, [lambda s=s: hip.call(
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
            measure("C4", "CE forward composed", 4 * n + small,
                    [lambda s=s: composed_forward(s) for s in sets], n)
            measure("C4", "CE backward composed", 8 * n + rows * 24,
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
                measure("C5", f"LN forward chain {label}", 2 * T,
                        [lambda k=k: forward(view_of(label, k), Gs[k]) for k in range(count)], n)
                losses = []

                def prepare():
                    for leaf in (gamma, beta, bases[label][0]):
                        leaf.zero_grad()
                    losses[:] = [forward(view_of(label), Gs[0])]

                def backward_runs(make_loss, runs):
                    # `runs` losses built over the rotated sets in turn; each run
                    # clears its leaves' gradients (host only: no device work) so
                    # that every backward writes fresh gradients, as a cold one does.
                    built = [(k % count, make_loss(k % count)) for k in range(runs)]

                    def run(k, loss):
                        for leaf in (gamma, beta, bases[label][k]):
                            leaf.zero_grad()
                        loss.backward()

                    return [lambda k=k, loss=loss: run(k, loss) for k, loss in built], count

                measure("C5", f"LN backward chain {label}", 3 * T,
                        lambda: losses[0].backward(), n, prepare=prepare,
                        build_runs=lambda runs: backward_runs(
                            lambda k: forward(view_of(label, k), Gs[k]), runs))

                # The same LayerNorm fused (spar.layer_norm); a non-contiguous view is
                # first made contiguous, inside the timed op.
                measure("C5", f"fused LN forward {label}", 2 * T,
                        [lambda k=k: spar.layer_norm(view_of(label, k), gamma, beta, 1e-5)
                         for k in range(count)], n)

                def prepare_fused():
                    for leaf in (gamma, beta, bases[label][0]):
                        leaf.zero_grad()
                    y = spar.layer_norm(view_of(label), gamma, beta, 1e-5)
                    losses[:] = [spar.sum(spar.multiply(y, Gs[0]), None, False)]

                def fused_loss(k):
                    y = spar.layer_norm(view_of(label, k), gamma, beta, 1e-5)
                    return spar.sum(spar.multiply(y, Gs[k]), None, False)

                measure("C5", f"fused LN backward {label}", 3 * T,
                        lambda: losses[0].backward(), n, prepare=prepare_fused,
                        build_runs=lambda runs: backward_runs(fused_loss, runs))
                del losses
            if self.with_cpu:
                import oracle.reference as R

                # The same chain on the reference's CPU path for rows 0-255 of each
                # view: the transposed view of columns 0-255 of the base, and the
                # block of rows 256-511 of the sliced base's first 512 rows.
                k = 256
                cpu_device = spar.Device.cpu()

                def host(t):
                    return np.ascontiguousarray(t.to(cpu_device).numpy())

                g_host, b_host = host(gamma), host(beta)
                G_host = host(Gs[0])[:k].copy()
                blocks = {"transposed": host(bases["transposed"][0])[:, :k].copy(),
                          "sliced": host(bases["sliced"][0])[:256 + k].copy()}
                cpu_ops, graphs = [], {}
                for label, block in blocks.items():
                    leaves = [R.RTensor.of(block, True), R.RTensor.of(g_host, True),
                              R.RTensor.of(b_host, True)]
                    G_r = R.RTensor.of(G_host)

                    def cpu_forward(label=label, leaves=leaves, G_r=G_r):
                        for leaf in leaves:
                            leaf.meta.leaf_grad = None
                        base, w, b = leaves
                        x = base.transpose(0, 1) if label == "transposed" else \
                            base.narrow(0, 256, k).narrow(1, 512, cols)
                        mu = R.mean(x, [1], True)
                        xc = R.subtract(x, mu)
                        var = R.mean(R.square(xc), [1], True)
                        xhat = R.divide(xc, R.sqrt(R.add_scalar(var, 1e-5)))
                        y = R.add(R.multiply(xhat, w), b)
                        graphs[label] = R.sum(R.multiply(y, G_r), None, False)

                    T_s = 4 * k * cols
                    cpu_ops += [(f"LN forward chain {label}", 2 * T_s, cpu_forward),
                                (f"LN backward chain {label}", 3 * T_s,
                                 lambda label=label: graphs[label].backward())]
                self.cpu_baseline("C5", f"the LN chain, forward and backward, on rows 0-{k - 1} "
                                  f"of each view", cpu_ops)

        def optim():
            # Optimizer: one AdamW step, the gradient-norm summary and the clip scaling
            # over GPT-2 small's 124,439,808 fp32 parameters held as one flat buffer.
            n = 124_439_808
            count = rotation(16 * n)
            sets = [(normal(n, 81 + 100 * k), normal(n, 82 + 100 * k, 1e-2),
                     normal(n, 83 + 100 * k, 1e-3), uniform(n, 84 + 100 * k, 0.0, 1e-5),
                     hip.DeviceBuffer(64)) for k in range(count)]
            c1, c2 = 1.0 - 0.9 ** 1000, 1.0 - 0.95 ** 1000
            measure("optim", "adamw step", 28 * n, [
                lambda p=p, g=g, m=m, v=v: hip.call(
                    "spar_hip_launch_adamw", p.ptr, g.ptr, m.ptr, v.ptr, n, F, 3e-4, 0.9, 0.95, 1e-8, 0.1,
                    c1, c2, 0) for p, g, m, v, _ in sets], n)
            measure("optim", "grad norm summary", 4 * n, [lambda g=g, summary=summary: hip.call(
                "spar_hip_launch_gradient_norm_summary", summary.ptr, g.ptr, n, F, 0)
                for _, g, _, _, summary in sets], n)
            measure("optim", "scale in place", 8 * n, [lambda g=g: hip.call(
                "spar_hip_launch_scale_in_place", g.ptr, n, F, 1.0, 0) for _, g, _, _, _ in sets], n)
            if self.with_cpu:
                import oracle.ops as O

                k = 1 << 24  # parameters 0 to 2^24 - 1
                p, g, m, v = (buf.to_numpy(np.float32, (n,))[:k].copy() for buf in sets[0][:4])
                self.cpu_baseline("optim", f"parameters 0 to 2^24 - 1 of {n:,}", [
                    ("adamw step", 28 * k, lambda: O.adamw(p, g, m, v, 3e-4, 0.9, 0.95, 1e-8, 0.1, c1, c2)),
                    ("grad norm summary", 4 * k, lambda: O.SumSquares().add(g)),
                    ("scale in place", 8 * k, lambda: O.scale(g, 1.0))])
            del sets

        return {"C1": c1, "C1L": c1l, "C3": c3, "C4": c4, "C5": c5, "optim": optim}


if __name__ == "__main__":
    main()
