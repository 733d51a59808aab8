"""Profiles bench.py's default workload with rocprofv3 and writes two
markdown summaries: per-kernel durations, and HBM bytes per dispatch from the
FETCH_SIZE / WRITE_SIZE counters.

    python3 rocprof_summary.py run --raw DIR --out DIR

runs, as child processes (this process never touches the GPU):

1. ``rocprofv3 --kernel-trace --stats`` over ``bench.py --no-cpu-baseline``;
2. ``rocprofv3 --pmc FETCH_SIZE`` over ``bench.py --profile-loop 2``;
3. ``rocprofv3 --pmc WRITE_SIZE`` over the same command.

``bench.py --profile-loop`` runs the workload steps and then one plain
contiguous copy of a 512 MiB tensor.  That copy's counter values calibrate
the counters: it must move exactly 512 MiB each way, so each counter is
scaled by 512 MiB / (its value on the copy).  A kernel's HBM traffic per
launch is then scaled FETCH + scaled WRITE.

``bench.py`` reads the ``hbm_bytes_per_launch`` lines of the traffic summary
for its roofline ``traffic`` field.

``summarize`` regenerates the markdown from an existing raw directory.

    python3 rocprof_summary.py suite --section optim --raw DIR --out DIR

profiles one ``bench.py --suite-only SECTION`` run with ``--kernel-trace
--stats`` and runs the same command without a profiler, then writes a
per-kernel duration table next to the suite's own event-timed lines.

    python3 rocprof_summary.py traffic --section C3 --raw DIR --out DIR

measures every op of a suite section alone (``bench.py --suite-op
SECTION/OP --profile-launches 4``): one ``--pmc FETCH_SIZE`` and one ``--pmc
WRITE_SIZE`` pass per op, each ending with the calibration copy, and one pass
of gfx950's request-size counters per section.  Dispatches between the
bench's marker dispatches belong to the op; the summary gives each op's HBM
bytes per launch, which bench.py reports as the op's ``traffic``.

Why FETCH_SIZE needs the calibration factor on gfx950: rocprofv3 defines it
(counter_defs.yaml) as (TCC_BUBBLE*128 + (TCC_EA0_RDREQ - TCC_BUBBLE -
TCC_EA0_RDREQ_32B)*64 + TCC_EA0_RDREQ_32B*32) / 1024 KiB, where TCC_BUBBLE
counts 128-byte read requests.  On gfx950 TCC_BUBBLE reads 0 while the
streaming kernels' reads arrive as 128-byte requests, counted by
TCC_EA0_RDREQ_128B: FETCH_SIZE prices each at 64 bytes and reports half the
bytes read.  The request-size pass shows it directly: 32*RDREQ_32B +
64*RDREQ_64B + 128*RDREQ_128B equals the algorithmic read bytes, and
calibration against the 512 MiB copy gives the same factor, 2.0.
"""
from __future__ import annotations

import argparse
import collections
import csv
import json
import os
import re
import shlex
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent


def shown(path: Path) -> str:
    """A path as the profile headers print it: relative to the repository
    root when it lies inside it (the raw directories of a GPU run do)."""
    try:
        return str(path.relative_to(ROOT))
    except ValueError:
        return str(path)

# bench.py's kernel classes: a regex over the demangled kernel name, and
# whether dispatches of that kernel count as launches of the class (helper
# kernels such as the partial-sum combine add traffic but no launch).
CLASSES = {
    "broadcast_binary": [(r"::row_tile_kernel<|::row_vector_kernel<", True)],
    "column_reduction": [(r"::column_kernel<|::column_wide_kernel<", True),
                         (r"::combine_columns_kernel<", False)],
}
COPY_PATTERN = r"CopyOp"
CALIBRATION_BYTES = 512 << 20

TRACE_ARGS = ["--no-cpu-baseline", "--no-suite", "--steps", "20"]
LOOP_ARGS = ["--profile-loop", "2"]
STATS_FILE = "kernel_stats_x32x1024x4096.md"
TRAFFIC_FILE = "hbm_traffic_x32x1024x4096.md"


def short(name: str) -> str:
    """Kernel name without namespaces, return type and argument list."""
    name = re.sub(r"spar_hip::\(anonymous namespace\)::", "", name)
    name = name.replace("spar_hip::", "")
    if name.startswith("void "):
        name = name[5:]
    depth = 0
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            return name[:i]
    return name


def commands(raw: Path):
    bench = [sys.executable, str(ROOT / "bench.py")]
    return {
        "trace": ["rocprofv3", "--kernel-trace", "--stats", "--output-format", "csv", "-d",
                  str(raw / "trace"), "-o", "trace", "--"] + bench + TRACE_ARGS,
        "fetch": ["rocprofv3", "--pmc", "FETCH_SIZE", "--output-format", "csv", "-d",
                  str(raw / "fetch"), "-o", "fetch", "--"] + bench + LOOP_ARGS,
        "write": ["rocprofv3", "--pmc", "WRITE_SIZE", "--output-format", "csv", "-d",
                  str(raw / "write"), "-o", "write", "--"] + bench + LOOP_ARGS,
        # The same benchmark without a profiler: the tracer slows launches
        # bracketed by events, so bench.py's own timing is compared unprofiled.
        "plain": bench + TRACE_ARGS,
    }


def shell(argv) -> str:
    """The command as typed from the repository root."""
    text = " ".join(shlex.quote(str(a)) for a in argv)
    text = text.replace(sys.executable, "python3").replace(str(ROOT) + "/", "")
    return text


def run(raw: Path, out: Path, limit: int) -> None:
    raw.mkdir(parents=True, exist_ok=True)
    for name, argv in commands(raw).items():
        print(f"pass {name}: {shell(argv)}", flush=True)
        log = raw / f"{name}.log"
        with open(log, "w") as handle:
            # rocprofv3 writes temporary files under TMPDIR; run it from /tmp.
            proc = subprocess.run(["timeout", "-s", "KILL", str(limit)] + argv, cwd="/tmp",
                                  env=dict(os.environ, TMPDIR="/tmp"), stdout=handle,
                                  stderr=subprocess.STDOUT)
        print(f"pass {name}: exit {proc.returncode}", flush=True)
        if proc.returncode != 0:
            sys.stdout.write(log.read_text()[-4000:])
            raise SystemExit(proc.returncode)
    summarize(raw, out)


def bench_line(log: Path):
    if not log.exists():
        return None
    for line in reversed(log.read_text().splitlines()):
        line = line.strip()
        if line.startswith("{") and '"roofline"' in line:
            return json.loads(line)
    return None


def kernel_class(full_name: str):
    if re.search(COPY_PATTERN, full_name):
        return None, False
    for cls, patterns in CLASSES.items():
        for pattern, counts in patterns:
            if re.search(pattern, full_name):
                return cls, counts
    return None, False


def counters(path: Path):
    rows = collections.defaultdict(list)
    for r in csv.DictReader(open(path)):
        rows[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    return rows


def summarize(raw: Path, out: Path) -> None:
    out.mkdir(parents=True, exist_ok=True)
    cmds = commands(raw)
    bench = bench_line(raw / "plain.log")
    traced = bench_line(raw / "trace.log")

    # --- kernel durations
    stats = list(csv.DictReader(open(raw / "trace" / "trace_kernel_stats.csv")))
    lines = [
        "# Kernel durations: bench.py default workload, x[32,1024,4096] fp32",
        "",
        "Command (from the repository root):",
        "",
        "    " + shell(cmds["trace"]),
        "",
        "Every launch of the run: data generation, warm-up, the timed steps and the",
        "per-op event timing.  Durations from the kernel trace.",
        "",
        "| kernel | class | calls | avg us | min us | max us | % time |",
        "|---|---|---|---|---|---|---|",
    ]
    class_ns = collections.defaultdict(float)
    class_calls = collections.defaultdict(int)
    for r in stats:
        cls, counts = kernel_class(r["Name"])
        lines.append(
            f"| `{short(r['Name'])}` | {cls or ''} | {r['Calls']} | "
            f"{float(r['AverageNs']) / 1e3:.1f} | {float(r['MinNs']) / 1e3:.1f} | "
            f"{float(r['MaxNs']) / 1e3:.1f} | {float(r['Percentage']):.2f} |")
        if cls is not None:
            class_ns[cls] += float(r["TotalDurationNs"])
            if counts:
                class_calls[cls] += int(r["Calls"])
    lines += ["", "Average duration per launch of each bench.py kernel class (rocprofv3):", ""]
    for cls in CLASSES:
        if class_calls[cls]:
            lines.append(f"- {cls}: {class_ns[cls] / class_calls[cls] / 1e3:.1f} us "
                         f"over {class_calls[cls]} launches")
    for label, line in (("without a profiler (`" + shell(cmds["plain"]) + "`)", bench),
                        ("under the kernel trace above", traced)):
        if line is None:
            continue
        roof = line["roofline"]
        lines += ["", f"bench.py's own line {label}, timed with HIP events on the backend stream:",
                  "",
                  f"- value {line['value']} GB/s, {line['ms_per_step']} ms per step",
                  f"- roofline kernel {roof['kernel']}: avg launch "
                  f"{roof['avg_launch_ms'] * 1e3:.1f} us, achieved {roof['achieved']} GB/s "
                  f"({roof['frac'] * 100:.1f}% of {roof['peak']:.0f} GB/s)"]
    (out / STATS_FILE).write_text("\n".join(lines) + "\n")

    # --- HBM traffic
    fetch = counters(raw / "fetch" / "fetch_counter_collection.csv")
    write = counters(raw / "write" / "write_counter_collection.csv")
    copy = [k for k in fetch if re.search(COPY_PATTERN, k)]
    if len(copy) != 1:
        raise SystemExit(f"expected one calibration copy kernel, found {copy}")
    copy = copy[0]
    cal_kib = CALIBRATION_BYTES / 1024
    fetch_copy = sum(fetch[copy]) / len(fetch[copy])
    write_copy = sum(write[copy]) / len(write[copy])
    f_scale = cal_kib / fetch_copy
    w_scale = cal_kib / write_copy
    lines = [
        "# L2-fabric (HBM + Infinity Cache) traffic per dispatch: bench.py --profile-loop 2, "
        "x[32,1024,4096] fp32",
        "",
        "FETCH_SIZE and WRITE_SIZE count what the L2 reads from and writes to the data",
        "fabric, that is HBM plus Infinity Cache (MALL) hits; gfx950 exposes no counter",
        "that tells the two apart.  This workload's 537 MB tensors rotate through more",
        "than the 256 MB cache, so here the figures are close to HBM bytes.",
        "",
        "Commands (from the repository root), one counter per run:",
        "",
        "    " + shell(cmds["fetch"]),
        "    " + shell(cmds["write"]),
        "",
        "Calibration: the run ends with a plain contiguous copy of 512 MiB "
        f"(`{short(copy)}`), which reads FETCH_SIZE {fetch_copy:.0f} KiB and WRITE_SIZE "
        f"{write_copy:.0f} KiB per dispatch; every counter value below is scaled by "
        f"{f_scale:.4f} (fetch) and {w_scale:.4f} (write) to bytes.",
        "",
        "| kernel | class | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | L2-fabric MB per dispatch |",
        "|---|---|---|---|---|---|",
    ]
    class_bytes = collections.defaultdict(float)
    class_launches = collections.defaultdict(int)
    for name, values in fetch.items():
        fv = sum(values) / len(values)
        wv = sum(write.get(name, [0.0])) / max(len(write.get(name, [])), 1)
        per = (fv * f_scale + wv * w_scale) * 1024
        cls, counts = kernel_class(name)
        lines.append(f"| `{short(name)}` | {cls or ''} | {len(values)} | {fv:.0f} | {wv:.0f} | "
                     f"{per / 1e6:.1f} |")
        if cls is not None:
            class_bytes[cls] += per * len(values)
            if counts:
                class_launches[cls] += len(values)
    lines += ["", "L2-fabric bytes per launch of each bench.py kernel class (all dispatches",
              "of the class over its launches; bench.py reads these lines as its roofline's",
              "traffic):", ""]
    for cls in CLASSES:
        if class_launches[cls]:
            lines.append(f"- hbm_bytes_per_launch[{cls}] = "
                         f"{round(class_bytes[cls] / class_launches[cls])}")
    (out / TRAFFIC_FILE).write_text("\n".join(lines) + "\n")
    print(f"wrote {out / STATS_FILE} and {out / TRAFFIC_FILE}", flush=True)


# Suite sections: the workload each one times, for the summary's name and title.
SUITE_WORKLOADS = {
    "C1": ("c1_4096x4096", "C1 contiguous elementwise on [4096, 4096] fp32"),
    "C1L": ("c1l_8192x8192", "C1L contiguous elementwise on [8192, 8192] fp32"),
    "C3": ("c3_8192x8192", "C3 axis reductions on [8192, 8192] and full reductions of 2^28 fp32"),
    "C4": ("c4_8192x32768", "C4 softmax, log-softmax and cross entropy on [8192, 32768] fp32"),
    "C5": ("c5_4096x8192", "C5 LayerNorm chain and fused layer_norm on [4096, 8192] fp32 views"),
    "optim": ("optim_124439808", "AdamW, gradient-norm summary and scaling over 124,439,808 fp32"),
}
SUITE_ARGS = ["--no-cpu-baseline", "--steps", "2", "--warmup", "1", "--suite-only"]


def suite_file(section: str) -> str:
    return f"kernel_stats_suite_{SUITE_WORKLOADS[section][0]}.md"


def suite_commands(raw: Path, section: str):
    bench = [sys.executable, str(ROOT / "bench.py")] + SUITE_ARGS + [section]
    return {
        "trace": ["rocprofv3", "--kernel-trace", "--stats", "--output-format", "csv", "-d",
                  str(raw / "trace"), "-o", "trace", "--"] + bench,
        "plain": bench + ["--suite"],
    }


def run_suite(raw: Path, out: Path, section: str, limit: int) -> None:
    raw.mkdir(parents=True, exist_ok=True)
    for name, argv in suite_commands(raw, section).items():
        print(f"pass {name}: {shell(argv)}", flush=True)
        log = raw / f"{name}.log"
        with open(log, "w") as handle:
            proc = subprocess.run(["timeout", "-s", "KILL", str(limit)] + argv, cwd="/tmp",
                                  env=dict(os.environ, TMPDIR="/tmp"), stdout=handle,
                                  stderr=subprocess.STDOUT)
        print(f"pass {name}: exit {proc.returncode}", flush=True)
        if proc.returncode != 0:
            sys.stdout.write(log.read_text()[-4000:])
            raise SystemExit(proc.returncode)
    summarize_suite(raw, out, section)


def summarize_suite(raw: Path, out: Path, section: str) -> None:
    out.mkdir(parents=True, exist_ok=True)
    cmds = suite_commands(raw, section)
    stats = list(csv.DictReader(open(raw / "trace" / "trace_kernel_stats.csv")))
    title = SUITE_WORKLOADS[section][1]
    lines = [
        f"# Kernel durations: bench.py suite section {section}, {title}",
        "",
        "Generated (from the repository root) by",
        "",
        f"    python3 rocprof_summary.py suite --section {section} "
        f"--raw {shown(raw)} --out profiles",
        "",
        "which runs",
        "",
        "    " + shell(cmds["trace"]),
        "",
        "Every launch of the run, including bench.py's default workload (two steps)",
        "and the cache-evicting reads (`touch_kernel`) before each timed launch.",
        "Durations from the kernel trace.",
        "",
        "| kernel | calls | avg us | min us | max us | % time |",
        "|---|---|---|---|---|---|",
    ]
    for r in stats:
        lines.append(
            f"| `{short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
            f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | "
            f"{float(r['Percentage']):.2f} |")
    suite_lines = [line for line in (raw / "plain.log").read_text().splitlines()
                   if line.startswith('{"suite"')]
    lines += ["", "The suite's own lines without a profiler (`" + shell(cmds["plain"]) + "`),",
              "each op timed with HIP events (`timing` says how: back to back over rotated",
              "input sets, or cold single launches, median of 20):", "", "```"]
    lines += suite_lines
    lines += ["```"]
    (out / suite_file(section)).write_text("\n".join(lines) + "\n")
    print(f"wrote {out / suite_file(section)}", flush=True)


def read_traffic(path: Path):
    """{class: bytes per launch} from a traffic summary, or {} if absent."""
    if not path.exists():
        return {}
    found = {}
    for m in re.finditer(r"^- hbm_bytes_per_launch\[(\w+)\] = (\d+)$", path.read_text(), re.M):
        found[m.group(1)] = int(m.group(2))
    return found


SUITE_FILES = {"C1": "c1_4096x4096", "C1L": "c1l_8192x8192", "C3": "c3_8192x8192",
               "C4": "c4_8192x32768",
               "C5": "c5_4096x8192", "optim": "optim_124439808"}
MARKER = r"touch_kernel"
GENERATORS = r"normal_kernel<|uniform_f32_kernel|uniform_kernel<"
REQUEST_COUNTERS = ["TCC_EA0_RDREQ_32B_sum", "TCC_EA0_RDREQ_64B_sum", "TCC_EA0_RDREQ_128B_sum",
                    "TCC_BUBBLE_sum"]


def suite_traffic_file(config: str) -> str:
    return f"hbm_traffic_suite_{SUITE_FILES[config]}.md"


def read_op_traffic(path: Path):
    """{op: HBM bytes per launch} from a suite traffic summary ({} if absent)."""
    if not path.exists():
        return {}
    found = {}
    for m in re.finditer(r"^- op_hbm_bytes_per_launch\[(.+)\] = (\d+)$", path.read_text(), re.M):
        found[m.group(1)] = int(m.group(2))
    return found


def dispatches(path: Path):
    """[(dispatch id, kernel name, {counter: value})] in dispatch order."""
    by_id = {}
    for r in csv.DictReader(open(path)):
        key = int(r["Dispatch_Id"])
        entry = by_id.setdefault(key, (key, r["Kernel_Name"], {}))
        entry[2][r["Counter_Name"]] = float(r["Counter_Value"])
    return [by_id[k] for k in sorted(by_id)]


def op_window(rows, launches=None):
    """The dispatches inside each (opening, closing) marker pair, markers
    excluded, and the calibration copy (the last dispatch).  Markers come in
    pairs, one pair per launch; whatever runs between a closing marker and
    the next opening one (a fresh graph's forward, say) is left out."""
    marks = [i for i, (_, name, _) in enumerate(rows) if re.search(MARKER, name)]
    if len(marks) < 2 or len(marks) % 2:
        raise SystemExit(f"expected marker pairs around each launch, found {len(marks)} markers")
    if launches is not None and len(marks) != 2 * launches:
        raise SystemExit(f"expected {2 * launches} markers for {launches} launches, "
                         f"found {len(marks)}")
    copy = rows[-1]
    if not re.search(COPY_PATTERN, copy[1]):
        raise SystemExit(f"last dispatch is not the calibration copy: {copy[1]}")
    window = []
    for opening, closing in zip(marks[0::2], marks[1::2]):
        window += rows[opening + 1:closing]
    return window, copy


def bench_info(log: Path):
    """The JSON line bench.py printed at the end of a --suite-op pass."""
    if not log.exists():
        return {}
    for line in reversed(log.read_text().splitlines()):
        line = line.strip()
        if line.startswith('{"suite_op"'):
            return json.loads(line)
    return {}


def suite_bench(op_spec: str, launches: int):
    return [sys.executable, str(ROOT / "bench.py"), "--suite-op", op_spec,
            "--profile-launches", str(launches)]


def run_traffic(raw: Path, out: Path, section: str, limit: int, launches: int) -> None:
    """Counter passes over every op of a section, then the summary."""
    raw.mkdir(parents=True, exist_ok=True)
    listing = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--list-suite-ops"],
                             capture_output=True, text=True, check=True)
    ops = json.loads(listing.stdout)[section]
    plan = []
    for k, op in enumerate(ops):
        spec = f"{section}/{op}"
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            tag = f"op{k:02d}_{counter.lower()}"
            plan.append((tag, ["rocprofv3", "--pmc", counter, "--output-format", "csv", "-d",
                               str(raw / tag), "-o", tag, "--"] + suite_bench(spec, launches)))
    largest = f"{section}/{ops[0]}"
    plan.append(("requests", ["rocprofv3", "--pmc", *REQUEST_COUNTERS, "--output-format", "csv",
                              "-d", str(raw / "requests"), "-o", "requests", "--"]
                 + suite_bench(largest, launches)))
    for tag, argv in plan:
        print(f"pass {tag}: {shell(argv)}", flush=True)
        with open(raw / f"{tag}.log", "w") as handle:
            proc = subprocess.run(["timeout", "-s", "KILL", str(limit)] + argv, cwd="/tmp",
                                  env=dict(os.environ, TMPDIR="/tmp"), stdout=handle,
                                  stderr=subprocess.STDOUT)
        if proc.returncode != 0:
            sys.stdout.write((raw / f"{tag}.log").read_text()[-3000:])
            raise SystemExit(f"pass {tag}: exit {proc.returncode}")
    (raw / "plan.json").write_text(json.dumps({"section": section, "ops": ops,
                                               "launches": launches,
                                               "commands": {t: shell(a) for t, a in plan}}))
    summarize_traffic(raw, out)


def summarize_traffic(raw: Path, out: Path) -> None:
    plan = json.loads((raw / "plan.json").read_text())
    section, ops, launches = plan["section"], plan["ops"], plan["launches"]
    cal_kib = CALIBRATION_BYTES / 1024
    lines = [
        f"# L2-fabric (HBM + Infinity Cache) traffic per launch: bench.py suite section {section}, "
        f"{SUITE_WORKLOADS[section][1]}",
        "",
        "Generated (from the repository root) by",
        "",
        f"    python3 rocprof_summary.py traffic --section {section} "
        f"--raw {shown(raw)} --out profiles",
        "",
        f"which runs two counter passes per op, for example (op `{ops[0]}`):",
        "",
        "    " + plan["commands"]["op00_fetch_size"],
        "    " + plan["commands"]["op00_write_size"],
        "",
        f"Each pass runs the op alone {launches} times, each launch between an opening and a",
        "closing marker dispatch, and ends with a plain contiguous copy of 512 MiB; each",
        "pass's FETCH_SIZE and WRITE_SIZE are scaled by 512 MiB over the copy's reading, and",
        "the dispatches inside the marker pairs (random generators excluded) are summed and",
        "divided by the launches.  Work a launch needs first (a fresh graph's forward for a",
        "backward) runs outside the pairs and is not counted.",
        "",
        "What the counters see: FETCH_SIZE and WRITE_SIZE count the L2's traffic to and from",
        "the data fabric, that is HBM plus Infinity Cache (MALL) hits; gfx950 exposes no",
        "counter that separates the two.  For a kernel that re-reads data from the Infinity",
        "Cache the figures below are L2-fabric bytes, an upper bound on its HBM bytes.",
        "",
        "| op | kernels per launch | FETCH_SIZE scale | L2-fabric read MB | L2-fabric write MB | "
        "L2-fabric MB per launch | algorithmic MB | ratio |",
        "|---|---|---|---|---|---|---|---|",
    ]
    results = []
    for k, op in enumerate(ops):
        fetch_rows = dispatches(raw / f"op{k:02d}_fetch_size" / f"op{k:02d}_fetch_size_counter_collection.csv")
        write_rows = dispatches(raw / f"op{k:02d}_write_size" / f"op{k:02d}_write_size_counter_collection.csv")
        fwin, fcopy = op_window(fetch_rows, launches)
        wwin, wcopy = op_window(write_rows, launches)
        f_scale = cal_kib / fcopy[2]["FETCH_SIZE"]
        w_scale = cal_kib / wcopy[2]["WRITE_SIZE"]
        fwin = [r for r in fwin if not re.search(GENERATORS, r[1])]
        wwin = [r for r in wwin if not re.search(GENERATORS, r[1])]
        read = sum(r[2]["FETCH_SIZE"] for r in fwin) * f_scale * 1024 / launches
        write = sum(r[2]["WRITE_SIZE"] for r in wwin) * w_scale * 1024 / launches
        kernels = sorted({short(r[1]) for r in fwin})
        results.append((op, round(read + write)))
        info = bench_info(raw / f"op{k:02d}_fetch_size.log")
        algorithmic = info.get("bytes")
        ratio = f"{(read + write) / algorithmic:.3f}" if algorithmic else ""
        alg_mb = f"{algorithmic / 1e6:.1f}" if algorithmic else ""
        lines.append(f"| {op} | {'<br>'.join('`' + n + '`' for n in kernels)} | {f_scale:.3f} | "
                     f"{read / 1e6:.1f} | {write / 1e6:.1f} | {(read + write) / 1e6:.1f} | "
                     f"{alg_mb} | {ratio} |")
    lines += ["", "L2-fabric bytes per launch of each op (bench.py reads these lines as the op's",
              "traffic):", ""]
    lines += [f"- op_hbm_bytes_per_launch[{op}] = {value}" for op, value in results]
    req = dispatches(raw / "requests" / "requests_counter_collection.csv")
    rwin, rcopy = op_window(req, launches)

    def request_bytes(c):
        return 32 * c["TCC_EA0_RDREQ_32B_sum"] + 64 * c["TCC_EA0_RDREQ_64B_sum"] + \
            128 * c["TCC_EA0_RDREQ_128B_sum"]

    lines += ["", "Read requests by size (gfx950 TCC counters; one pass, op `" + ops[0] + "`):",
              "", "    " + plan["commands"]["requests"], "",
              "| dispatch | 32 B | 64 B | 128 B | TCC_BUBBLE | bytes by request size |",
              "|---|---|---|---|---|---|"]
    for _, name, c in rwin[:6] + [rcopy]:
        lines.append(f"| `{short(name)}` | {c['TCC_EA0_RDREQ_32B_sum']:.0f} | "
                     f"{c['TCC_EA0_RDREQ_64B_sum']:.0f} | {c['TCC_EA0_RDREQ_128B_sum']:.0f} | "
                     f"{c['TCC_BUBBLE_sum']:.0f} | {request_bytes(c) / 1e6:.1f} MB |")
    lines += ["", "TCC_BUBBLE stays 0 on gfx950 while reads go out as 128-byte requests, so",
              "FETCH_SIZE (which prices non-32-byte requests not counted by TCC_BUBBLE at 64",
              "bytes) reads half; the request sizes give the copy's 536.9 MB directly."]
    out.mkdir(parents=True, exist_ok=True)
    target = out / suite_traffic_file(section)
    target.write_text("\n".join(lines) + "\n")
    print(f"wrote {target}", flush=True)


def main():
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    sub = p.add_subparsers(dest="mode", required=True)
    r = sub.add_parser("run")
    r.add_argument("--raw", type=Path, required=True, help="directory for raw rocprofv3 output")
    r.add_argument("--out", type=Path, required=True, help="directory for the markdown")
    r.add_argument("--limit", type=int, default=240, help="seconds per rocprofv3 pass")
    s = sub.add_parser("summarize")
    s.add_argument("--raw", type=Path, required=True)
    s.add_argument("--out", type=Path, required=True)
    q = sub.add_parser("suite")
    q.add_argument("--section", required=True, choices=sorted(SUITE_WORKLOADS))
    q.add_argument("--raw", type=Path, required=True)
    q.add_argument("--out", type=Path, required=True)
    q.add_argument("--limit", type=int, default=240, help="seconds per pass")
    t = sub.add_parser("traffic")
    t.add_argument("--section", required=True, choices=sorted(SUITE_FILES))
    t.add_argument("--raw", type=Path, required=True)
    t.add_argument("--out", type=Path, required=True)
    t.add_argument("--limit", type=int, default=120, help="seconds per pass")
    t.add_argument("--launches", type=int, default=4)
    ts = sub.add_parser("summarize-traffic")
    ts.add_argument("--raw", type=Path, required=True)
    ts.add_argument("--out", type=Path, required=True)
    args = p.parse_args()
    if args.mode == "run":
        run(args.raw.resolve(), args.out.resolve(), args.limit)
    elif args.mode == "suite":
        run_suite(args.raw.resolve(), args.out.resolve(), args.section, args.limit)
    elif args.mode == "traffic":
        run_traffic(args.raw.resolve(), args.out.resolve(), args.section, args.limit,
                    args.launches)
    elif args.mode == "summarize-traffic":
        summarize_traffic(args.raw.resolve(), args.out.resolve())
    else:
        summarize(args.raw.resolve(), args.out.resolve())


if __name__ == "__main__":
    main()
