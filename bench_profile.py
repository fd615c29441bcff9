"""rocprofv3 evidence behind bench.py's roofline figures (run on the MI355X).

  python3 bench_profile.py [--steps K] [--prompt P] [--out profiles]

Runs bench.py under rocprofv3, each pass as a child process with its own
time limit:
  1. --kernel-trace --stats over the default bench command: the summary of the
     kernels of the run, and the mean duration of the timed decode dispatches
     (the last K launches of the step kernel; prefill launches of the same
     kernel come first), to compare with bench.py's event timing;
  2. --pmc FETCH_SIZE, then --pmc WRITE_SIZE, over bench.py with the same
     prompt (KiB per dispatch, averaged over the timed decode dispatches);
  3. the same two counters over `bench.py --copy-calibration` (1 GiB device
     copies): factor = 1 GiB / counter reading, which scales 2.
Writes <out>/decode_step_kernel_trace.md, <out>/decode_step_traffic.md and
<out>/decode_step_traffic.json (read by bench.py for roofline.traffic).
Every pass must end with rocprofv3's exit status 0; any other status fails
the run, whatever the profiled program printed.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import statistics
import subprocess
import sys
import tempfile

ROOT = os.path.dirname(os.path.abspath(__file__))
BENCH = os.path.join(ROOT, "bench.py")
KERNEL = "decode_step_kernel"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def rocprof(tag, prof_args, bench_args, tmp, limit):
    out = os.path.join(tmp, tag)
    cmd = ["timeout", "-s", "KILL", str(limit), "rocprofv3", *prof_args, "--output-format", "csv",
           "-d", out, "-o", "run", "--", sys.executable, BENCH, *bench_args]
    log(f"[profile] {tag}: {' '.join(cmd[4:])}")
    env = dict(os.environ, TMPDIR="/tmp")
    # stdout carries the JSON line; stderr (progress of bench.py and of the
    # profiler) passes through
    r = subprocess.run(cmd, cwd="/tmp", env=env, stdout=subprocess.PIPE, text=True)
    lines = [l for l in r.stdout.splitlines() if l.startswith("{")]
    if r.returncode != 0 or not lines:
        log(r.stdout[-2000:])
        raise SystemExit(f"[profile] {tag}: rocprofv3 exited with status {r.returncode}"
                         + ("" if lines else " before the program printed its line"))
    log(f"[profile] {tag}: done (rocprofv3 exit status 0)")
    return out, json.loads(lines[-1]), " ".join(["rocprofv3", *prof_args, "--", "python3", "bench.py", *bench_args])


def one_csv(d, suffix):
    f = sorted(glob.glob(os.path.join(d, "**", f"*{suffix}"), recursive=True))
    if not f:
        raise SystemExit(f"[profile] no {suffix} under {d}")
    return list(csv.DictReader(open(f[0])))


def per_dispatch(rows, name_part, counter):
    """{dispatch id: counter value summed over its rows} for kernels whose name contains name_part."""
    vals = {}
    for r in rows:
        if name_part in r.get("Kernel_Name", "") and r.get("Counter_Name") == counter:
            d = int(r["Dispatch_Id"])
            vals[d] = vals.get(d, 0.0) + float(r["Counter_Value"])
    return vals


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=64, help="timed steps of the counter passes")
    ap.add_argument("--prompt", type=int, default=2048)
    ap.add_argument("--out", default=os.path.join(ROOT, "profiles"))
    args = ap.parse_args()
    os.makedirs(args.out, exist_ok=True)
    tmp = tempfile.mkdtemp(prefix="lyk_prof_", dir="/tmp")

    # 1. kernel trace of the default bench command
    d, line, cmd_trace = rocprof("trace", ["--kernel-trace", "--stats"], [], tmp, 600)
    steps = line["steps"]
    stats = one_csv(d, "kernel_stats.csv")
    trace = [r for r in one_csv(d, "kernel_trace.csv") if KERNEL in r["Kernel_Name"]]
    trace.sort(key=lambda r: int(r["Start_Timestamp"]))
    timed = trace[-steps:]
    dur = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in timed]
    total = sum(float(r["TotalDurationNs"]) for r in stats)
    md = ["# decode_step_kernel: kernel trace of the bench command", "",
          f"Command (from the repo root, on one MI355X): `{cmd_trace}` (rocprofv3 exit status 0)", "",
          "bench.py line of this run:", "", "```", json.dumps(line), "```", "",
          "rocprofv3 --stats (every dispatch of the run, prefill included):", "",
          "| kernel | calls | total ms | avg us | share |", "|---|---:|---:|---:|---:|"]
    for r in sorted(stats, key=lambda r: -float(r["TotalDurationNs"]))[:8]:
        md.append(f"| `{r['Name'][:90]}` | {r['Calls']} | {float(r['TotalDurationNs']) / 1e6:.1f} | "
                  f"{float(r['AverageNs']) / 1e3:.2f} | {float(r['TotalDurationNs']) / total * 100:.1f}% |")
    md += ["", f"Timed decode dispatches (the last {steps} launches of `{KERNEL}`, from the per-dispatch "
           f"trace): mean {statistics.mean(dur):.2f} us, median {statistics.median(dur):.2f} us, "
           f"min {min(dur):.2f} us, max {max(dur):.2f} us. bench.py's HIP-event figure for the same "
           f"steps: {line['roofline_kernel']['avg_us']} us (the events also span the launch gaps).", ""]
    open(os.path.join(args.out, "decode_step_kernel_trace.md"), "w").write("\n".join(md))
    log("\n".join(md))

    # 2./3. HBM counters of the decode step and of a plain copy
    bargs = ["--no-cpu-baseline", "--steps", str(args.steps), "--warmup", "4", "--prompt", str(args.prompt)]
    res, cmds = {}, {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        d, bl, cmds[counter] = rocprof(f"pmc_{counter}", ["--pmc", counter], bargs, tmp, 900)
        vals = per_dispatch(one_csv(d, "counter_collection.csv"), KERNEL, counter)
        ids = sorted(vals)[-args.steps:]
        res[counter] = statistics.mean(vals[i] for i in ids)
        d, _, cmds[counter + "_copy"] = rocprof(f"cal_{counter}", ["--pmc", counter], ["--copy-calibration"], tmp, 300)
        rows = one_csv(d, "counter_collection.csv")
        vals = per_dispatch(rows, "", counter)
        top = sorted(vals.values())[-4:]   # the four 1 GiB copies are the largest dispatches
        res[counter + "_copy"] = statistics.median(top)
        kernel, workload = bl["roofline_kernel"]["kernel"], bl["roofline_kernel"]["workload"]
        alg = bl["roofline_kernel"]["bytes_per_launch"]
    kib = 1 << 30 >> 10
    f_fetch, f_write = kib / res["FETCH_SIZE_copy"], kib / res["WRITE_SIZE_copy"]
    fetch_b = res["FETCH_SIZE"] * 1024 * f_fetch
    write_b = res["WRITE_SIZE"] * 1024 * f_write
    out = {"kernel": kernel, "workload": workload, "timed_steps": args.steps,
           "fetch_kib_per_launch": round(res["FETCH_SIZE"], 1), "write_kib_per_launch": round(res["WRITE_SIZE"], 1),
           "copy_fetch_kib": round(res["FETCH_SIZE_copy"], 1), "copy_write_kib": round(res["WRITE_SIZE_copy"], 1),
           "fetch_factor": round(f_fetch, 4), "write_factor": round(f_write, 4),
           "traffic_bytes_per_launch": int(fetch_b + write_b),
           "algorithmic_bytes_per_launch": alg, "commands": cmds}
    json.dump(out, open(os.path.join(args.out, "decode_step_traffic.json"), "w"), indent=1)
    md = ["# decode_step_kernel: HBM traffic per launch", "",
          f"Kernel `{kernel}`, workload `{workload}`; counters averaged over the last {args.steps} "
          "(timed, greedy) launches.", "",
          "| pass | command (from the repo root) | reading |", "|---|---|---:|",
          f"| FETCH_SIZE | `{cmds['FETCH_SIZE']}` | {res['FETCH_SIZE']:.0f} KiB/launch |",
          f"| WRITE_SIZE | `{cmds['WRITE_SIZE']}` | {res['WRITE_SIZE']:.0f} KiB/launch |",
          f"| FETCH_SIZE, 1 GiB copy | `{cmds['FETCH_SIZE_copy']}` | {res['FETCH_SIZE_copy']:.0f} KiB |",
          f"| WRITE_SIZE, 1 GiB copy | `{cmds['WRITE_SIZE_copy']}` | {res['WRITE_SIZE_copy']:.0f} KiB |", "",
          f"Calibration factors (1 GiB / copy reading): fetch {f_fetch:.4f}, write {f_write:.4f}.", "",
          f"Traffic per launch = {fetch_b / 1e9:.4f} GB read + {write_b / 1e9:.4f} GB written = "
          f"{(fetch_b + write_b) / 1e9:.4f} GB, against {alg / 1e9:.4f} GB algorithmic "
          f"({(fetch_b + write_b) / alg:.3f}x).", ""]
    open(os.path.join(args.out, "decode_step_traffic.md"), "w").write("\n".join(md))
    log("\n".join(md))


if __name__ == "__main__":
    main()
