"""rocprofv3 evidence for the bench.py workloads other than the headline decode.

    python profile_workloads.py run --workload W [--steps K] [--warmup N]
        One 256 MiB device-to-device copy (torch; the runtime's copy kernel reads and writes exactly
        256 MiB: the calibration of the byte counters), then bench.py's workload W in this process
        (no CPU leg; for matvec, `steps` hot launches of each sweep shape, no cold copies).  Run it under
        rocprofv3 three times: --kernel-trace --stats, --pmc FETCH_SIZE, --pmc WRITE_SIZE -- except the
        long-context workload, which takes the kernel trace only: a --pmc FETCH_SIZE pass over it once
        ended in a SIGSEGV on a thread of the runtime or profiler (not the program's), with no cause
        shown, so the tool refuses that workload under counter collection (ROCPROF_COUNTER_COLLECTION).

    python profile_workloads.py summarize --trace T --fetch F --write W --marker KERNEL --skip N
                                          --title TITLE --command CMD --out FILE
        Per-step kernel times (from the (N+1)-th launch of KERNEL, the first kernel of a step, on),
        and per-step HBM bytes of every kernel from the two counter passes, each counter scaled by
        what it reads for the copy kernel.  With --marker "" every launch counts (per-launch
        figures for the matvec sweep, grouped by grid).  Writes a markdown summary ending in a JSON
        block that bench.py reads for its `roofline.traffic`.

    python profile_workloads.py mall [--iters N] --out FILE
        How much of a weight stream the 256 MB last-level cache ("Infinity Cache", MALL) serves: the
        151936x896 Q4_0 head matvec cycling through 1..13 device copies of its weights (footprints
        78 MB .. 1 GB), each read in the same order on every pass, as the decode reads its weights
        once per token.  The counters of the L2 <-> fabric boundary (FETCH_SIZE, TCC_EA0_RDREQ_DRAM)
        count cache hits and misses of that cache alike, so the share comes from the rate: with the
        hot rate b_h (one copy, cache-resident) and the cold rate b_c (footprint far above 256 MB),
        a footprint read at rate b has a served fraction h = (1/b_c - 1/b) / (1/b_c - 1/b_h).
"""
import argparse
import csv
import glob
import json
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, HERE)

COPY_BYTES = 256 << 20


def _calibration_copy() -> None:
    import torch
    x = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device="cuda").normal_()
    y = torch.empty_like(x)
    y.copy_(x)                                        # runs as the runtime's copy kernel
    torch.cuda.synchronize()
    del x, y


MATVEC_SHAPES = [(896, 896), (128, 896), (4864, 896), (896, 4864), (151936, 896)]


def run_matvec(launches: int) -> None:
    """The matvec sweep's kernels without the cold copies (a counter pass serializes every launch, and
    the cold timing's thousands of copies of the small shapes would take minutes): per shape, the
    same seeded weights as bench.py, `launches` timed launches on the same x."""
    import numpy as np
    import q4hip
    import synth
    for N, K in MATVEC_SHAPES:
        raw = synth.quantize_q4_0(np.random.default_rng([1, N, K]).standard_normal(N * K, dtype=np.float32)
                                  * np.float32(0.02))
        mv = q4hip.Matvec(raw, N, K)
        mv.run(np.random.default_rng(1).standard_normal(K, dtype=np.float32))
        us = mv.time(launches)
        mv.close()
        print(json.dumps({"shape": [N, K], "us": round(us, 2)}), flush=True)


def run(a) -> None:
    if a.workload == "long-context" and (os.environ.get("ROCPROF_COUNTER_COLLECTION") == "1"
                                         or "ROCPROF_COUNTERS" in os.environ):
        sys.exit("profile_workloads.py: the long-context workload takes the kernel trace only (a counter "
                 "pass over it once ended in a SIGSEGV with no cause shown); it is not run under --pmc")
    _calibration_copy()
    if a.workload == "matvec":
        run_matvec(a.steps or 20)
        return
    sys.path.insert(0, REPO)
    import bench
    argv = ["bench.py", "--workload", a.workload, "--no-cpu"]
    if a.steps is not None:
        argv += ["--steps", str(a.steps)]
    if a.warmup is not None:
        argv += ["--warmup", str(a.warmup)]
    sys.argv = argv
    bench.main()


def _rows(d: str, pattern: str):
    files = glob.glob(os.path.join(d, "**", pattern), recursive=True)
    if not files:
        raise SystemExit(f"no {pattern} under {d}")
    with open(files[0]) as f:
        return list(csv.DictReader(f))


def _short(name: str) -> str:
    if name.startswith("_Z"):                 # some trace names come mangled
        try:
            # c++filt may not know _Float16 (DF16_): demangle it as half (Dh) and rename that back
            alias = name.replace("DF16_", "Dh")
            out = subprocess.run(["c++filt", alias], capture_output=True, text=True, timeout=10).stdout.strip()
            if out and not out.startswith("_Z"):
                name = out.replace("half", "_Float16") if alias != name else out
        except (OSError, subprocess.SubprocessError):
            pass
    if name.startswith("_Z"):                 # c++filt without _Float16 support: the bare name
        m = re.match(r"_Z(\d+)", name)
        if m:
            n = int(m.group(1))
            base = name[m.end():m.end() + n]
            name = base + ("<..., _Float16>" if "DF16_" in name else "<...>")
    name = name.replace("(anonymous namespace)::", "")
    return name.split("(")[0].replace("void ", "")


def _dispatches(rows, id_key: str, name_key: str, marker: str, skip: int):
    """Dispatch ids, in launch order, from the (skip+1)-th launch of `marker` on (all with no marker);
    returns (ids, number of steps)."""
    order = sorted({(int(r[id_key]), r[name_key]) for r in rows})
    if not marker:
        return [i for i, _ in order], 1
    marks = [k for k, (_, n) in enumerate(order) if marker in n]
    if len(marks) <= skip:
        raise SystemExit(f"fewer than {skip + 1} launches of {marker}")
    return [i for i, _ in order[marks[skip]:]], len(marks) - skip


def _grid(r) -> str:
    """Total threads of a dispatch (the counter files give Grid_Size, the trace its x, y, z), with the
    shared memory it was given (two launches of one kernel on different shapes may share a grid)."""
    if r.get("Grid_Size"):
        g = int(float(r["Grid_Size"]))
    else:
        g = int(r.get("Grid_Size_X", 1)) * int(r.get("Grid_Size_Y", 1)) * int(r.get("Grid_Size_Z", 1))
    lds = r.get("LDS_Block_Size") or r.get("Lds_Size") or ""
    return f"{g}" + (f", LDS {int(float(lds))}" if lds not in ("", "0") else "")


def _run_index(rows):
    """{dispatch id: k} where k numbers the runs of consecutive launches of the same (kernel, grid) in
    launch order; two shapes of the matvec sweep can share a grid, and their launches form separate
    runs (the same numbering in the trace and in the counter files, whose launch order is the same)."""
    order = sorted({(int(r["Dispatch_Id"]), (_short(r["Kernel_Name"]), _grid(r))) for r in rows})
    out, runs, prev = {}, {}, None
    for i, key in order:
        if key != prev:
            runs[key] = runs.get(key, -1) + 1
            prev = key
        out[i] = runs[key]
    return out


def _key(r, marker: str, runs):
    k = (_short(r["Kernel_Name"]), _grid(r))
    return k if marker else k + (runs[int(r["Dispatch_Id"])],)


def _counter_by_kernel(d: str, counter: str, marker: str, skip: int):
    rows = [r for r in _rows(d, "*counter_collection.csv") if r["Counter_Name"] == counter]
    ids, nsteps = _dispatches(rows, "Dispatch_Id", "Kernel_Name", marker, skip)
    keep = set(ids)
    runs = _run_index(rows)
    per = {}
    for r in rows:
        if int(r["Dispatch_Id"]) in keep:
            key = _key(r, marker, runs)
            per.setdefault(key, {}).setdefault(r["Dispatch_Id"], 0.0)
            per[key][r["Dispatch_Id"]] += float(r["Counter_Value"])
    return per, nsteps


def _sum_by_dispatch(rows, counter: str, name_part: str):
    out = {}
    for r in rows:
        if r["Counter_Name"] == counter and name_part in r["Kernel_Name"]:
            out[r["Dispatch_Id"]] = out.get(r["Dispatch_Id"], 0.0) + float(r["Counter_Value"])
    return out


def _calibration(d: str, counter: str) -> float:
    """Counter reading (KiB) of the 256 MiB copy, as a multiple of the bytes copied."""
    per = _sum_by_dispatch(_rows(d, "*counter_collection.csv"), counter, "copyBuffer")
    if not per:
        raise SystemExit(f"no copy kernel in {d}")
    return max(per.values()) * 1024 / COPY_BYTES


def summarize(a) -> None:
    trace = _rows(a.trace, "*kernel_trace.csv")
    ids, nsteps = _dispatches(trace, "Dispatch_Id", "Kernel_Name", a.marker, a.skip)
    keep = set(ids)
    runs = _run_index(trace)
    times = {}
    for r in trace:
        if int(r["Dispatch_Id"]) in keep:
            key = _key(r, a.marker, runs)
            c = times.setdefault(key, [0, 0.0])
            c[0] += 1
            c[1] += (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    if a.fetch and a.write:
        f_cal, w_cal = _calibration(a.fetch, "FETCH_SIZE"), _calibration(a.write, "WRITE_SIZE")
        fetch, _ = _counter_by_kernel(a.fetch, "FETCH_SIZE", a.marker, a.skip)
        write, _ = _counter_by_kernel(a.write, "WRITE_SIZE", a.marker, a.skip)
    else:                                     # kernel trace only
        f_cal = w_cal = None
        fetch, write = {}, {}

    def per_step(d, key, cal):
        """Bytes per step, or per launch of this kernel with no marker (the matvec sweep)."""
        v = d.get(key)
        if v is None:
            return None
        return sum(v.values()) * 1024 / cal / (nsteps if a.marker else len(v))

    lines = [f"# {a.title}", "", "Commands (repository root on the MI355X host, `cd /tmp && export TMPDIR=/tmp` "
             "first; paths absolute):", "", "```"]
    tools = ["--kernel-trace --stats -d T -o t"]
    if f_cal is not None:
        tools += ["--pmc FETCH_SIZE -d F -o f", "--pmc WRITE_SIZE -d W -o w"]
    for tool in tools:
        lines.append(f"rocprofv3 {tool} --output-format csv -- python3 e2e-browser-voice-agent_amd/py/"
                     f"profile_workloads.py run {a.command}")
    counters = "--fetch F --write W " if f_cal is not None else ""
    lines += [f"python3 e2e-browser-voice-agent_amd/py/profile_workloads.py summarize --trace T {counters}"
              f"--marker '{a.marker}' --skip {a.skip}" + (f" --only '{a.only}'" if a.only else "") +
              f" --title ... --command '{a.command}' --out <this file>", "```", ""]
    unit = "step" if a.marker else "launch"
    cal = (f" Byte counters scaled by the 256 MiB copy kernel: FETCH_SIZE reads {f_cal:.3f} x, WRITE_SIZE "
           f"{w_cal:.3f} x the bytes copied." if f_cal is not None else " Kernel trace only.")
    if a.marker:
        lines += [f"{nsteps} steps counted.{cal}", "",
                  "| kernel | grid (threads) | launches per step | us per step | us per launch | fetch MB per step | "
                  "write MB per step |", "|---|---|---|---|---|---|---|"]
    else:
        lines += [f"Every launch counted.{cal}", "",
                  "| kernel | grid (threads) | launches | us per launch | fetch MB per launch | write MB per launch |",
                  "|---|---|---|---|---|---|"]
    tot_us = tot_f = tot_w = 0.0
    only = re.compile(a.only) if a.only else None
    per_launch = []
    for key, (n, t) in sorted(times.items(), key=lambda kv: -kv[1][1]):
        if only and not only.search(key[0]):
            continue
        fb, wb = per_step(fetch, key, f_cal), per_step(write, key, w_cal)
        per = nsteps if a.marker else n            # no marker: every figure per launch of the kernel
        tot_us += t / per
        tot_f += fb or 0.0
        tot_w += wb or 0.0
        if not a.marker:
            if n < 2:                         # a lone launch (the sweep's first run of a shape)
                continue
            per_launch.append({"kernel": key[0], "grid": key[1], "launches": n, "us": t / n,
                               "fetch_bytes": fb, "write_bytes": wb})
            lines.append(f"| {key[0]} | {key[1]} | {n} | {t / n:.2f} | "
                         f"{'-' if fb is None else f'{fb / 1e6:.3f}'} | {'-' if wb is None else f'{wb / 1e6:.3f}'} |")
            continue
        lines.append(f"| {key[0]} | {key[1]} | {n / per:g} | {t / per:.1f} | {t / n:.1f} | "
                     f"{'-' if fb is None else f'{fb / 1e6:.2f}'} | {'-' if wb is None else f'{wb / 1e6:.2f}'} |")
    traffic = tot_f + tot_w if f_cal is not None else None
    if a.marker:
        lines += ["", f"Per step: kernel time {tot_us:.1f} us" +
                  (f", HBM traffic {traffic / 1e6:.2f} MB (fetch {tot_f / 1e6:.2f}, write {tot_w / 1e6:.2f})."
                   if traffic is not None else "."), ""]
    else:
        lines += [""]
    blob = {"unit": unit, "count": nsteps, "kernel_us": tot_us, "fetch_bytes": tot_f if traffic else None,
            "write_bytes": tot_w if traffic else None, "traffic_bytes": traffic, "fetch_calibration": f_cal,
            "write_calibration": w_cal}
    if not a.marker:
        blob["per_launch"] = per_launch
    import q4hip
    blob["kernel_sources_sha"] = q4hip.sources_sha()
    lines += ["```json", json.dumps(blob, indent=1), "```", ""]
    with open(a.out, "w") as f:
        f.write("\n".join(lines))
    print("\n".join(lines[:60]))


def mall(a) -> None:
    import numpy as np
    import q4hip
    import synth
    N, K = 151936, 896
    raw = synth.quantize_q4_0(np.random.default_rng([1, N, K]).standard_normal(N * K, dtype=np.float32)
                              * np.float32(0.02))
    mv = q4hip.Matvec(raw, N, K)
    mv.run(np.random.default_rng(1).standard_normal(K, dtype=np.float32))
    mv.time(a.iters)
    hot = mv.time(a.iters)
    alg = N * K // 32 * 18
    rows = [{"copies": 1, "footprint_mb": None, "us": hot}]
    for copies in (2, 3, 4, 5, 6, 8, 13):
        us, n = mv.time_cold(a.iters, rotate_bytes=int(copies * 77.832e6) - (1 << 20))
        rows.append({"copies": n, "us": us})
    mv.close()
    per_copy = 77.832e6    # repacked bytes of one copy (qs + scales, tile padding included)
    for r in rows:
        r["footprint_mb"] = round(r["copies"] * per_copy / 1e6, 1)
        r["gbps"] = round(alg / (r["us"] * 1e-6) / 1e9, 1)
    b_h, b_c = rows[0]["gbps"], rows[-1]["gbps"]
    for r in rows:
        b = r["gbps"]
        r["served_fraction"] = round(min(1.0, max(0.0, (1 / b_c - 1 / b) / (1 / b_c - 1 / b_h))), 3)
    lines = ["# Last-level cache (MALL) share of a weight stream: Q4_0 head matvec over rotating weight copies", "",
             "Command (repository root on the MI355X host):", "", "```",
             f"python3 e2e-browser-voice-agent_amd/py/profile_workloads.py mall --iters {a.iters} --out <this file>",
             "```", "",
             "151936 x 896 Q4_0 head (76.6 MB algorithmic, 77.8 MB repacked), x quantized once; each row "
             "cycles through `copies` device copies of the weights in the same order. Rate = algorithmic "
             "bytes / mean launch time (HIP events). served fraction h = (1/b_c - 1/b) / (1/b_c - 1/b_h), "
             "with b_h the one-copy rate and b_c the 13-copy (1 GB) rate.", "",
             "| copies | footprint MB | us per launch | GB/s | served fraction |", "|---|---|---|---|---|"]
    for r in rows:
        lines.append(f"| {r['copies']} | {r['footprint_mb']} | {r['us']:.2f} | {r['gbps']} | {r['served_fraction']} |")
    import q4hip
    lines += ["", "```json", json.dumps({"rows": rows, "kernel_sources_sha": q4hip.sources_sha()}, indent=1), "```", ""]
    with open(a.out, "w") as f:
        f.write("\n".join(lines))
    print("\n".join(lines))


def main() -> None:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    r = sub.add_parser("run")
    r.add_argument("--workload", required=True, choices=["long-context", "prefill", "matvec", "batched"])
    r.add_argument("--steps", type=int, default=None)
    r.add_argument("--warmup", type=int, default=None)
    s = sub.add_parser("summarize")
    for k in ("--trace", "--title", "--command", "--out"):
        s.add_argument(k, required=True)
    s.add_argument("--fetch", default=None)
    s.add_argument("--write", default=None)
    s.add_argument("--marker", default="")
    s.add_argument("--only", default="", help="regular expression: list only the kernels it matches")
    s.add_argument("--skip", type=int, default=0)
    m = sub.add_parser("mall")
    m.add_argument("--iters", type=int, default=200)
    m.add_argument("--out", required=True)
    a = ap.parse_args()
    {"run": run, "summarize": summarize, "mall": mall}[a.cmd](a)


if __name__ == "__main__":
    main()
