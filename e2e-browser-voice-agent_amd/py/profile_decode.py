"""Workload and summariser for the rocprofv3 evidence of the decode kernel.

    python profile_decode.py run [--steps 64]
        One 256 MiB device-to-device copy (torch; it runs as the runtime's copy kernel, which
        reads and writes exactly 256 MiB: the calibration), then the headline decode workload: Qwen2.5-0.5B shape, 64-token prompt,
        one warmup launch and one timed launch of `steps` greedy steps of the persistent decode
        kernel.  Prints the HIP-event time of the timed launch.

    python profile_decode.py summarize --trace DIR --fetch DIR --write DIR [--dram DIR] --steps K --out FILE
        Reads the rocprofv3 CSV outputs (kernel trace with --stats; one --pmc FETCH_SIZE pass; one
        --pmc WRITE_SIZE pass; optionally one --pmc TCC_EA0_RDREQ_DRAM_sum TCC_EA0_RDREQ_sum pass),
        scales each byte counter by what it reads for the copy kernel, and writes a short markdown
        summary with per-launch and per-step figures.

    python profile_decode.py steps --trace DIR --marker KERNEL --skip N --title T --command C --out FILE
        Per-step kernel times of a multi-kernel workload from a rocprofv3 kernel trace: the dispatches
        from the (N+1)-th launch of KERNEL (the first kernel of a step) on, grouped by kernel name
        and grid, averaged per step (e.g. the batched decode steps of bench.py --workload batched).

The counters are read by rocprofv3 per dispatch, in KiB.  For the persistent kernel they include
every byte the launch moves between the L2s and the memory fabric: weights, K/V, logits and the
polling of the exchange area between workgroups.
"""
import argparse
import csv
import glob
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

COPY_BYTES = 256 << 20
PROMPT = 64


def run(steps: int) -> None:
    import torch
    import q4hip
    import synth

    x = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device="cuda").normal_()
    y = torch.empty_like(x)
    y.copy_(x)                                        # runs as the runtime's copy kernel
    torch.cuda.synchronize()
    del x, y

    shape = synth.SHAPES["qwen2.5-0.5b"]
    m = q4hip.Model(shape, ctx=max(256, PROMPT + steps + 2))
    m.load(synth.make_model(shape, 1))
    ids = synth.prompt_ids(1, PROMPT, shape.vocab)
    first = m.forward(ids, 0)
    m.generate(first, PROMPT, steps)                  # warmup launch, same length
    toks, ms = m.time_generate(first, PROMPT, steps)  # timed launch
    print(json.dumps({"steps": steps, "launch_ms": ms, "ms_per_step": ms / steps,
                      "decode_mode": m.decode_mode_used(), "tokens": toks[:8]}), flush=True)
    m.close()


def _rows(d: str, pattern: str):
    files = glob.glob(os.path.join(d, "**", pattern), recursive=True)
    if not files:
        raise SystemExit(f"no {pattern} under {d}")
    with open(files[0]) as f:
        return list(csv.DictReader(f))


def _counter(d: str, name: str):
    """{kernel name: [value per dispatch]} for one counter."""
    out = {}
    for r in _rows(d, "*counter_collection.csv"):
        if r["Counter_Name"] != name:
            continue
        out.setdefault(r["Kernel_Name"], {}).setdefault(r["Dispatch_Id"], 0.0)
        out[r["Kernel_Name"]][r["Dispatch_Id"]] += float(r["Counter_Value"])
    return {k: list(v.values()) for k, v in out.items()}


def _find(d: dict, key: str):
    for k, v in d.items():
        if key in k:
            return k, v
    raise SystemExit(f"no kernel matching {key!r}")


def summarize(a) -> None:
    trace = _rows(a.trace, "*kernel_stats.csv")
    pers = next(r for r in trace if "k_decode_persistent" in r["Name"])
    calls = int(pers["Calls"])
    avg_ns = float(pers["AverageNs"])
    fetch = _counter(a.fetch, "FETCH_SIZE")
    write = _counter(a.write, "WRITE_SIZE")
    # the 256 MiB device copy is the largest dispatch of the runtime's copy kernel
    copy_name, copy_f = _find(fetch, "copyBuffer")
    _, copy_w = _find(write, "copyBuffer")
    f_cal = max(copy_f) * 1024 / COPY_BYTES
    w_cal = max(copy_w) * 1024 / COPY_BYTES
    _, pf = _find(fetch, "k_decode_persistent")
    _, pw = _find(write, "k_decode_persistent")
    steps = a.steps
    fetch_b = sum(pf) / len(pf) * 1024 / f_cal
    write_b = sum(pw) / len(pw) * 1024 / w_cal
    sys.path.insert(0, os.path.dirname(HERE))
    import synth
    shape = synth.SHAPES["qwen2.5-0.5b"]
    repo = os.path.dirname(os.path.dirname(HERE))
    sys.path.insert(0, repo)
    from bench import algorithmic_bytes
    alg = sum(algorithmic_bytes(shape, PROMPT + i + 1)["total"] for i in range(steps))
    lines = [
        f"# Persistent decode kernel, Qwen2.5-0.5B shape, {steps} greedy steps per launch",
        "",
        "Commands (repository root on the MI355X host, `cd /tmp && export TMPDIR=/tmp` first; paths absolute):",
        "",
        "```",
        f"rocprofv3 --kernel-trace --stats -d T -o t --output-format csv -- python3 e2e-browser-voice-agent_amd/py/profile_decode.py run --steps {steps}",
        f"rocprofv3 --pmc FETCH_SIZE -d F -o f --output-format csv -- python3 e2e-browser-voice-agent_amd/py/profile_decode.py run --steps {steps}",
        f"rocprofv3 --pmc WRITE_SIZE -d W -o w --output-format csv -- python3 e2e-browser-voice-agent_amd/py/profile_decode.py run --steps {steps}",
        f"rocprofv3 --pmc TCC_EA0_RDREQ_DRAM_sum TCC_EA0_RDREQ_sum -d D -o d --output-format csv -- python3 e2e-browser-voice-agent_amd/py/profile_decode.py run --steps {steps}",
        f"python3 e2e-browser-voice-agent_amd/py/profile_decode.py summarize --trace T --fetch F --write W --dram D --steps {steps} --out <this file>",
        "```",
        "",
        "| | value |",
        "|---|---|",
        f"| k_decode_persistent launches (warmup + timed) | {calls} |",
        f"| average launch duration (kernel trace) | {avg_ns / 1e3:.1f} us |",
        f"| per step | {avg_ns / 1e3 / steps:.2f} us ({steps * 1e9 / avg_ns:.0f} tokens/s) |",
        f"| algorithmic bytes per launch | {alg / 1e6:.1f} MB ({alg / steps / 1e6:.2f} MB per step) |",
        f"| achieved algorithmic bandwidth | {alg / (avg_ns * 1e-9) / 1e9:.1f} GB/s ({alg / (avg_ns * 1e-9) / 8e12 * 100:.2f}% of 8 TB/s) |",
        f"| calibration: copy kernel `{copy_name[:40]}` of {COPY_BYTES >> 20} MiB | FETCH_SIZE reads {f_cal:.3f} x, WRITE_SIZE {w_cal:.3f} x the bytes copied |",
        f"| FETCH_SIZE per launch, scaled | {fetch_b / 1e6:.1f} MB ({fetch_b / steps / 1e6:.2f} MB per step) |",
        f"| WRITE_SIZE per launch, scaled | {write_b / 1e6:.1f} MB ({write_b / steps / 1e6:.2f} MB per step) |",
        f"| traffic / algorithmic bytes | {(fetch_b + write_b) / alg:.3f} |",
        "",
        "Top kernels by total time (kernel trace --stats):",
        "",
        "| kernel | calls | total us | average us |",
        "|---|---|---|---|",
    ]
    for r in sorted(trace, key=lambda r: -float(r["TotalDurationNs"]))[:8]:
        lines.append(f"| {r['Name'][:70]} | {r['Calls']} | {float(r['TotalDurationNs']) / 1e3:.1f} | "
                     f"{float(r['AverageNs']) / 1e3:.1f} |")
    traffic = {"steps": steps, "launch_us": avg_ns / 1e3, "fetch_bytes_per_step": fetch_b / steps,
               "write_bytes_per_step": write_b / steps, "algorithmic_bytes_per_step": alg / steps,
               "fetch_calibration": f_cal, "write_calibration": w_cal}
    if a.dram:
        dram = _counter(a.dram, "TCC_EA0_RDREQ_DRAM_sum")
        req = _counter(a.dram, "TCC_EA0_RDREQ_sum")
        _, cd = _find(dram, "copyBuffer")
        _, pdr = _find(dram, "k_decode_persistent")
        _, prq = _find(req, "k_decode_persistent")
        bytes_per_req = COPY_BYTES / max(cd)            # the 256 MiB copy reads COPY_BYTES
        dram_b = sum(pdr) / len(pdr) * bytes_per_req
        traffic["dram_read_bytes_per_step"] = dram_b / steps
        traffic["dram_read_share_of_requests"] = sum(pdr) / sum(prq)
        lines += [
            "",
            f"`TCC_EA0_RDREQ_DRAM_sum` (L2 read requests sent to the memory side) per launch: {sum(pdr) / len(pdr):.4g}, "
            f"{sum(pdr) / sum(prq):.4f} of all L2 read requests (`TCC_EA0_RDREQ_sum`); the 256 MiB copy reads "
            f"{max(cd):.0f} requests = {bytes_per_req:.1f} bytes each, so {dram_b / steps / 1e6:.2f} MB per step go to the "
            f"memory side. That path includes the 256 MB last-level cache (MALL): hits there are counted too, so this "
            f"counter bounds the DRAM reads from above and does not split them (the MALL share is measured by weight "
            f"rotation, `profiles/mall_weight_rotation_head.md`).",
        ]
    import q4hip
    traffic["kernel_sources_sha"] = q4hip.sources_sha()
    lines += ["", "```json", json.dumps(traffic, indent=1), "```", ""]
    with open(a.out, "w") as f:
        f.write("\n".join(lines))
    print("\n".join(lines))


def steps(a) -> None:
    rows = _rows(a.trace, "*kernel_trace.csv")
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    marks = [i for i, r in enumerate(rows) if a.marker in r["Kernel_Name"]]
    if len(marks) <= a.skip:
        raise SystemExit(f"fewer than {a.skip + 1} launches of {a.marker}")
    rest = rows[marks[a.skip]:]
    nsteps = len(marks) - a.skip
    agg = {}
    for r in rest:
        name = r["Kernel_Name"].split("(")[0]
        key = (name, r.get("Grid_Size_X", "?") + "x" + r.get("Grid_Size_Y", "?"))
        d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        c = agg.setdefault(key, [0, 0.0])
        c[0] += 1
        c[1] += d
    busy = sum(v[1] for v in agg.values()) / nsteps
    span = (int(rest[-1]["End_Timestamp"]) - int(rest[0]["Start_Timestamp"])) / 1e3 / nsteps
    lines = [f"# {a.title}", "", "Commands (repository root on the MI355X host, `cd /tmp && export TMPDIR=/tmp` first; paths absolute):",
             "", "```", a.command,
             f"python3 e2e-browser-voice-agent_amd/py/profile_decode.py steps --trace T --marker {a.marker} --skip {a.skip} "
             f"--title ... --command ... --out <this file>", "```", "",
             f"{nsteps} steps; kernel time {busy:.1f} us per step; first kernel start to last kernel end {span:.1f} us per step.",
             "", "| kernel | grid (threads x, y) | launches per step | us per step | us per launch |", "|---|---|---|---|---|"]
    for (name, grid), (n, t) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        lines.append(f"| {name} | {grid} | {n / nsteps:g} | {t / nsteps:.1f} | {t / n:.1f} |")
    lines.append("")
    with open(a.out, "w") as f:
        f.write("\n".join(lines))
    print("\n".join(lines))


def main() -> None:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    r = sub.add_parser("run")
    r.add_argument("--steps", type=int, default=64)
    s = sub.add_parser("summarize")
    s.add_argument("--trace", required=True)
    s.add_argument("--fetch", required=True)
    s.add_argument("--write", required=True)
    s.add_argument("--dram", default=None)
    s.add_argument("--steps", type=int, default=64)
    s.add_argument("--out", required=True)
    t = sub.add_parser("steps")
    t.add_argument("--trace", required=True)
    t.add_argument("--marker", required=True)
    t.add_argument("--skip", type=int, default=0)
    t.add_argument("--title", required=True)
    t.add_argument("--command", required=True)
    t.add_argument("--out", required=True)
    a = ap.parse_args()
    if a.cmd == "run":
        run(a.steps)
    elif a.cmd == "steps":
        steps(a)
    else:
        summarize(a)


if __name__ == "__main__":
    main()
