"""Decode throughput of the Qwen2 Q4_0 token loop on one MI355X.

Workload (the headline configuration): Qwen2.5-0.5B shape (hidden 896, 24 layers, 14/2 heads,
head_dim 64, FFN 4864, vocab 151936), random-init N(0,0.02) weights in GGUF Q4_0, batch 1,
a 64-token seeded prompt, then greedy decode.  One step = one decode token.  W warmup steps run
from position 64; then K timed steps run again from position 64 (same tokens, K/V overwritten),
bracketed by device synchronisation.  value = K / elapsed seconds.

The K timed steps are one launch of the persistent decode kernel (every workgroup resident, one
role per workgroup, the whole greedy loop on the device); its duration comes from HIP events on the
library's stream.  Also reported: algorithmic HBM bytes per token / time per token (achieved GB/s),
the roofline of that kernel (the only kernel in the timed region), the HBM traffic per launch from
the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary, the same K steps on the multi-kernel
hipGraph path for comparison, the same greedy decode driven from Node.js through the N-API addon
(engine/llm.js generateIds, one forward() call per token: node_forward_ms_per_step), and the oracle
timed on the host cores as the CPU baseline.

Other workloads of the same model (one JSON line each, same keys):
  --workload long-context  batch-1 decode after a 4096-position cache filled with seeded fp16-valued
                           K/V (written through q4hip_set_kv), 256 greedy steps by default
                           (fp16 K/V cache by default; --kv-cache f32 for the reference's cache type)
  --workload prefill       one 1024-token seeded prompt per step
  --workload matvec        the isolated Q4_0 matvec at the model's five shapes, 1000 launches each
  --workload batched       32 independent sequences on the Qwen2.5-1.5B shape, each after a
                           1024-token seeded prompt, decoded together; one step = 32 tokens
                           (fp16 K/V cache by default; --kv-cache f32 for the reference's cache type)

Usage: python bench.py [--gpus 1] [--steps 64] [--warmup 8] [--workload decode]
"""
import argparse
import json
import math
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "e2e-browser-voice-agent_amd", "py"))

HBM_PEAK_GBPS = 8000.0
PROMPT = 64
SEED = 1


def algorithmic_bytes(shape, T):
    """HBM bytes one decode step must move at context length T: GGUF Q4_0 weights (18 B per 32),
    fp32 norms and bias, one embedding row, the logits write and the fp32 K/V read."""
    D, F, L, V, QKV = shape.dim, shape.ffn, shape.layers, shape.vocab, shape.qkv
    q4 = lambda n, k: n * k // 32 * 18  # noqa: E731
    layers = L * (q4(QKV, D) + q4(D, D) + q4(2 * F, D) + q4(D, F))
    head = q4(V, D)
    norms = (2 * L + 1) * D * 4
    bias = L * QKV * 4
    emb = D // 32 * 18
    logits = V * 4
    kv = L * shape.kv_heads * shape.head_dim * 4 * 2 * T
    return {"layers": layers, "head": head, "other": norms + bias + emb + logits, "kv": kv,
            "total": layers + head + norms + bias + emb + logits + kv}


def repacked_weight_bytes(shape):
    """Device bytes of the layers' and the head's Q4_0 matrices in the library's layout: per row,
    16 bytes of nibbles per 4 blocks (64-byte words of 4 lanes) and 16 bytes of fp16 scales per 8
    blocks, the block counts rounded up to whole groups; rows in tiles of 64."""
    def mat(n, k):
        nb = k // 32
        return (n + 63) // 64 * 64 * (((nb + 3) // 4) * 64 + ((nb + 7) // 8) * 16)
    D, F = shape.dim, shape.ffn
    return shape.layers * (mat(shape.qkv, D) + mat(D, D) + mat(2 * F, D) + mat(D, F)) + mat(shape.vocab, D)


PROFILE = os.path.join(REPO, "profiles", "decode_persistent_qwen05b_prompt64_steps64.md")


def profile_blob(name):
    """The JSON block at the end of a committed rocprofv3 summary profiles/<name>, or None when there
    is none or it was measured on other kernels: the block records the hash of the device code's
    sources it was made with (kernel_sources_sha), and a figure from a summary of other kernels is
    not reported (profile_source says which)."""
    try:
        text = open(os.path.join(REPO, "profiles", name)).read()
        blob = text[text.index("```json") + 7:]
        data = json.loads(blob[:blob.index("```")])
    except (OSError, ValueError):
        return None
    import q4hip
    if not isinstance(data, dict) or data.get("kernel_sources_sha") != q4hip.sources_sha():
        return None
    return data


def profile_source(name):
    """Where a profile-derived figure comes from: the summary, the kernels it measured, and whether
    those are the kernels this run uses (else the figure is null)."""
    import q4hip
    try:
        text = open(os.path.join(REPO, "profiles", name)).read()
        blob = text[text.index("```json") + 7:]
        data = json.loads(blob[:blob.index("```")])
        sha = data.get("kernel_sources_sha") if isinstance(data, dict) else None
    except (OSError, ValueError):
        sha = None
    return {"profile": "profiles/" + name, "kernel_sources_sha": sha, "current_kernels": q4hip.sources_sha(),
            "matches": sha is not None and sha == q4hip.sources_sha()}


def profiled_traffic():
    """Per-step HBM bytes (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration) from
    the committed rocprofv3 summary of the headline workload, or None."""
    data = profile_blob(os.path.basename(PROFILE))
    try:
        return data["fetch_bytes_per_step"] + data["write_bytes_per_step"]
    except (TypeError, KeyError):
        return None


MALL_PROFILE = "mall_weight_rotation_head.md"


def mall_share(footprint_bytes):
    """Fraction of a weight stream of this footprint, read in the same order every pass, that the
    256 MB last-level cache serves: the committed rotation sweep's row of the smallest footprint
    at or above it (None without the summary)."""
    data = profile_blob(MALL_PROFILE)
    rows = data.get("rows") if data else None
    if not rows:
        return None
    above = [r for r in rows if r["footprint_mb"] * 1e6 >= footprint_bytes]
    row = min(above, key=lambda r: r["footprint_mb"]) if above else rows[-1]
    return {"served_fraction": row["served_fraction"], "footprint_mb": round(footprint_bytes / 1e6, 1),
            "measured_at_mb": row["footprint_mb"], "method": "weight-copy rotation of the head matvec",
            "profile_source": profile_source(MALL_PROFILE)}


def cpu_baseline(shape, tensors, ids, first_tokens):
    """The oracle on the host cores: prompt with every logical core, decode with ceil(cores/2)
    threads (the reference's policy, engine/cpu.js:21-23); median ms per decode token."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    cores = min(cores, 16)
    decode_threads = max(1, math.ceil(cores / 2))
    o = oracle.Model(shape, tensors, ctx=256, threads=cores)
    nxt = o.forward(ids, 0)
    o.set_threads(decode_threads)
    times, toks = [], [nxt]
    pos = len(ids)
    budget = time.time() + 20.0
    while len(times) < 32 and time.time() < budget:
        t0 = time.perf_counter()
        nxt = o.forward([nxt], pos)
        times.append(time.perf_counter() - t0)
        toks.append(nxt)
        pos += 1
    # the same decode on one thread (a few tokens)
    o.set_threads(1)
    one = []
    budget = time.time() + 6.0
    while len(one) < 8 and time.time() < budget:
        t0 = time.perf_counter()
        o.forward([toks[len(one)]], len(ids) + len(one))
        one.append(time.perf_counter() - t0)
    o.close()
    agree = toks[:len(first_tokens)] == first_tokens[:len(toks)]
    med = statistics.median(times)
    med1 = statistics.median(one)
    return {"value": round(1.0 / med, 3), "unit": "tokens/s", "cores": decode_threads, "kind": "port",
            "sample": f"oracle (C restatement of kernels.c) decode of {len(times)} greedy tokens after the same "
                      f"64-token prompt, median ms/token {med * 1e3:.1f}, {decode_threads} of {cores} threads "
                      f"(logical cores capped at 16, this host's CPU share per GPU)",
            "tokens_agree_with_gpu": bool(agree),
            "one_thread": {"value": round(1.0 / med1, 3), "unit": "tokens/s", "tokens": len(one)},
            "cpu_model": cpu_model()}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="decode", choices=["decode", "long-context", "prefill", "matvec", "batched"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-node", action="store_true", help="skip the Node.js host leg of the decode workload")
    ap.add_argument("--kv-cache", default=None, choices=["f32", "f16"],
                    help="K/V cache storage of the long-context and batched workloads: f16 (half the K/V "
                         "bytes; parity against the oracle with the same fp16 rounding; the default, as "
                         "both configurations name an fp16 cache) or f32 (the reference's cache type)")
    args = ap.parse_args()
    if args.kv_cache is None:
        args.kv_cache = "f16" if args.workload in ("batched", "long-context") else "f32"
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the batch-1 decode loop runs on a single device "
              "(multi-GPU sharding is not run)", file=sys.stderr)
        sys.exit(2)
    defaults = {"decode": (64, 8), "long-context": (256, 8), "prefill": (3, 1), "matvec": (1000, 10),
                "batched": (32, 4)}[args.workload]
    args.steps = defaults[0] if args.steps is None else args.steps
    args.warmup = defaults[1] if args.warmup is None else args.warmup
    if args.steps < 1 or args.warmup < 0:
        sys.exit("--steps must be >= 1 and --warmup >= 0")
    {"decode": bench_decode, "long-context": bench_long_context, "prefill": bench_prefill,
     "matvec": bench_matvec, "batched": bench_batched}[args.workload](args)


def _oracle():
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle
    return oracle


def _cores():
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return min(cores, 16)


def bench_decode(args):
    import q4hip
    import synth

    shape = synth.SHAPES["qwen2.5-0.5b"]
    ctx = max(256, PROMPT + max(args.steps, args.warmup) + 2)
    t0 = time.time()
    tensors = synth.make_model(shape, SEED)
    t_gen = time.time() - t0
    m = q4hip.Model(shape, ctx=ctx)
    m.load(tensors)
    ids = synth.prompt_ids(SEED, PROMPT, shape.vocab)

    t0 = time.perf_counter()
    first = m.forward(ids, 0)                      # prefill (not timed for the metric)
    prefill_ms = (time.perf_counter() - t0) * 1e3

    if args.warmup:
        m.generate(first, PROMPT, args.warmup)
    # timed region: K greedy steps from position 64, device synchronised on both sides
    t0 = time.perf_counter()
    toks, dev_ms = m.time_generate(first, PROMPT, args.steps)
    wall_ms = (time.perf_counter() - t0) * 1e3
    ms_per_step = dev_ms / args.steps
    value = args.steps / (dev_ms / 1e3)

    mode = m.decode_mode_used()

    # algorithmic bytes over the timed steps (T = 65 .. 64+K)
    tot = sum(algorithmic_bytes(shape, PROMPT + i + 1)["total"] for i in range(args.steps))
    achieved_gbps = tot / (dev_ms / 1e3) / 1e9

    # the timed region is one launch of the persistent kernel: its roofline is the whole region's
    per_step_traffic = profiled_traffic()
    roofline = {"bound": "hbm", "kernel": "k_decode_persistent" if mode == 2 else "decode graph",
                "achieved": round(achieved_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(achieved_gbps / HBM_PEAK_GBPS, 4),
                "traffic": round(per_step_traffic * args.steps) if per_step_traffic and mode == 2 else None,
                "bytes_per_launch": tot, "avg_launch_us": round(dev_ms * 1e3, 1), "steps_per_launch": args.steps,
                "traffic_source": profile_source(os.path.basename(PROFILE))}
    # how much of the weight set the 256 MB last-level cache can serve when it is read once per token
    share = mall_share(repacked_weight_bytes(shape))
    if share:
        roofline["infinity_cache_share"] = share

    # the same K steps on the multi-kernel path (hipGraph replay per step), for comparison
    m.set_decode_mode(q4hip.DECODE_GRAPH)
    m.generate(first, PROMPT, min(args.warmup, 4) or 1)
    toks_g, graph_ms = m.time_generate(first, PROMPT, args.steps)
    m.set_decode_mode(q4hip.DECODE_AUTO)

    out = {
        "metric": "decode tokens/s at batch 1 (Qwen2.5-0.5B Q4_0 shape); achieved HBM GB/s",
        "value": round(value, 2), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "i8xq4/f32", "data": "synthetic",
        "config": {"workload": "qwen2.5-0.5b-shape Q4_0 greedy decode, batch 1, 64-token prompt",
                   "global_batch": 1, "seq_len": PROMPT + args.steps, "prompt": PROMPT,
                   "parallelism": "single-gpu",
                   "decode_path": {2: "persistent", 1: "graph"}.get(mode, str(mode))},
        "achieved_gbps": round(achieved_gbps, 1),
        "hbm_roofline_frac": round(achieved_gbps / HBM_PEAK_GBPS, 4),
        "algorithmic_mb_per_token": round(tot / args.steps / 1e6, 2),
        "wall_ms_timed": round(wall_ms, 2),
        "prefill64_ms": round(prefill_ms, 2),
        "graph_path_ms_per_step": round(graph_ms / args.steps, 4),
        "graph_path_tokens_identical": toks_g == toks,
        "roofline": roofline,
        "model_gen_s": round(t_gen, 1),
    }
    m.close()
    if not args.no_node:
        out.update(node_host_decode(shape, tensors, ids, args.steps, [first] + toks))
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(shape, tensors, ids, [first] + toks)
    print(json.dumps(out))


def node_host_decode(shape, tensors, ids, steps, want):
    """The same greedy decode driven from Node.js as an application does (engine/llm.js generateIds:
    one forward() call through the N-API addon per token, each a one-step launch), on a GGUF file of
    the same model.  Reports the median host-side milliseconds per decode call."""
    import shutil
    import subprocess
    import tempfile
    import synth
    d = tempfile.mkdtemp(prefix="q4hip-bench-")
    try:
        path = os.path.join(d, "model.gguf")
        synth.write_gguf(path, shape, tensors)
        with open(os.path.join(d, "ids.json"), "w") as f:
            json.dump(list(ids), f)
        script = os.path.join(REPO, "e2e-browser-voice-agent_amd", "node", "host_decode.js")
        r = subprocess.run(["node", script, path, str(max(256, len(ids) + steps + 2)), os.path.join(d, "ids.json"),
                            str(steps + 1)], capture_output=True, text=True, timeout=600)
        if r.returncode != 0:
            raise RuntimeError(f"Node host decode failed: {r.stderr.strip()[-2000:]}")
        res = json.loads(r.stdout.strip().splitlines()[-1])
    finally:
        shutil.rmtree(d, ignore_errors=True)
    return {"node_forward_ms_per_step": round(res["medianStepMs"], 4),
            "node_tokens_identical": res["tokens"] == want,
            "node_decode_path": res["decodePath"]}


LONG_CTX = 4096


def fill_cache(shape, P, seed=SEED):
    """fp16-valued N(0, 1) K and V rows for positions [0, P), seeded per (layer, kv head)."""
    import numpy as np
    for l in range(shape.layers):
        for kh in range(shape.kv_heads):
            rng = np.random.default_rng([seed, l, kh])
            k = rng.standard_normal((P, shape.head_dim), dtype=np.float32).astype(np.float16).astype(np.float32)
            v = rng.standard_normal((P, shape.head_dim), dtype=np.float32).astype(np.float16).astype(np.float32)
            yield l, kh, k, v


def bench_long_context(args):
    """Decode after a 4096-position cache of seeded fp16 K/V (an fp16 cache by default, fp32 with
    --kv-cache f32): the attention role streams past rows through its LDS ring."""
    import q4hip
    import synth
    shape = synth.SHAPES["qwen2.5-0.5b"]
    P = LONG_CTX
    ctx = P + max(args.steps, args.warmup) + 2
    tensors = synth.make_model(shape, SEED)
    kv16 = args.kv_cache == "f16"
    m = q4hip.Model(shape, ctx=ctx, kv_type=q4hip.KV_F16 if kv16 else q4hip.KV_F32)
    m.load(tensors)
    for l, kh, k, v in fill_cache(shape, P):
        m.set_kv(l, kh, 0, k, v)
    first = synth.prompt_ids(SEED + 1, 1, shape.vocab)[0]
    if args.warmup:
        m.generate(first, P, args.warmup)
    toks, dev_ms = m.time_generate(first, P, args.steps)
    mode = m.decode_mode_used()
    # algorithmic bytes: the step's weights and logits, then every cached position's K and V row at the
    # byte width of the cache (fp32: 24,576 B per position; fp16: 12,288 B)
    base = algorithmic_bytes(shape, 0)["total"]
    per_pos = shape.layers * shape.kv_heads * shape.head_dim * 2 * (2 if kv16 else 4)
    tot = sum(base + per_pos * (P + i + 1) for i in range(args.steps))
    gbps = tot / (dev_ms / 1e3) / 1e9
    out = {
        "metric": "decode tokens/s at batch 1 (Qwen2.5-0.5B Q4_0 shape) after a 4096-position KV cache; achieved HBM GB/s",
        "value": round(args.steps / (dev_ms / 1e3), 2), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(dev_ms / args.steps, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "i8xq4/f32", "data": "synthetic",
        "config": {"workload": "qwen2.5-0.5b-shape Q4_0 greedy decode, batch 1, 4096-position cache + 256 steps",
                   "global_batch": 1, "seq_len": P + args.steps, "cache_positions": P,
                   "kv_cache": "fp16" if kv16 else "fp32 (fp16-valued rows)", "parallelism": "single-gpu",
                   "decode_path": {2: "persistent", 1: "graph"}.get(mode, str(mode))},
        "achieved_gbps": round(gbps, 1),
        "roofline": {"bound": "hbm", "kernel": "k_decode_persistent" if mode == 2 else "decode graph",
                     "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None, "bytes_per_launch": tot,
                     "avg_launch_us": round(dev_ms * 1e3, 1), "steps_per_launch": args.steps,
                     "profile": "profiles/decode_long_context_qwen05b_ctx4096.md (kernel trace; the byte-counter "
                                "pass of this workload ended the profiled process, so traffic is not measured)"},
    }
    if not args.no_cpu:
        oracle = _oracle()
        cores = _cores()
        th = max(1, math.ceil(cores / 2))
        o = oracle.Model(shape, tensors, ctx=ctx, threads=th)
        if kv16:
            o.set_variant(oracle.V_KV_F16)
        ok, ov = o.kv()
        for l, kh, k, v in fill_cache(shape, P):
            ok[l, kh, :P] = k
            ov[l, kh, :P] = v
        times, got, tok = [], [], first
        budget = time.time() + 20.0
        while len(times) < 16 and time.time() < budget:
            t0 = time.perf_counter()
            tok = o.forward([tok], P + len(times))
            times.append(time.perf_counter() - t0)
            got.append(tok)
        o.close()
        med = statistics.median(times)
        out["cpu_baseline"] = {"value": round(1.0 / med, 3), "unit": "tokens/s", "cores": th, "kind": "port",
                               "sample": f"oracle decode of {len(times)} greedy tokens after the same 4096-position cache, "
                                         f"median ms/token {med * 1e3:.1f}, {th} of {cores} threads",
                               "tokens_agree_with_gpu": got == toks[:len(got)]}
    m.close()
    print(json.dumps(out))


def bench_prefill(args):
    """One 1024-token prompt per step, a whole-prompt device pass: tiled exact Q4 GEMMs and tiled
    causal attention; the roofline is the integer dot throughput of the largest projection."""
    import q4hip
    import synth
    shape = synth.SHAPES["qwen2.5-0.5b"]
    n = 1024
    tensors = synth.make_model(shape, SEED)
    m = q4hip.Model(shape, ctx=n + 2)
    m.load(tensors)
    ids = synth.prompt_ids(SEED + 2, n, shape.vocab)
    for _ in range(args.warmup):
        m.forward(ids, 0)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        nxt = m.forward(ids, 0)
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    prof = m.profile_pass(ids, 0)
    gu_us = prof["matvec gate+up"] / shape.layers
    macs = n * 2 * shape.ffn * shape.dim
    tops = 2 * macs / (gu_us * 1e-6) / 1e12
    # the pass's FLOPs: every projection over the n tokens, causal attention (q.k and p.v over
    # t = 1..n positions per head), the head for the last token
    D, F, L, H, HD, QKV = shape.dim, shape.ffn, shape.layers, shape.heads, shape.head_dim, shape.qkv
    gemm = 2 * n * L * (QKV * D + D * D + 2 * F * D + D * F)
    attn = 4 * L * H * HD * n * (n + 1) // 2
    flops = gemm + attn + 2 * shape.vocab * D
    pass_tflops = flops / (ms * 1e-3) / 1e12
    pf = profile_blob("prefill_qwen05b_1024.md")
    out = {
        "metric": "prefill tokens/s of a 1024-token prompt (Qwen2.5-0.5B Q4_0 shape)",
        "value": round(n / (ms / 1e3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "i8xq4/f32", "data": "synthetic",
        "config": {"workload": "qwen2.5-0.5b-shape Q4_0 prefill of 1024 seeded ids", "global_batch": 1,
                   "seq_len": n, "parallelism": "single-gpu"},
        "profile_us_per_pass": {k: round(v, 1) for k, v in prof.items()},
        "roofline": {"bound": "mfma", "kernel": "whole prefill pass (projections on k_gemm_sk: exact block dots on the "
                                                 "matrix cores, fp32 lane chains on the VALU)",
                     "achieved": round(pass_tflops, 2), "peak": 2500.0, "unit": "TFLOP/s (dense bf16 MFMA peak)",
                     "frac": round(pass_tflops / 2500.0, 5),
                     "traffic": round(pf["traffic_bytes"] * args.steps) if pf and pf.get("traffic_bytes") else None,
                     "flops_per_pass": flops, "ops_per_launch": flops * args.steps,
                     "avg_launch_us": round(ms * 1e3, 1), "traffic_source": profile_source("prefill_qwen05b_1024.md")},
        "gate_up_int8_dot_tops": {"achieved": round(tops, 2), "peak": 5000.0, "frac": round(tops / 5000.0, 5),
                                  "us_per_layer": round(gu_us, 1)},
        "next_token": nxt,
    }
    if not args.no_cpu:
        oracle = _oracle()
        cores = _cores()
        o = oracle.Model(shape, tensors, ctx=n + 2, threads=cores)
        k = n                                   # the whole prompt (a few seconds with the SSE2 block dots)
        t0 = time.perf_counter()
        cpu_next = o.forward(ids[:k], 0)
        sec = time.perf_counter() - t0
        o.close()
        out["cpu_baseline"] = {"value": round(k / sec, 2), "unit": "tokens/s", "cores": cores, "kind": "port",
                               "tokens_agree_with_gpu": cpu_next == nxt,
                               "sample": f"oracle prefill of all {k} of the 1024 ids (16-token chunks), "
                                         f"{sec:.1f} s, {cores} threads"}
    m.close()
    print(json.dumps(out))


def bench_matvec(args):
    """The isolated matvec (y = W x, x quantized per 32-block) at the model's five shapes: cache-hot (the
    same weights every launch) and cold (launches cycle through copies of the weights totalling more than
    the 256 MB last-level cache)."""
    import numpy as np
    import q4hip
    import synth
    shapes = [(896, 896), (128, 896), (4864, 896), (896, 4864), (151936, 896)]
    rows = []
    for N, K in shapes:
        raw = synth.quantize_q4_0((np.random.default_rng([SEED, N, K]).standard_normal(N * K, dtype=np.float32)
                                   * np.float32(0.02)))
        mv = q4hip.Matvec(raw, N, K)
        mv.time(args.warmup)
        us = mv.time(args.steps)
        cold_us, copies = mv.time_cold(args.steps)
        mv.close()
        nbytes = N * K // 32 * 18 + K * 4 + N * 4
        rows.append({"shape": [N, K], "us": round(us, 2), "gbps": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "cold_us": round(cold_us, 2), "cold_gbps": round(nbytes / (cold_us * 1e-6) / 1e9, 1),
                     "cold_copies": copies})
    head = rows[-1]
    # value: the head streamed from HBM (launches cycle through weight copies larger than the 256 MB
    # last-level cache); the cache-hot rate, where repeated launches find the weights in that cache,
    # is reported beside it
    out = {
        "metric": "isolated Q4_0 matvec achieved GB/s (Qwen2.5-0.5B shapes, fp32 x quantized per 32-block)",
        "value": head["cold_gbps"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(head["cold_us"] / 1e3, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "i8xq4/f32", "data": "synthetic",
        "config": {"workload": "Q4_0 matvec sweep, value = the 151936x896 head shape read from HBM "
                               f"(launches rotate over {head['cold_copies']} weight copies)",
                   "shapes": [r["shape"] for r in rows], "parallelism": "single-gpu"},
        "per_shape": rows,
        "cache_hot": {"value": head["gbps"], "us": head["us"],
                      "note": "the same weights every launch: served largely by the 256 MB last-level cache"},
        "roofline": {"bound": "hbm", "kernel": "k_matvec_stream<28> 151936x896", "achieved": head["cold_gbps"],
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(head["cold_gbps"] / HBM_PEAK_GBPS, 4),
                     "traffic": _matvec_head_traffic(), "avg_launch_us": head["cold_us"],
                     "traffic_source": profile_source("matvec_sweep_qwen05b.md")},
    }
    if not args.no_cpu:
        oracle = _oracle()
        N, K = 151936, 896
        raw = synth.quantize_q4_0((np.random.default_rng([SEED, N, K]).standard_normal(N * K, dtype=np.float32)
                                   * np.float32(0.02)))
        x = np.random.default_rng(SEED).standard_normal(K, dtype=np.float32)
        qs, d = synth.q4_0_blocks(raw)          # the weights as the reference holds them after loading
        oracle.matvec_q4_blocks(qs, d, N, K, x)
        t0 = time.perf_counter()
        reps = 20
        for _ in range(reps):
            oracle.matvec_q4_blocks(qs, d, N, K, x)
        sec = (time.perf_counter() - t0) / reps
        out["cpu_baseline"] = {"value": round((N * K // 32 * 18) / sec / 1e9, 3), "unit": "GB/s", "cores": 1,
                               "kind": "port", "sample": f"oracle matvec of the 151936x896 head (SSE2 lane dots, "
                                                          f"weights split into nibbles and scales beforehand), "
                                                          f"{reps} calls, {sec * 1e3:.1f} ms each, one thread"}
    print(json.dumps(out))



def _matvec_head_traffic():
    """HBM bytes of one head-shape matvec launch from the committed sweep profile, or None."""
    pm = profile_blob("matvec_sweep_qwen05b.md")
    groups = 151936 // 16                               # 16-row groups; k_matvec_stream's grid, in threads
    per = -(-groups // 2048)
    grid = str(-(-(-(-groups // per)) // 4) * 256)
    for r in (pm or {}).get("per_launch", []):
        if r["grid"].split(",")[0] == grid and r.get("fetch_bytes") is not None:
            return round(r["fetch_bytes"] + r["write_bytes"])
    return None


BATCH = 32
BATCH_PROMPT = 1024


def bench_batched(args):
    """32 sequences of the Qwen2.5-1.5B shape (hidden 1536, 28 layers, 12/2 heads, head_dim 128,
    FFN 8960), each prefilled with its own 1024-token seeded prompt, then decoded together: every
    step runs the 32 tokens through one pass of B-token GEMMs, per-sequence attention over 1025+
    positions and a per-row greedy argmax.  Warmup steps run from position 1024, then the timed
    steps again from 1024 (same tokens, K/V overwritten)."""
    import q4hip
    import synth
    shape = synth.SHAPES["qwen2.5-1.5b"]
    ctx = BATCH_PROMPT + max(args.steps, args.warmup) + 2
    t0 = time.time()
    tensors = synth.make_model(shape, SEED)
    kv16 = args.kv_cache == "f16"
    m = q4hip.Model(shape, ctx=ctx, kv_type=q4hip.KV_F16 if kv16 else q4hip.KV_F32)
    m.load(tensors)
    bt = q4hip.Batch(m, BATCH)
    first = [bt.prefill(b, synth.prompt_ids(SEED + 10 + b, BATCH_PROMPT, shape.vocab), 0) for b in range(BATCH)]
    print(f"batched: model and {BATCH} prefills ready in {time.time() - t0:.1f} s", file=sys.stderr, flush=True)
    pos = [BATCH_PROMPT] * BATCH
    if args.warmup:
        bt.generate(first, pos, args.warmup)
    toks, dev_ms = bt.time_generate(first, pos, args.steps)
    tok_s = BATCH * args.steps / (dev_ms / 1e3)
    # algorithmic bytes per step: the weights once, then every sequence's K/V rows at the byte width
    # of the cache
    base = algorithmic_bytes(shape, 0)
    weights = base["layers"] + base["head"] + base["other"] - shape.vocab * 4
    per_pos = shape.layers * shape.kv_heads * shape.head_dim * 2 * (2 if kv16 else 4)
    logits = BATCH * shape.vocab * 4
    tot = sum(weights + logits + BATCH * per_pos * (BATCH_PROMPT + i + 1) for i in range(args.steps))
    gbps = tot / (dev_ms / 1e3) / 1e9
    pb = profile_blob("batched_decode_qwen15b_b32_ctx1024.md")   # measured with the fp16 cache
    # matrix-core work of the step's projections: one v_mfma_f32_16x16x16_f16 (8192 flops) per
    # 16 weight rows x 16-token tile x block x reference lane chain (k_gemm_sk), over qkv, o, gate|up,
    # down and the head
    D, F, L, V, QKV = shape.dim, shape.ffn, shape.layers, shape.vocab, shape.qkv
    tiles = (BATCH + 15) // 16
    pad16 = lambda n: (n + 63) // 64 * 64 // 16          # noqa: E731  16-row groups of a 64-row-padded matrix
    mfmas = tiles * 4 * (L * (pad16(QKV) * (D // 32) + pad16(D) * (D // 32) + pad16(2 * F) * (D // 32)
                              + pad16(D) * (F // 32)) + pad16(V) * (D // 32))
    mfma_tflops = mfmas * 8192 * args.steps / (dev_ms / 1e3) / 1e12
    out = {
        "metric": "batched decode tokens/s, 32 sequences at 1024-token context (Qwen2.5-1.5B Q4_0 shape)",
        "value": round(tok_s, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(dev_ms / args.steps, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "i8xq4/f32", "data": "synthetic",
        "config": {"workload": "qwen2.5-1.5b-shape Q4_0 greedy decode, 32 sequences, 1024-token prompts",
                   "global_batch": BATCH, "seq_len": BATCH_PROMPT + args.steps,
                   "kv_cache": "fp16" if kv16 else "fp32 (the reference's cache type)",
                   "parallelism": "single-gpu"},
        "achieved_gbps": round(gbps, 1),
        "mfma": {"instructions_per_step": mfmas, "flops_per_step": mfmas * 8192,
                 "achieved_tflops": round(mfma_tflops, 2), "peak_tflops": 2500.0,
                 "frac": round(mfma_tflops / 2500.0, 5),
                 "note": "v_mfma_f32_16x16x16_f16 issued by the step's projections over the whole step time, "
                         "against the dense fp16 matrix peak; 10 of each instruction's 16 k-slots carry data "
                         "(the exact integer encoding of the reference's lane dots)"},
        "roofline": {"bound": "hbm", "kernel": "batched decode step (all kernels)",
                     "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4),
                     "traffic": round(pb["traffic_bytes"] * args.steps) if pb and kv16 else None,
                     "bytes_per_launch": tot, "avg_launch_us": round(dev_ms * 1e3, 1), "steps_per_launch": args.steps,
                     "traffic_source": profile_source("batched_decode_qwen15b_b32_ctx1024.md")},
        "first_tokens": toks[0, :4].tolist(),
    }
    bt.close()
    m.close()
    if not args.no_cpu:
        oracle = _oracle()
        cores = _cores()
        th = max(1, math.ceil(cores / 2))
        o = oracle.Model(shape, tensors, ctx=ctx, threads=th)
        times, tok = [], first[0]
        budget = time.time() + 20.0
        while len(times) < 8 and time.time() < budget:
            t1 = time.perf_counter()
            tok = o.forward([tok], BATCH_PROMPT + len(times))
            times.append(time.perf_counter() - t1)
        o.close()
        med = statistics.median(times)
        out["cpu_baseline"] = {"value": round(1.0 / med, 3), "unit": "tokens/s", "cores": th, "kind": "port",
                               "sample": f"oracle decode of {len(times)} tokens of one sequence at positions "
                                         f"{BATCH_PROMPT}.. (the reference decodes one sequence at a time; cache "
                                         f"contents not matched, timing only), median ms/token {med * 1e3:.1f}, "
                                         f"{th} of {cores} threads"}
    print(json.dumps(out))


if __name__ == "__main__":
    main()
