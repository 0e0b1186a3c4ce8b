"""How far other floating-point operation orders move the reference's logits (CPU, the oracle).

The reference quantizes every activation to int8 per 32-block before each projection, so a
reassociated sum that differs in the last bit can flip an int8 rounding, and the flip moves the
logits by a weight times a quantization step.  This measures that on the benchmark workloads:

    python oracle/reassoc_study.py [--steps 64] [--threads 8] [--positions 4096]

  * decode: Qwen2.5-0.5B shape, seeded random Q4_0 weights, 64-token prompt, then `steps` steps;
  * long:   the same model after `positions` cached fp16-valued K/V rows, then `steps` steps.

Each variant model (oracle.h ORC_V_*) is fed the exact model's tokens (teacher forcing), so every
step compares logits at the same inputs.  Per variant: the largest max-abs logit error over the
steps, the steps whose error exceeds 1e-3, the steps whose greedy token differs, and the smallest
top-2 logit margin of the exact model (how close the greedy choice is to flipping).  Prints one
JSON line per (workload, variant).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.join(os.path.dirname(HERE), "e2e-browser-voice-agent_amd", "py"))

import oracle  # noqa: E402
import synth  # noqa: E402

VARIANTS = {
    "norm_tree": oracle.V_NORM_TREE,
    "dot_splitk": oracle.V_DOT_SPLITK,
    "attn_split": oracle.V_ATTN_SPLIT,
    "kv_f16": oracle.V_KV_F16,
    "all_reassociated": oracle.V_NORM_TREE | oracle.V_DOT_SPLITK | oracle.V_ATTN_SPLIT,
}


def fill_cache(models, shape, P, seed=1):
    """The same fp16-valued N(0, 1) K/V rows for positions [0, P) in every model."""
    for l in range(shape.layers):
        for kh in range(shape.kv_heads):
            rng = np.random.default_rng([seed, l, kh])
            k = rng.standard_normal((P, shape.head_dim), dtype=np.float32).astype(np.float16).astype(np.float32)
            v = rng.standard_normal((P, shape.head_dim), dtype=np.float32).astype(np.float16).astype(np.float32)
            for m in models:
                kc, vc = m.kv()
                kc[l, kh, :P] = k
                vc[l, kh, :P] = v


def run(workload, shape, tensors, steps, threads, positions):
    ctx = (positions if workload == "long" else 64) + steps + 8
    exact = oracle.Model(shape, tensors, ctx=ctx, mt=16, threads=threads)
    var = {}
    for name, flags in VARIANTS.items():
        m = oracle.Model(shape, tensors, ctx=ctx, mt=16, threads=threads)
        m.set_variant(flags)
        var[name] = m
    stats = {n: {"max_abs": 0.0, "steps_over_1e-3": 0, "token_flips": 0, "errors": []} for n in var}
    margins = []
    if workload == "long":
        fill_cache([exact, *var.values()], shape, positions)
        tok, pos = 7, positions
        inputs = [([tok], pos)]
    else:
        ids = synth.prompt_ids(1, 64, shape.vocab)
        inputs = [(ids, 0)]
    t0 = time.time()
    for step in range(steps + 1):
        ids_in, pos = inputs[-1]
        nxt = exact.forward(ids_in, pos)
        le = exact.logits()
        top2 = np.partition(le, -2)[-2:]
        margins.append(float(top2[1] - top2[0]))
        for name, m in var.items():
            nv = m.forward(ids_in, pos)
            err = float(np.max(np.abs(m.logits() - le)))
            s = stats[name]
            s["max_abs"] = max(s["max_abs"], err)
            s["steps_over_1e-3"] += err > 1e-3
            s["token_flips"] += nv != nxt
            s["errors"].append(err)
        inputs.append(([nxt], pos + len(ids_in)))
    out = []
    for name, s in stats.items():
        e = np.array(s.pop("errors"))
        out.append(dict(workload=workload, variant=name, steps=steps + 1, median_abs=float(np.median(e)),
                        min_top2_margin=min(margins), seconds=round(time.time() - t0, 1), **s))
    for m in [exact, *var.values()]:
        m.close()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--threads", type=int, default=8)
    ap.add_argument("--positions", type=int, default=4096)
    ap.add_argument("--workloads", default="decode,long")
    a = ap.parse_args()
    shape = synth.SHAPES["qwen2.5-0.5b"]
    tensors = synth.make_model(shape, 1)
    for w in a.workloads.split(","):
        for row in run(w, shape, tensors, a.steps, a.threads, a.positions):
            print(json.dumps(row), flush=True)


if __name__ == "__main__":
    main()
