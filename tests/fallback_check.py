"""Multi-token passes under a kernel-selection switch, against the oracle, in a process of their own.

The switches are read once per process (Q4HIP_GEMM=valu keeps the matrix cores out: k_gemm_rows for
passes of 9..64 tokens, k_gemm_q4 above, unfused SwiGLU and RoPE launches; Q4HIP_ATTN_ROWS=0 runs a
prompt's attention in three launches instead of k_attn_rows; Q4HIP_PV_TILES=0 on k_attn_pv_list), so
tests/test_gpu_fallbacks.py starts this script as a
child with the switch set.  Prompts of 12, 40 and 150 tokens on two shapes (head_dim 64 and 128),
then decode steps; a ragged batch of 12 sequences for two steps.  Tokens equal and logits bit
for bit, as in the other GPU tests.  Prints the first mismatch and exits 1 on failure.
"""
import os
import sys

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(REPO, "e2e-browser-voice-agent_amd", "py"))
sys.path.insert(0, os.path.join(REPO, "oracle"))

import oracle  # noqa: E402
import q4hip  # noqa: E402
import synth  # noqa: E402


def same(lg, lo, what):
    a = np.ascontiguousarray(lg, np.float32).view(np.uint32)
    b = np.ascontiguousarray(lo, np.float32).view(np.uint32)
    bad = np.flatnonzero(a != b)
    if bad.size:
        raise AssertionError(f"{what}: {bad.size} logits differ, max-abs {float(np.max(np.abs(lg - lo)))}")


def prompts(name, seed):
    shape = synth.SHAPES[name]
    t = synth.make_model(shape, seed)
    for n in (12, 40, 150):
        g = q4hip.Model(shape, ctx=256)
        g.load(t)
        g.set_decode_mode(q4hip.DECODE_GRAPH)
        o = oracle.Model(shape, t, ctx=256, mt=16, threads=8)
        try:
            ids = synth.prompt_ids(seed + n, n, shape.vocab)
            ng, no = g.forward(ids, 0), o.forward(ids, 0)
            assert ng == no, f"{name} prompt {n}: token {ng} != {no}"
            same(g.read_logits(), o.logits(), f"{name} prompt {n}")
            for step in range(3):
                ng, no = g.forward([ng], n + step), o.forward([no], n + step)
                assert ng == no, f"{name} prompt {n} step {step}: token {ng} != {no}"
            same(g.read_logits(), o.logits(), f"{name} prompt {n} step 2")
            print(f"{name} prompt {n}: ok", flush=True)
        finally:
            g.close()
            o.close()


def batch(name, seed):
    shape = synth.SHAPES[name]
    t = synth.make_model(shape, seed)
    rng = np.random.default_rng(seed)
    lens = [int(n) for n in rng.integers(1, 30, 12)]
    ps = [rng.integers(0, shape.vocab, n).astype(np.int32) for n in lens]
    g = q4hip.Model(shape, ctx=96)
    g.load(t)
    o = oracle.Model(shape, t, ctx=96, mt=16, threads=8)
    bt = q4hip.Batch(g, len(lens))
    try:
        first = [bt.prefill(b, ps[b], 0) for b in range(len(lens))]
        out = bt.generate(first, lens, 2)
        lg = bt.read_logits()
        for b in range(len(lens)):
            tok = o.forward(ps[b], 0)
            want = [tok]
            for i in range(2):
                tok = o.forward([tok], lens[b] + i)
                want.append(tok)
            assert first[b] == want[0] and out[:, b].tolist() == want[1:], f"{name} batch sequence {b}: tokens"
            same(lg[b], o.logits(), f"{name} batch sequence {b}")
        print(f"{name} batch of {len(lens)}: ok", flush=True)
    finally:
        bt.close()
        g.close()
        o.close()


def main():
    print("switches:", {k: os.environ.get(k) for k in ("Q4HIP_GEMM", "Q4HIP_ATTN_ROWS", "Q4HIP_PV_TILES")}, flush=True)
    try:
        prompts("small", 71)
        prompts("small128", 72)
        batch("small", 73)
        batch("small128", 74)
    except AssertionError as e:
        print("MISMATCH:", e, flush=True)
        sys.exit(1)
    print("all ok", flush=True)


if __name__ == "__main__":
    main()
