"""Phase timeline of one persistent decode step (q4hip_profile_persistent), per layer.

    python profile_phases.py                   # Qwen2.5-0.5B shape, 64-token prompt, steps from position 64
    python profile_phases.py --positions 4096  # the same after a 4096-position cache of seeded fp16-valued K/V
    python profile_phases.py --positions 4096 --kv-cache f16   # ... stored as an fp16 cache

Prints, for the middle layers (median over layers 1 .. L-2), when each role's phases end, in microseconds after
the last down-projection store of the previous layer: the per-workgroup timestamps (min / median / max over the
role's workgroups) and the attention marks of the first attention workgroup.  Needs a GPU.
"""
import argparse
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

# per-workgroup timestamp slots k of each role (q4hip_profile_persistent)
WG_SLOTS = {
    "OD": {0: "att received", 4: "o terms (wave 0)", 1: "x1 stored", 2: "act received", 5: "down terms (w0)",
           6: "down terms (all)", 3: "x2 stored"},
    "A": {0: "x received", 2: "past K scored", 3: "scores exchanged", 6: "past sum done", 4: "new K/V received",
          5: "p formed",
          1: "att stored"},
    "KV": {0: "x received", 7: "norm chain done", 2: "normalised", 3: "rows formed", 1: "K/V rows stored"},
    "GU": {0: "x1 received", 7: "norm chain done", 2: "normalised", 3: "rows formed", 1: "act stored"},
}
# slots of the first attention workgroup's timeline (l * 16 + k)
A_MARKS = [(9, "normalised"), (5, "q rows"), (11, "RoPE"), (15, "new K/V received"), (12, "maximum"),
           (13, "softmax sum"), (14, "division"), (6, "att stored")]


def fill_cache(m, shape, P, seed=1):
    """fp16-valued N(0, 1) K and V rows for positions [0, P), seeded per (layer, kv head) (bench.py's cache)."""
    for l in range(shape.layers):
        for kh in range(shape.kv_heads):
            rng = np.random.default_rng([seed, l, kh])
            k = rng.standard_normal((P, shape.head_dim), dtype=np.float32).astype(np.float16).astype(np.float32)
            v = rng.standard_normal((P, shape.head_dim), dtype=np.float32).astype(np.float16).astype(np.float32)
            m.set_kv(l, kh, 0, k, v)


def main() -> None:
    import q4hip
    import synth

    ap = argparse.ArgumentParser()
    ap.add_argument("--positions", type=int, default=0, help="cached positions (0: the 64-token prompt)")
    ap.add_argument("--runs", type=int, default=5)
    ap.add_argument("--kv-cache", default="f32", choices=["f32", "f16"], help="K/V cache storage")
    args = ap.parse_args()
    shape = synth.SHAPES["qwen2.5-0.5b"]
    L = shape.layers
    P = args.positions
    m = q4hip.Model(shape, ctx=max(256, P + 40), kv_type=q4hip.KV_F16 if args.kv_cache == "f16" else q4hip.KV_F32)
    m.load(synth.make_model(shape, 1))
    m.set_decode_mode(q4hip.DECODE_PERSISTENT)
    if P:
        fill_cache(m, shape, P)
        tok, pos = 7, P
    else:
        ids = synth.prompt_ids(1, 64, shape.vocab)
        tok, pos = m.forward(ids, 0), 64
    m.generate(tok, pos, 2)
    runs = [m.profile_persistent(tok, pos + i, per_workgroup=True) for i in range(args.runs)]
    tl = np.median(np.stack([r[0] for r in runs]), axis=0)
    wg = np.median(np.stack([r[1] for r in runs]), axis=0)
    split_from = int(os.environ.get("Q4HIP_SPLIT_FROM", "512"))
    asplit = 2 if P >= split_from else 1
    nOD, nA, nKV, nGU = shape.dim // 16, shape.heads * asplit, 8 * shape.kv_heads, shape.ffn // 32
    roles = {"OD": slice(0, nOD), "A": slice(nOD, nOD + nA), "KV": slice(nOD + nA, nOD + nA + nKV),
             "GU": slice(nOD + nA + nKV, nOD + nA + nKV + nGU)}
    base = wg[:, roles["OD"], 3].max(axis=1)          # last x2 store of each layer
    mid = range(1, L - 1)
    print(f"cached positions {P or 64}, attention workgroups per head {asplit}; per layer "
          f"{np.median(np.diff(base)):.2f} us; whole step {tl[L, 2]:.2f} us; shader clock {tl[L, 4]:.0f} MHz")
    for role, slots in WG_SLOTS.items():
        for k, name in slots.items():
            raw = wg[1:L - 1, roles[role], k]
            if np.count_nonzero(raw) < raw.size // 2:
                continue                                 # slot not written in this mode
            off = np.stack([wg[l, roles[role], k] - base[l - 1] for l in mid])
            if np.median(off) < 0:
                continue                                 # slot not written by this kernel (no stamp)
            print(f"{role:>3} {name:<18} min {np.median(off.min(1)):7.2f}  median {np.median(np.median(off, 1)):7.2f}"
                  f"  max {np.median(off.max(1)):7.2f}")
    hb = base[L - 1]
    print(f"head: x received {tl[L, 0] - hb:.2f}, (value, index) sent {tl[L, 1] - hb:.2f}, token known "
          f"{tl[L, 2] - hb:.2f} us after the last layer's down stores; layer 0's down stores end {base[0]:.2f} us "
          f"after the kernel starts")
    marks = np.median(np.stack([[tl[l, k] - base[l - 1] for k, _ in A_MARKS] for l in mid]), axis=0)
    print("first attention workgroup: " + ", ".join(f"{n} {v:.2f}" for (_, n), v in zip(A_MARKS, marks)))
    m.close()


if __name__ == "__main__":
    main()
