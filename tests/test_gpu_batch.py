"""Batched decode (q4hip_batch_*) on the GPU against the oracle run one sequence at a time.

The reference decodes one sequence per backend (engine/cpu.js, engine/llm.js:86-97); a batch of B
sequences must give every sequence the greedy tokens and bit-identical logits its own loop gives.
Prompts are ragged (positions differ per sequence) and include a one-token prompt.
"""
import numpy as np
import pytest

import oracle
import synth

pytestmark = pytest.mark.gpu

_cache = {}


def _model(name, seed, head_type=synth.GGML_Q4_0):
    key = (name, seed, head_type)
    if key not in _cache:
        _cache[key] = synth.make_model(synth.SHAPES[name], seed, head_type=head_type)
    return _cache[key]


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _same_logits(lg, lo, what):
    diff = float(np.max(np.abs(lg - lo)))
    assert diff <= 1e-3, f"{what}: max-abs logit error {diff}"
    bad = np.flatnonzero(_bits(lg) != _bits(lo))
    assert bad.size == 0, f"{what}: {bad.size} logits differ (max-abs {diff}), first {bad[:5]}"


def _oracle_loop(o, prompt, steps):
    """Greedy loop of one sequence on the oracle: (tokens after the prompt, logits of the last step)."""
    tok = o.forward(prompt, 0)
    toks = [tok]
    for i in range(steps):
        tok = o.forward([tok], len(prompt) + i)
        toks.append(tok)
    return toks, o.logits().copy()


@pytest.mark.parametrize("name,seed,lens,head_type", [
    ("tiny", 41, [1, 7, 20, 33, 3], synth.GGML_Q4_0),
    ("small", 42, [12, 5, 40], synth.GGML_Q4_0),
    ("small128", 43, [9, 30, 1, 17], synth.GGML_Q4_0),
    ("small", 44, [6, 19], synth.GGML_Q8_0),
])
def test_batch_matches_independent_loops(name, seed, lens, head_type):
    import q4hip
    print(f"batch {name} seed {seed} lens {lens} head {head_type}", flush=True)
    shape = synth.SHAPES[name]
    t = _model(name, seed, head_type)
    B, steps, ctx = len(lens), 6, 96
    rng = np.random.default_rng(seed)
    prompts = [rng.integers(0, shape.vocab, n).astype(np.int32) for n in lens]
    g = q4hip.Model(shape, ctx=ctx)
    g.load(t)
    o = oracle.Model(shape, t, ctx=ctx, mt=16, threads=8)
    bt = q4hip.Batch(g, B)
    try:
        first = [bt.prefill(b, prompts[b], 0) for b in range(B)]
        out = bt.generate(first, lens, steps)
        lg = bt.read_logits()
        for b in range(B):
            want, lo = _oracle_loop(o, prompts[b], steps)
            assert first[b] == want[0], f"sequence {b}: prefill token"
            assert out[:, b].tolist() == want[1:], f"sequence {b}: tokens"
            _same_logits(lg[b], lo, f"sequence {b} last step")
    finally:
        bt.close()
        g.close()
        o.close()


def test_batch_steps_continue():
    """Two generate calls in a row continue each sequence where the first left it, and a batch's
    decode leaves the context's own cache and single-sequence decode untouched."""
    import q4hip
    shape = synth.SHAPES["tiny"]
    t = _model("tiny", 45)
    lens = [4, 11, 2]
    rng = np.random.default_rng(45)
    prompts = [rng.integers(0, shape.vocab, n).astype(np.int32) for n in lens]
    g = q4hip.Model(shape, ctx=64)
    g.load(t)
    o = oracle.Model(shape, t, ctx=64, mt=16, threads=8)
    bt = q4hip.Batch(g, 3)
    try:
        single = g.forward(prompts[1], 0)
        first = [bt.prefill(b, prompts[b], 0) for b in range(3)]
        a = bt.generate(first, lens, 3)
        pos2 = [n + 3 for n in lens]
        b2 = bt.generate(a[-1], pos2, 4)
        both = np.concatenate([a, b2])
        for b in range(3):
            want, _ = _oracle_loop(o, prompts[b], 7)
            assert both[:, b].tolist() == want[1:], f"sequence {b}"
        # the context's own sequence continues as if no batch had run
        want1, lo = _oracle_loop(o, prompts[1], 1)
        assert g.forward([single], lens[1]) == want1[1]
        _same_logits(g.read_logits(), lo, "context after batch")
    finally:
        bt.close()
        g.close()
        o.close()


def test_batch_prefilled_cache():
    """Sequences whose caches were written through q4hip_batch_set_kv (a 300-position cache per
    sequence, different contents) decode as the oracle does over the same cache."""
    import q4hip
    shape = synth.SHAPES["small128"]
    t = _model("small128", 46)
    P, B, ctx, steps = 300, 3, 320, 4
    g = q4hip.Model(shape, ctx=ctx)
    g.load(t)
    o = oracle.Model(shape, t, ctx=ctx, mt=16, threads=8)
    bt = q4hip.Batch(g, B)
    try:
        caches = []
        for b in range(B):
            r = np.random.default_rng(100 + b)
            k = r.standard_normal((shape.layers, shape.kv_heads, P, shape.head_dim)).astype(np.float16).astype(np.float32)
            v = r.standard_normal((shape.layers, shape.kv_heads, P, shape.head_dim)).astype(np.float16).astype(np.float32)
            caches.append((k, v))
            for l in range(shape.layers):
                for kh in range(shape.kv_heads):
                    bt.set_kv(b, l, kh, 0, k[l, kh], v[l, kh])
        first = [5, 17, 900]
        pos = [P, P - 40, P - 7]
        out = bt.generate(first, pos, steps)
        lg = bt.read_logits()
        for b in range(B):
            ok, ov = o.kv()
            ok[:, :, :P] = caches[b][0]
            ov[:, :, :P] = caches[b][1]
            tok = first[b]
            for i in range(steps):
                tok = o.forward([tok], pos[b] + i)
                assert out[i, b] == tok, f"sequence {b} step {i}"
            _same_logits(lg[b], o.logits(), f"sequence {b}")
    finally:
        bt.close()
        g.close()
        o.close()


def test_batch_errors():
    import q4hip
    shape = synth.SHAPES["tiny"]
    g = q4hip.Model(shape, ctx=32, mt=4)
    g.load(_model("tiny", 47))
    try:
        with pytest.raises(q4hip.Q4Error):
            q4hip.Batch(g, 5)                      # more sequences than the pass size
        bt = q4hip.Batch(g, 2)
        try:
            with pytest.raises(q4hip.Q4Error) as e:
                bt.generate([1, 2], [3, 30], 2)    # 30 + 2 >= ctx
            assert e.value.code == q4hip.ECONTEXT
            with pytest.raises(q4hip.Q4Error):
                bt.generate([1, shape.vocab], [0, 0], 1)
            with pytest.raises(q4hip.Q4Error):
                bt.prefill(2, [1, 2], 0)
            with pytest.raises(q4hip.Q4Error):
                bt.set_kv(0, 0, 0, 31, np.zeros((2, shape.head_dim)), np.zeros((2, shape.head_dim)))
            assert bt.generate([1, 2], [0, 5], 2).shape == (2, 2)
        finally:
            bt.close()
    finally:
        g.close()


@pytest.mark.parametrize("B,kv", [(16, "f32"), (12, "f16")])
def test_batch_qwen05b_sixteen_sequences(B, kv):
    """16 (or 12: a partial 16-token tile) sequences of the Qwen2.5-0.5B shape: the output head
    (151,936 rows) runs as a matrix-core GEMM and the q|k|v projection with RoPE and the cache
    append fused; every sequence's tokens and last logits equal the oracle's (with an fp16 cache,
    the oracle over the same fp16 rounding)."""
    import q4hip
    shape = synth.SHAPES["qwen2.5-0.5b"]
    t = _model("qwen2.5-0.5b", 48)
    steps, ctx = 3, 64
    rng = np.random.default_rng(48)
    lens = [int(n) for n in rng.integers(1, 12, B)]
    prompts = [rng.integers(0, shape.vocab, n).astype(np.int32) for n in lens]
    print(f"qwen05b batch of {B}, kv {kv}, prompt lengths {lens}", flush=True)
    g = q4hip.Model(shape, ctx=ctx, kv_type=q4hip.KV_F16 if kv == "f16" else q4hip.KV_F32)
    g.load(t)
    o = oracle.Model(shape, t, ctx=ctx, mt=16, threads=8)
    if kv == "f16":
        o.set_variant(oracle.V_KV_F16)
    bt = q4hip.Batch(g, B)
    try:
        first = [bt.prefill(b, prompts[b], 0) for b in range(B)]
        out = bt.generate(first, lens, steps)
        lg = bt.read_logits()
        for b in range(B):
            want, lo = _oracle_loop(o, prompts[b], steps)
            assert first[b] == want[0] and out[:, b].tolist() == want[1:], f"sequence {b}"
            _same_logits(lg[b], lo, f"sequence {b}")
    finally:
        bt.close()
        g.close()
        o.close()


def test_batch_full_size_matches_single_sequence():
    """The batched-decode configuration at full size (Qwen2.5-1.5B shape, 32 sequences; prompts
    shortened to 16 tokens): each sequence decoded in the batch of 32 (multi-token GEMMs, list
    attention) gives the same tokens and logit bits as the same sequence decoded alone (batch of
    one: single-token matvecs), and equal prompts give equal rows."""
    import q4hip
    shape = synth.SHAPES["qwen2.5-1.5b"]
    t = _model("qwen2.5-1.5b", 49)
    B, steps, ctx, P = 32, 4, 64, 16
    prompts = [np.asarray(synth.prompt_ids(500 + b, P, shape.vocab), np.int32) for b in range(B)]
    prompts[7] = prompts[3].copy()
    g = q4hip.Model(shape, ctx=ctx)
    g.load(t)
    try:
        bt = q4hip.Batch(g, B)
        first = [bt.prefill(b, prompts[b], 0) for b in range(B)]
        out = bt.generate(first, [P] * B, steps)
        lg = bt.read_logits()
        bt.close()
        assert out[:, 7].tolist() == out[:, 3].tolist()
        assert np.array_equal(_bits(lg[7]), _bits(lg[3]))
        one = q4hip.Batch(g, 1)
        for b in (0, 3, 31):
            f1 = one.prefill(0, prompts[b], 0)
            o1 = one.generate([f1], [P], steps)
            assert f1 == first[b] and o1[:, 0].tolist() == out[:, b].tolist(), f"sequence {b}"
            _same_logits(one.read_logits()[0], lg[b], f"sequence {b}")
        one.close()
    finally:
        g.close()


def test_batch_qwen15b_prefilled_1024():
    """The batched-decode configuration's shape and cache length (Qwen2.5-1.5B, 1024 cached positions
    per sequence written through q4hip_batch_set_kv, different contents and positions): every
    sequence's tokens and last logits equal the oracle's over the same cache."""
    import q4hip
    shape = synth.SHAPES["qwen2.5-1.5b"]
    t = _model("qwen2.5-1.5b", 50)
    P, B, ctx, steps = 1024, 4, 1040, 2
    print(f"qwen15b batch of {B}, {P}-position caches", flush=True)
    g = q4hip.Model(shape, ctx=ctx)
    g.load(t)
    o = oracle.Model(shape, t, ctx=ctx, mt=16, threads=16)
    bt = q4hip.Batch(g, B)
    try:
        caches = []
        for b in range(B):
            r = np.random.default_rng(200 + b)
            k = r.standard_normal((shape.layers, shape.kv_heads, P, shape.head_dim)).astype(np.float16).astype(np.float32)
            v = r.standard_normal((shape.layers, shape.kv_heads, P, shape.head_dim)).astype(np.float16).astype(np.float32)
            caches.append((k, v))
            for l in range(shape.layers):
                for kh in range(shape.kv_heads):
                    bt.set_kv(b, l, kh, 0, k[l, kh], v[l, kh])
        first = [5, 17, 900, 4242]
        pos = [P, P - 1, P - 100, P - 511]
        out = bt.generate(first, pos, steps)
        lg = bt.read_logits()
        for b in range(B):
            ok, ov = o.kv()
            ok[:, :, :P] = caches[b][0]
            ov[:, :, :P] = caches[b][1]
            tok = first[b]
            for i in range(steps):
                tok = o.forward([tok], pos[b] + i)
                assert out[i, b] == tok, f"sequence {b} step {i}"
            _same_logits(lg[b], o.logits(), f"sequence {b}")
    finally:
        bt.close()
        g.close()
        o.close()


def _seq_cache(shape, P, seed):
    """K and V rows [layers][kv_heads][P][head_dim] of one sequence: fp16-valued N(0, 1)."""
    r = np.random.default_rng(seed)
    dims = (shape.layers, shape.kv_heads, P, shape.head_dim)
    k = r.standard_normal(dims, dtype=np.float32).astype(np.float16).astype(np.float32)
    v = r.standard_normal(dims, dtype=np.float32).astype(np.float16).astype(np.float32)
    return k, v


def test_batch_qwen15b_b32_ctx1024():
    """The batched-decode configuration as defined: Qwen2.5-1.5B shape, 32 sequences, each with its
    own cache of about 1024 positions (different contents, written through q4hip_batch_set_kv) and
    its own position (ragged: 1024 down to 725), then 3 greedy steps of all 32 together.  Every
    sequence's tokens and last-step logits equal the oracle's, run one sequence at a time over the
    same cache (engine/llm.js:86-97, engine/kernels.c:355-377)."""
    import q4hip
    shape = synth.SHAPES["qwen2.5-1.5b"]
    t = _model("qwen2.5-1.5b", 51)
    P, B, ctx, steps = 1024, 32, 1040, 3
    pos = [P - (b * 37) % 300 for b in range(B)]
    first = [int(x) for x in np.random.default_rng(51).integers(0, shape.vocab, B)]
    print(f"qwen15b batch of {B}, {P}-position caches, positions {min(pos)}..{max(pos)}", flush=True)
    g = q4hip.Model(shape, ctx=ctx)
    g.load(t)
    bt = q4hip.Batch(g, B)
    o = None
    try:
        for b in range(B):
            k, v = _seq_cache(shape, P, 300 + b)
            for l in range(shape.layers):
                for kh in range(shape.kv_heads):
                    bt.set_kv(b, l, kh, 0, k[l, kh], v[l, kh])
        out = bt.generate(first, pos, steps)
        lg = bt.read_logits()
        print("batch done; oracle per sequence", flush=True)
        o = oracle.Model(shape, t, ctx=ctx, mt=16, threads=16)
        for b in range(B):
            k, v = _seq_cache(shape, P, 300 + b)
            ok, ov = o.kv()
            ok[:, :, :P] = k
            ov[:, :, :P] = v
            tok = first[b]
            for i in range(steps):
                tok = o.forward([tok], pos[b] + i)
                assert out[i, b] == tok, f"sequence {b} step {i}"
            _same_logits(lg[b], o.logits(), f"sequence {b}")
    finally:
        bt.close()
        g.close()
        if o is not None:
            o.close()


def test_batch_qwen15b_b32_ctx1024_fp16():
    """The batched-decode configuration with the fp16 cache: Qwen2.5-1.5B shape, 32 sequences with
    their own ~1024-position caches (written through q4hip_batch_set_kv), 3 steps of all 32.  Every
    sequence's tokens and last logits equal, bit for bit, the oracle's over a cache holding the same
    fp16-rounded values (ORC_V_KV_F16), run one sequence at a time."""
    import q4hip
    shape = synth.SHAPES["qwen2.5-1.5b"]
    t = _model("qwen2.5-1.5b", 51)
    P, B, ctx, steps = 1024, 32, 1040, 3
    pos = [P - (b * 37) % 300 for b in range(B)]
    first = [int(x) for x in np.random.default_rng(52).integers(0, shape.vocab, B)]
    print(f"qwen15b batch of {B}, {P}-position fp16 caches", flush=True)
    g = q4hip.Model(shape, ctx=ctx, kv_type=q4hip.KV_F16)
    g.load(t)
    bt = q4hip.Batch(g, B)
    o = None
    try:
        for b in range(B):
            k, v = _seq_cache(shape, P, 400 + b)
            for l in range(shape.layers):
                for kh in range(shape.kv_heads):
                    bt.set_kv(b, l, kh, 0, k[l, kh], v[l, kh])
        out = bt.generate(first, pos, steps)
        lg = bt.read_logits()
        print("batch done; oracle per sequence", flush=True)
        o = oracle.Model(shape, t, ctx=ctx, mt=16, threads=16)
        o.set_variant(oracle.V_KV_F16)
        for b in range(B):
            k, v = _seq_cache(shape, P, 400 + b)
            ok, ov = o.kv()
            ok[:, :, :P] = k
            ov[:, :, :P] = v
            tok = first[b]
            for i in range(steps):
                tok = o.forward([tok], pos[b] + i)
                assert out[i, b] == tok, f"sequence {b} step {i}"
            _same_logits(lg[b], o.logits(), f"sequence {b}")
    finally:
        bt.close()
        g.close()
        if o is not None:
            o.close()
