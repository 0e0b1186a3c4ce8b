"""The Node.js host (engine/gguf.js, engine/hip.js, engine/llm.js) driven through tests/js/cli.js.

CPU: GGUF parsing and Qwen2 config match what the file holds; type checks throw the reference's
messages before the GPU is touched; sampling follows cpu-worker.js.  GPU: LLM.generateIds through
the N-API addon gives the oracle's tokens and logits.
"""
import json
import os
import struct
import subprocess

import numpy as np
import pytest

import synth

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(REPO, "tests", "js", "cli.js")


def node(*args, timeout=300):
    r = subprocess.run(["node", CLI, *map(str, args)], capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout)


@pytest.fixture(scope="module")
def tiny_gguf(tmp_path_factory):
    shape = synth.SHAPES["tiny"]
    t = synth.make_model(shape, 77)
    p = str(tmp_path_factory.mktemp("m") / "tiny.gguf")
    synth.write_gguf(p, shape, t)
    return shape, t, p


def test_parse_matches_file(tiny_gguf):
    shape, t, p = tiny_gguf
    r = node("parse", p)
    cfg = r["cfg"]
    assert cfg["arch"] == "qwen2" and cfg["dim"] == shape.dim and cfg["layers"] == shape.layers
    assert cfg["ffn"] == shape.ffn and cfg["heads"] == shape.heads and cfg["kvHeads"] == shape.kv_heads
    assert cfg["vocab"] == shape.vocab and cfg["eos"] == shape.vocab - 1
    assert cfg["ropeTheta"] == shape.rope_theta and abs(cfg["eps"] - shape.eps) < 1e-12
    _, infos = synth.read_gguf(p)
    for name, (typ, shp, start, nbytes) in r["tensors"].items():
        dims, typ2, off, nb2 = infos[name]
        assert typ == typ2 and tuple(shp) == tuple(dims) and start == off and nbytes == nb2


def test_wrong_tensor_type_rejected_before_gpu(tmp_path):
    shape = synth.SHAPES["tiny"]
    t = synth.make_model(shape, 3)
    bad = dict(t)
    w = t["blk.1.ffn_up.weight"]
    bad["blk.1.ffn_up.weight"] = synth.Tensor(w.name, w.dims, synth.GGML_Q8_0, synth.q4_to_q8_0(w.data))
    p = str(tmp_path / "bad.gguf")
    synth.write_gguf(p, shape, bad)
    r = node("load", p, 64)
    assert r["error"] == "blk.1.ffn_up.weight: expected Q4_0"
    bad = dict(t)
    n = t["blk.0.attn_norm.weight"]
    bad["blk.0.attn_norm.weight"] = synth.Tensor(n.name, n.dims, synth.GGML_F16, n.data.astype(np.float16))
    synth.write_gguf(p, shape, bad)
    assert node("load", p, 64)["error"] == "blk.0.attn_norm.weight: expected F32"


def test_not_a_gguf(tmp_path):
    p = tmp_path / "x.gguf"
    p.write_bytes(struct.pack("<IIQQ", 0x12345678, 3, 0, 0))
    assert node("load", str(p), 64)["error"] == "not a GGUF file"


def test_sampling_follows_reference(tmp_path):
    """Greedy = first maximum; temperature > 0 is deterministic in the seed (cpu-worker.js:154-167)."""
    lg = np.random.default_rng(0).standard_normal(5000).astype(np.float32)
    lg[[10, 20]] = 9.0
    p = tmp_path / "lg.f32"
    p.write_bytes(lg.tobytes())
    assert node("sample", p, 0, 1)["id"] == 10
    a, b = node("sample", p, 0.8, 42)["id"], node("sample", p, 0.8, 42)["id"]
    assert a == b and 0 <= a < 5000


@pytest.mark.gpu
def test_generate_through_napi_matches_oracle(tiny_gguf, tmp_path):
    import oracle
    shape, t, p = tiny_gguf
    ids = synth.prompt_ids(77, 25, shape.vocab)
    (tmp_path / "ids.json").write_text(json.dumps(ids))
    out = node("generate", p, 128, tmp_path / "ids.json", 20, tmp_path / "lg.f32")
    o = oracle.Model(shape, t, ctx=128)
    ref = o.generate(ids, 20)
    assert out["tokens"] == ref and out["device"] == ref
    lg = np.frombuffer((tmp_path / "lg.f32").read_bytes(), np.float32)
    assert np.array_equal(lg.view(np.uint32), o.logits().view(np.uint32))
    assert out["ctxError"] == "context full"
    o.close()


@pytest.mark.gpu
def test_q8_head_through_napi_matches_oracle(tmp_path):
    """A GGUF with a Q8_0 output head, the type real Qwen2.5 files carry, loads through createHIP
    and decodes to the oracle's tokens and logits."""
    import oracle
    shape = synth.SHAPES["tiny"]
    t = synth.make_model(shape, 78, head_type=synth.GGML_Q8_0)
    p = str(tmp_path / "q8head.gguf")
    synth.write_gguf(p, shape, t)
    ids = synth.prompt_ids(78, 17, shape.vocab)
    (tmp_path / "ids.json").write_text(json.dumps(ids))
    out = node("generate", p, 128, tmp_path / "ids.json", 12, tmp_path / "lg.f32")
    o = oracle.Model(shape, t, ctx=128)
    ref = o.generate(ids, 12)
    assert out["tokens"] == ref and out["device"] == ref
    lg = np.frombuffer((tmp_path / "lg.f32").read_bytes(), np.float32)
    assert np.array_equal(lg.view(np.uint32), o.logits().view(np.uint32))
    o.close()
