"""CPU checks of the native boundary: the C-ABI library and the N-API addon load and export what
include/q4hip.h declares; the Python binding refuses to run without the HIP library; GGUF I/O."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import q4hip
import synth

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "q4hip.h")
ADDON = os.path.join(REPO, "e2e-browser-voice-agent_amd", "lib", "q4hip.node")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\**\s*(q4hip_[a-z_0-9]+)\s*\(", text, re.M)))


def test_header_declarations_found():
    names = declared()
    assert "q4hip_create" in names and "q4hip_forward" in names and len(names) >= 15


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(q4hip.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(declared()) == set(q4hip.EXPORTS)


def test_last_error_without_calls():
    q4hip.lib()
    assert q4hip.lib().q4hip_last_error() == b""


def test_binding_fails_loudly_without_library(monkeypatch):
    monkeypatch.setattr(q4hip, "_lib", None)
    monkeypatch.setattr(q4hip, "LIB_PATH", "/nonexistent/libq4hip.so")
    with pytest.raises(RuntimeError, match="not built"):
        q4hip.lib()


def test_addon_loads_and_exports():
    out = subprocess.run(["node", "-e", f"const a = require({ADDON!r}); console.log(Object.keys(a).sort().join(','))"],
                         capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stderr
    keys = out.stdout.strip().split(",")
    for k in ["create", "destroy", "setTensor", "setRope", "forward", "readLogits", "generate", "profile", "deviceCount",
              "setKv", "setDecodeMode", "decodeModeUsed", "batchCreate", "batchDestroy", "batchPrefill", "batchSetKv",
              "batchGenerate", "batchReadLogits"]:
        assert k in keys


def test_addon_rejects_bad_handles():
    js = f"""
    const a = require({ADDON!r});
    let msgs = [];
    try {{ a.forward({{}}, new Int32Array([1]), 0); }} catch (e) {{ msgs.push(e.message); }}
    try {{ a.create(1, 2); }} catch (e) {{ msgs.push(e.message); }}
    console.log(JSON.stringify(msgs));
    """
    out = subprocess.run(["node", "-e", js], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stderr
    assert "expected a q4hip handle" in out.stdout and "10 arguments" in out.stdout


def test_gguf_roundtrip(tmp_path):
    shape = synth.SHAPES["tiny"]
    t = synth.make_model(shape, 5)
    path = str(tmp_path / "m.gguf")
    synth.write_gguf(path, shape, t)
    meta, infos = synth.read_gguf(path)
    assert meta["general.architecture"] == "qwen2"
    assert meta["qwen2.embedding_length"] == shape.dim and meta["qwen2.block_count"] == shape.layers
    assert len(meta["tokenizer.ggml.tokens"]) == shape.vocab
    raw = np.memmap(path, dtype=np.uint8, mode="r")
    for name, tensor in t.items():
        dims, typ, off, nbytes = infos[name]
        assert tuple(dims) == tuple(tensor.dims) and typ == tensor.type
        assert np.array_equal(raw[off:off + nbytes], np.frombuffer(tensor.raw_bytes(), np.uint8))
        assert off % 32 == 0


def test_synthetic_model_is_deterministic():
    shape = synth.SHAPES["tiny"]
    a, b = synth.make_model(shape, 9), synth.make_model(shape, 9)
    c = synth.make_model(shape, 10)
    for n in a:
        assert np.array_equal(a[n].data, b[n].data)
    assert not np.array_equal(a["output.weight"].data, c["output.weight"].data)
    assert synth.prompt_ids(3, 64, 151936) == synth.prompt_ids(3, 64, 151936)


@pytest.mark.parametrize("kv_f16", [False, True])
@pytest.mark.parametrize("ring_slots", [3, 7])
@pytest.mark.parametrize("split,half", [(False, 0), (True, 0), (True, 1)])
@pytest.mark.parametrize("kv_tile", [0, 140, 192])
def test_attention_ring_reads_only_past_rows(kv_tile, split, half, ring_slots, kv_f16):
    """Every row the attention role's ring loads read is a past position (< pos), at every position
    of a 4200-position context: the loads past a stream's end are redirected to its last row, not to
    ctx - 1 (rows at and past pos are written during the step by the K/V role, possibly on another
    XCD; the reference reads exactly pos + 1 positions, engine/kernels.c:355-360)."""
    if split and kv_tile:
        pytest.skip("the split pair stages no tile")
    for pos in range(0, 4201):
        lo, hi, n = q4hip.attn_ring_rows(pos, kv_tile, ring_slots, split, half, kv_f16)
        if n == 0:
            continue
        assert 0 <= lo <= hi < pos, (pos, lo, hi, n)


def test_attention_ring_bound_is_tight():
    """The clamp is exercised: near a stream's end the ring still loads (the last row read is
    exactly pos - 1), and positions past the staged tile are all streamed."""
    lo, hi, n = q4hip.attn_ring_rows(1000, 140, 7, False, 0, False)
    assert n > 0 and hi == 999 and lo == 140
    lo, hi, n = q4hip.attn_ring_rows(100, 140, 7, False, 0, False)
    assert n == 0          # everything staged
    lo, hi, n = q4hip.attn_ring_rows(4096, 0, 7, True, 1, True)
    assert n > 0 and hi == 4095
