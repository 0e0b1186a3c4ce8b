"""Seeded synthetic Qwen2-shaped models in GGUF Q4_0, and a minimal GGUF v3 writer/reader.

There is no network and no checkpoint, so every weight is random: matrices, embedding, head and
the q/k/v biases are N(0, 0.02) fp32, quantized to GGUF Q4_0 (32 values per block, fp16 scale);
norm weights are 1.0.  Each tensor has its own PCG64 stream keyed by (seed, crc32(name)), so a
tensor does not change when the model around it does.

Tensor names, shapes and metadata keys are the ones the reference engine reads from a real
Qwen2 GGUF file (h2-own-inference-engine/engine/gguf.js:72-88, engine/cpu-worker.js:57-128).
"""
from __future__ import annotations

import concurrent.futures
import dataclasses
import math
import os
import struct
import zlib

import numpy as np

GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0 = 0, 1, 2, 8
BLOCK = {GGML_Q4_0: (32, 18), GGML_Q8_0: (32, 34), GGML_F32: (1, 4), GGML_F16: (1, 2)}


@dataclasses.dataclass(frozen=True)
class Shape:
    dim: int
    layers: int
    ffn: int
    heads: int
    kv_heads: int
    vocab: int
    eps: float = 1e-6
    rope_theta: float = 1e6
    context_length: int = 32768

    @property
    def head_dim(self) -> int:
        return self.dim // self.heads

    @property
    def qkv(self) -> int:
        return self.dim + 2 * self.kv_heads * self.head_dim


SHAPES = {
    # Qwen2.5-0.5B: hidden 896, 24 layers, 14 q-heads / 2 kv-heads, head_dim 64, FFN 4864
    "qwen2.5-0.5b": Shape(896, 24, 4864, 14, 2, 151936),
    # Qwen2.5-1.5B: hidden 1536, 28 layers, 12 q-heads / 2 kv-heads, head_dim 128, FFN 8960
    "qwen2.5-1.5b": Shape(1536, 28, 8960, 12, 2, 151936),
    # small shapes for fast tests, same head_dim families (64 and 128)
    "tiny": Shape(128, 2, 256, 2, 1, 512),
    "small": Shape(256, 3, 512, 4, 1, 4096),
    "small128": Shape(256, 2, 512, 2, 1, 1024),
}


# ---------------------------------------------------------------------------- quantizers

def quantize_q4_0(x: np.ndarray) -> np.ndarray:
    """GGUF Q4_0 of float32 values (length a multiple of 32) -> uint8 [nblocks, 18].

    Block rule of the GGUF format: the value of largest magnitude (first one on ties) is max,
    d = max / -8, q = min(15, trunc(x/d + 8.5)), stored d as fp16; byte j of the 16 value bytes
    holds q[j] in its low nibble and q[16+j] in its high nibble.
    """
    b = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, 32)
    idx = np.argmax(np.abs(b), axis=1)
    mx = b[np.arange(b.shape[0]), idx]
    d = (mx / np.float32(-8.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, np.float32(1.0)), np.float32(0.0)).astype(np.float32)
    v = b * inv[:, None] + np.float32(8.5)
    q = np.minimum(np.trunc(v).astype(np.int32), 15).astype(np.uint8)
    out = np.empty((b.shape[0], 18), dtype=np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q[:, :16] | (q[:, 16:] << 4)
    return out


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    """GGUF Q8_0 of float32 values (length a multiple of 32) -> uint8 [nblocks, 34].

    Block rule of the GGUF format: amax = max |x|, d = amax / 127, q = round(x / d) with halves
    away from zero (computed as x * (1/d)), d stored as fp16 in the first two bytes.
    """
    b = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, 32)
    amax = np.max(np.abs(b), axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, np.float32(1.0)), np.float32(0.0)).astype(np.float32)
    v = b * inv[:, None]
    q = (np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))).astype(np.int32)
    q = np.clip(q, -127, 127).astype(np.int8)
    out = np.empty((b.shape[0], 34), dtype=np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out


def dequantize_q8_0(raw: np.ndarray) -> np.ndarray:
    raw = raw.reshape(-1, 34)
    d = raw[:, 0:2].copy().view(np.float16).reshape(-1).astype(np.float32)
    return (raw[:, 2:].copy().view(np.int8).astype(np.float32) * d[:, None]).reshape(-1)


def q4_0_blocks(raw: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """uint8 [nb,18] -> (nibble bytes [nb,16], fp32 scales [nb]), as copyBlocks does
    (engine/cpu-worker.js:97-104)."""
    raw = raw.reshape(-1, 18)
    return np.ascontiguousarray(raw[:, 2:]), raw[:, 0:2].copy().view(np.float16).reshape(-1).astype(np.float32)


def dequantize_q4_0(raw: np.ndarray) -> np.ndarray:
    qs, d = q4_0_blocks(raw)
    lo = (qs & 15).astype(np.int32) - 8
    hi = (qs >> 4).astype(np.int32) - 8
    vals = np.concatenate([lo, hi], axis=1).astype(np.float32)
    return (vals * d[:, None]).reshape(-1)


def q4_to_q8_0(raw: np.ndarray) -> np.ndarray:
    """Lossless Q8_0 re-encoding of Q4_0 blocks: same fp16 scale, int8 = nibble - 8."""
    raw = raw.reshape(-1, 18)
    qs = raw[:, 2:]
    vals = np.concatenate([(qs & 15).astype(np.int16) - 8, (qs >> 4).astype(np.int16) - 8], axis=1)
    out = np.empty((raw.shape[0], 34), dtype=np.uint8)
    out[:, 0:2] = raw[:, 0:2]
    out[:, 2:] = vals.astype(np.int8).view(np.uint8)
    return out


# ---------------------------------------------------------------------------- generator

def _rng(seed: int, name: str) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64([seed & 0xFFFFFFFF, zlib.crc32(name.encode())]))


def _normal_q(seed: int, name: str, count: int, quant, std: float = 0.02, chunk: int = 1 << 24) -> np.ndarray:
    rng = _rng(seed, name)
    parts = []
    done = 0
    while done < count:
        n = min(chunk, count - done)
        parts.append(quant(rng.standard_normal(n, dtype=np.float32) * np.float32(std)))
        done += n
    return np.concatenate(parts) if len(parts) > 1 else parts[0]


def _normal_q4(seed: int, name: str, count: int, std: float = 0.02) -> np.ndarray:
    return _normal_q(seed, name, count, quantize_q4_0, std)


@dataclasses.dataclass
class Tensor:
    name: str
    dims: tuple          # GGUF order: dims[0] = row length
    type: int
    data: np.ndarray     # uint8 blocks (quantized) or float32 values

    @property
    def rows(self) -> int:
        n = 1
        for d in self.dims[1:]:
            n *= d
        return n

    def raw_bytes(self) -> bytes:
        return self.data.tobytes()


def make_model(shape: Shape, seed: int = 1234, head_type: int = GGML_Q4_0, workers: int = 0) -> dict:
    """All tensors of a synthetic Qwen2 model, keyed by GGUF tensor name.  head_type GGML_Q8_0
    gives the output head the type real Qwen2.5 GGUF files use.  Tensors are generated on
    `workers` threads (0: up to 8); each has its own stream, so the result does not depend on it."""
    D, F, KV = shape.dim, shape.ffn, shape.kv_heads * shape.head_dim
    jobs = []   # (name, dims, type, thunk) in GGUF order

    def q4(name, k, n):
        jobs.append((name, (k, n), GGML_Q4_0, lambda: _normal_q4(seed, name, k * n)))

    def f32(name, n, value=None):
        def make():
            data = np.full(n, value, dtype=np.float32) if value is not None else \
                _rng(seed, name).standard_normal(n, dtype=np.float32) * np.float32(0.02)
            return data.astype(np.float32)
        jobs.append((name, (n,), GGML_F32, make))

    q4("token_embd.weight", D, shape.vocab)
    for layer in range(shape.layers):
        p = f"blk.{layer}."
        f32(p + "attn_norm.weight", D, 1.0)
        q4(p + "attn_q.weight", D, D)
        q4(p + "attn_k.weight", D, KV)
        q4(p + "attn_v.weight", D, KV)
        f32(p + "attn_q.bias", D)
        f32(p + "attn_k.bias", KV)
        f32(p + "attn_v.bias", KV)
        q4(p + "attn_output.weight", D, D)
        f32(p + "ffn_norm.weight", D, 1.0)
        q4(p + "ffn_gate.weight", D, F)
        q4(p + "ffn_up.weight", D, F)
        q4(p + "ffn_down.weight", F, D)
    f32("output_norm.weight", D, 1.0)
    if head_type == GGML_Q8_0:
        jobs.append(("output.weight", (D, shape.vocab), GGML_Q8_0,
                     lambda: _normal_q(seed, "output.weight", D * shape.vocab, quantize_q8_0)))
    else:
        q4("output.weight", D, shape.vocab)
    n = workers if workers > 0 else min(8, os.cpu_count() or 1)
    if n > 1:
        with concurrent.futures.ThreadPoolExecutor(n) as pool:
            data = list(pool.map(lambda j: j[3](), jobs))
    else:
        data = [j[3]() for j in jobs]
    return {name: Tensor(name, dims, typ, d) for (name, dims, typ, _), d in zip(jobs, data)}


def prompt_ids(seed: int, n: int, vocab: int) -> list:
    """Seeded uniform-random prompt ids in [0, vocab)."""
    return [int(v) for v in _rng(seed, "prompt").integers(0, vocab, size=n)]


def rope_table(ctx: int, head_dim: int, theta: float) -> np.ndarray:
    """fp32 [ctx][head_dim/2][2] of cos/sin(pos / theta^(2i/head_dim)) computed in double with the
    C library's pow/cos/sin, then rounded to fp32 (engine/cpu-worker.js:130-135)."""
    half = head_dim // 2
    inv = [math.pow(theta, (2.0 * i) / head_dim) for i in range(half)]
    out = np.empty((ctx, half, 2), dtype=np.float64)
    for pos in range(ctx):
        for i in range(half):
            a = pos / inv[i]
            out[pos, i, 0] = math.cos(a)
            out[pos, i, 1] = math.sin(a)
    return out.astype(np.float32)


# ---------------------------------------------------------------------------- GGUF v3 I/O

_GGUF_MAGIC = 0x46554747


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


# ---------------------------------------------------------------------------- tokenizer

CONTROL_TOKEN = 3
SPECIALS = ["<|endoftext|>", "<|im_start|>", "<|im_end|>"]
_CORPUS = (
    "The quick brown fox jumps over the lazy dog. It's a sunny day; we're going to the park, "
    "aren't we? She'll read 3 books and 12 poems in 2024. Numbers like 42, 7 and 1000 appear often.\n"
    "Caf\u00e9 cr\u00e8me br\u00fbl\u00e9e, na\u00efve r\u00e9sum\u00e9, \u00fcber stra\u00dfe. "
    "\u4f60\u597d\uff0c\u4e16\u754c\uff01 \u3053\u3093\u306b\u3061\u306f "
    "\u041f\u0440\u0438\u0432\u0435\u0442 \U0001f600\U0001f680 hello world\n\n"
    "You are a helpful assistant. The user asks a question and the assistant answers it. "
    "system user assistant hello hello hello the the the and and of of to to in in is is it it\n"
)


def byte_chars() -> list:
    """GPT-2's printable stand-in for each byte value (printable Latin-1 bytes stand for themselves,
    the other 68 take code points 256, 257, ... in byte order)."""
    printable = lambda b: 33 <= b <= 126 or 161 <= b <= 172 or 174 <= b <= 255  # noqa: E731
    out, extra = [], 0
    for b in range(256):
        if printable(b):
            out.append(chr(b))
        else:
            out.append(chr(256 + extra))
            extra += 1
    return out


def make_tokenizer(vocab: int, seed: int = 0) -> dict:
    """A byte-level BPE tokenizer in GGUF form for a synthetic model of `vocab` ids: the 256 byte
    symbols, merges learned greedily from a small built-in multilingual corpus, the three ChatML
    special tokens, and reserved control tokens up to `vocab`.  Deterministic (`seed` only names the
    reserved tokens).  Returns {tokens, token_type, merges, eos}."""
    import regex
    split = regex.compile(r"""(?:'[sS]|'[tT]|'[rR][eE]|'[vV][eE]|'[mM]|'[lL][lL]|'[dD])|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+""")
    bc = byte_chars()
    words = {}
    for piece in split.findall(_CORPUS):
        w = tuple(bc[b] for b in piece.encode("utf-8"))
        words[w] = words.get(w, 0) + 1
    tokens = list(bc)
    n_merges = max(0, vocab - 256 - len(SPECIALS) - 8)
    merges = []
    while len(merges) < n_merges:
        pairs = {}
        for w, c in words.items():
            for a, b in zip(w, w[1:]):
                pairs[(a, b)] = pairs.get((a, b), 0) + c
        if not pairs:
            break
        (a, b), _ = max(pairs.items(), key=lambda kv: (kv[1], kv[0]))
        merges.append(f"{a} {b}")
        tokens.append(a + b)
        nw = {}
        for w, c in words.items():
            out, i = [], 0
            while i < len(w):
                if i + 1 < len(w) and w[i] == a and w[i + 1] == b:
                    out.append(a + b)
                    i += 2
                else:
                    out.append(w[i])
                    i += 1
            nw[tuple(out)] = nw.get(tuple(out), 0) + c
        words = nw
    types = [1] * len(tokens)
    for sp in SPECIALS:
        tokens.append(sp)
        types.append(CONTROL_TOKEN)
    k = 0
    while len(tokens) < vocab:
        tokens.append(f"<|reserved_{seed}_{k}|>")
        types.append(CONTROL_TOKEN)
        k += 1
    if len(tokens) > vocab:
        raise ValueError(f"vocab {vocab} too small for the tokenizer")
    return {"tokens": tokens, "token_type": types, "merges": merges, "eos": tokens.index("<|im_end|>")}


def write_gguf(path: str, shape: Shape, tensors: dict, align: int = 32, tokenizer: dict = None) -> None:
    """Write a GGUF v3 file with the Qwen2 metadata the reference's qwen2Config reads; with
    `tokenizer` (make_tokenizer) also its vocabulary, token types and merges."""
    meta = [
        ("general.architecture", 8, "qwen2"),
        ("general.alignment", 4, align),
        ("qwen2.embedding_length", 4, shape.dim),
        ("qwen2.block_count", 4, shape.layers),
        ("qwen2.feed_forward_length", 4, shape.ffn),
        ("qwen2.attention.head_count", 4, shape.heads),
        ("qwen2.attention.head_count_kv", 4, shape.kv_heads),
        ("qwen2.rope.freq_base", 6, shape.rope_theta),
        ("qwen2.attention.layer_norm_rms_epsilon", 6, shape.eps),
        ("qwen2.context_length", 4, shape.context_length),
        ("tokenizer.ggml.eos_token_id", 4, tokenizer["eos"] if tokenizer else shape.vocab - 1),
    ]
    kv = bytearray()
    for k, typ, v in meta:
        kv += _str(k) + struct.pack("<I", typ)
        if typ == 8:
            kv += _str(v)
        elif typ == 4:
            kv += struct.pack("<I", v)
        elif typ == 6:
            kv += struct.pack("<f", v)
    names = tokenizer["tokens"] if tokenizer else [f"t{i}" for i in range(shape.vocab)]
    kv += _str("tokenizer.ggml.tokens") + struct.pack("<IIQ", 9, 8, len(names))
    kv += b"".join(_str(t) for t in names)
    n_kv = len(meta) + 1
    if tokenizer:
        kv += _str("tokenizer.ggml.token_type") + struct.pack("<IIQ", 9, 5, len(tokenizer["token_type"]))
        kv += b"".join(struct.pack("<i", t) for t in tokenizer["token_type"])
        kv += _str("tokenizer.ggml.merges") + struct.pack("<IIQ", 9, 8, len(tokenizer["merges"]))
        kv += b"".join(_str(m) for m in tokenizer["merges"])
        n_kv += 2

    infos = bytearray()
    offset = 0
    order = list(tensors.values())
    offsets = []
    for t in order:
        nbytes = t.data.nbytes
        infos += _str(t.name) + struct.pack("<I", len(t.dims)) + b"".join(struct.pack("<Q", d) for d in t.dims)
        infos += struct.pack("<IQ", t.type, offset)
        offsets.append(offset)
        offset += (nbytes + align - 1) // align * align
    header = struct.pack("<IIQQ", _GGUF_MAGIC, 3, len(order), n_kv) + bytes(kv) + bytes(infos)
    pad = (-len(header)) % align
    with open(path, "wb") as f:
        f.write(header + b"\0" * pad)
        for t, off in zip(order, offsets):
            b = t.raw_bytes()
            f.write(b)
            f.write(b"\0" * ((-len(b)) % align))


def read_gguf(path: str) -> tuple:
    """(meta, {name: (dims, type, offset_in_file, nbytes)}) of a GGUF file (engine/gguf.js:15-69)."""
    data = np.memmap(path, dtype=np.uint8, mode="r")
    p = [0]

    def rd(fmt):
        n = struct.calcsize(fmt)
        v = struct.unpack(fmt, data[p[0]:p[0] + n].tobytes())
        p[0] += n
        return v

    def s():
        (n,) = rd("<Q")
        b = bytes(data[p[0]:p[0] + n])
        p[0] += n
        return b.decode()

    def val(t):
        if t in (0, 1, 7):
            return rd("<" + "BbB"[[0, 1, 7].index(t)])[0]
        if t in (2, 3):
            return rd("<" + "Hh"[t - 2])[0]
        if t in (4, 5, 6):
            return rd("<" + "Iif"[t - 4])[0]
        if t == 8:
            return s()
        if t == 9:
            et, n = rd("<IQ")
            return [val(et) for _ in range(n)]
        if t in (10, 11, 12):
            return rd("<" + "Qqd"[t - 10])[0]
        raise ValueError(f"unknown GGUF value type {t}")

    magic, version, nt, nkv = rd("<IIQQ")
    if magic != _GGUF_MAGIC:
        raise ValueError("not a GGUF file")
    meta = {}
    for _ in range(nkv):
        k = s()
        (t,) = rd("<I")
        meta[k] = val(t)
    infos = {}
    for _ in range(nt):
        name = s()
        (nd,) = rd("<I")
        dims = rd("<" + "Q" * nd)
        typ, off = rd("<IQ")
        infos[name] = [tuple(dims), typ, off]
    align = meta.get("general.alignment", 32)
    start = (p[0] + align - 1) // align * align
    out = {}
    for name, (dims, typ, off) in infos.items():
        count = 1
        for d in dims:
            count *= d
        per, nbytes = BLOCK[typ]
        out[name] = (dims, typ, start + off, count // per * nbytes)
    return meta, out
