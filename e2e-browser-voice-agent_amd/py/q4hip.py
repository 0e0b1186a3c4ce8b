"""ctypes binding of the q4hip C ABI (include/q4hip.h) for Python callers: the tests and bench.py.

The JavaScript backend (engine/hip.js) is the product's host; this module exposes the same C ABI
to Python.  It loads the in-tree libq4hip.so and fails loudly when it is missing: there is no
CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
import weakref

import numpy as np

import synth

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "lib", "libq4hip.so")

OK, EINVAL, ECONTEXT, ETYPE, EHIP, ESTATE = 0, 1, 2, 3, 4, 5
DECODE_AUTO, DECODE_GRAPH, DECODE_PERSISTENT = 0, 1, 2
KV_F32, KV_F16 = 0, 1
NOALLOC_MAX_K = 65536          # include/q4hip.h Q4HIP_NOALLOC_MAX_K
PROF_NAMES = ["embed", "norm+quantize", "matvec qkv", "rope+kv", "attention", "quantize", "matvec o",
              "matvec gate+up", "swiglu+quantize", "matvec down", "matvec output", "sample"]

EXPORTS = [
    "q4hip_last_error", "q4hip_device_count", "q4hip_create", "q4hip_set_tensor", "q4hip_set_rope",
    "q4hip_forward", "q4hip_read_logits", "q4hip_generate", "q4hip_profile", "q4hip_time_generate",
    "q4hip_time_head", "q4hip_destroy", "q4hip_mv_create", "q4hip_mv_run", "q4hip_mv_time",
    "q4hip_mv_destroy", "q4hip_set_decode_mode", "q4hip_decode_mode_used", "q4hip_profile_persistent",
    "q4hip_set_kv", "q4hip_profile_pass", "q4hip_batch_create", "q4hip_batch_destroy",
    "q4hip_batch_prefill", "q4hip_batch_set_kv", "q4hip_batch_generate", "q4hip_batch_time_generate",
    "q4hip_batch_read_logits", "q4hip_mv_time_cold", "q4hip_check_division", "q4hip_mv_run_noalloc",
    "q4hip_attn_ring_rows",
]

_lib = None


class Q4Error(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build() first")
    L = ctypes.CDLL(LIB_PATH)
    P, I, I64, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
    sig = {
        "q4hip_last_error": (ctypes.c_char_p, []),
        "q4hip_device_count": (I, [ctypes.POINTER(I)]),
        "q4hip_check_division": (I, [I, P, I]),
        "q4hip_create": (I, [ctypes.POINTER(P), I, I, I, I, I, I, I, I, F, I, I]),
        "q4hip_set_tensor": (I, [P, I, I, I, I, P, I64, ctypes.c_size_t]),
        "q4hip_set_rope": (I, [P, P, I64]),
        "q4hip_forward": (I, [P, P, I, I, ctypes.POINTER(I)]),
        "q4hip_read_logits": (I, [P, P, I]),
        "q4hip_generate": (I, [P, I, I, I, P]),
        "q4hip_profile": (I, [P, I, I, P, I]),
        "q4hip_time_generate": (I, [P, I, I, I, P, ctypes.POINTER(F)]),
        "q4hip_time_head": (I, [P, I, ctypes.POINTER(F)]),
        "q4hip_destroy": (None, [P]),
        "q4hip_mv_create": (I, [ctypes.POINTER(P), I, I, P, I]),
        "q4hip_mv_run": (I, [P, P, P]),
        "q4hip_mv_time": (I, [P, I, ctypes.POINTER(F)]),
        "q4hip_mv_destroy": (None, [P]),
        "q4hip_set_decode_mode": (I, [P, I]),
        "q4hip_decode_mode_used": (I, [P, ctypes.POINTER(I)]),
        "q4hip_profile_persistent": (I, [P, I, I, P, I]),
        "q4hip_set_kv": (I, [P, I, I, I, I, P, P]),
        "q4hip_profile_pass": (I, [P, P, I, I, P, I]),
        "q4hip_batch_create": (I, [ctypes.POINTER(P), P, I]),
        "q4hip_batch_destroy": (None, [P]),
        "q4hip_batch_prefill": (I, [P, I, P, I, I, ctypes.POINTER(I)]),
        "q4hip_batch_set_kv": (I, [P, I, I, I, I, I, P, P]),
        "q4hip_batch_generate": (I, [P, P, P, I, P]),
        "q4hip_batch_time_generate": (I, [P, P, P, I, P, ctypes.POINTER(F)]),
        "q4hip_batch_read_logits": (I, [P, P, I64]),
        "q4hip_mv_time_cold": (I, [P, I64, I, ctypes.POINTER(F), ctypes.POINTER(I)]),
        "q4hip_mv_run_noalloc": (I, [P, P, P, P]),
        "q4hip_attn_ring_rows": (I, [I, I, I, I, I, I, ctypes.POINTER(I), ctypes.POINTER(I), ctypes.POINTER(I)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _check(rc: int) -> None:
    if rc != OK:
        raise Q4Error(rc, lib().q4hip_last_error().decode())


def _ptr(a: np.ndarray) -> ctypes.c_void_p:
    return ctypes.c_void_p(a.ctypes.data)


def sources_sha() -> str:
    """First 16 hex digits of the SHA-256 of the device code's sources (csrc/*.h and csrc/*.hip, by
    name): what a rocprofv3 summary records as the kernels it measured, so that a figure taken from a
    summary can be dropped once the kernels have changed."""
    import hashlib
    d = os.path.join(os.path.dirname(_HERE), "csrc")
    h = hashlib.sha256()
    for name in sorted(os.listdir(d)):
        if name.endswith((".h", ".hip")):
            h.update(name.encode())
            with open(os.path.join(d, name), "rb") as f:
                h.update(f.read())
    return h.hexdigest()[:16]


def device_count() -> int:
    n = ctypes.c_int(0)
    _check(lib().q4hip_device_count(ctypes.byref(n)))
    return n.value


DIVISION_FORMS = ["a / 127", "d ? 1/d : 0", "g / (1 + fast_exp(-g))", "a / 896", "1 / d"]


def check_division(device: int = 0) -> dict:
    """Mismatch counts of the device's quotient forms against IEEE division over their whole
    input domains (q4hip_check_division)."""
    out = np.zeros(len(DIVISION_FORMS), np.uint64)
    _check(lib().q4hip_check_division(device, _ptr(out), len(DIVISION_FORMS)))
    return dict(zip(DIVISION_FORMS, (int(v) for v in out)))


def attn_ring_rows(pos: int, kv_tile: int, ring_slots: int, split: bool, half: int, kv_f16: bool) -> tuple:
    """(lowest row, highest row, loads) the persistent kernel's attention ring reads at position
    pos, from the kernel's row arithmetic run on the host (q4hip_attn_ring_rows; no GPU)."""
    lo, hi, n = ctypes.c_int(0), ctypes.c_int(0), ctypes.c_int(0)
    _check(lib().q4hip_attn_ring_rows(pos, kv_tile, ring_slots, int(split), half, int(kv_f16), ctypes.byref(lo),
                                      ctypes.byref(hi), ctypes.byref(n)))
    return lo.value, hi.value, n.value


class Model:
    """One loaded model on one GPU: the backend object's C side."""

    def __init__(self, shape: synth.Shape, ctx: int = 2048, mt: int = 0, device: int = 0, kv_type: int = KV_F32):
        self.shape, self.ctx, self.kv_type = shape, ctx, kv_type
        h = ctypes.c_void_p()
        _check(lib().q4hip_create(ctypes.byref(h), shape.dim, shape.layers, shape.ffn, shape.heads,
                                  shape.kv_heads, shape.vocab, ctx, mt, ctypes.c_float(shape.eps), device, kv_type))
        self.h = h

    def close(self) -> None:
        if self.h:
            for bt in list(getattr(self, "_batches", ())):   # batches go before their context
                bt.close()
            lib().q4hip_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_tensor(self, kind: int, layer: int, row0: int, t: synth.Tensor) -> None:
        data = np.ascontiguousarray(t.data)
        rows = t.rows if t.type != synth.GGML_F32 else data.size
        _check(lib().q4hip_set_tensor(self.h, kind, layer, row0, t.type, _ptr(data), rows, data.nbytes))

    def load(self, tensors: dict, rope: np.ndarray | None = None) -> None:
        """Upload a model dict from synth.make_model, fusing q|k|v and gate|up as
        engine/cpu-worker.js:106-128 does."""
        s = self.shape
        D, F, KV = s.dim, s.ffn, s.kv_heads * s.head_dim
        for layer in range(s.layers):
            p = f"blk.{layer}."
            for kind, names, offs in [(0, ["attn_q", "attn_k", "attn_v"], [0, D, D + KV]), (1, ["attn_output"], [0]),
                                      (2, ["ffn_gate", "ffn_up"], [0, F]), (3, ["ffn_down"], [0])]:
                for n, o in zip(names, offs):
                    self.set_tensor(kind, layer, o, tensors[p + n + ".weight"])
            self.set_tensor(4, layer, 0, tensors[p + "attn_norm.weight"])
            self.set_tensor(5, layer, 0, tensors[p + "ffn_norm.weight"])
            for n, o in zip(["attn_q", "attn_k", "attn_v"], [0, D, D + KV]):
                self.set_tensor(6, layer, o, tensors[p + n + ".bias"])
        self.set_tensor(7, 0, 0, tensors["token_embd.weight"])
        self.set_tensor(8, 0, 0, tensors["output.weight"])
        self.set_tensor(9, 0, 0, tensors["output_norm.weight"])
        if rope is None:
            rope = synth.rope_table(self.ctx, s.head_dim, s.rope_theta)
        rope = np.ascontiguousarray(rope, dtype=np.float32)
        _check(lib().q4hip_set_rope(self.h, _ptr(rope), rope.size))

    def set_kv(self, layer: int, kv_head: int, pos0: int, k: np.ndarray, v: np.ndarray) -> None:
        """Write K and V rows [n][head_dim] of one layer and kv head at positions pos0.."""
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        assert k.shape == v.shape and k.shape[1] == self.shape.head_dim
        _check(lib().q4hip_set_kv(self.h, layer, kv_head, pos0, k.shape[0], _ptr(k), _ptr(v)))

    def set_decode_mode(self, mode: int) -> None:
        _check(lib().q4hip_set_decode_mode(self.h, mode))

    def decode_mode_used(self) -> int:
        m = ctypes.c_int(0)
        _check(lib().q4hip_decode_mode_used(self.h, ctypes.byref(m)))
        return m.value

    def forward(self, ids, pos: int) -> int:
        a = np.ascontiguousarray(ids, dtype=np.int32)
        nxt = ctypes.c_int(0)
        _check(lib().q4hip_forward(self.h, _ptr(a), a.size, pos, ctypes.byref(nxt)))
        return nxt.value

    def read_logits(self) -> np.ndarray:
        out = np.empty(self.shape.vocab, dtype=np.float32)
        _check(lib().q4hip_read_logits(self.h, _ptr(out), out.size))
        return out

    def generate(self, first: int, pos: int, steps: int) -> list:
        out = np.empty(steps, dtype=np.int32)
        _check(lib().q4hip_generate(self.h, first, pos, steps, _ptr(out)))
        return out.tolist()

    def time_generate(self, first: int, pos: int, steps: int) -> tuple:
        out = np.empty(steps, dtype=np.int32)
        ms = ctypes.c_float(0)
        _check(lib().q4hip_time_generate(self.h, first, pos, steps, _ptr(out), ctypes.byref(ms)))
        return out.tolist(), ms.value

    def profile(self, token: int, pos: int) -> dict:
        us = np.zeros(len(PROF_NAMES), dtype=np.float32)
        _check(lib().q4hip_profile(self.h, token, pos, _ptr(us), us.size))
        return dict(zip(PROF_NAMES, us.tolist()))

    def profile_pass(self, ids, pos: int) -> dict:
        """Device microseconds per kernel class of one eager pass over `ids` at positions pos.."""
        a = np.ascontiguousarray(ids, dtype=np.int32)
        us = np.zeros(len(PROF_NAMES), dtype=np.float32)
        _check(lib().q4hip_profile_pass(self.h, _ptr(a), a.size, pos, _ptr(us), us.size))
        return dict(zip(PROF_NAMES, us.tolist()))

    def profile_persistent(self, token: int, pos: int, per_workgroup: bool = False):
        """Timeline of one persistent decode step, microseconds from kernel start,
        shape (layers + 1, 16); with per_workgroup also the (layers, grid, 8) workgroup
        timestamps.  See q4hip_profile_persistent in include/q4hip.h."""
        L = self.shape.layers
        n = (L + 1) * 16 + 8 * L * 256
        us = np.zeros(n, dtype=np.float32)
        _check(lib().q4hip_profile_persistent(self.h, token, pos, _ptr(us), n))
        tl = us[:(L + 1) * 16].reshape(L + 1, 16)
        if not per_workgroup:
            return tl
        G = int(tl[L, 5])
        return tl, us[(L + 1) * 16:(L + 1) * 16 + 8 * L * G].reshape(L, G, 8)

    def time_head(self, iters: int) -> float:
        us = ctypes.c_float(0)
        _check(lib().q4hip_time_head(self.h, iters, ctypes.byref(us)))
        return us.value


class Batch:
    """B sequences decoded together with one Model's weights, each with its own K/V cache.
    Holds a reference to the model; close the batch before closing the model explicitly."""

    def __init__(self, model: Model, B: int):
        self.model, self.B = model, B
        h = ctypes.c_void_p()
        _check(lib().q4hip_batch_create(ctypes.byref(h), model.h, B))
        self.h = h
        if not hasattr(model, "_batches"):
            model._batches = weakref.WeakSet()
        model._batches.add(self)

    def prefill(self, seq: int, ids, pos: int) -> int:
        """Prompt of sequence `seq` at positions pos..; returns its greedy next token."""
        a = np.ascontiguousarray(ids, dtype=np.int32)
        nxt = ctypes.c_int(0)
        _check(lib().q4hip_batch_prefill(self.h, seq, _ptr(a), a.size, pos, ctypes.byref(nxt)))
        return nxt.value

    def set_kv(self, seq: int, layer: int, kv_head: int, pos0: int, k: np.ndarray, v: np.ndarray) -> None:
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        assert k.shape == v.shape and k.shape[1] == self.model.shape.head_dim
        _check(lib().q4hip_batch_set_kv(self.h, seq, layer, kv_head, pos0, k.shape[0], _ptr(k), _ptr(v)))

    def _args(self, first, pos):
        f = np.ascontiguousarray(first, dtype=np.int32)
        p = np.ascontiguousarray(pos, dtype=np.int32)
        assert f.size == self.B and p.size == self.B
        return f, p

    def generate(self, first, pos, steps: int) -> np.ndarray:
        """[steps][B] greedy tokens: row i holds every sequence's token at its position pos[b]+1+i."""
        f, p = self._args(first, pos)
        out = np.empty((steps, self.B), dtype=np.int32)
        _check(lib().q4hip_batch_generate(self.h, _ptr(f), _ptr(p), steps, _ptr(out)))
        return out

    def time_generate(self, first, pos, steps: int) -> tuple:
        f, p = self._args(first, pos)
        out = np.empty((steps, self.B), dtype=np.int32)
        ms = ctypes.c_float(0)
        _check(lib().q4hip_batch_time_generate(self.h, _ptr(f), _ptr(p), steps, _ptr(out), ctypes.byref(ms)))
        return out, ms.value

    def read_logits(self) -> np.ndarray:
        out = np.empty((self.B, self.model.shape.vocab), dtype=np.float32)
        _check(lib().q4hip_batch_read_logits(self.h, _ptr(out), out.size))
        return out

    def close(self) -> None:
        if self.h:
            lib().q4hip_batch_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Matvec:
    """Isolated Q4_0 matvec y = W x (N x K, W in GGUF Q4_0 blocks)."""

    def __init__(self, raw_q4: np.ndarray, N: int, K: int, device: int = 0):
        self.N, self.K = N, K
        data = np.ascontiguousarray(raw_q4, dtype=np.uint8)
        assert data.size == N * (K // 32) * 18
        h = ctypes.c_void_p()
        _check(lib().q4hip_mv_create(ctypes.byref(h), N, K, _ptr(data), device))
        self.h = h

    def run(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        assert x.size == self.K
        y = np.empty(self.N, dtype=np.float32)
        _check(lib().q4hip_mv_run(self.h, _ptr(x), _ptr(y)))
        return y

    def run_device(self, x_dev: int, y_dev: int, stream: int = 0) -> None:
        """y = W x on device buffers (addresses), allocating nothing; waits unless `stream` is given."""
        _check(lib().q4hip_mv_run_noalloc(self.h, ctypes.c_void_p(x_dev), ctypes.c_void_p(y_dev),
                                          ctypes.c_void_p(stream or None)))

    def time(self, iters: int) -> float:
        us = ctypes.c_float(0)
        _check(lib().q4hip_mv_time(self.h, iters, ctypes.byref(us)))
        return us.value

    def time_cold(self, iters: int, rotate_bytes: int = 320 << 20) -> tuple:
        """(us per launch, copies): launches cycling through copies of W totalling >= rotate_bytes."""
        us, n = ctypes.c_float(0), ctypes.c_int(0)
        _check(lib().q4hip_mv_time_cold(self.h, rotate_bytes, iters, ctypes.byref(us), ctypes.byref(n)))
        return us.value, n.value

    def close(self) -> None:
        if self.h:
            lib().q4hip_mv_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
