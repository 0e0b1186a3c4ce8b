"""The matvec entry point that allocates nothing (q4hip_mv_run_noalloc) against q4hip_mv_run.

Both quantize x to int8 per 32-block as quantize_row does (engine/kernels.c:90-114) and accumulate
each output as matmul_q4 does (engine/kernels.c:200-229); the no-allocation one keeps the
activation blocks in the library's static device buffer instead of the handle's.  The bar is
bit-exact equality, on two calls in a row where the second has the smaller input (so it runs over
the first call's leftovers in the shared buffer), then again on a caller-given stream.  Device
buffers come from the HIP runtime through ctypes; no torch.
"""
import ctypes

import numpy as np
import pytest

import oracle
import synth

pytestmark = pytest.mark.gpu


def _hip():
    import q4hip
    q4hip.lib()                       # loads libamdhip64 as a dependency
    h = ctypes.CDLL("libamdhip64.so.7")
    P, I, S = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    for name, args in {"hipMalloc": [ctypes.POINTER(P), S], "hipFree": [P], "hipMemcpy": [P, P, S, I],
                       "hipSetDevice": [I], "hipStreamCreate": [ctypes.POINTER(P)],
                       "hipStreamSynchronize": [P], "hipStreamDestroy": [P]}.items():
        getattr(h, name).argtypes = args
        getattr(h, name).restype = I
    return h


H2D, D2H = 1, 2


class DevBuf:
    def __init__(self, hip, nbytes):
        self.hip, self.p = hip, ctypes.c_void_p()
        assert hip.hipMalloc(ctypes.byref(self.p), nbytes) == 0
        self.nbytes = nbytes

    def put(self, a):
        assert a.nbytes <= self.nbytes
        assert self.hip.hipMemcpy(self.p, a.ctypes.data, a.nbytes, H2D) == 0

    def get(self, n):
        out = np.empty(n, np.float32)
        assert self.hip.hipMemcpy(out.ctypes.data, self.p, out.nbytes, D2H) == 0
        return out

    def free(self):
        if self.p:
            self.hip.hipFree(self.p)
            self.p = None


def _weights(N, K, seed):
    rng = np.random.default_rng(seed)
    return synth.quantize_q4_0(rng.standard_normal(N * K, dtype=np.float32) * np.float32(0.02))


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_noalloc_matches_run_twice_second_smaller():
    import q4hip
    hip = _hip()
    assert hip.hipSetDevice(0) == 0
    shapes = [(896, 4864), (1152, 896)]             # down, then qkv: the second input is smaller
    bufs, mvs = [], []
    try:
        xb = DevBuf(hip, 4864 * 4)
        yb = DevBuf(hip, 1152 * 4)
        bufs += [xb, yb]
        for call, (N, K) in enumerate(shapes):
            print(f"no-alloc matvec call {call}: {N}x{K}", flush=True)
            raw = _weights(N, K, 7 + call)
            mv = q4hip.Matvec(raw, N, K)
            mvs.append(mv)
            x = np.random.default_rng(50 + call).standard_normal(K, dtype=np.float32)
            ref = mv.run(x)
            xb.put(x)
            mv.run_device(xb.p.value, yb.p.value)
            y = yb.get(N)
            bad = np.flatnonzero(_bits(y) != _bits(ref))
            assert bad.size == 0, f"call {call}: {bad.size} outputs differ, first {bad[:5]}"
            assert np.array_equal(_bits(y), _bits(oracle.matvec_q4(raw, N, K, x)))
        # the same two handles again, in the same order, on a caller-given stream
        s = ctypes.c_void_p()
        assert hip.hipStreamCreate(ctypes.byref(s)) == 0
        try:
            for call, ((N, K), mv) in enumerate(zip(shapes, mvs)):
                x = np.random.default_rng(60 + call).standard_normal(K, dtype=np.float32)
                ref = mv.run(x)
                xb.put(x)
                mv.run_device(xb.p.value, yb.p.value, stream=s.value)
                assert hip.hipStreamSynchronize(s) == 0
                assert np.array_equal(_bits(yb.get(N)), _bits(ref)), f"stream call {call}"
        finally:
            hip.hipStreamDestroy(s)
    finally:
        for mv in mvs:
            mv.close()
        for b in bufs:
            b.free()


def test_noalloc_at_the_largest_k():
    """K = Q4HIP_NOALLOC_MAX_K (65536: 2048 activation blocks, 128 KB of shared memory in the
    one-token matvec), bit-equal to q4hip_mv_run and to the oracle's matmul_q4."""
    import q4hip
    hip = _hip()
    assert hip.hipSetDevice(0) == 0
    N, K = 64, q4hip.NOALLOC_MAX_K
    print(f"no-alloc matvec {N}x{K}", flush=True)
    raw = _weights(N, K, 11)
    mv = q4hip.Matvec(raw, N, K)
    xb, yb = DevBuf(hip, K * 4), DevBuf(hip, N * 4)
    try:
        x = np.random.default_rng(12).standard_normal(K, dtype=np.float32)
        ref = mv.run(x)
        xb.put(x)
        mv.run_device(xb.p.value, yb.p.value)
        assert np.array_equal(_bits(yb.get(N)), _bits(ref))
        assert np.array_equal(_bits(ref), _bits(oracle.matvec_q4(raw, N, K, x)))
    finally:
        mv.close()
        xb.free()
        yb.free()


def test_noalloc_rejects_bad_buffers_and_sizes():
    """Host pointers, short buffers and K above the limit are refused before any launch."""
    import q4hip
    hip = _hip()
    N, K = 4864, 896
    mv = q4hip.Matvec(_weights(N, K, 3), N, K)
    xb, yb = DevBuf(hip, K * 4), DevBuf(hip, N * 4)
    host = np.zeros(max(N, K), np.float32)
    try:
        with pytest.raises(q4hip.Q4Error, match="not device memory"):
            mv.run_device(host.ctypes.data, yb.p.value)
        with pytest.raises(q4hip.Q4Error, match="bytes needed"):
            mv.run_device(xb.p.value, yb.p.value + 8192)   # y starts 8 KB in: 8 KB short
        big_k = q4hip.NOALLOC_MAX_K + 32
        big = q4hip.Matvec(_weights(64, big_k, 4), 64, big_k)
        try:
            with pytest.raises(q4hip.Q4Error, match="no-allocation limit"):
                big.run_device(xb.p.value, yb.p.value)
        finally:
            big.close()
        # the handle still works after the refusals
        x = np.random.default_rng(1).standard_normal(K, dtype=np.float32)
        xb.put(x)
        mv.run_device(xb.p.value, yb.p.value)
        assert np.array_equal(_bits(yb.get(N)), _bits(mv.run(x)))
    finally:
        mv.close()
        xb.free()
        yb.free()
