"""Isolated Q4_0 matvec on the GPU against the oracle's matmul_q4 (engine/kernels.c:200-273).

Sweep shapes are the model's projections: [896x896] o, [128x896] k/v, [4864x896] gate/up,
[896x4864] down and [151936x896] output head; [1536x1536] and [8960x1536] are the 1.5B shape's (the
second width the one-token stream kernel is built for), and [200x896] a row count that is not a
multiple of the 64-row tile.  The activation is quantized to int8 per 32-block
on the device exactly as quantize_row does, and each output is accumulated in the reference's lane
order, so the bar is bit-exact equality.
"""
import numpy as np
import pytest

import oracle
import synth

pytestmark = pytest.mark.gpu

SHAPES = [(896, 896), (128, 896), (4864, 896), (896, 4864), (151936, 896), (1536, 1536), (8960, 1536),
          (200, 896)]


def _weights(N, K, seed):
    rng = np.random.default_rng(seed)
    return synth.quantize_q4_0(rng.standard_normal(N * K, dtype=np.float32) * np.float32(0.02))


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("N,K", SHAPES)
def test_matvec_bit_exact(N, K):
    import q4hip
    print(f"matvec {N}x{K}", flush=True)
    raw = _weights(N, K, N + K)
    mv = q4hip.Matvec(raw, N, K)
    try:
        for seed in range(3):
            x = np.random.default_rng(100 + seed).standard_normal(K, dtype=np.float32)
            y = mv.run(x)
            ref = oracle.matvec_q4(raw, N, K, x)
            bad = np.flatnonzero(_bits(y) != _bits(ref))
            assert bad.size == 0, f"{bad.size} outputs differ, first {bad[:5]}: {y[bad[:5]]} vs {ref[bad[:5]]}"
    finally:
        mv.close()


def test_matvec_edge_inputs():
    """amax = 0 blocks (d = 0, id = 0), exact .5 ties, saturating magnitudes, tiny values."""
    import q4hip
    N, K = 256, 512
    raw = _weights(N, K, 5)
    mv = q4hip.Matvec(raw, N, K)
    try:
        rng = np.random.default_rng(9)
        cases = [np.zeros(K, np.float32)]
        x = rng.standard_normal(K).astype(np.float32)
        x[:32] = 0.0                                             # one all-zero block
        x[32:64] = np.arange(32, dtype=np.float32) - 15.5        # ties after scaling
        x[64:96] = np.float32(127.0)                             # all at amax
        x[96:128] = np.float32(1e-30) * np.arange(32)            # denormal-range products
        x[128:160] = np.float32(3e38) * np.sign(rng.standard_normal(32))  # near fp32 max
        cases.append(x)
        for x in cases:
            y = mv.run(x)
            ref = oracle.matvec_q4(raw, N, K, x)
            assert np.array_equal(_bits(y), _bits(ref))
    finally:
        mv.close()
