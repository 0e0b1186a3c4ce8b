"""Pins for the oracle (oracle/oracle.c), CPU only.

The reference ships no golden vectors for synthetic weights (its reference.json needs the real
429 MB GGUF), so each oracle function is pinned by something other than its own formula:
  * a numpy emulation of the wasm SIMD128 instructions the reference uses (i16x8.extend_*,
    i32x4.dot_i16x8_s, f32x4.* lane arithmetic, saturating narrows), applied to the reference's
    own expressions (kernels.c:80-170) -- this fixes the lane partition and rounding order;
  * closed forms, exhaustive sweeps (all 16 nibbles x all 65,536 fp16 scales), special cases;
  * float64 references with derived error bounds, and invariants (chunking/threads independence).
A plausible slip (wrong lane set, dropped -8 offset, swapped operands, FMA contraction, ties to
away instead of even) fails at least one of them.
"""
import math

import numpy as np
import pytest

import oracle
import synth

f32 = np.float32


# ------------------------------------------------------------------ wasm SIMD emulation (spec semantics)

def ext_lo(v):          # i16x8.extend_low_i8x16_s
    return v[:8].astype(np.int32)


def ext_hi(v):          # i16x8.extend_high_i8x16_s
    return v[8:].astype(np.int32)


def dot_i16x8(a, b):    # i32x4.dot_i16x8_s: lane j = a[2j]*b[2j] + a[2j+1]*b[2j+1]
    p = a * b
    return p[0::2] + p[1::2]


def simd_q4_bdot(qs16, xq32):
    """kernels.c:127-136 / :178-185 with emulated instructions."""
    lo = ((qs16 & 0x0F).astype(np.int16) - 8).astype(np.int8)        # v128_and, i8x16_sub
    hi = ((qs16 >> 4).astype(np.int16) - 8).astype(np.int8)          # u8x16_shr, i8x16_sub
    x0, x1 = xq32[:16], xq32[16:]
    return (dot_i16x8(ext_lo(lo), ext_lo(x0)) + dot_i16x8(ext_hi(lo), ext_hi(x0))) + \
           (dot_i16x8(ext_lo(hi), ext_lo(x1)) + dot_i16x8(ext_hi(hi), ext_hi(x1)))


def simd_dot_q4_q8(wq, wd, xq, xd):
    """dot_q4_q8 (kernels.c:121-139): f32x4 acc = acc + convert(p) * splat(wd*xd); hsum."""
    acc = np.zeros(4, f32)
    for b in range(wd.size):
        p = simd_q4_bdot(wq[16 * b:16 * b + 16], xq[32 * b:32 * b + 32])
        acc = (acc + p.astype(f32) * (f32(wd[b]) * f32(xd[b]))).astype(f32)
    return f32(f32(f32(acc[0] + acc[1]) + acc[2]) + acc[3])


def simd_dot_q8_q8(wq, wd, xq, xd):
    """dot_q8_q8 (kernels.c:157-170) with emulated instructions."""
    acc = np.zeros(4, f32)
    for b in range(wd.size):
        w0, w1 = wq[32 * b:32 * b + 16], wq[32 * b + 16:32 * b + 32]
        x0, x1 = xq[32 * b:32 * b + 16], xq[32 * b + 16:32 * b + 32]
        p = (dot_i16x8(ext_lo(w0), ext_lo(x0)) + dot_i16x8(ext_hi(w0), ext_hi(x0))) + \
            (dot_i16x8(ext_lo(w1), ext_lo(x1)) + dot_i16x8(ext_hi(w1), ext_hi(x1)))
        acc = (acc + p.astype(f32) * (f32(wd[b]) * f32(xd[b]))).astype(f32)
    return f32(f32(f32(acc[0] + acc[1]) + acc[2]) + acc[3])


def simd_quantize_row(x):
    """quantize_row (kernels.c:90-114) with emulated f32x4 ops."""
    n = x.size
    q = np.empty(n, np.int8)
    d = np.empty(n // 32, f32)
    for b in range(n // 32):
        xb = x[32 * b:32 * b + 32].astype(f32)
        mx = np.zeros(4, f32)
        for i in range(0, 32, 4):
            mx = np.maximum(mx, np.abs(xb[i:i + 4]))                   # f32x4_max(mx, abs)
        amax = mx[0] if mx[0] > mx[1] else mx[1]
        amax = mx[2] if mx[2] > amax else amax
        amax = mx[3] if mx[3] > amax else amax
        dd = f32(amax / f32(127.0))
        idv = f32(f32(1.0) / dd) if dd != 0 else f32(0.0)
        v = np.rint((xb * idv).astype(f32))                             # f32x4_nearest: ties to even
        i32 = np.clip(v, -2147483648.0, 2147483647.0).astype(np.int64)  # trunc_sat
        i16 = np.clip(i32, -32768, 32767)                               # i16x8.narrow_i32x4_s
        q[32 * b:32 * b + 32] = np.clip(i16, -128, 127).astype(np.int8)  # i8x16.narrow_i16x8_s
        d[b] = dd
    return q, d


def _bits(a):
    return np.ascontiguousarray(a, f32).view(np.uint32)


# ------------------------------------------------------------------ fp16 / Q4_0 dequantization

def test_f16_table_exhaustive():
    """cpu-worker.js:93-96 vs numpy's IEEE half conversion, all 65,536 encodings."""
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(v)) for v in h], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(_bits(got[~nan]), _bits(ref[~nan]))


def test_q4_dequant_exhaustive():
    """Embedding dequant (kernels.c:312-322) over every nibble in both positions x every finite
    fp16 scale: (nib - 8) * d, bit-exact against numpy."""
    scales = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    scales = scales[np.isfinite(scales)]
    nb = scales.size
    byte = np.array([j | ((15 - j) << 4) for j in range(16)], np.uint8)     # low = j, high = 15 - j
    qs = np.tile(byte, nb)
    got = oracle.embed_row(qs, scales).reshape(nb, 32)
    lo = (np.arange(16) - 8).astype(np.float32)
    hi = ((15 - np.arange(16)) - 8).astype(np.float32)
    ref = np.concatenate([lo[None, :] * scales[:, None], hi[None, :] * scales[:, None]], axis=1)
    assert np.array_equal(_bits(got), _bits(ref))


def test_q4_0_quantizer_roundtrip():
    """The synthetic-weight quantizer (GGUF Q4_0 rule): |x - deq| <= |d|/2 where the nibble is not
    clipped at 15 (<= |d| where it is, the far side of the range), and the max-magnitude element
    maps to nibble 0 (value -8*d = max)."""
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(32 * 500) * 0.02).astype(np.float32)
    raw = synth.quantize_q4_0(x)
    deq = synth.dequantize_q4_0(raw).reshape(-1, 32)
    xb = x.reshape(-1, 32)
    _, d = synth.q4_0_blocks(raw)
    err = np.abs(deq - xb)
    nib = np.concatenate([raw[:, 2:] & 15, raw[:, 2:] >> 4], axis=1)
    tol = np.where(nib == 15, 1.0, 0.5) * np.abs(d)[:, None] * 1.01 + np.abs(xb) * 2e-3
    assert np.all(err <= tol)
    idx = np.argmax(np.abs(xb), axis=1)
    assert np.all((raw[np.arange(raw.shape[0]), 2 + idx % 16] >> (4 * (idx // 16)) & 15) == 0)


# ------------------------------------------------------------------ quantize_row

def test_quantize_row_matches_simd_emulation():
    rng = np.random.default_rng(1)
    for scale in (1e-3, 1.0, 37.0, 1e20):
        x = (rng.standard_normal(32 * 40) * scale).astype(f32)
        q, d, s = oracle.quantize_row(x)
        qe, de = simd_quantize_row(x)
        assert np.array_equal(q, qe) and np.array_equal(_bits(d), _bits(de))
        # s = d * (float)sum(q) per block (kernels.c:112)
        sums = q.reshape(-1, 32).astype(np.int64).sum(axis=1).astype(f32)
        assert np.array_equal(_bits(s), _bits((d * sums).astype(f32)))


def test_quantize_row_invariants():
    rng = np.random.default_rng(2)
    x = rng.standard_normal(32 * 64).astype(f32)
    q, d, _ = oracle.quantize_row(x)
    xb, qb = x.reshape(-1, 32), q.reshape(-1, 32).astype(np.int32)
    assert np.all(np.abs(qb) <= 127)
    amax_idx = np.argmax(np.abs(xb), axis=1)
    assert np.all(np.abs(qb[np.arange(64), amax_idx]) == 127)         # amax -> +-127
    assert np.all(np.sign(qb) * np.sign(xb) >= 0)                       # no sign flips
    assert np.all(np.abs(xb - qb * d[:, None]) <= d[:, None] * (0.5 + 1e-5))
    # all-zero block: d = 0, id = 0, q = 0 (kernels.c:98)
    z = np.zeros(64, f32)
    q, d, s = oracle.quantize_row(z)
    assert not q.any() and not d.any() and not s.any()


def test_quantize_row_ties_to_even():
    """Values landing exactly on k + 0.5 after scaling round to the even integer."""
    x = np.zeros(32, f32)
    x[0] = 127.0                                   # amax 127 -> d = 1, id = 1 exactly
    x[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -3.5]
    q, d, _ = oracle.quantize_row(x)
    assert d[0] == 1.0
    assert q[1:9].tolist() == [0, 2, 2, 0, -2, -2, 126, -4]


# ------------------------------------------------------------------ integer block dot and dot products

def test_block_lanes_match_simd_emulation():
    rng = np.random.default_rng(3)
    for _ in range(400):
        qs = rng.integers(0, 256, 16, dtype=np.uint8)
        x = rng.integers(-128, 128, 32).astype(np.int8)
        got = oracle.block_lanes_q4(qs, x)
        assert np.array_equal(got, simd_q4_bdot(qs, x))
        # the four lanes sum to the full block dot of (nib-8)*x
        nib = np.concatenate([(qs & 15), (qs >> 4)]).astype(np.int64) - 8
        assert int(got.sum()) == int(nib @ x.astype(np.int64))


def test_dot_q4_q8_matches_emulation_and_float64():
    rng = np.random.default_rng(4)
    for nb in (1, 3, 28, 152):
        wq = rng.integers(0, 256, 16 * nb, dtype=np.uint8)
        wd = (rng.standard_normal(nb) * 0.003).astype(np.float16).astype(f32)
        x = rng.standard_normal(32 * nb).astype(f32)
        xq, xd, _ = oracle.quantize_row(x)
        got = f32(oracle.dot_q4_q8(wq, wd, xq, xd))
        assert _bits(np.array([got]))[0] == _bits(np.array([simd_dot_q4_q8(wq, wd, xq, xd)]))[0]
        nib = np.stack([(wq.reshape(nb, 16) & 15), (wq.reshape(nb, 16) >> 4)], 1).reshape(nb, 32).astype(np.float64) - 8
        exact = float(np.sum(nib * wd[:, None] * xq.reshape(nb, 32) * xd[:, None]))
        mag = float(np.sum(np.abs(nib * wd[:, None] * xq.reshape(nb, 32) * xd[:, None])))
        assert abs(float(got) - exact) <= (nb + 4) * 1.2e-7 * mag + 1e-30


def test_dot_q8_equals_dot_q4_on_reencoded_head():
    """The lossless Q4_0 -> Q8_0 re-encoding gives bit-identical dots (shared lane partition)."""
    rng = np.random.default_rng(5)
    raw = synth.quantize_q4_0((rng.standard_normal(32 * 28 * 8) * 0.02).astype(f32)).reshape(8, 28, 18)
    x = rng.standard_normal(896).astype(f32)
    xq, xd, _ = oracle.quantize_row(x)
    for row in raw:
        qs, d = synth.q4_0_blocks(row)
        r8 = synth.q4_to_q8_0(row)
        q8 = np.ascontiguousarray(r8[:, 2:]).view(np.int8)
        a = oracle.dot_q4_q8(qs.reshape(-1), d, xq, xd)
        b = oracle.dot_q8_q8(q8.reshape(-1), d, xq, xd)
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32)


def test_dot_q8_q8_matches_emulation_on_full_int8_range():
    """The Q8_0 head of real files: int8 weights over the whole range, not only re-encoded nibbles."""
    rng = np.random.default_rng(15)
    for nb in (1, 5, 28):
        wq = rng.integers(-128, 128, 32 * nb).astype(np.int8)
        wd = (rng.standard_normal(nb) * 0.002).astype(np.float16).astype(f32)
        x = rng.standard_normal(32 * nb).astype(f32)
        xq, xd, _ = oracle.quantize_row(x)
        got = f32(oracle.dot_q8_q8(wq, wd, xq, xd))
        assert np.float32(got).view(np.uint32) == np.float32(simd_dot_q8_q8(wq, wd, xq, xd)).view(np.uint32)
        exact = float(np.sum(wq.reshape(nb, 32).astype(np.float64) * wd[:, None] * xq.reshape(nb, 32) * xd[:, None]))
        mag = float(np.sum(np.abs(wq.reshape(nb, 32).astype(np.float64) * wd[:, None] * xq.reshape(nb, 32) * xd[:, None])))
        assert abs(float(got) - exact) <= (nb + 4) * 1.2e-7 * mag + 1e-30


def test_synthetic_q8_0_quantizer():
    """The GGUF Q8_0 block rule of the synthetic heads: amax -> +-127, error within half a step of
    the fp32 scale (plus its fp16 rounding), zero blocks stay zero."""
    rng = np.random.default_rng(16)
    x = (rng.standard_normal(32 * 64) * 0.02).astype(f32)
    x[:32] = 0.0
    raw = synth.quantize_q8_0(x)
    q = raw[:, 2:].copy().view(np.int8).astype(np.int64)
    d16 = raw[:, 0:2].copy().view(np.float16).reshape(-1).astype(np.float64)
    xb = x.reshape(-1, 32).astype(np.float64)
    assert not q[0].any() and d16[0] == 0
    idx = np.argmax(np.abs(xb[1:]), axis=1)
    assert np.all(np.abs(q[1:][np.arange(63), idx]) == 127)
    d32 = np.abs(xb).max(1) / 127.0
    assert np.all(np.abs(xb - q * d32[:, None]) <= d32[:, None] * 0.5 * (1 + 1e-5))
    assert np.allclose(synth.dequantize_q8_0(raw).reshape(-1, 32), q * d16[:, None])


def test_matvec_vs_float64():
    rng = np.random.default_rng(6)
    N, K = 64, 896
    raw = synth.quantize_q4_0((rng.standard_normal(N * K) * 0.02).astype(f32))
    x = rng.standard_normal(K).astype(f32)
    y = oracle.matvec_q4(raw, N, K, x)
    W = synth.dequantize_q4_0(raw).reshape(N, K).astype(np.float64)
    xq, xd, _ = oracle.quantize_row(x)
    xdeq = xq.astype(np.float64) * np.repeat(xd.astype(np.float64), 32)
    ref = W @ xdeq
    mag = np.abs(W) @ np.abs(xdeq)
    assert np.all(np.abs(y - ref) <= 40 * 1.2e-7 * mag)
    # and against the activation itself: the int8 quantization error bound
    assert np.all(np.abs(y - W @ x.astype(np.float64)) <= np.abs(W) @ np.repeat(xd, 32) * 0.5 + 40 * 1.2e-7 * mag)


# ------------------------------------------------------------------ elementwise ops

def test_fast_exp():
    xs = np.concatenate([np.linspace(-87.0, 88.0, 20001), [0.0, -1e-8, 1e-8, 1.0, -1.0]]).astype(f32)
    got = np.array([oracle.fast_exp(float(v)) for v in xs], np.float64)
    ref = np.exp(xs.astype(np.float64))
    assert np.max(np.abs(got - ref) / ref) < 2.5e-7
    assert oracle.fast_exp(0.0) == 1.0
    assert oracle.fast_exp(-87.5) == 0.0 and oracle.fast_exp(-1000.0) == 0.0
    assert oracle.fast_exp(1000.0) == oracle.fast_exp(88.0)


def test_rmsnorm():
    rng = np.random.default_rng(7)
    x = rng.standard_normal(896).astype(f32) * 3
    w = rng.standard_normal(896).astype(f32)
    got = oracle.rmsnorm(x, w, 1e-6)
    # SIMD emulation: lane sums of x*x over i = j mod 4, ((l0+l1)+l2)+l3 (kernels.c:81-85)
    s = np.zeros(4, f32)
    for i in range(0, 896, 4):
        s = (s + (x[i:i + 4] * x[i:i + 4]).astype(f32)).astype(f32)
    ss = f32(f32(f32(s[0] + s[1]) + s[2]) + s[3])
    r = f32(f32(1.0) / f32(np.sqrt(f32(f32(ss / f32(896)) + f32(1e-6)))))
    assert np.array_equal(_bits(got), _bits(((x * r).astype(f32) * w).astype(f32)))
    ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * w
    assert np.allclose(got, ref, rtol=2e-6, atol=1e-7)
    c = np.full(64, 2.0, f32)
    assert np.allclose(oracle.rmsnorm(c, np.ones(64, f32), 0.0), 1.0, rtol=1e-7)


@pytest.mark.parametrize("hd", [64, 128])
def test_rope_head(hd):
    """NEOX pairs (i, i + hd/2) (kernels.c:340-344) at both head dims the configurations use."""
    rng = np.random.default_rng(8 + hd)
    v = rng.standard_normal(hd).astype(f32)
    table = oracle.rope_table(8, hd, 1e6)
    assert np.array_equal(oracle.rope_head(v, table[0].reshape(-1)), v)          # pos 0: identity
    got = oracle.rope_head(v, table[5].reshape(-1))
    c, s = table[5, :, 0].astype(np.float64), table[5, :, 1].astype(np.float64)
    x0, x1 = v[:hd // 2].astype(np.float64), v[hd // 2:].astype(np.float64)
    ref = np.concatenate([x0 * c - x1 * s, x1 * c + x0 * s])
    assert np.allclose(got, ref, rtol=1e-6, atol=1e-7)
    assert np.allclose(got[:hd // 2] ** 2 + got[hd // 2:] ** 2, v[:hd // 2] ** 2 + v[hd // 2:] ** 2, rtol=1e-5)


@pytest.mark.parametrize("hd", [64, 128])
def test_rope_table_vs_float64(hd):
    """cos/sin(pos / theta^(2i/hd)) (cpu-worker.js:130-135) within one fp32 ulp of float64."""
    t = oracle.rope_table(300, hd, 1e6)
    pos = np.arange(300)[:, None].astype(np.float64)
    a = pos / np.power(1e6, 2.0 * np.arange(hd // 2)[None, :] / hd)
    assert np.all(np.abs(t[:, :, 0] - np.cos(a)) <= np.spacing(np.float32(1.0)))
    assert np.all(np.abs(t[:, :, 1] - np.sin(a)) <= np.spacing(np.float32(1.0)))
    assert np.all(t[0, :, 0] == 1.0) and np.all(t[0, :, 1] == 0.0)
    # the Python host's table (synth.rope_table) is bit-identical to the oracle's
    assert np.array_equal(_bits(synth.rope_table(300, hd, 1e6)), _bits(t))


@pytest.mark.parametrize("hd", [64, 128])
def test_attention(hd):
    """Softmax attention of one head (kernels.c:354-378) against float64 at both head dims (scale
    1/sqrt(hd), four lane sums of hd/4 products), with its two closed forms: one position gives
    that position's V row exactly, q = 0 gives the mean of V."""
    rng = np.random.default_rng(9 + hd)
    for T in (1, 2, 7, 65, 300):
        q = rng.standard_normal(hd).astype(f32)
        k = rng.standard_normal((T, hd)).astype(f32)
        v = rng.standard_normal((T, hd)).astype(f32)
        got = oracle.attend(q, k, v, T, hd)
        if T == 1:
            assert np.array_equal(got, v[0])                                      # softmax of one = 1
        s = (k.astype(np.float64) @ q.astype(np.float64)) / math.sqrt(hd)
        p = np.exp(s - s.max())
        ref = (p / p.sum()) @ v.astype(np.float64)
        assert np.allclose(got, ref, rtol=2e-5, atol=2e-6)
    # q = 0: uniform weights, output = mean of V
    v = rng.standard_normal((50, hd)).astype(f32)
    got = oracle.attend(np.zeros(hd, f32), rng.standard_normal((50, hd)).astype(f32), v, 50, hd)
    assert np.allclose(got, v.astype(np.float64).mean(0), rtol=1e-5, atol=1e-6)


def test_attention_float64_bound_catches_a_wrong_scale():
    """The float64 bound above is sharp enough to see the plausible head-dim mistakes: the hd = 64
    scale (1/8) used at hd = 128, or only half of the dimensions in the scores."""
    rng = np.random.default_rng(99)
    hd, T = 128, 65
    q = rng.standard_normal(hd).astype(f32)
    k = rng.standard_normal((T, hd)).astype(f32)
    v = rng.standard_normal((T, hd)).astype(f32)
    got = oracle.attend(q, k, v, T, hd)
    for s in ((k.astype(np.float64) @ q.astype(np.float64)) / 8.0,
              (k[:, :64].astype(np.float64) @ q[:64].astype(np.float64)) / math.sqrt(hd)):
        p = np.exp(s - s.max())
        wrong = (p / p.sum()) @ v.astype(np.float64)
        assert not np.allclose(got, wrong, rtol=2e-5, atol=2e-6)


def test_swiglu():
    rng = np.random.default_rng(10)
    g = (rng.standard_normal(4864) * 4).astype(f32)
    u = rng.standard_normal(4864).astype(f32)
    got = oracle.swiglu(g, u)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.allclose(got, ref, rtol=1e-6, atol=1e-12)


def test_argmax_first_max_wins():
    rng = np.random.default_rng(11)
    for _ in range(50):
        x = rng.standard_normal(151936).astype(f32)
        i, j = sorted(rng.integers(0, x.size, 2))
        x[i] = x[j] = f32(10.0)
        assert oracle.argmax(x) == int(np.argmax(x)) == i
    assert oracle.argmax(np.array([-0.0, 0.0], f32)) == 0


# ------------------------------------------------------------------ whole-model invariants

def test_model_independent_of_threads_and_chunking():
    shape = synth.SHAPES["tiny"]
    t = synth.make_model(shape, 31)
    ids = synth.prompt_ids(31, 37, shape.vocab)
    runs = []
    for mt, th in ((16, 1), (5, 3), (1, 2)):
        m = oracle.Model(shape, t, ctx=96, mt=mt, threads=th)
        toks = m.generate(ids, 6)
        runs.append((toks, m.logits()))
        m.close()
    for toks, lg in runs[1:]:
        assert toks == runs[0][0] and np.array_equal(_bits(lg), _bits(runs[0][1]))


def test_model_context_full():
    shape = synth.SHAPES["tiny"]
    m = oracle.Model(shape, synth.make_model(shape, 1), ctx=16)
    with pytest.raises(RuntimeError, match="context full"):
        m.forward(list(range(16)), 0)
    m.close()


@pytest.mark.parametrize("name,seed", [("tiny", 41), ("small128", 42)])
def test_model_logits_near_float64_reference(name, seed):
    """End to end on a tiny model (head_dim 64) and on small128 (head_dim 128, the 1.5B shape's): the oracle's logits against a float64 model that quantizes the
    activations at the same points (quantize_row) and computes everything else exactly, except
    RMSNorm, which it takes in fp32 from the oracle: embedding rows are multiples of their Q4
    scale, so after the norm many values sit exactly on a .5 tie of the int8 grid and a 1-ulp
    difference would flip them (each flip moves a logit by ~5e-4)."""
    shape = synth.SHAPES[name]
    t = synth.make_model(shape, seed)
    ids = synth.prompt_ids(seed, 9, shape.vocab)
    m = oracle.Model(shape, t, ctx=32)
    m.forward(ids, 0)
    lg = m.logits()
    m.close()
    ref = _float64_model(shape, t, ids)
    diff = np.abs(lg - ref)
    assert np.max(diff) < 2e-3 and np.mean(diff) < 1e-4, (np.max(diff), np.mean(diff))
    assert int(np.argmax(ref)) == int(np.argmax(lg)) or np.sort(ref)[-1] - np.sort(ref)[-2] < 2e-3


def _float64_model(shape, t, ids):
    D, F, H, KVH, HD = shape.dim, shape.ffn, shape.heads, shape.kv_heads, shape.head_dim
    W = lambda n: synth.dequantize_q4_0(t[n].data).reshape(t[n].dims[1], t[n].dims[0]).astype(np.float64)  # noqa: E731

    def qz(v):
        q, d, _ = oracle.quantize_row(v.astype(f32))
        return q.astype(np.float64) * np.repeat(d.astype(np.float64), 32)

    def norm(v, w):
        return oracle.rmsnorm(v.astype(f32), w, shape.eps).astype(np.float64)

    emb = synth.dequantize_q4_0(t["token_embd.weight"].data).reshape(shape.vocab, D).astype(np.float64)
    rope = oracle.rope_table(32, HD, shape.rope_theta).astype(np.float64)
    T = len(ids)
    x = emb[ids]
    for layer in range(shape.layers):
        p = f"blk.{layer}."
        Wqkv = np.concatenate([W(p + "attn_q.weight"), W(p + "attn_k.weight"), W(p + "attn_v.weight")])
        b = np.concatenate([t[p + n + ".bias"].data for n in ("attn_q", "attn_k", "attn_v")]).astype(np.float64)
        qkv = np.stack([Wqkv @ qz(norm(x[i], t[p + "attn_norm.weight"].data)) + b for i in range(T)])
        heads = qkv[:, :H * HD].reshape(T, H, HD).copy()
        ks = qkv[:, D:D + KVH * HD].reshape(T, KVH, HD).copy()
        vs = qkv[:, D + KVH * HD:].reshape(T, KVH, HD)
        for i in range(T):
            c, s = rope[i, :, 0], rope[i, :, 1]
            for arr in (heads[i], ks[i]):
                x0, x1 = arr[:, :HD // 2].copy(), arr[:, HD // 2:].copy()
                arr[:, :HD // 2] = x0 * c - x1 * s
                arr[:, HD // 2:] = x1 * c + x0 * s
        att = np.zeros((T, D))
        for i in range(T):
            for h in range(H):
                kh = h // (H // KVH)
                sc = ks[:i + 1, kh] @ heads[i, h] / math.sqrt(HD)
                pr = np.exp(sc - sc.max())
                att[i, h * HD:(h + 1) * HD] = (pr / pr.sum()) @ vs[:i + 1, kh]
        x = x + np.stack([W(p + "attn_output.weight") @ qz(att[i]) for i in range(T)])
        Wg, Wu, Wd = W(p + "ffn_gate.weight"), W(p + "ffn_up.weight"), W(p + "ffn_down.weight")
        for i in range(T):
            hn = qz(norm(x[i], t[p + "ffn_norm.weight"].data))
            g, u = Wg @ hn, Wu @ hn
            x[i] = x[i] + Wd @ qz(g / (1 + np.exp(-g)) * u)
    head = synth.dequantize_q4_0(t["output.weight"].data).reshape(shape.vocab, D).astype(np.float64)
    return head @ qz(norm(x[-1], t["output_norm.weight"].data))


def test_round_f16_matches_ieee_conversion():
    """orc_round_f16 (the oracle's half-precision KV cache rounding) against numpy's IEEE 754
    float32 -> float16 conversion (round to nearest, ties to even): 2^20 bit patterns spread over
    the whole float32 range, every float16 tie point (the midpoints between neighbouring halves)
    and their neighbours, the overflow and subnormal boundaries, signed zeros, inf and NaN."""
    import ctypes
    f = oracle.lib().orc_round_f16
    pats = np.arange(0, 1 << 32, 1 << 12, dtype=np.uint64).astype(np.uint32)
    h = np.arange(0, 0x7c00, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    mids = ((h[:-1].astype(np.float64) + h[1:].astype(np.float64)) / 2).astype(np.float32)
    extra = np.array([65504.0, 65519.0, 65519.99, 65520.0, 65536.0, 6.1035156e-05, 6.097555e-05, 5.9604645e-08,
                      2.9802322e-08, 2.9802326e-08, 0.0, -0.0, np.inf, -np.inf], np.float32)
    vals = np.concatenate([pats.view(np.float32), mids, np.nextafter(mids, np.float32(np.inf)),
                           np.nextafter(mids, np.float32(-np.inf)), extra, -mids, -extra])
    vals = vals[np.isfinite(vals) | np.isinf(vals)]
    got = np.array([f(ctypes.c_float(v)) for v in vals], np.float32)
    want = vals.astype(np.float16).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.isnan(f(ctypes.c_float(float("nan"))))


def test_variant_zero_is_the_reference_arithmetic():
    """orc_set_variant(0) leaves every result as before; each variant changes the logits of a tiny
    model (the variants are measuring tools, so they must actually differ from the reference)."""
    shape = synth.SHAPES["tiny"]
    t = synth.make_model(shape, 5)
    ids = synth.prompt_ids(5, 300, shape.vocab)
    base = oracle.Model(shape, t, ctx=512)
    n0 = base.forward(ids, 0)
    l0 = base.logits()
    for flags in (oracle.V_NORM_TREE, oracle.V_DOT_SPLITK, oracle.V_ATTN_SPLIT, oracle.V_KV_F16):
        m = oracle.Model(shape, t, ctx=512)
        m.set_variant(0)
        assert m.forward(ids, 0) == n0 and np.array_equal(m.logits().view(np.uint32), l0.view(np.uint32))
        m.set_variant(flags)
        m.forward(ids, 0)
        assert not np.array_equal(m.logits().view(np.uint32), l0.view(np.uint32)), flags
        m.close()
    base.close()
