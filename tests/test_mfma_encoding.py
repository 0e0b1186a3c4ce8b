"""The exact-integer fp16 encoding of the Q4_0 x Q8 lane dot that k_gemm_sk feeds to the matrix cores.

One v_mfma_f32_16x16x16_f16 sums, for each (token, weight row), 16 products A[k] * B[k].  The kernel's
weight operand (SkB in csrc/gemm_sk.h) and activation operand (quantize_item in csrc/kernels.h) are
built so that this sum is exactly p_j = sum_k (n_k - 8) q_k, the integer dot of reference lane j
(engine/kernels.c:179-185, the i32x4.dot_i16x8_s lanes of q4_bdot).  This test rebuilds both operands
byte by byte on the CPU -- v_perm_b32 emulated, the constants read from the header -- and checks
that every product is an integer, that no ordering of the partial sums can leave the range where
fp32 integers are exact, and that the total is p_j.
"""
import pathlib
import re

import numpy as np

CSRC = pathlib.Path(__file__).resolve().parent.parent / "e2e-browser-voice-agent_amd" / "csrc"


def skb_constants():
    """mask, orv, sel0, sel1 for lane quarters kg = 0..3, parsed from SkB's constructor."""
    text = (CSRC / "gemm_sk.h").read_text()
    body = text[text.index("struct SkB"):]
    body = body[:body.index("operator()")]

    def line(name):
        m = re.search(r"\b%s = ([^;]+);" % name, body)
        assert m, name
        return m.group(1)

    return [tuple(_ternary(line(n), kg) for n in ("mask", "orv", "sel0", "sel1")) for kg in range(4)]


def _ternary(expr, kg):
    """Evaluate a C chain `c1 ? a : c2 ? b : d` of integer literals and comparisons of kg."""
    expr = expr.strip()
    if "?" not in expr:
        return int(expr.rstrip("u"), 0)
    cond, rest = expr.split("?", 1)
    a, b = rest.split(":", 1)
    c = cond.strip()
    m = re.fullmatch(r"kg\s*(==|<)\s*(\d+)", c)
    assert m, c
    ok = kg == int(m.group(2)) if m.group(1) == "==" else kg < int(m.group(2))
    return _ternary(a, kg) if ok else _ternary(b, kg)


def perm(s0, s1, sel):
    """v_perm_b32 D, s0, s1, sel for the selector values used: 0-3 bytes of s1, 4-7 bytes of s0, 0x0c zero."""
    src = s1 | (s0 << 32)
    out = 0
    for i in range(4):
        b = (sel >> (8 * i)) & 0xFF
        if b <= 7:
            v = (src >> (8 * b)) & 0xFF
        elif b == 0x0C:
            v = 0x00
        else:
            raise AssertionError("selector byte %#x not used by the kernel" % b)
        out |= v << (8 * i)
    return out


def f16_pair(word):
    return np.array([word & 0xFFFF, word >> 16], dtype=np.uint16).view(np.float16).astype(np.float64)


def weight_operand(wv, consts, kg):
    mask, orv, sel0, sel1 = consts[kg]
    v = (wv & mask) | orv
    return np.concatenate([f16_pair(perm(0x64646464, v, sel0)), f16_pair(perm(0x64646464, v, sel1))])


def activation_operand(q):
    """The four quarters quantize_item writes for one (chain, token): k = 0..15."""
    q = [int(x) for x in q]
    a = np.zeros(16, dtype=np.float64)
    a[0:4] = np.float16(q[0:4])
    a[4:8] = np.array([np.float16(np.float32(x) * np.float32(0.0625)) for x in q[4:8]], dtype=np.float64)
    a[8] = np.float16(-(q[0] + q[1] + q[2] + q[3]))
    a[9] = np.float16(-(q[4] + q[5] + q[6] + q[7]))
    return a


def lane_word(nibbles):
    """The repacked weight word of one reference lane: byte i holds n_i (low) and n_{i+4} (high)."""
    return sum((int(nibbles[i]) | (int(nibbles[i + 4]) << 4)) << (8 * i) for i in range(4))


def check(nibbles, q, consts):
    b = np.concatenate([weight_operand(lane_word(nibbles), consts, kg) for kg in range(4)])
    a = activation_operand(q)
    prod = a * b                                             # float64: exact for fp16 x fp16
    assert np.all(prod == np.round(prod)), (nibbles, q, prod)
    assert np.sum(np.abs(prod)) < 2 ** 24                    # any order of fp32 partial sums is exact
    want = sum((int(n) - 8) * int(x) for n, x in zip(nibbles, q))
    assert int(np.sum(prod)) == want, (nibbles, q, int(np.sum(prod)), want)


def test_constants_parsed():
    consts = skb_constants()
    assert consts[3] == (0, 0, 0x0C0C0C0C, 0x0C0C0C0C)      # quarter 3 is all zero
    for kg in range(2):
        assert consts[kg][1] == 0                            # nibble quarters: no constant or-ed in


def test_weight_operand_values():
    consts = skb_constants()
    nib = [1, 2, 3, 4, 5, 6, 7, 15]
    w = lane_word(nib)
    assert list(weight_operand(w, consts, 0)) == [1024 + n for n in nib[:4]]
    assert list(weight_operand(w, consts, 1)) == [1024 + 16 * n for n in nib[4:]]
    assert list(weight_operand(w, consts, 2)) == [1032, 72, 0, 0]
    assert list(weight_operand(w, consts, 3)) == [0, 0, 0, 0]


def test_lane_dot_exact_extremes_and_random():
    consts = skb_constants()
    for n in (0, 8, 15):
        for x in (-127, -128 + 1, 0, 1, 127):
            check([n] * 8, [x] * 8, consts)
    check([0, 15] * 4, [127, -127] * 4, consts)
    check([15, 0] * 4, [127, -127] * 4, consts)
    rng = np.random.default_rng(7)
    for _ in range(4000):
        check(rng.integers(0, 16, 8), rng.integers(-127, 128, 8), consts)


def test_a_wrong_correction_fails():
    """The check catches a slip in the high quarter's correction (72 -> 64) or a missing /16."""
    consts = skb_constants()
    bad = list(consts)
    m, o, s0, s1 = bad[2]
    bad[2] = (m, (o & 0x0000FFFF) | 0x54000000, s0, s1)      # fp16 64 instead of 72
    try:
        check([3, 5, 7, 9, 11, 13, 15, 1], [10, -20, 30, -40, 50, -60, 70, -80], bad)
    except AssertionError:
        pass
    else:
        raise AssertionError("a wrong k = 9 constant went unnoticed")
