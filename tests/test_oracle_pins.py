"""Pins the CPU oracle (the checker) before anything is compared against it.

Each check is a known answer the reference itself fixes, or a property the
mathematics fixes, chosen so that a plausible slip in the oracle (a wrong
rounding tie, a swapped operand, a dropped term) fails:
  - the KAT vectors of the reference's Rust unit tests (file:line cited);
  - the reference's three forward op conformance vectors, hash-checked first
    exactly as golden_runner.rs:48-87 does;
  - SHA-256 of the LUTs against the reference scale packs;
  - closed forms / brute force for what those leave open.
"""
from __future__ import annotations

import hashlib
import json
import math
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---- fixed_point.rs -----------------------------------------------------------

# fixed_point.rs:251-275 (division_semantics_vector): (value, shift, expected)
DIVISION_VECTOR = [
    (0, 3, 0), (1, 1, 0), (2, 1, 1), (3, 1, 2), (4, 1, 2), (5, 1, 2), (6, 1, 3), (7, 1, 4), (8, 3, 1),
    (12, 3, 2), (1_000_000, 8, 3906), (-1, 1, 0), (-2, 1, -1), (-3, 1, -2), (-4, 1, -2), (-5, 1, -2),
    (-6, 1, -3), (-7, 1, -4), (-8, 3, -1), (-12, 3, -2), (-1_000_000, 8, -3906),
]


def test_division_semantics_vector(oracle):
    for v, s, e in DIVISION_VECTOR:
        assert oracle.rshift_round(v, s) == e, (v, s)
        assert oracle.rshift_round_i64(v, s) == e, (v, s)
        assert oracle.rshift_round_i128(v, s) == e, (v, s)


def test_rshift_round_basic_kats(oracle):
    # fixed_point.rs:210-222, 225-228
    assert [oracle.rshift_round(v, 1) for v in (4, 3, 5, 7)] == [2, 2, 2, 4]
    assert [oracle.rshift_round(v, 1) for v in (-5, -4, -3)] == [-2, -2, -2]
    assert oracle.rescale(127 * 127, 13, 6) == 126


def test_rshift_round_is_exact_rne_bruteforce(oracle):
    # Closed form: round(v / 2^s), ties to even, for every v in a window.
    for s in (1, 2, 3, 7, 13):
        for v in range(-300, 301):
            q = Fraction(v, 1 << s)
            f = math.floor(q)
            r = q - f
            exp = f + 1 if (r > Fraction(1, 2) or (r == Fraction(1, 2) and f % 2 == 1)) else f
            assert oracle.rshift_round(v, s) == exp
            assert oracle.rshift_round_i64(v * (1 << 33), s + 33) == exp
            assert oracle.rshift_round_i128(v * (1 << 90), s + 90) == exp


def test_overflow_saturation_vector(oracle):
    # fixed_point.rs:303-333
    L = oracle.lib()
    assert L.or_clamp_i8(2**31 - 1) == 127 and L.or_clamp_i8(-2**31) == -128
    assert L.or_clamp_i8(128) == 127 and L.or_clamp_i8(-129) == -128
    assert L.or_clamp_i16(2**31 - 1) == 32767 and L.or_clamp_i16(-2**31) == -32768
    assert L.or_clamp_i16(32768) == 32767 and L.or_clamp_i16(-32769) == -32768
    assert L.or_clamp_i16_from_i64(2**63 - 1) == 32767 and L.or_clamp_i16_from_i64(-2**63) == -32768
    assert L.or_clamp_i32(2**63 - 1) == 2**31 - 1 and L.or_clamp_i32(-2**63) == -2**31
    assert L.or_clamp_i32(2**31) == 2**31 - 1 and L.or_clamp_i32(-2**31 - 1) == -2**31


def test_inv_sqrt_q15_and_isqrt_round(oracle):
    # fixed_point.rs:336-362, 382-395
    assert [oracle.inv_sqrt_q15(h) for h in (4, 16, 64, 256)] == [1 << 14, 1 << 13, 1 << 12, 1 << 11]
    assert oracle.inv_sqrt_q15(128) == 2896 and oracle.inv_sqrt_q15(512) == 1448 and oracle.inv_sqrt_q15(2) == 23170
    assert [oracle.isqrt_round(n) for n in (0, 1, 2, 3, 4)] == [0, 1, 1, 2, 2]
    assert oracle.isqrt_round(8_388_608) == 2896 and oracle.isqrt_round(16_777_216) == 4096
    for n in (5, 99, 1000, 123_456, 1 << 40, 2**64 - 1, 2**62 + 12345):
        r = math.isqrt(n)
        exp = r + 1 if (r + 1) ** 2 - n < n - r * r else r
        assert oracle.isqrt_round(n) == exp, n


def test_multiplier_equals_shift_for_powers_of_two(oracle):
    # fixed_point.rs:364-379
    for x in (-100_003, -8, -7, -1, 0, 1, 7, 8, 9, 100_003, 1 << 30):
        for n in (1, 3, 5, 8, 16):
            assert oracle.rshift_round_i64(x, n) == oracle.rshift_round_i64(x * (1 << 12), n + 12)


def test_rescale_negative_shift_is_plain_left_shift(oracle):
    # fixed_point.rs:173-191: in_frac < out_frac -> unrounded left shift (wrapping).
    assert oracle.rescale(3, 2, 5) == 24
    assert oracle.rescale_i64(-3, 0, 7) == -384
    assert oracle.rescale(1 << 30, 0, 2) == 0          # bits shifted out of i32 are lost
    assert oracle.rescale(0x40000001, 0, 1) == -2147483646  # wraps like Rust release


# ---- dot.rs / linear.rs ---------------------------------------------------------

@pytest.mark.parametrize("simd", [0, 1])
def test_dot_extremes_and_order(oracle, simd):
    # dot.rs:306-327: extremes beyond i32; any order gives the same exact sum.
    # Both dot forms: the scalar i64 loop and the i32 blocks of 256 products,
    # whose worst block (-128 * -32768 * 256 = 2^30) must not wrap.
    rng = np.random.default_rng(0)
    w = rng.integers(-128, 128, 4096).astype(np.int8)
    x = rng.integers(-32768, 32768, 4096).astype(np.int16)
    L = oracle.lib()
    L.or_set_simd(simd)
    try:
        exact = int(np.dot(w.astype(np.int64), x.astype(np.int64)))
        assert L.or_dot_i8_i16(w.ctypes.data, x.ctypes.data, 4096) == exact
        for n in (20000, 256, 257, 255, 1):
            w2 = np.full(n, -128, np.int8)
            x2 = np.full(n, -32768, np.int16)
            assert L.or_dot_i8_i16(w2.ctypes.data, x2.ctypes.data, n) == n * 128 * 32768
            x2[:] = 32767
            assert L.or_dot_i8_i16(w2.ctypes.data, x2.ctypes.data, n) == -n * 128 * 32767
    finally:
        L.or_set_simd(1)


def test_requant_of_exact_sums_equals_the_linear_forms(oracle):
    # The requant steps on precomputed sums give what linear_w8a16 and the
    # multiplier form give on the same operands.
    rng = np.random.default_rng(12)
    M, N, K = 3, 70, 300
    W = rng.integers(-128, 128, (N, K)).astype(np.int8)
    x = rng.integers(-32768, 32768, (M, K)).astype(np.int16)
    x[0, :3] = (-32768, 32767, 0)
    acc = x.astype(np.int64) @ W.astype(np.int64).T
    ws = rng.integers(0, 14, N).astype(np.uint8)
    assert np.array_equal(oracle.requant_shift(acc, ws, 11, 4), oracle.linear_batch(x, W, ws, 11, 4))
    assert np.array_equal(oracle.requant_shift(acc, ws, 2, 9), oracle.linear_batch(x, W, ws, 2, 9))
    mult = rng.integers(1 << 29, (1 << 30) + 1, N).astype(np.int32)
    sh = rng.integers(20, 41, N).astype(np.uint8)
    assert np.array_equal(oracle.requant_mult(acc, mult, sh), oracle.linear_mult(x, W, mult, sh))


def test_linear_kats(oracle):
    # linear.rs:151-222
    assert list(oracle.linear_w8a16([64, -64], [127, 0, 0, 127], 2, [7, 7], 6, 6)) == [64, -64]
    assert list(oracle.linear_w8a16([64], [64, 64], 1, [7, 6], 6, 6)) == [32, 64]
    assert list(oracle.linear_w8a16([32767] * 896, [127] * 896, 896, [7], 5, 3)) == [32767]
    x, W, ws = [100, -50, 25], [64, -32, 16, 10, 20, -30], [6, 5]
    assert list(oracle.linear_w8a16(x, W, 3, ws, 4, 6)) == list(oracle.linear_w8a16_pc(x, W, 3, ws, 4, [6, 6]))
    assert list(oracle.linear_w8a16_pc([100, 100], [64] * 4, 2, [6, 6], 0, [6, 3])) == [12800, 1600]


def test_linear_matches_closed_form(oracle):
    # y = clamp16(round_half_even(dot / 2^(w_shift + act - out))) with exact Fractions.
    rng = np.random.default_rng(1)
    N, K = 37, 53
    W = rng.integers(-127, 128, (N, K)).astype(np.int8)
    x = rng.integers(-32768, 32768, K).astype(np.int16)
    ws = rng.integers(0, 12, N).astype(np.uint8)
    y = oracle.linear_w8a16(x, W.ravel(), K, ws, 9, 4)
    for r in range(N):
        d = int(np.dot(W[r].astype(np.int64), x.astype(np.int64)))
        s = int(ws[r]) + 9 - 4
        q = Fraction(d, 1 << s)
        f = math.floor(q)
        fr = q - f
        v = f + 1 if (fr > Fraction(1, 2) or (fr == Fraction(1, 2) and f % 2)) else f
        assert y[r] == max(-32768, min(32767, v))


def test_bias_kats(oracle):
    # linear.rs:225-254
    assert list(oracle.add_bias_i16([10, -10], [1, 1], [2, 2], 4)) == [14, -6]
    assert list(oracle.add_bias_i16([0, 0], [3, -3], [3, 3], 1)) == [1, -1]
    assert list(oracle.add_bias_i16([0, 0], [4, 4], [1, 0], 0)) == [2, 4]
    assert list(oracle.add_bias_i16([32766, -32767, 0], [4, -4, 0], [1, 1, 1], 0)) == [32767, -32768, 0]


def test_multiplier_requant_reduces_to_shift(oracle):
    # Build-defined multiplier requant: M = 2^k, s = k + s_ref equals the reference.
    rng = np.random.default_rng(2)
    N, K = 64, 96
    W = rng.integers(-127, 128, (N, K)).astype(np.int8)
    x = rng.integers(-32768, 32768, (3, K)).astype(np.int16)
    ws = rng.integers(0, 10, N).astype(np.uint8)
    ref = oracle.linear_batch(x, W, ws, 8, 3)
    k = 29
    got = oracle.linear_mult(x, W, np.full(N, 1 << k, np.int32), (ws.astype(np.int32) + 8 - 3 + k).astype(np.uint8))
    assert np.array_equal(ref, got)
    # and a general multiplier against exact rational rounding
    mult = rng.integers(1 << 29, 1 << 30, N).astype(np.int32)
    sh = rng.integers(20, 41, N).astype(np.uint8)
    got = oracle.linear_mult(x, W, mult, sh)
    for m in range(3):
        for r in range(N):
            d = int(np.dot(W[r].astype(np.int64), x[m].astype(np.int64))) * int(mult[r])
            q = Fraction(d, 1 << int(sh[r]))
            f = math.floor(q)
            fr = q - f
            v = f + 1 if (fr > Fraction(1, 2) or (fr == Fraction(1, 2) and f % 2)) else f
            assert got[m, r] == max(-32768, min(32767, v))


# ---- rmsnorm.rs -----------------------------------------------------------------

def spec_rsqrt_lut(n):
    # rmsnorm.rs:169-180 (test helper): lut[x] = round(2^12 / sqrt(x)), lut[0] = 256
    return [256] + [int(round(4096.0 / math.sqrt(x))) for x in range(1, n)]


def test_rmsnorm_kats(oracle):
    # rmsnorm.rs:183-249
    inv = oracle.inv_n_q20
    assert inv(896) == 1170 and inv(1) == 1 << 20
    lut1k, lut = spec_rsqrt_lut(1024), spec_rsqrt_lut(32768)
    r = lambda x, xs, g, gs, L, n, of: list(oracle.rmsnorm_i16(x, xs, g, gs, L, 8, 8, inv(n), of))
    assert r([0, 0, 0], [0] * 3, [64] * 3, [6] * 3, lut1k, 3, 6) == [0, 0, 0]
    assert r([16, 16], [0, 0], [64, 64], [6, 6], lut, 2, 6) == [64, 64]
    assert r([-16, -16], [0, 0], [64, 64], [6, 6], lut, 2, 6) == [-64, -64]
    out = r([12000, 12000], [0, 0], [32, 32], [5, 5], lut, 2, 3)
    assert all(abs(o - 8) <= 1 for o in out)
    out = r([16, 0], [0, 0], [32, 32], [5, 5], lut, 2, 6)
    assert out[0] in (90, 91) and out[1] == 0
    assert r([16, 16], [0, 0], [32, 32], [5, 5], lut, 2, 6) == [64, 64]
    assert r([16, 16], [0, 0], [64, 64], [5, 5], lut, 2, 6) == [128, 128]
    assert r([16, 16], [0, 0], [32, 32], [5, 4], lut, 2, 6) == [64, 128]


def test_rmsnorm_invariances(oracle):
    # rmsnorm.rs:252-376
    inv = oracle.inv_n_q20
    lut = spec_rsqrt_lut(32768)
    ref = list(oracle.rmsnorm_i16([3000, -500, 7, 12000], [0] * 4, [32, 40, 20, 8], [5] * 4, lut, 8, 8, inv(4), 6))
    for s in (1, 5, 9, 14):
        assert list(oracle.rmsnorm_i16([3000, -500, 7, 12000], [s] * 4, [32, 40, 20, 8], [5] * 4, lut, 8, 8, inv(4),
                                       6)) == ref
    g, gs = [64] * 4, [6] * 4
    out = oracle.rmsnorm_i16([9600, 1024, -2048, 3072], [1, 12, 12, 12], g, gs, lut, 8, 8, inv(4), 8)
    assert abs(abs(out[0] / 256.0) - 2.0) < 0.1
    a = oracle.rmsnorm_i16([9600, 1024, -2048, 3072], [1, 12, 12, 12], g, gs, lut, 8, 8, inv(4), 8)
    b = oracle.rmsnorm_i16([19200, 256, -512, 768], [2, 10, 10, 10], g, gs, lut, 8, 8, inv(4), 8)
    assert list(a) == list(b)
    out = oracle.rmsnorm_i16([9600, 1024, 4800, 4], [2, 10, 1, 2], g, gs, lut, 8, 8, inv(4), 8)
    assert out[1] == out[3] and out[0] == out[2]
    out = oracle.rmsnorm_i16([32767, 32767, 1, 1], [0, 20, 0, 20], [127] * 4, [20] * 4, lut, 8, 8, inv(4), 0)
    assert all(v >= 0 for v in out)


def test_rmsnorm_rejects_what_the_reference_panics_on(oracle):
    lut = spec_rsqrt_lut(1024)
    with pytest.raises(ValueError):
        oracle.rmsnorm_i16([1, 2], [0, 0], [1, 1], [0, 0], lut, 7, 8, 1 << 19, 6)  # odd input shift (:76)
    with pytest.raises(ValueError):
        oracle.rmsnorm_i16([], [], [], [], lut, 8, 8, 1, 6)  # empty x_shifts (:96)


# ---- rope.rs ------------------------------------------------------------------------

def test_rope_kats(oracle):
    # rope.rs:69-121
    v = [100, -200, 32000, -32000]
    assert list(oracle.rotate_half_split_i16(v, [256, 256], [0, 0], 8)) == v
    assert list(oracle.rotate_half_split_i16([100, 200, 300, 400], [0, 0], [256, 256], 8)) == [-300, -400, 100, 200]
    assert list(oracle.rotate_half_split_i16([4096, 0, 0, 0], [256, 256], [0, 0], 8)) == [4096, 0, 0, 0]
    cos = np.full(8, 256, np.int16)
    sin = np.zeros(8, np.int16)
    qo, ko = oracle.apply_rope_i16([[10, 20, 30, 40]], [[50, 60, 70, 80]], cos, sin, [0], 8)
    assert list(qo[0]) == [10, 20, 30, 40] and list(ko[0]) == [50, 60, 70, 80]


def test_rope_position_wraps_modulo_rows(oracle):
    # model.rs:469-473 / rope.rs:46,52: position p uses LUT row p % n_pos.
    rng = np.random.default_rng(3)
    cos = rng.integers(-256, 257, 4 * 3).astype(np.int16)
    sin = rng.integers(-256, 257, 4 * 3).astype(np.int16)
    q = rng.integers(-30000, 30000, (1, 6)).astype(np.int16)
    a, _ = oracle.apply_rope_i16(q, q, cos, sin, [1], 8)
    b, _ = oracle.apply_rope_i16(q, q, cos, sin, [5], 8)  # 5 % 4 == 1
    assert np.array_equal(a, b)
    # pair (j, j+half) rotation against the closed form
    j = 2
    x0, x1 = int(q[0, j]), int(q[0, j + 3])
    c, s = int(cos[3 + j]), int(sin[3 + j])
    for val, exp in ((a[0, j], x0 * c - x1 * s), (a[0, j + 3], x1 * c + x0 * s)):
        f = Fraction(exp, 256)
        fl = math.floor(f)
        r = f - fl
        e = fl + 1 if (r > Fraction(1, 2) or (r == Fraction(1, 2) and fl % 2)) else fl
        assert val == max(-32768, min(32767, e))


# ---- softmax.rs / attention.rs ------------------------------------------------------------

def test_softmax_properties(oracle):
    from myelith_amd.luts import exp_lut
    lut = exp_lut()
    # equal logits -> uniform; sum of probabilities within n/2 of 2^14
    p = oracle.softmax_int([5, 5, 5, 5], lut, 6, 14)
    assert list(p) == [4096] * 4
    rng = np.random.default_rng(4)
    z = rng.integers(-200000, 200000, 300).astype(np.int32)
    p = oracle.softmax_int(z, lut, 6, 14)
    assert abs(int(p.sum()) - (1 << 14)) <= 150
    assert p[np.argmax(z)] == p.max()
    # shift invariance: adding a constant to all logits changes nothing
    assert np.array_equal(p, oracle.softmax_int(z + 12345, lut, 6, 14))
    # all-masked (out of LUT range) -> the uniform fallback with the remainder on the lowest indices
    p = oracle.softmax_int([0, -10_000_000, -10_000_000], np.array([0], np.int16), 6, 14)
    assert list(p) == [5462, 5461, 5461]


def test_softmax_division_rounds_half_to_even(oracle):
    # p_j = RNE(e_j * one / S) with a true integer division (softmax.rs:50-63)
    lut = np.array([3, 1, 2], np.int16)  # e for diffs 0, 1, 2 with shift 0
    p = oracle.softmax_int([2, 1, 0], lut, 0, 2)  # e = [3, 1, 2], S = 6, one = 4
    exp = []
    for e in (3, 1, 2):
        q = Fraction(e * 4, 6)
        f = math.floor(q)
        r = q - f
        exp.append(f + 1 if (r > Fraction(1, 2) or (r == Fraction(1, 2) and f % 2)) else f)
    assert list(p) == exp


def test_attention_tolerance_kats(oracle):
    # attention.rs:96-140
    exp_lut = [int(round(math.exp(-i / 256.0) * 256)) for i in range(129)]
    out = oracle.attention_int([[64, 0], [64, 0]], [[64, 0], [64, 0]], [[100, -50], [100, -50]], 1 << 15, 4 + 15,
                               exp_lut, 0, 8, mask=[[1, 0], [1, 1]])
    assert abs(out[0][0] - 100) <= 1 and abs(out[0][1] + 50) <= 1 and abs(out[1][0] - 100) <= 1
    out = oracle.attention_int([[64, 0]], [[64, 0]] * 3, [[100, 0], [200, 0], [300, 0]], 1 << 15, 19, exp_lut, 0, 8)
    assert abs(out[0][0] - 200) <= 2 and abs(out[0][1]) <= 1
    L = oracle.lib()
    a = np.full(64, 30000, np.int16)
    assert L.or_dot_int(a.ctypes.data, a.ctypes.data, 64) == 64 * 30000 * 30000


def test_attention_selects_the_dominant_key(oracle):
    # One key far ahead of the rest -> the output is exactly that key's value row.
    from myelith_amd.luts import exp_lut
    lut = exp_lut()
    q = np.array([[1000, 0, 0, 0]], np.int16)
    k = np.array([[0, 0, 0, 0], [30000, 0, 0, 0], [0, 0, 0, 0]], np.int16)
    v = np.array([[7, 7, 7, 7], [111, -222, 333, -444], [9, 9, 9, 9]], np.int16)
    out = oracle.attention_int(q, k, v, 1 << 12, 14, lut, 6, 14)
    assert list(out[0]) == [111, -222, 333, -444]


# ---- integer_math.rs / mlp.rs / sampling.rs / prng.rs ---------------------------------------

def test_lut_lookup_and_mlp_smoke(oracle):
    lut = np.arange(100, 612, dtype=np.int16)  # 512 entries
    assert oracle.lut_lookup(0, lut, 0, 256) == lut[256]
    assert oracle.lut_lookup(-1000, lut, 0, 256) == lut[0]
    assert oracle.lut_lookup(1000, lut, 0, 256) == lut[511]
    # mlp.rs:91-121 smoke: deterministic, right length
    silu = [int(round(((x / 2.0) / (1 + math.exp(-x / 2.0))) * 64)) for x in range(-256, 256)]
    args = ([64, -32], [64, 0, 0, 64], [64, 0, 0, 64], [64, 32, 32, 64], 2, 2, [6, 6], [6, 6], [6, 6], silu,
            6, 6, 6, 6, 1, 256, 6, [6, 6])
    a, b = oracle.mlp_int(*args), oracle.mlp_int(*args)
    assert len(a) == 2 and list(a) == list(b)


def test_mlp_composes_linear_silu_linear(oracle):
    # mlp_int == linear(gate), linear(up), SiLU-LUT product, linear_pc(down): composition of pinned parts.
    rng = np.random.default_rng(5)
    H, I = 16, 24
    x = rng.integers(-3000, 3000, H).astype(np.int16)
    Wg, Wu = rng.integers(-127, 128, (I, H)).astype(np.int8), rng.integers(-127, 128, (I, H)).astype(np.int8)
    Wd = rng.integers(-127, 128, (H, I)).astype(np.int8)
    gs, us, ds = [rng.integers(5, 9, n).astype(np.uint8) for n in (I, I, H)]
    from myelith_amd.luts import silu_lut
    silu = silu_lut()
    of = rng.integers(7, 11, H).astype(np.uint8)
    out = oracle.mlp_int(x, Wg, Wu, Wd, H, I, gs, us, ds, silu, 10, 11, 10, 12, 6, 8192, 8, of)
    g = oracle.linear_w8a16(x, Wg.ravel(), H, gs, 10, 11)
    u = oracle.linear_w8a16(x, Wu.ravel(), H, us, 10, 10)
    wrap16 = lambda v: ((v + 32768) & 0xFFFF) - 32768
    h = []
    for gi, ui in zip(g, u):
        gd = oracle.rescale(int(gi), 11, 6)            # mlp.rs:56, i32 rescale
        idx = wrap16(wrap16(gd) + 8192)                # `as i16`, then the i16 add (integer_math.rs:45)
        a = int(silu[max(0, min(16383, idx))])
        h.append(max(-32768, min(32767, oracle.rescale_i64(a * int(ui), 8 + 10, 12))))
    ref = oracle.linear_w8a16_pc(np.array(h, np.int16), Wd.ravel(), I, ds, 12, of)
    assert np.array_equal(out, ref)


def test_argmax_first_maximum(oracle):
    assert oracle.argmax_int([1, 9, 3]) == 1           # sampling.rs:287-291
    assert oracle.argmax_int([5, 9, 9, 2, 9]) == 1      # ties: lowest index (spec.json tie_breaking)
    assert oracle.argmax_int([-2**31] * 4) == 0


def test_splitmix64(oracle):
    # prng.rs:332-349 reproducibility + known SplitMix64 outputs for state 0
    s1, z1 = oracle.splitmix64(42)
    s1b, z1b = oracle.splitmix64(42)
    assert (s1, z1) == (s1b, z1b)
    s2, z2 = oracle.splitmix64(s1)
    assert s1 != 42 and s2 != s1 and z1 != z2
    _, z = oracle.splitmix64(0)
    assert z == 0xE220A8397B1DCDAF  # first output of SplitMix64 seeded with 0 (published test value)


def test_sample_integer_cdf_closed_forms(oracle):
    """sample_integer_cdf (sampling.rs:27-46) against what its definition
    fixes, with SplitMix64 pinned above: constant logits (all weights 1: the
    token is r % n), the reference's own example [10, 20, 30] (weights 1, 11,
    21), a total of zero from a wrapped weight (token 0, state unchanged),
    an empty row, and determinism (sampling.rs:58-66)."""
    for n, state in ((1, 0), (7, 42), (152064, 2**64 - 1), (1000, 123456789)):
        ns, r = oracle.splitmix64(state)
        assert oracle.sample_integer_cdf([77] * n, state) == (r % n, ns)
    ns, r = oracle.splitmix64(42)
    t = r % 33
    assert oracle.sample_integer_cdf([10, 20, 30], 42) == (0 if t < 1 else 1 if t < 12 else 2, ns)
    assert oracle.sample_integer_cdf([10, 20, 30], 42) == oracle.sample_integer_cdf([10, 20, 30], 42)
    # z - min + 1 = 2^32 - 1 wraps to -1 in i32: total 1 - 1 = 0
    assert oracle.sample_integer_cdf([-2**31, 2**31 - 2], 99) == (0, 99)
    # a weight of 2^32 wraps to 0: total 1, threshold 0, token 0, state advanced
    ns, _ = oracle.splitmix64(5)
    assert oracle.sample_integer_cdf([-2**31, 2**31 - 1], 5) == (0, ns)
    assert oracle.sample_integer_cdf([], 7) == (0, 7)


def test_sample_integer_cdf_against_a_binary_search(oracle):
    """For positive weights the token is where the threshold falls in the
    cumulative weights: numpy's binary search (side right) over cumsum(w),
    on random logits and states."""
    rng = np.random.default_rng(8)
    for trial in range(40):
        n = int(rng.integers(1, 3000))
        z = rng.integers(-50000, 50000, n).astype(np.int32)
        state = int(rng.integers(0, 2**63)) * 2 + int(rng.integers(0, 2))
        w = z.astype(np.int64) - int(z.min()) + 1
        ns, r = oracle.splitmix64(state)
        thr = r % int(w.sum())
        want = int(np.searchsorted(np.cumsum(w), thr, side="right"))
        assert oracle.sample_integer_cdf(z, state) == (want, ns), trial


# ---- conformance vectors and LUT hashes --------------------------------------------------------

def _hash_tensor(data, dtype):
    # golden_runner.rs:48-66
    fmt = {"int8": "<i1", "int16": "<i2", "int32": "<i4"}[dtype]
    return hashlib.sha256(np.asarray(data, dtype=np.int64).astype(fmt).tobytes()).hexdigest()


def test_conformance_vectors(oracle):
    vecs = json.loads((GOLDEN / "op_vectors.json").read_text())
    for name, gv in vecs.items():
        for t in list(gv["inputs"].values()) + list(gv["outputs"].values()):
            assert _hash_tensor(t["data"], t["dtype"]) == t["hash"], name
    v = vecs["linear_w8a16_identity"]
    m = v["metadata"]
    W = np.array(m["W"], np.int8)
    y = oracle.linear_w8a16(v["inputs"]["x"]["data"], W.ravel(), W.shape[1], [m["weight_frac"]] * W.shape[0],
                            m["act_frac"], m["out_frac"])
    assert list(y) == v["outputs"]["y"]["data"]
    v = vecs["rmsnorm_basic"]
    m = v["metadata"]
    x = v["inputs"]["x"]["data"]
    y = oracle.rmsnorm_i16(x, [0] * len(x), v["inputs"]["gamma"]["data"], [m["gamma_shift"]] * len(x),
                           m["rsqrt_lut"], m["lut_input_shift"], m["lut_output_frac"], m["inv_n_q20"], m["out_frac"])
    assert list(y) == v["outputs"]["y"]["data"]
    v = vecs["softmax_basic"]
    m = v["metadata"]
    y = oracle.softmax_int(v["inputs"]["logits"]["data"], m["exp_lut"], m["lut_shift"], m["frac_bits"])
    assert list(y) == v["outputs"]["probs"]["data"]


def test_conformance_luts_are_the_closed_forms():
    # The LUTs embedded in the vectors are generate_rsqrt_lut(1023, 8, 8) and
    # generate_exp_lut(1024, 4, 8) (calibrate/src/luts.py).
    from myelith_amd.luts import exp_lut, rsqrt_lut
    vecs = json.loads((GOLDEN / "op_vectors.json").read_text())
    assert list(rsqrt_lut(1023, 8, 8)) == vecs["rmsnorm_basic"]["metadata"]["rsqrt_lut"]
    assert list(exp_lut(1024, 4, 8)) == vecs["softmax_basic"]["metadata"]["exp_lut"]


def test_lut_hashes_match_scale_packs():
    from myelith_amd.luts import LutSet
    hashes = json.loads((GOLDEN / "lut_hashes.json").read_text())
    for pack, hd in (("qwen2.5-0.5b", 64), ("qwen2.5-7b", 128)):
        got = LutSet.for_head_dim(hd).hashes()
        for name, meta in hashes[pack].items():
            assert got[name] == meta["sha256"], (pack, name)


def test_digest_byte_layout():
    # generate.rs:173-201: logits i32 LE, then the token u32 LE, no separators.
    steps = [([7, -3, 1], 0), ([2, 9, -1], 1)]
    b = b"".join(np.array(l, "<i4").tobytes() + np.uint32(t).astype("<u4").tobytes() for l, t in steps)
    assert b[:4] == (7).to_bytes(4, "little", signed=True)
    assert b[12:16] == (0).to_bytes(4, "little")
    assert len(b) == 2 * 4 * 4
    # FIPS 180-4 KAT for the hash itself ("abc")
    assert hashlib.sha256(b"abc").hexdigest() == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"


# ---- integer log-softmax (build-defined; pinned by closed forms) ---------------

def _samples_u64(seed=5):
    r = np.random.default_rng(seed)
    s = [1, 2, 3, 5, 16383, 16384, 16385, (1 << 40) - 1, 1 << 40, (1 << 46) + 12345]
    s += [1 << k for k in range(0, 47)] + [(1 << k) - 1 for k in range(2, 47)] + [(1 << k) + 1 for k in range(1, 47)]
    s += [int(v) for v in r.integers(1, 1 << 46, 2000, dtype=np.int64)]
    return s


def test_log2_q16_closed_form(oracle):
    """e = floor(log2 S) exactly; f = the first 16 fraction bits of log2(S / 2^e)
    up to the truncation of each squaring (which can only lower it, by at
    most one unit at these widths); powers of two have f = 0."""
    for S in _samples_u64():
        e, f = oracle.log2_q16(S)
        assert e == S.bit_length() - 1, S
        true = (math.log2(S) - e) * 65536
        assert 0 <= f <= 65535
        assert math.floor(true) - 1 <= f <= math.floor(true + 1e-9), (S, f, true)
        if S & (S - 1) == 0:
            assert f == 0
    assert oracle.log2_q16(0) == (0, 0)  # S = 0 is taken as 1


def test_ln_q16_closed_form(oracle):
    """ln(S / 2^14) in Q16 to within two units; exact zero at S = 2^14 and the
    exact RNE of k * ln2 at powers of two."""
    for S in _samples_u64(6):
        got = oracle.ln_q16(S)
        assert abs(got - math.log(S / 16384) * 65536) <= 2.0, S
    assert oracle.ln_q16(16384) == 0
    for k in range(0, 47):
        v = (k - 14) * 65536 * 744261118
        assert oracle.ln_q16(1 << k) == oracle.rshift_round_i64(v, 30)


def test_logsoftmax_matches_float_log_softmax(oracle):
    """Against the float64 log-softmax of the same Q6 logits: the exp LUT is
    exp(-x) to Q14, so the integer result is within 2e-3 nats."""
    from myelith_amd.luts import exp_lut
    lut = exp_lut()
    r = np.random.default_rng(11)
    for n in (1, 2, 17, 1000, 152064):
        z = r.integers(-20000, 20000, n).astype(np.int32)
        if n > 2:
            z[1] = z[0]  # ties
        zf = z.astype(np.float64) / 64.0
        mx = zf.max()
        lse = mx + math.log(np.exp(zf - mx).sum())
        for t in {0, n // 2, n - 1, int(np.argmax(z))}:
            got = oracle.logsoftmax_at(z, lut, t)
            assert abs(got / 65536.0 - (zf[t] - lse)) < 2e-3, (n, t)
    # one dominant logit: S = 2^14 exactly, so the maximum scores 0
    z = np.array([5000, -100000, -200000], np.int32)
    assert oracle.logsoftmax_at(z, lut, 0) == 0
    assert oracle.logsoftmax_at(z, lut, 3) == 0 and oracle.logsoftmax_at(z, lut, -1) == 0


def test_probability_sums_bound_the_i32_pv_path(oracle):
    """The decode P.V kernel for exp tables without negative entries sums
    p_j v_j in i32 (wrapping partial sums, exact when the total fits).  Its
    premise, checked on the oracle's softmax_int (softmax.rs:12-64) with the
    contract's exp table: every p_j lies in [0, 2^14] and sum_j p_j <= 2^14 +
    L/2 (each p_j is e_j 2^14 / S rounded to nearest), so |sum_j p_j v_j| <=
    (2^14 + L/2) 2^15 < 2^31 for L <= 65536.  Rows: equal scores (every p_j
    rounded up the most), two levels, a spike, spreads at the table's edge,
    and random rows, at lengths up to 4097."""
    from myelith_amd.luts import LutSet
    lut = np.asarray(LutSet.for_head_dim(128).exp, np.int16)
    assert lut.min() >= 0
    shift = 14 - 8  # score frac 14, exp-table input frac 8
    r = np.random.default_rng(11)
    rows = []
    for L in (1, 2, 3, 7, 100, 257, 1000, 2049, 4097):
        rows.append(np.zeros(L, np.int32))                                  # all equal
        rows.append(np.where(np.arange(L) % 2 == 0, 0, -(1 << 12)).astype(np.int32))  # two levels
        spike = np.full(L, -(1 << 30), np.int32)
        spike[L // 2] = 5
        rows.append(spike)
        edge = len(lut) << shift
        rows.append((-r.integers(0, edge + 64, L)).astype(np.int32))        # around the table's end
        rows.append(r.integers(-(1 << 20), 1 << 20, L).astype(np.int32))
    for z in rows:
        p = oracle.softmax_int(z, lut, shift, 14).astype(np.int64)
        L = len(z)
        assert p.min() >= 0 and p.max() <= 1 << 14, L
        assert p.sum() <= (1 << 14) + L // 2, (L, int(p.sum()))
        assert ((1 << 14) + L / 2) * 32768 < 2 ** 31 or L > 65536
