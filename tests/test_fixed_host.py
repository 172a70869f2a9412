"""The device fixed-point helpers of csrc/fixed.h, compiled for the host with
hipcc and checked against their general forms (no GPU needed).

softmax_div_round_pos (the probability division of the matrix-core
attention, softmax.rs:50-63 for a non-negative numerator and a positive sum,
with a 32-bit reciprocal) must equal softmax_div_round (the general signed
form, itself pinned against exact rational rounding in test_oracle_pins.py)
on edge cases -- s = 1, 2, near 2^31, ties, remainders whose doubling wraps
in i32 -- and on a million seeded pairs."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]

SRC = r"""
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
#include "fixed.h"
static uint64_t sm = 0x9E3779B97F4A7C15ull;
static uint64_t next() {
    uint64_t z = (sm += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static long bad = 0, n = 0;
static void check(int32_t num, int32_t s) {
    const int32_t a = softmax_div_round_pos(num, s, recip32_u32((uint32_t)s));
    const int32_t b = softmax_div_round(num, s, recip32((uint32_t)s));
    ++n;
    if (a != b && bad++ < 10) printf("num=%d s=%d fast=%d general=%d\n", num, s, a, b);
}
int main() {
    const int32_t ss[] = {1, 2, 3, 7, 16384, 32767, 65536, 1 << 30, (1 << 30) + 1, 2147483646, 2147483647};
    for (int32_t s : ss) {
        const int64_t S = s;
        const int64_t nums[] = {0, 1, 2, S / 2, S / 2 + 1, S - 1, S, S + 1, 3 * (S / 2), 1 << 29, (1 << 29) - 1,
                                2147483647, 2147483646, 1 << 30, (1 << 30) + 7};
        for (int64_t num : nums)
            if (num >= 0 && num <= 2147483647) check((int32_t)num, s);
    }
    for (int i = 0; i < 1000000; ++i) {
        const uint64_t z = next();
        const int32_t s = 1 + (int32_t)((z >> 1) % (i & 1 ? 2147483647u : 1u << (1 + (z & 30))));
        const int32_t num = (int32_t)((next() >> 33) % (i & 2 ? 2147483648ull : (1ull << 29) + 1));
        check(num, s);
        // ties: num = q * s + s / 2 for even s
        if ((s & 1) == 0 && s < (1 << 29)) check((int32_t)((uint32_t)((next() >> 40) % ((1u << 29) / (uint32_t)s + 1)) * (uint32_t)s + (uint32_t)s / 2), s);
    }
    printf("checked %ld, mismatches %ld\n", n, bad);
    return bad != 0;
}
"""


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(), reason="hipcc absent")
def test_softmax_div_round_pos_matches_general(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    src = tmp_path / "t.hip"
    src.write_text(SRC)
    exe = tmp_path / "t"
    subprocess.run([hipcc, "-O2", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
                    "-packed-fp32-ops", "-I", str(ROOT / "myelith_amd" / "csrc"), str(src), "-o", str(exe)],
                   check=True, capture_output=True, timeout=300)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout
    assert "mismatches 0" in r.stdout


RECIP_SRC = r"""
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
#include "fixed.h"
// the plain 33-step restoring division of 2^32 by d
static uint64_t recip_plain(uint32_t d) {
    uint64_t q = 0, r = 0;
    for (int bit = 32; bit >= 0; --bit) {
        r = (r << 1) | (bit == 32 ? 1u : 0u);
        q <<= 1;
        if (r >= d) { r -= d; q |= 1; }
    }
    return q;
}
int main() {
    long bad = 0, n = 0;
    auto check = [&](uint32_t d) {
        ++n;
        const uint64_t a = recip32(d), b = recip_plain(d);
        if (a != b && bad++ < 10) printf("d=%u fast=%llu plain=%llu\n", d, (unsigned long long)a, (unsigned long long)b);
        if (d && b != (d == 1 ? (1ull << 32) : (1ull << 32) / d) && bad++ < 10) printf("d=%u plain wrong\n", d);
    };
    for (uint32_t d = 0; d < 70000; ++d) check(d);
    for (int k = 1; k < 32; ++k)
        for (int e = -3; e <= 3; ++e) check((uint32_t)((1ull << k) + (int64_t)e));
    check(0xFFFFFFFFu);
    check(0xFFFFFFFEu);
    uint64_t s = 0x243F6A8885A308D3ull;
    for (int i = 0; i < 2000000; ++i) {
        s ^= s << 13; s ^= s >> 7; s ^= s << 17;
        check((uint32_t)(s >> (s & 31)));
    }
    printf("checked %ld, mismatches %ld\n", n, bad);
    return bad != 0;
}
"""


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(), reason="hipcc absent")
def test_recip32_matches_long_division(tmp_path):
    """recip32 starts its long division at the divisor's bit length; it must
    equal the plain 33-step division (and floor(2^32 / d)) for every d."""
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    src = tmp_path / "r.hip"
    src.write_text(RECIP_SRC)
    exe = tmp_path / "r"
    subprocess.run([hipcc, "-O2", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
                    "-packed-fp32-ops", "-I", str(ROOT / "myelith_amd" / "csrc"), str(src), "-o", str(exe)],
                   check=True, capture_output=True, timeout=300)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout
    assert "mismatches 0" in r.stdout



RSQRT_SRC = r"""
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
#include "ops.h"
int main(int argc, char** argv) {
    const uint32_t f = (uint32_t)atoi(argv[1]), sh = (uint32_t)atoi(argv[2]), n = (uint32_t)atoi(argv[3]);
    for (uint32_t x = 0; x < n; ++x) printf("%d\n", myl::rsqrt_closed(x, f, sh));
    return 0;
}
"""


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(), reason="hipcc absent")
def test_rsqrt_closed_form_equals_the_table(tmp_path):
    """rsqrt_closed (the norm setup's integer closed form) against the
    reference's float64 table generator (luts.py:32-49) at every entry, for
    the contract's parameters (input shift 8, 8 fraction bits) and for two
    others, one with an odd input shift."""
    from myelith_amd.luts import rsqrt_lut
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    src = tmp_path / "q.hip"
    src.write_text(RSQRT_SRC)
    exe = tmp_path / "q"
    subprocess.run([hipcc, "-O2", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
                    "-packed-fp32-ops", "-I", str(ROOT / "myelith_amd" / "csrc"), "-I", str(ROOT / "include"),
                    str(src), "-o", str(exe)], check=True, capture_output=True, timeout=300)
    for frac, shift, n in ((8, 8, 32768), (6, 4, 20000), (10, 3, 9000)):
        r = subprocess.run([str(exe), str(frac), str(shift), str(n)], capture_output=True, text=True, timeout=120)
        assert r.returncode == 0
        got = np.array([int(v) for v in r.stdout.split()], dtype=np.int64)
        want = rsqrt_lut(n - 1, shift, frac).astype(np.int64)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, (frac, shift, bad[:10], got[bad[:10]], want[bad[:10]])


RNE_SRC = r"""
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
#include "ops.h"
int main() {
    long bad = 0, n = 0;
    auto check = [&](int64_t v, uint32_t s) {
        ++n;
        const int64_t a = myl::rne_shift64_small(v, s), b = rshift_round64(v, (uint8_t)s);
        if (a != b && bad++ < 10) printf("v=%lld s=%u fast=%lld general=%lld\n", (long long)v, s, (long long)a, (long long)b);
    };
    const int64_t lim = (1ll << 62) - 1;
    uint64_t z = 0x9E3779B97F4A7C15ull;
    auto next = [&]() { z ^= z << 13; z ^= z >> 7; z ^= z << 17; return z; };
    for (uint32_t s = 0; s <= 62; ++s) {
        const int64_t half = s ? (1ll << (s - 1)) : 0;
        for (int64_t v : {(int64_t)0, (int64_t)1, (int64_t)-1, (int64_t)2, (int64_t)-2, (int64_t)3, (int64_t)-3, lim, -lim, lim - 1, -lim + 1}) check(v, s);
        for (int i = 0; i < 20000; ++i) {
            // ties and their neighbours: v = q 2^s + 2^(s-1) + d for q of either sign
            // |q| < 2^(61 - s) keeps |v| below 2^62
            const uint64_t qmax = s < 61 ? (1ull << (61 - s)) : 1ull;
            const int64_t q = (int64_t)(next() % qmax) * ((next() & 1) ? 1 : -1);
            const int64_t base = q * (int64_t)(1ull << s);
            for (int64_t d = -1; d <= 1; ++d) {
                const int64_t v = base + half + d;
                if (v <= lim && v >= -lim) check(v, s);
            }
            const int64_t r = (int64_t)(next() >> 2) * ((next() & 1) ? 1 : -1);  // |r| < 2^62
            check(r, s);
            check(r >> (next() % 62), s);
        }
    }
    printf("checked %ld, mismatches %ld\n", n, bad);
    return bad != 0;
}
"""


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(), reason="hipcc absent")
def test_rne_shift64_small_matches_rshift_round64(tmp_path):
    """The short round-half-even shift of the norm outputs (rms_out) equals
    rshift_round64 (fixed_point.rs:140-153) for every shift 0..62 on values
    below 2^62: ties of both signs and their neighbours, random values of
    every magnitude, the range ends."""
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    src = tmp_path / "n.hip"
    src.write_text(RNE_SRC)
    exe = tmp_path / "n"
    subprocess.run([hipcc, "-O2", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
                    "-packed-fp32-ops", "-I", str(ROOT / "myelith_amd" / "csrc"), "-I", str(ROOT / "include"),
                    str(src), "-o", str(exe)], check=True, capture_output=True, timeout=300)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout
    assert "mismatches 0" in r.stdout


def _rsqrt_wave_search(x: int, f: int, s: int) -> tuple[int, int]:
    """rsqrt_closed_wave (csrc/ops.h) step by step: 64 lanes test evenly
    spaced candidates of [lo, hi) per round, the ballot count moves the
    bounds.  Returns (value, rounds)."""
    if x == 0:
        return 1 << f, 0
    e = 2 * f + s + 2
    lo, hi = 0, (1 << (f + (s + 1) // 2)) + 1
    rounds = 0
    while hi - lo > 1:
        step = (hi - lo + 63) >> 6
        k = 0
        for lane in range(64):
            c = lo + step * (lane + 1)
            t = 2 * c - 1
            if c < hi and t * t * x <= (1 << e):
                k += 1
        nlo = lo + step * k
        hi = min(hi, nlo + step)
        lo = nlo
        rounds += 1
    return lo, rounds


def test_rsqrt_wave_search_equals_the_table():
    """The wave-wide rsqrt search of the decode norm staging (64 candidates per
    round) against the reference's float64 table generator (luts.py:32-49) at
    every entry of the contract's table and on the two other parameter sets,
    and it finishes in at most three rounds for the contract's range (4097
    candidates); the ballot count is a prefix of holding lanes, so a planted
    non-monotone test would fail here first."""
    from myelith_amd.luts import rsqrt_lut
    for frac, shift, n in ((8, 8, 32768), (6, 4, 4000), (10, 3, 3000)):
        want = rsqrt_lut(n - 1, shift, frac).astype(np.int64)
        worst = 0
        for x in range(n):
            v, rounds = _rsqrt_wave_search(x, frac, shift)
            assert v == want[x], (frac, shift, x, v, want[x])
            worst = max(worst, rounds)
        if (frac, shift) == (8, 8):
            assert worst <= 3


def _planes(x):
    """x = 256 hi + lo' + 128 with hi = x >> 8 (signed) and lo' = (x & 255) - 128,
    the byte planes of the matrix-core score product (csrc/qk_planes.h)."""
    x = x.astype(np.int64)
    return x >> 8, (x & 255) - 128


@pytest.mark.parametrize("hd", [64, 128])
def test_score_byte_plane_identity(hd):
    """The exact score of the decode-batch kernels' int8 matrix-core form:
    q . k = 65536 hh + 256 (hl + lh) + ll + 128 sum(q) + 128 sum(k) - 16384 hd,
    with sum(k) recovered from the products of an all-ones query row as
    256 sum(k_hi) + sum(k_lo') + 128 hd; every plane sum fits i32.  Random
    int16 vectors and the extremes (all -32768, all 32767, alternating)."""
    r = np.random.default_rng(hd)
    cases = [r.integers(-32768, 32768, (2, hd)) for _ in range(200)]
    for a in (-32768, 32767):
        cases.append(np.full((2, hd), a))
    alt = np.where(np.arange(hd) % 2 == 0, -32768, 32767)
    cases.append(np.stack([alt, -alt - 1]))
    for q, k in cases:
        qh, ql = _planes(q)
        kh, kl = _planes(k)
        assert np.array_equal(256 * qh + ql + 128, q) and np.array_equal(256 * kh + kl + 128, k)
        assert qh.min() >= -128 and qh.max() <= 127 and ql.min() >= -128 and ql.max() <= 127
        hh, mid, ll = int(qh @ kh), int(qh @ kl + ql @ kh), int(ql @ kl)
        for v in (hh, mid, ll):
            assert abs(v) < 2**31
        ones = np.ones(hd, dtype=np.int64)
        ksum = 256 * int(ones @ kh) + int(ones @ kl) + 128 * hd
        assert ksum == int(k.sum())
        dot = 65536 * hh + 256 * mid + ll + 128 * int(q.sum()) + 128 * ksum - 16384 * hd
        assert dot == int(q.astype(np.int64) @ k.astype(np.int64))
