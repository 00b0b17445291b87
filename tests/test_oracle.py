"""The CPU oracle (oracle/kt_oracle.c) pinned against the reference's golden vectors, known answers and the
mathematics -- before anything is compared with it. CPU only.

Each test names the reference test or golden it restates (paths relative to the tritify repository root).
"""
import json
import os
from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as O

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "goldens.json")))

KT_DEMO_HASH = "de67ba758bd0d1fb574fa64d7ff326e9d17f536d7725659228bebddcc6478bfa"  # README.md:74, REPRODUCE.md:15
CORPUS_HASH = "781285bb99bcd9cb5233f708466676db41e717b6971ce70508b57ed291478352"  # kt-runtime/src/tests_cuda.rs:9


# ----------------------------------------------------------------------------------------------------------------
# goldens of the reference


def test_kt_demo_default_hash():
    """apps/kt-demo: 64x768x768, seed 42, SHA-256 over the i64 outputs (README.md:74)."""
    qx, qw = O.gen_demo(64, 768, 768, 42)
    assert qx.min() >= -127 and qx.max() <= 127 and set(np.unique(qw)) == {-1, 0, 1}
    y = O.linear_cpu(qx, qw, 64, 768, 768)
    assert O.sha256_hex(y) == KT_DEMO_HASH


def test_config1_hashes():
    """benchmark config 1 (64x1024x1024, seed 42): the kt-demo generator at that shape, hashed over i64 and i32."""
    g = GOLD["config1"]
    qx, qw = O.gen_demo(64, 1024, 1024, 42)
    assert O.sha256_hex(qx) == g["x_sha256"] and O.sha256_hex(qw) == g["w_sha256"]
    y = O.linear_cpu(qx, qw, 64, 1024, 1024)
    assert O.sha256_hex(y) == g["y_i64_sha256"] == "0a86cb0cbfa63f2bb495cb70c4d166d6434f2114ba8ac69a4fe211bbc1ba6847"
    assert O.sha256_hex(y.astype(np.int32)) == g["y_i32_sha256"]
    assert g["y_i32_sha256"] == "54f29151282de81f8d1dfd028c3281cf5f063228fa94ffd2fa7a8e243ea61146"
    assert int(np.abs(y).max()) == 8413


@pytest.mark.parametrize("variant", [0, 1, 2])
def test_corpus_hash_on_every_cpu_variant(variant):
    """kt-runtime/src/tests.rs:33-45 (every_available_backend_is_byte_identical) with tests_cuda.rs:9's hash."""
    if not O.lib().kt_cpu_variant_available(variant):
        pytest.skip("this host lacks the variant")
    ys = [O.linear_cpu(c.x, c.w, c.rows, c.out, c.k, variant) for c in O.corpus()]
    assert O.sha256_hex(np.concatenate(ys)) == CORPUS_HASH


def test_corpus_shapes_and_extremes():
    """gate.rs:38-55: eight cases in order; the extremes are exactly +-WLEVELS."""
    cs = O.corpus()
    assert [c.label for c in cs] == ["k=1", "odd tail", "k=33", "k=1023", "k=4099 (long)", "threaded 8×512×2048",
                                     "extremes ±WLEVELS", "all +WLEVELS"]
    for c in cs:
        assert np.abs(c.x).max() <= O.WLEVELS and np.abs(c.w).max() <= O.WLEVELS
    assert set(np.abs(cs[6].x)) == {O.WLEVELS}


def test_flush_case_closed_form():
    """gate.rs:61-66: k = 1,342,192, every code +WLEVELS against rows +-WLEVELS gives +-k*WLEVELS^2."""
    c = O.flush_case()
    assert c.k == 1_342_192 == (O.KT_FLUSH + 1) * 16
    y = O.linear_cpu(c.x, c.w, 1, 2, c.k)
    want = c.k * O.WLEVELS**2
    assert want == 94_768_309_459_532_800
    assert list(y) == [want, -want]


def test_sha256_against_hashlib():
    """The C SHA-256 against Python's hashlib on every padding boundary."""
    rng = np.random.default_rng(5)
    for n in [0, 1, 3, 55, 56, 57, 63, 64, 65, 119, 120, 128, 1000, 4099]:
        a = rng.integers(0, 256, size=n, dtype=np.uint8)
        assert O.sha256_hex(a) == O.sha256_py(a)


# ----------------------------------------------------------------------------------------------------------------
# the CPU partition (crates/01-engine/kt-core/src/tests_partition.rs)


def _codes20(n, seed):
    s = np.random.default_rng(seed)
    return s.integers(-(1 << 20), 1 << 20, size=n).astype(np.int32)


def test_every_partition_gives_the_serial_loop():
    """tests_partition.rs:31-41; the serial reference is numpy's int64 matmul, independent of the flat indexing."""
    for rows in [0, 1, 2, 3, 7, 16, 31]:
        for out in [0, 1, 2, 17, 64]:
            for k in [0, 1, 5, 33]:
                x, w = _codes20(rows * k, 1 + rows), _codes20(out * k, 7 + out)
                want = (x.reshape(rows, k).astype(np.int64) @ w.reshape(out, k).astype(np.int64).T).reshape(-1)
                for threads in [1, 2, 3, 16, 64]:
                    assert np.array_equal(O.linear_threads(x, w, rows, out, k, threads), want), (rows, out, k, threads)
                assert np.array_equal(O.linear_cpu(x, w, rows, out, k), want)


def test_the_plan_follows_the_work():
    """tests_partition.rs:43-69."""
    wps, serial = 1 << 17, 1 << 20
    assert O.plan_threads(0, 0) == 1
    assert O.plan_threads(1, 2**64 - 1) == 1
    assert O.plan_threads(1 << 20, serial - 1) == 1
    assert O.plan_threads(1 << 20, 896 * 896) == 1
    assert O.plan_threads(1 << 20, 9 * wps) <= 3
    assert O.plan_threads(1 << 20, 10_000 * wps) <= 100
    assert O.plan_threads(2, 2**64 - 1) <= 2
    assert O.plan_threads(4864, 4864 * 896) <= 5


def test_every_planted_partition_is_caught():
    """kt-runtime/src/tests.rs:182-209: each planted partition is wrong on some shape of the grid."""
    for bad in (1, 2, 3):
        wrong = 0
        for rows, out, k in [(1, 17, 5), (3, 17, 5), (7, 64, 33), (16, 2, 33), (31, 17, 1)]:
            x = np.array([(i * 7919) % 1001 - 500 for i in range(rows * k)], dtype=np.int32)
            w = np.array([(i * 104729) % 997 - 498 for i in range(out * k)], dtype=np.int32)
            want = O.portable(x, w, rows, out, k)
            for t in (2, 3, 16, 64):
                if not np.array_equal(O.planted_partition(x, w, rows, out, k, bad, t), want):
                    wrong += 1
        assert wrong > 0, bad


def test_the_gate_catches_wrapping_and_float_accumulators():
    """kt-runtime/src/tests.rs:47-60 and the control that cannot fail (94-102)."""
    cs = O.corpus()
    diverged = lambda which: [c.label for c in cs
                              if not np.array_equal(O.planted_dot(c.x, c.w, c.rows, c.out, c.k, which),
                                                    O.portable(c.x, c.w, c.rows, c.out, c.k))]
    assert "extremes ±WLEVELS" in diverged(10)
    assert diverged(11)
    for c in cs:  # a reversed exact sum is no defect
        x, w = c.x.reshape(c.rows, c.k)[:, ::-1].copy(), c.w.reshape(c.out, c.k)[:, ::-1].copy()
        assert np.array_equal(O.portable(x, w, c.rows, c.out, c.k), O.portable(c.x, c.w, c.rows, c.out, c.k))


# ----------------------------------------------------------------------------------------------------------------
# digits


def test_every_code_splits_into_three_base81_digits_and_back():
    """kt-cuda/src/tests.rs:21-34 (the reference's digit scheme, kt-cuda/src/digits.rs:40-53)."""
    lv = O.WLEVELS
    step = 37  # a stride coprime to 81 visits every residue; the ends are checked exactly below
    for v in list(range(-lv, lv + 1, step)) + [-lv, -lv + 1, -1, 0, 1, lv - 1, lv]:
        d = O.split81(v)
        assert d is not None and all(abs(x) <= 40 for x in d) and O.join81(d) == v, v
    assert O.split81(lv) == [40, 40, 40] and O.split81(-lv) == [-40, -40, -40]
    for v in [lv + 1, -lv - 1, 2**31 - 1, -(2**31)]:
        assert O.split81(v) is None


def test_balanced_base256_digits_round_trip():
    """This build's digit scheme: p balanced base-256 digits reach exactly [lo_p, hi_p], each digit in [-128,127]."""
    lo, hi = -128, 127
    rng = np.random.default_rng(1)
    for p in range(1, 6):
        vals = list(range(lo, min(lo + 300, hi + 1))) + list(range(max(hi - 300, lo), hi + 1)) + [0, 1, -1]
        vals += [int(v) for v in rng.integers(max(lo, -(2**31)), min(hi, 2**31 - 1) + 1, size=2000)]
        for v in vals:
            if -(2**31) <= v < 2**31:
                d = O.split256(v, p)
                assert d is not None and all(-128 <= x <= 127 for x in d), (p, v)
                assert sum(x * 256**i for i, x in enumerate(d)) == v
        for v in (lo - 1, hi + 1):
            if -(2**31) <= v < 2**31:
                assert O.split256(v, p) is None, (p, v)
        lo, hi = lo * 256 - 128, hi * 256 + 127
    # every i32 fits five digits
    for v in (-(2**31), 2**31 - 1):
        assert O.split256(v, 5) is not None
    # the plane count of a slice is the fewest digits that hold all of it
    assert O.planes_for([0, 127, -128]) == 1
    assert O.planes_for([128]) == 2
    assert O.planes_for([O.WLEVELS, -O.WLEVELS]) == 3
    assert O.planes_for([2**31 - 1]) == 5


def test_every_small_code_splits_exhaustively():
    """Exhaustive over the whole 1- and 2-digit ranges."""
    for v in range(-32896, 32640):
        d = O.split256(v, 2)
        assert d is not None and d[0] + 256 * d[1] == v


def test_pack_puts_each_digit_where_the_layout_reads_it():
    """kt-cuda/src/tests.rs:36-52 for this build's layout [plane][row][kp], zero padding beyond k."""
    rows, k = 17, 35
    c = O.codes(rows * k, 3)
    p = O.pack_planes(c, rows, k, 3)
    assert p.shape == (3, rows, 64)
    for r in range(rows):
        for col in range(64):
            d = O.split256(int(c[r * k + col]), 3) if col < k else [0, 0, 0]
            assert list(p[:, r, col]) == d, (r, col)


# ----------------------------------------------------------------------------------------------------------------
# the plane emulator (the analogue of kt-cuda/src/host.rs)


def test_emulator_equals_portable_on_tails_and_extremes():
    """kt-cuda/src/tests.rs:54-65."""
    for rows, out, k in [(1, 1, 1), (3, 5, 7), (2, 17, 33), (16, 16, 16), (17, 33, 50), (1, 9, 4099), (20, 40, 300)]:
        x, w = O.codes(rows * k, rows), O.codes(out * k, 7 + out)
        assert np.array_equal(O.emu_linear(x, w, rows, out, k), O.portable(x, w, rows, out, k))
    lv, k = O.WLEVELS, 1027
    x = np.array([-lv if i % 3 == 0 else lv for i in range(2 * k)], dtype=np.int32)
    w = np.array([lv if i % 2 == 0 else -lv for i in range(3 * k)], dtype=np.int32)
    assert np.array_equal(O.emu_linear(x, w, 2, 3, k), O.portable(x, w, 2, 3, k))
    # any i32 codes: five planes, wrapping i64 exactly as the reference's release-mode sum
    x = np.array([2**31 - 1, -(2**31), 12345, -7], dtype=np.int32)
    w = np.array([2**31 - 1, 2**31 - 1, -(2**31), 3], dtype=np.int32)
    assert np.array_equal(O.emu_linear(x, w, 1, 1, 4), O.portable(x, w, 1, 1, 4))


def test_the_flush_sits_at_the_int32_bound():
    """Each (px, pw) flush interval is the last 256-multiple at which an int32 group sum cannot wrap: at the bound
    the unflushed product is exact, one chunk more wraps (the analogue of kt-cuda/src/tests.rs:67-77 and the
    NoFlush firing control, tests_cuda.rs:63-68, for this build's accumulator)."""
    for px, pw, code in [(1, 1, -128), (3, 3, -8_421_504)]:
        fk = O.flush_k(px, pw)
        n = min(px, pw)
        assert fk * n * 16384 <= 2**31 - 1 < (fk + 256) * n * 16384
        assert O.split256(code, px) == [-128] * px  # every digit at its largest magnitude
        for k, wraps in [(fk, False), (fk + 256, True)]:
            x = np.full(k, code, dtype=np.int32)
            want = O.portable(x, x, 1, 1, k)
            assert int(want[0]) == k * code * code
            assert np.array_equal(O.emu_linear(x, x, 1, 1, k, px, pw), want)
            no_flush = O.emu_linear(x, x, 1, 1, k, px, pw, flush=0)
            assert (not np.array_equal(no_flush, want)) == wraps, (px, pw, k)


def test_every_planted_emulator_defect_fires_where_it_should():
    """kt-cuda/src/tests.rs:109-132."""
    x, w = O.codes(4 * 300, 5), O.codes(20 * 300, 6)
    want = O.portable(x, w, 4, 20, 300)
    assert not np.array_equal(O.emu_linear(x, w, 4, 20, 300, drop_top=True), want)
    assert not np.array_equal(O.emu_linear(x, w, 4, 20, 300, wrong_carry=True), want)
    assert np.array_equal(O.emu_linear(x, w, 4, 20, 300, flush=0), want)


# ----------------------------------------------------------------------------------------------------------------
# kt-int (crates/00-kernels/kt-int/src/lib.rs)


def test_kt_int_doc_known_answers():
    """lib.rs:35-39."""
    three_quarters = O.from_ratio(3, 4)
    assert O.scale_apply(three_quarters, 8) == 6
    assert O.scale_apply(O.scale_mul(three_quarters, O.from_ratio(4, 3)), 9) == 9
    assert O.isqrt_u128(144) == 12


def test_requant_round_half_away_by_hand():
    """requant (lib.rs:78-86) on values worked by hand: x.5 goes away from zero, shifts <= 0 are exact."""
    assert O.requant(5, 1, 1) == 3 and O.requant(-5, 1, 1) == -3
    assert O.requant(3, 1, 1) == 2 and O.requant(-3, 1, 1) == -2
    assert O.requant(7, 1, 2) == 2 and O.requant(-6, 1, 2) == -2 and O.requant(5, 1, 2) == 1
    assert O.requant(9, 3, 0) == 27 and O.requant(-9, 3, -2) == -108
    m, s = O.frexp_scale(3.0, 53)
    for a in [-1_000_000, -7, 0, 1, 42, 999_999, 1_000_000_000_000]:  # lib.rs:557-566
        assert O.requant(a, m, s) == 3 * a


def test_requant_against_exact_rationals():
    rng = np.random.default_rng(11)
    for _ in range(3000):
        a = int(rng.integers(-(2**41), 2**41))
        m = int(rng.integers(0, 2**31))
        s = int(rng.integers(1, 70))
        q = Fraction(a * m, 2**s)
        want = (abs(q.numerator) * 2 + q.denominator) // (2 * q.denominator)  # floor(|q| + 1/2)
        want = want if q >= 0 else -want
        want = (want + 2**63) % 2**64 - 2**63  # `r as i64` (lib.rs:85) keeps the low 64 bits
        assert O.requant(a, m, s) == want


EDGE_ACC = [0, 1, -1, 2**31 - 1, -(2**31), 2**31, 12345, -98765, 2**40 + 3, 2**62, -(2**63), 2**63 - 1]
EDGE_MANT = [0, 1, -1, 3, 2**31 - 1, -(2**31), 1 << 30, -12345]
EDGE_SHIFT = [-(2**31), -200, -128, -64, -63, -62, -40, -33, -1, 0, 1, 2, 30, 31, 32, 33, 62, 63, 64, 65, 94, 95,
              96, 126, 127, 128, 200, 2**31 - 1]


def _exact_requant(a: int, m: int, s: int) -> int:
    """round(a * m / 2^s) half away from zero, saturated to i64, with exact rationals. |a * m| <= 2^126, so for
    s > 300 the value is below 2^-174 and rounds to 0; for s < -300 any nonzero product saturates."""
    p = a * m
    if p == 0:
        return 0
    if s > 300:
        return 0
    if s < -300:
        return 2**63 - 1 if p > 0 else -(2**63)
    q = Fraction(p) / Fraction(2) ** s
    r = (abs(q.numerator) * 2 + q.denominator) // (2 * q.denominator)  # floor(|q| + 1/2)
    r = r if q > 0 else -r
    return max(-(2**63), min(2**63 - 1, r))


def test_requant_sat_against_exact_rationals_on_every_edge():
    """The per-channel epilogue's requant (no i64 wrap) over the edges of i64 accumulators, int32 multipliers and
    every class of int32 shift, including shifts outside the 128-bit product's range."""
    for a in EDGE_ACC:
        for m in EDGE_MANT:
            for s in EDGE_SHIFT:
                assert O.requant_sat(a, m, s) == _exact_requant(a, m, s), (a, m, s)


def test_requant_sat_equals_requant_where_the_value_fits():
    """Where round(a * m / 2^s) fits i64, the saturating form and the reference's wrapping form agree."""
    rng = np.random.default_rng(12)
    for _ in range(4000):
        a = int(rng.integers(-(2**62), 2**62)) >> int(rng.integers(0, 62))
        m = int(rng.integers(-(2**31), 2**31))
        s = int(rng.integers(-40, 127))
        want = _exact_requant(a, m, s)
        if -(2**63) < want < 2**63 - 1:
            assert O.requant(a, m, s) == want == O.requant_sat(a, m, s), (a, m, s)


def _lcg(s):
    s = (s * 6364136223846793005 + 1442695040888963407) % 2**64
    return s


def test_requant_matches_float_baseline():
    """lib.rs:490-507: within 1 of round(accum * scale) in f64, exact on > 99%."""
    s, exact, n = 0xC0FFEE, 0, 20000
    for _ in range(n):
        s = _lcg(s); bits = (s % 42)
        s = _lcg(s); mag = s & max((1 << bits) - 1, 1)
        s = _lcg(s); accum = mag if s & 1 == 0 else -mag
        s = _lcg(s); e = -(s % 41)
        s = _lcg(s); frac = 1.0 + (s >> 40) / (1 << 24)
        sc = frac * 2.0**e
        m, sh = O.frexp_scale(sc, 53)
        got = O.requant(accum, m, sh)
        ref = round_away(accum * sc)
        assert abs(got - ref) <= 1
        exact += got == ref
    assert exact / n > 0.99


def round_away(v: float) -> int:
    import math

    return int(math.floor(abs(v) + 0.5)) * (1 if v >= 0 else -1)


def test_scale_arithmetic_against_f64():
    """lib.rs:590-650: from_ratio, mul/apply, recip, rsqrt, zero and exact scales."""
    rng = np.random.default_rng(3)
    for _ in range(3000):
        num, den = int(rng.integers(1, 2**50)), int(rng.integers(1, 2**50))
        sc = O.from_ratio(num, den)
        assert abs(sc.mant * 2.0**-sc.shift / (num / den) - 1) < 1e-8
        a = O.from_f64(1e-6 + float(rng.random()) * 16)  # the reference's ranges (lib.rs:605-606)
        b = O.from_f64(1e-3 + float(rng.random()))
        p = O.scale_mul(a, b)
        fa, fb, fp = (t.mant * 2.0**-t.shift for t in (a, b, p))
        assert abs(fp / (fa * fb) - 1) < 1e-8
        v = int(rng.integers(-(2**39), 2**39))
        assert abs(O.scale_apply(p, v) - round_away(v * fp)) <= 1
        x = 1e-7 + float(rng.random()) * 4096  # lib.rs:626
        r = O.scale_recip(O.from_f64(x))
        assert abs(r.mant * 2.0**-r.shift * x - 1) < 1e-8
        vv = 2.0 ** (-20 + 40 * float(rng.random()))
        q = O.scale_rsqrt(O.from_f64(vv))
        assert abs(q.mant * 2.0**-q.shift * vv**0.5 - 1) < 2e-9
    assert O.scale_apply(O.from_ratio(0, 5), 123) == 0
    four = O.from_ratio(4, 1)
    for v in [-7, 0, 1, 1000, 1_000_000_000]:
        assert O.scale_apply(four, v) == 4 * v
    assert O.scale_ge(O.from_ratio(3, 4), O.from_ratio(2, 3)) and not O.scale_ge(O.from_ratio(2, 3), O.from_ratio(3, 4))
    s = O.scale_add(O.from_ratio(1, 4), O.from_ratio(1, 2))
    assert O.scale_apply(s, 1000) == 750


def test_scale_to_i32_keeps_the_value():
    """The int32 multiplier of the per-channel epilogue: mant in [2^30, 2^31), value within one ulp of 2^-30."""
    rng = np.random.default_rng(4)
    for _ in range(2000):
        num, den = int(rng.integers(1, 2**40)), int(rng.integers(1, 2**40))
        a = O.from_ratio(num, den)
        b = O.scale_to_i32(a)
        assert 2**30 <= b.mant < 2**31
        assert abs(Fraction(b.mant, 2**b.shift) - Fraction(a.mant, 2**a.shift)) <= Fraction(1, 2**b.shift)


def test_quant_to_and_requant_dyn_against_rationals():
    """layers.rs:23-39 against exact rational rounding (half away from zero)."""
    rng = np.random.default_rng(9)
    for xmax in [1, 2, 3, 7, 1000, 65537, 2**28, 2**31 - 1]:
        d = rng.integers(-xmax, xmax + 1, size=200).astype(np.int64)
        d[:3] = [xmax, -xmax, 0]
        got = O.quant_to(d.astype(np.int32), xmax)
        for v, g in zip(d, got):
            q = Fraction(int(v) * O.WLEVELS, xmax)
            want = int((abs(q) + Fraction(1, 2)).__floor__()) * (1 if q >= 0 else -1)
            assert g == want
        assert got[0] == O.WLEVELS and got[1] == -O.WLEVELS
    for _ in range(2000):
        v = int(rng.integers(-(2**45), 2**45))
        den = int(rng.integers(1, 2**46))
        den = max(den, abs(v))
        q = Fraction(v * O.ACT_LEVELS, den)
        want = int((abs(q) + Fraction(1, 2)).__floor__()) * (1 if q >= 0 else -1)
        assert O.requant_dyn(v, O.ACT_LEVELS, den) == want


# ----------------------------------------------------------------------------------------------------------------
# the 12-bit weight path


def test_w12_layout_round_trips_every_code():
    """Exhaustive: all 4096 codes, placed so each (row, k) position class is hit, decode back exactly; and the
    fragment rule the kernels use holds on the packed bytes: lane l = (n % 32) + 32 h of block (n // 32, k // 32)
    carries k = 32 kb + 16 h + t, t = 0..15, as 16 lo bytes in t order and 8 nib bytes whose dwords D0, D1 give
    hi(t) for t = 0..15 as D0 & 0x0F0F0F0F, (D0 >> 4) & .., D1 & .., (D1 >> 4) & .. ."""
    n, k = 64, 64
    codes = np.arange(-2048, 2048, dtype=np.int32).reshape(n, k)
    lo, nib = O.w12_pack(codes, n, k)
    for r in range(n):
        for c in range(k):
            assert O.w12_get(lo, nib, k, r, c) == codes[r, c]
    KB = k // 32
    his = ((codes + 2048) >> 8).astype(np.int64)
    los = (codes & 255) - 128
    for nb in range(n // 32):
        for kb in range(KB):
            for l in range(64):
                frag = (nb * KB + kb) * 64 + l
                row, ks = nb * 32 + l % 32, kb * 32 + 16 * (l // 32)
                assert list(lo[frag * 16:frag * 16 + 16]) == list(los[row, ks:ks + 16])
                d0, d1 = (int(v) for v in nib[frag * 8:frag * 8 + 8].view(np.uint32))
                got = []
                for d in (d0 & 0x0F0F0F0F, (d0 >> 4) & 0x0F0F0F0F, d1 & 0x0F0F0F0F, (d1 >> 4) & 0x0F0F0F0F):
                    got += [(d >> (8 * b)) & 255 for b in range(4)]
                assert got == list(his[row, ks:ks + 16])
    # padding rows / k are zero digits
    lo2, nib2 = O.w12_pack(np.full(3 * 5, 7, np.int32), 3, 5)
    assert lo2.size == 32 * 64 and (lo2 != 0).sum() == 15 and (nib2 != 0).sum() > 0


def test_w12_recombination_equals_the_direct_sum():
    """S_lo + 256 S_hi - 1920 sum(x) equals the direct i64 sum, on tails (k not a multiple of 64) and extremes."""
    rng = np.random.default_rng(2)
    for m, n, k in [(1, 1, 1), (3, 5, 7), (2, 17, 33), (5, 9, 64), (4, 13, 100), (16, 40, 300)]:
        x = rng.integers(-128, 128, size=m * k).astype(np.int32)
        w = rng.integers(-2048, 2048, size=n * k).astype(np.int32)
        lo, nib = O.w12_pack(w, n, k)
        assert np.array_equal(O.w12_linear(x, lo, nib, m, n, k), O.portable(x, w, m, n, k))
    k = 4096
    for xv, wv in [(-128, -2048), (127, 2047), (-128, 2047), (127, -2048)]:
        x = np.full(k, xv, dtype=np.int32)
        w = np.full(k, wv, dtype=np.int32)
        lo, nib = O.w12_pack(w, 1, k)
        assert int(O.w12_linear(x, lo, nib, 1, 1, k)[0]) == k * xv * wv


def test_config2_generators_match_fixtures():
    """The benchmark config-2 inputs (this build's integer-only samplers) are stable: hashes pinned in goldens.json."""
    g = GOLD["config2"]
    w = O.gen_w12(g["w_seed"], 4096 * 4096)
    assert O.sha256_hex(w) == g["w_sha256"]
    assert w.min() == -2048 and w.max() == 2047
    x = O.gen_act_gauss(g["x_seed"], g["sigma"], 2048 * 4096)
    assert O.sha256_hex(x) == g["x_sha256"]
    assert abs(float(x.mean())) < 0.2 and 39.0 < float(x.std()) < 41.0 and np.abs(x).max() <= 127
    mant, shift = O.channel_scales(w, 4096, 4096, g["sigma"])
    assert O.sha256_hex(mant) == g["mant_sha256"] and O.sha256_hex(shift) == g["shift_sha256"]
    assert mant.min() >= 2**30 and mant.max() < 2**31
