"""The device Scale arithmetic (tritify_amd/csrc/kt_scale_dev.h), built for the host from the same source, against
Python's integers and against the oracle's restatement of kt-int (crates/00-kernels/kt-int/src/lib.rs:175-340).

Every kernel of the reference-semantics layers composes its Scales with these functions, so each arithmetic path
is exercised here on inputs chosen to reach it: udiv128's shift, double-estimate, 64-bit and long-division paths;
isqrt's double-root path (below 2^104) and the Newton iteration above it, around perfect squares; the 64-bit and
128-bit applies. Host and device share the source and IEEE double arithmetic (the estimates are corrected to the
exact integers, so their rounding details cannot change a result)."""
import ctypes as C
import math
import os
import shutil
import subprocess

import numpy as np
import pytest

from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
U64 = 2**64 - 1


@pytest.fixture(scope="module")
def sd(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("no g++ to build the host copy of the device Scale arithmetic")
    so = str(tmp_path_factory.mktemp("scale_dev") / "libscale_dev.so")
    subprocess.run([gxx, "-O2", "-std=c++17", "-shared", "-fPIC", "-I", os.path.join(ROOT, "tritify_amd", "csrc"),
                    os.path.join(ROOT, "tests", "scale_dev_host.cpp"), "-o", so], check=True)
    L = C.CDLL(so)
    u, i64, i32 = C.c_uint64, C.c_int64, C.c_int32
    pu, pi64, pi32 = C.POINTER(u), C.POINTER(i64), C.POINTER(i32)
    for name, res, args in (
        ("sd_udiv128", None, [u, u, u, u, pu, pu]),
        ("sd_isqrt", u, [u, u]),
        ("sd_from_ratio", None, [u, u, u, u, pi64, pi32]),
        ("sd_mul", None, [i64, i32, i64, i32, pi64, pi32]),
        ("sd_add", None, [i64, i32, i64, i32, pi64, pi32]),
        ("sd_recip", None, [i64, i32, pi64, pi32]),
        ("sd_rsqrt", None, [i64, i32, pi64, pi32]),
        ("sd_ge", C.c_int, [i64, i32, i64, i32]),
        ("sd_apply", i64, [i64, i32, i64]),
        ("sd_apply32", i64, [i64, i32, i32]),
        ("sd_requant_dyn", i32, [i64, i64]),
        ("sd_udiv_small_q", u, [u, u, i64]),
        ("sd_rq_apply", i32, [i64, i64]),
        ("sd_udiv64_small", u, [u, u]),
    ):
        f = getattr(L, name)
        f.restype, f.argtypes = res, args
    return L


def udiv(L, n, d):
    qh, ql = C.c_uint64(), C.c_uint64()
    L.sd_udiv128(n >> 64, n & U64, d >> 64, d & U64, C.byref(qh), C.byref(ql))
    return (qh.value << 64) | ql.value


def scale_out(f, *args):
    m, s = C.c_int64(), C.c_int32()
    f(*args, C.byref(m), C.byref(s))
    return m.value, s.value


def rand_bits(rng, bits):
    """A uniformly random integer of exactly `bits` bits (0 for bits == 0)."""
    if bits == 0:
        return 0
    v = 1 << (bits - 1)
    for b in range(0, bits - 1, 30):
        v |= int(rng.integers(0, 2**30)) << b
    return v & ((1 << bits) - 1) | (1 << (bits - 1))


def test_udiv128_every_path_is_floor_division(sd):
    rng = np.random.default_rng(11)
    cases = [(0, 1), (1, 1), (5, 7), (2**128 - 1, 1), (2**128 - 1, 3), (2**128 - 1, 2**64 - 1), (2**128 - 1, 2**64),
             (2**128 - 1, 2**127 + 1), (2**112 - 1, 2**63 + 1), (2**64 - 1, 2**64 - 1), (2**64 - 1, 3), (2**64, 3)]
    for _ in range(4000):
        db = int(rng.integers(1, 129))
        d = rand_bits(rng, db)
        path = int(rng.integers(0, 4))
        if path == 0:  # a power of two
            d = 1 << int(rng.integers(0, 64))
            n = rand_bits(rng, int(rng.integers(0, 129)))
        elif path == 1 and db <= 64:  # the double estimate: quotient below 2^49
            n = rand_bits(rng, min(128, db + int(rng.integers(0, 49))))
        elif path == 2 and db <= 64:  # both below 2^64, any quotient
            n = rand_bits(rng, int(rng.integers(db, 65)))
        else:  # long division
            n = rand_bits(rng, int(rng.integers(0, 129)))
        cases.append((n, d))
        # around exact multiples, where a rounded estimate lands one off
        q = n // d
        for nn in (q * d, q * d - 1, q * d + d - 1):
            if 0 <= nn < 2**128:
                cases.append((nn, d))
    for n, d in cases:
        assert udiv(sd, n, d) == n // d, (n, d)


def test_isqrt_is_the_floor_root_on_both_paths(sd):
    rng = np.random.default_rng(12)
    ns = [0, 1, 2, 3, 4, 2**104 - 1, 2**104, 2**104 + 1, 2**128 - 1, (2**52 - 1)**2, (2**52 + 1)**2 - 1]
    for _ in range(3000):
        ns.append(rand_bits(rng, int(rng.integers(1, 129))))
        k = rand_bits(rng, int(rng.integers(1, 65)))
        for v in (k * k - 1, k * k, k * k + 1, k * k + 2 * k):
            if 0 <= v < 2**128:
                ns.append(v)
    for n in ns:
        r = sd.sd_isqrt(n >> 64, n & U64)
        assert r == math.isqrt(n), n
        # the oracle restates the reference's Newton iteration: the same floor root
        assert O.isqrt_u128(n) == r, n


def rand_scale(rng, mant_bits=(1, 34), shift=(-40, 90)):
    return rand_bits(rng, int(rng.integers(*mant_bits))), int(rng.integers(*shift))


def test_scale_ops_equal_the_oracle(sd):
    rng = np.random.default_rng(13)
    for _ in range(3000):
        num = rand_bits(rng, int(rng.integers(0, 129)))
        den = rand_bits(rng, int(rng.integers(1, 129)))
        want = O.from_ratio(num, den)
        assert scale_out(sd.sd_from_ratio, num >> 64, num & U64, den >> 64, den & U64) == (want.mant, want.shift)
        (am, ash), (bm, bsh) = rand_scale(rng), rand_scale(rng)
        a, b = O.Scale(am, ash), O.Scale(bm, bsh)
        for f, g in ((sd.sd_mul, O.scale_mul), (sd.sd_add, O.scale_add)):
            w = g(a, b)
            assert scale_out(f, am, ash, bm, bsh) == (w.mant, w.shift), (f, am, ash, bm, bsh)
        assert bool(sd.sd_ge(am, ash, bm, bsh)) == O.scale_ge(a, b)
        for f, g in ((sd.sd_recip, O.scale_recip), (sd.sd_rsqrt, O.scale_rsqrt)):
            w = g(a)
            assert scale_out(f, am, ash) == (w.mant, w.shift), (f, am, ash)


def test_scale_ge_at_its_64_bit_bounds(sd):
    """Scale::ge's 64-bit comparison (mantissas below 2^33, shifts within 30) against the oracle at and beyond its
    bounds, including equal values written with different shifts."""
    rng = np.random.default_rng(19)
    cases = []
    for d in (-32, -31, -30, -29, -1, 0, 1, 29, 30, 31, 32):
        for ma, mb in ((2**33 - 1, 2**33 - 1), (2**33, 2**32), (1, 2**32), (2**32 + 1, 2**32)):
            cases.append((ma, 40, mb, 40 + d))
        for _ in range(40):
            ma = rand_bits(rng, int(rng.integers(1, 35)))
            cases.append((ma, 50, ma << max(d, 0) >> max(-d, 0) or 1, 50 + d))  # near-equal values
            cases.append((ma, 50, rand_bits(rng, int(rng.integers(1, 35))), 50 + d))
    for am, ash, bm, bsh in cases:
        if bm >= 2**62:  # mantissas are non-negative i64 values
            continue
        assert bool(sd.sd_ge(am, ash, bm, bsh)) == O.scale_ge(O.Scale(am, ash), O.Scale(bm, bsh)), (am, ash, bm, bsh)
        assert bool(sd.sd_ge(bm, bsh, am, ash)) == O.scale_ge(O.Scale(bm, bsh), O.Scale(am, ash)), (am, ash, bm, bsh)


def test_udiv64_small_at_exact_multiples(sd):
    """udiv64_small (d < 2^32, quotient < 2^40) on exact multiples k * d and their neighbours, where a rounded
    double quotient can land just below an integer or just above it."""
    rng = np.random.default_rng(18)
    cases = []
    for _ in range(20000):
        d = rand_bits(rng, int(rng.integers(1, 33)))
        k = rand_bits(rng, int(rng.integers(1, 41)))
        n = k * d
        cases += [(n + e, d) for e in (-1, 0, 1, d - 1) if 0 <= n + e < 2**64]
    for n, d in cases:
        assert sd.sd_udiv64_small(n, d) == n // d, (n, d)


def test_from_ratio_64_bit_paths_equal_the_oracle(sd):
    """from_ratio's 64-bit paths: den == 1 (Scale::mul and Scale::add; every bit length of num, the halves of a
    rounding at its boundary) and num < 2^62 with den < 2^32 (Scale::recip, the requant scales), either side of
    their bounds."""
    rng = np.random.default_rng(17)
    cases = []
    for bn in range(1, 129):
        for _ in range(12):
            cases.append((rand_bits(rng, bn), 1))
        k = max(bn - 32, 1)  # a value whose dropped bits are exactly one half, and one either side
        h = (rand_bits(rng, bn) >> k << k) | (1 << (k - 1))
        cases += [(h, 1), (h - 1, 1), (h + 1, 1)]
    for _ in range(4000):
        cases.append((rand_bits(rng, int(rng.integers(1, 66))), rand_bits(rng, int(rng.integers(1, 35)))))
    for num, den in cases:
        if num >= 2**128:
            continue
        want = O.from_ratio(num, den)
        assert scale_out(sd.sd_from_ratio, num >> 64, num & U64, den >> 64, den & U64) == (want.mant, want.shift), \
            (num, den)
    for _ in range(3000):
        (am, ash), (bm, bsh) = rand_scale(rng, (1, 33)), rand_scale(rng, (1, 33))
        w = O.scale_mul(O.Scale(am, ash), O.Scale(bm, bsh))
        assert scale_out(sd.sd_mul, am, ash, bm, bsh) == (w.mant, w.shift)


def test_from_ratio_general_path_equals_the_oracle(sd):
    """from_ratio past its 64-bit paths: a numerator past 2^62 or a denominator past 2^32 (the sums of squares over
    a row against its length, the fold's ratios), the halving of both past 64 bits, divisors of 60 to 64 bits, and
    quotients at a rounding boundary."""
    rng = np.random.default_rng(20)
    cases = []
    for _ in range(6000):
        cases.append((rand_bits(rng, int(rng.integers(60, 129))), rand_bits(rng, int(rng.integers(1, 129)))))
        cases.append((rand_bits(rng, int(rng.integers(1, 129))), rand_bits(rng, int(rng.integers(30, 66)))))
        cases.append((rand_bits(rng, int(rng.integers(64, 129))), int(rng.integers(1, 5000))))
    for bd in (60, 61, 62, 63, 64):
        for _ in range(300):
            d = rand_bits(rng, bd)
            q = rand_bits(rng, 32)
            cases += [(q * d + d // 2 + e, d) for e in (-1, 0, 1)]
    for num, den in cases:
        if num >= 2**128 or num <= 0 or den <= 0 or den >= 2**128:
            continue
        want = O.from_ratio(num, den)
        assert scale_out(sd.sd_from_ratio, num >> 64, num & U64, den >> 64, den & U64) == (want.mant, want.shift), \
            (num, den)


def test_applies_equal_the_oracle(sd):
    rng = np.random.default_rng(14)
    for _ in range(4000):
        am, ash = rand_scale(rng, (0, 34), (-8, 70))
        v32 = int(rng.integers(-(2**31), 2**31))
        want = O.scale_apply(O.Scale(am, ash), v32)
        assert sd.sd_apply(am, ash, v32) == want
        assert sd.sd_apply32(am, ash, v32) == want, (am, ash, v32)
        v64 = int(rng.integers(-(2**62), 2**62))
        assert sd.sd_apply(am, ash, v64) == O.scale_apply(O.Scale(am, ash), v64)
    for am, ash, v in ((2**32 - 1, 63, -(2**31)), (2**32 - 1, 0, 2**31 - 1), (1, 1, -1), (3, 1, -1), (2**31, 32, 1)):
        assert sd.sd_apply32(am, ash, v) == O.scale_apply(O.Scale(am, ash), v)


def test_requant_dyn_and_small_quotients(sd):
    rng = np.random.default_rng(15)
    for _ in range(4000):
        den = rand_bits(rng, int(rng.integers(1, 63)))
        v = int(rng.integers(-den, den + 1)) if den < 2**62 else den
        assert sd.sd_requant_dyn(v, den) == O.requant_dyn(v, 2**28, den), (v, den)
        d = rand_bits(rng, int(rng.integers(1, 63)))
        n = rand_bits(rng, min(127, d.bit_length() + int(rng.integers(0, 41))))
        if n // d < 2**40:
            assert sd.sd_udiv_small_q(n >> 64, n & U64, d) == n // d, (n, d)


def test_requant_by_reciprocal_equals_requant_dyn(sd):
    """rq_apply: the per-tensor requant without a division per value, on both sides of its 2^62 bound, at the
    rounding boundaries (|v| * 2^28 + den / 2 an exact multiple of den, and one below) and at |v| = den."""
    rng = np.random.default_rng(16)
    cases = [(1, 1), (1, -1), (1, 0), (2, 1), (3, 1), (3, 2), (2**62 - 1, 2**62 - 1), (2**62, 2**62 - 5),
             (2**63 - 1, -(2**63 - 1)), (2**63 - 1, 2**62), (5, 7)]
    for _ in range(6000):
        den = rand_bits(rng, int(rng.integers(1, 64)))
        v = int(rng.integers(-den, den + 1)) if den < 2**62 else rand_bits(rng, int(rng.integers(0, den.bit_length())))
        cases.append((den, v))
        # for odd den, the |v| with |v| * 2^28 + den / 2 an exact multiple of den, and its neighbours: the quotient
        # sits on a rounding boundary, where an estimate can land on either side
        if den % 2 == 1 and den > 2:
            a = (-(den // 2) * pow(2**28, -1, den)) % den
            for aa in (a - 1, a, a + 1):
                if 0 <= aa <= den:
                    cases += [(den, aa), (den, -aa)]
        cases.append((den, den))
        cases.append((den, -den))
    for den, v in cases:
        assert sd.sd_rq_apply(den, v) == O.requant_dyn(v, 2**28, den), (den, v)


def test_requant_outside_the_fast_range_is_the_references(sd):
    """rq_apply's cold path (|v| > den, den < 0, den >= 2^62) is layers.rs:33-39's i128 arithmetic, wrap to i32
    included: quotients far past 2^40, negative denominators (truncating division and half = den / 2 toward zero)
    and extreme v, against the oracle and against Python's integers."""
    rng = np.random.default_rng(17)

    def ref(v, den):  # layers.rs:33-39 with Python integers: truncating division, `as i32`
        prod, half = v * 2**28, (abs(den) // 2) * (1 if den > 0 else -1)
        t = lambda a, b: (abs(a) // abs(b)) * (1 if (a < 0) == (b < 0) else -1)
        r = t(prod + half, den) if prod >= 0 else -t(-prod + half, den)
        return (r + 2**31) % 2**32 - 2**31

    cases = [(1, 2**63 - 1), (1, -(2**63)), (3, -(2**63)), (-1, 5), (-3, 7), (-3, -7), (-(2**63), 2**63 - 1),
             (-(2**63) + 1, -(2**62)), (7, 2**40), (2**62, 2**63 - 1), (2**63 - 1, -(2**63)), (-2, 1), (-2, -1)]
    for _ in range(4000):
        den = rand_bits(rng, int(rng.integers(1, 64))) * (1 if rng.integers(0, 2) else -1)
        v = rand_bits(rng, int(rng.integers(0, 64))) * (1 if rng.integers(0, 2) else -1)
        v = max(min(v, 2**63 - 1), -(2**63))
        cases.append((den, v))
    for den, v in cases:
        want = O.requant_dyn(v, 2**28, den)
        assert want == ref(v, den), (den, v)
        assert sd.sd_rq_apply(den, v) == want, (den, v)
