"""The reference decoder at its own semantics, on the CPU: the oracle's restatement (oracle/kt_oracle_refdec.c) is
pinned by the reference's synthetic-decoder golden, by the properties the reference's own tests assert of a run,
and by closed forms of its ops; the product's offline tables (tritify_amd/csrc/kt_refdec.hip, host part) equal the
oracle's. No GPU call."""
import math

import numpy as np
import pytest

from oracle import oracle as O


@pytest.fixture(scope="module")
def synth():
    return O.RefModel(7)


def test_verify_repro_synthetic_golden(synth):
    """verify_repro --synthetic (seed 7, the fixed 12-token prompt, 32 greedy tokens) prints logits_hash
    8109ebad... (REPRODUCE.md:17; repro.rs:260-300; verify_repro.rs:71-78)."""
    toks, run, per_pos = synth.generate(O.SYNTH_PROMPT, 32)
    assert run == O.SYNTH_HASH
    assert len(toks) == 32 and all(0 <= t < 64 for t in toks)
    assert len(per_pos) == len(O.SYNTH_PROMPT) + 32 - 1  # the last token's logits are never computed


def test_run_properties_of_the_reference_tests(synth):
    """repro.rs's tests: a run twice gives the same bits; another seed is another model and differs at position 0;
    tests_generate.rs: a longer run extends a shorter one and the hash covers every step."""
    p9 = O.SYNTH_PROMPT[:9]
    a = synth.generate(p9, 12)
    assert synth.generate(p9, 12) == a
    assert len(a[2]) == 9 + 12 - 1
    b = O.RefModel(8).generate(p9, 4)
    assert b[2][0] != a[2][0]
    short, long_ = synth.generate([4, 5], 3), synth.generate([4, 5], 5)
    assert long_[0][:3] == short[0]
    assert long_[1] != short[1]
    assert long_[2][:len(short[2])] == short[2]


def real(codes, sc):
    return np.asarray(codes, dtype=np.float64) * sc[0] * 2.0 ** (-sc[1])


def test_rmsnorm_closed_forms():
    """A row of one repeated value normalizes to gamma exactly up to the output grid: every code is +-2^28 when
    gamma is constant, and the real value is gamma / sqrt(1 + eps / x^2). A zero row or a zero scale gives zeros at
    Scale::ZERO. Scaling x's codes by 3 changes nothing but the scale bookkeeping (within one output unit).

    The closed form holds while mean(x^2) and eps are within 2^32 of each other: Scale::add aligns the two mantissas
    and, when the aligned sum needs more than 64 bits, Scale::from_ratio's reduction (kt-int/src/lib.rs:196-203)
    halves the denominator 1 to 0 and resets it to 1, so the sum loses that power of two. The reference's RmsNorm
    carries this (the synthetic golden depends on it); the last case shows it: x real = 2^18, a 2^39 spread."""
    dim = 96
    g = np.full(dim, 200000, dtype=np.int32)
    gs, eps = (1342177280, 50), O.Scale(1125899907, 50)  # gamma real 200000 * 1.19e-6; eps = 1e-6
    xs = (1073741824, 40)
    y, ys = O.rd_rmsnorm(np.full(dim, 2**28, dtype=np.int32), 1, dim, xs, g, gs, (eps.mant, eps.shift))
    gam = 200000 * gs[0] * 2.0 ** -gs[1]
    # mean(x^2) = 2^36 = 2^31 * 2^5 against eps at shift 50: aligned, the sum has 32 + 55 = 87 bits and loses 2^23;
    # the inverse square root is then 2^11.5 too large
    assert abs(real(y[:1], ys)[0] - gam * 2**11.5) <= 1e-6 * gam * 2**11.5
    for v in (1, 5, -40, 300):
        y, ys = O.rd_rmsnorm(np.full(dim, v, dtype=np.int32), 1, dim, xs, g, gs, (eps.mant, eps.shift))
        assert (np.abs(y) == 2**28).all() and (np.sign(y) == np.sign(v)).all()
        xr = v * 2.0 ** -10
        want = 200000 * gs[0] * 2.0 ** -gs[1] / math.sqrt(1 + 1e-6 / xr**2)
        assert abs(real(y[:1], ys)[0] * np.sign(v) - want) <= 1e-6 * abs(want)
    y, ys = O.rd_rmsnorm(np.zeros(dim, dtype=np.int32), 1, dim, xs, g, gs, (eps.mant, eps.shift))
    assert not y.any() and ys == (0, 0)
    y, ys = O.rd_rmsnorm(np.full(dim, 7, dtype=np.int32), 1, dim, (0, 0), g, gs, (eps.mant, eps.shift))
    assert not y.any() and ys == (0, 0)
    rng = np.random.default_rng(3)
    x = rng.integers(-(2**14), 2**14, size=dim).astype(np.int32)  # mean(x^2) near 2^6: no bits lost in the add
    gr = rng.integers(-200000, 200000, size=dim).astype(np.int32)
    y1, s1 = O.rd_rmsnorm(x, 1, dim, xs, gr, gs, (eps.mant, eps.shift))
    y3, s3 = O.rd_rmsnorm(3 * x, 1, dim, (xs[0], xs[1] + 2), gr, gs, (eps.mant, eps.shift))  # 3x/4: scale-free
    r1, r3 = real(y1, s1), real(y3, s3)
    assert np.abs(r1 - r3).max() <= 4 * max(s1[0] * 2.0 ** -s1[1], s3[0] * 2.0 ** -s3[1]) + 1e-7 * np.abs(r1).max()


def test_add_closed_forms():
    """add equals the real sum within one unit of its output scale; adding a zero-scale tensor is the first tensor
    requantized by its own maximum (the identity when that maximum is 2^28); it is symmetric in its operands."""
    rng = np.random.default_rng(4)
    a = rng.integers(-(2**28), 2**28, size=300).astype(np.int32)
    b = rng.integers(-(2**28), 2**28, size=300).astype(np.int32)
    a[0] = 2**28
    sa, sb = (1610612736, 61), (1288490189, 63)
    y, ys = O.rd_add(a, sa, b, sb)
    unit = ys[0] * 2.0 ** -ys[1]
    assert np.abs(real(y, ys) - (real(a, sa) + real(b, sb))).max() <= unit * (1 + 1e-9)
    yb, sbb = O.rd_add(b, sb, a, sa)
    assert np.array_equal(yb, y) and sbb == ys
    y0, s0 = O.rd_add(a, sa, np.zeros(300, dtype=np.int32), (0, 0))
    assert np.array_equal(y0, a) and s0[0] * 2.0 ** -s0[1] == sa[0] * 2.0 ** -sa[1]  # same value, renormalized


def test_swiglu_tracks_silu_times_up(synth):
    """h = silu(g) * u in real values within the CodeLut's resolution (60 / 65535 in g), the right tail is the
    identity, the left tail is 0."""
    rng = np.random.default_rng(5)
    n = 4000
    g = rng.integers(-(2**28), 2**28, size=n).astype(np.int32)
    u = rng.integers(-(2**28), 2**28, size=n).astype(np.int32)
    gs = (1073741824, 53)  # g real in [-32, 32): both tails are reached
    us = (1073741824, 58)
    h, hs = O.rd_swiglu_act(synth, g, gs, u, us)
    gr, ur = real(g, gs), real(u, us)
    silu = gr / (1 + np.exp(-gr))
    want = np.where(gr > 30, gr, np.where(gr < -30, 0.0, silu)) * ur
    err = np.abs(real(h, hs) - want)
    tol = (60 / 65535) * 1.1 * np.abs(ur) + 2 * hs[0] * 2.0 ** -hs[1]
    assert (err <= tol).all()


def test_attention_first_step_returns_v(synth):
    """At position 0 the softmax has one entry: every head returns its kv head's v (rotated nothing), so the
    concatenated output is v repeated per group, requantized by its own maximum."""
    cache = O.RefCache(synth)
    c = synth.cfg
    rng = np.random.default_rng(6)
    q = rng.integers(-(2**28), 2**28, size=c["nh"] * c["hd"]).astype(np.int32)
    k = rng.integers(-(2**28), 2**28, size=c["nkv"] * c["hd"]).astype(np.int32)
    v = rng.integers(-(2**28), 2**28, size=c["nkv"] * c["hd"]).astype(np.int32)
    vs = (1288490189, 60)
    o, os_ = O.rd_attention_core(cache, q, (1073741824, 58), k, (1073741824, 59), v, vs, 0)
    group = c["nh"] // c["nkv"]
    want = np.concatenate([v[(h // group) * c["hd"]:(h // group + 1) * c["hd"]] for h in range(c["nh"])])
    assert np.abs(real(o, os_) - real(want, vs)).max() <= os_[0] * 2.0 ** -os_[1]


def test_product_tables_equal_the_oracle(synth):
    """The product's host-side CodeLut, RoPE and Scale::from_f64 builders give the oracle's integers."""
    from tritify_amd import backend as B

    for which, kind, lo, hi, rid in (("exp", B.LUT_EXP, -30.0, 0.0, False), ("silu", B.LUT_SILU, -30.0, 30.0, True)):
        codes, inv, lo_index, cs = synth.lut(which)
        pc, pl = B.ref_codelut(kind, lo, hi, 16, 20, rid)
        assert np.array_equal(pc, codes)
        assert (pl.inv_mant, pl.inv_shift, pl.lo_index, pl.code_mant, pl.code_shift, pl.n) == (
            inv[0], inv[1], lo_index, cs[0], cs[1], 1 << 16)
    (cm, csh, csg, sm, ssh, ssg), isq = synth.rope()
    c = synth.cfg
    pcos, psin = B.ref_rope_tables(c["max_seq"], c["hd"], c["theta"])
    assert np.array_equal(pcos["mant"], cm) and np.array_equal(pcos["shift"], csh)
    assert np.array_equal(pcos["sign"], csg.astype(np.int32))
    assert np.array_equal(psin["mant"], sm) and np.array_equal(psin["shift"], ssh)
    assert np.array_equal(psin["sign"], ssg.astype(np.int32))
    assert B.ref_scale_from_f64(1.0 / math.sqrt(c["hd"])) == isq
    assert B.ref_scale_from_f64(c["eps"]) == synth.norm(0, "in_norm")[2]
    # the tables' closed forms: exp(0) = 2^20 at the last entry; cos(0) = 1 with sign +, sin(0) = 0
    exp_codes = synth.lut("exp")[0]
    assert exp_codes[-1] == 2**20 and exp_codes[0] == round(math.exp(-30) * 2**20)
    assert (np.diff(exp_codes) >= 0).all()
    half = c["hd"] // 2
    assert (pcos["mant"][:half] == 2**30).all() and (pcos["shift"][:half] == 30).all()
    assert (psin["mant"][:half] == 0).all()


def test_the_oracle_model_from_given_codes_reproduces_the_golden():
    """RefModel.from_weights (the checker of device models built from other inputs) over the seed-7 model's own
    codes and Scales gives verify_repro's 8109ebad... and the same tokens."""
    m = O.RefModel(7)
    m2 = O.RefModel.from_weights(O.SYNTH_CFG, *m.weights())
    toks, run, pos = m2.generate(O.SYNTH_PROMPT, 32)
    assert run == O.SYNTH_HASH
    assert (toks, pos) == m.generate(O.SYNTH_PROMPT, 32)[::2]
