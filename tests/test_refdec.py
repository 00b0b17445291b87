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


# ---- the batched forward (CausalLM::forward_int: embed_int, blocks_int, head_int over a whole sequence) ----------


def test_a_one_token_forward_is_the_decode_step_at_position_zero():
    """Over one token the whole-sequence forward and decode_step at position 0 are the same integers (the
    attention's one cached step has the sequence's score and v scales); decode_step is pinned by 8109ebad..."""
    import hashlib

    for seed, cfg in ((7, O.SYNTH_CFG), (5, dict(dim=64, layers=2, nh=4, nkv=2, hd=16, hidden=96, vocab=40,
                                                 eps=1e-6, theta=1.0e6, max_seq=16))):
        m = O.RefModel(seed, cfg)
        for t in (0, 3, cfg["vocab"] - 1):
            lg, ls = m.forward([t])
            h = hashlib.sha256(np.int64(ls[0]).tobytes() + np.int32(ls[1]).tobytes() + lg.astype("<i4").tobytes())
            assert h.hexdigest() == m.generate([t], 1)[2][0], (seed, t)


def _dq(codes, sc):
    return np.asarray(codes, np.float64) * (sc[0] * 2.0 ** -sc[1])


def _lin_ref(x, w):
    """QuantLinear::forward_ref (layers.rs:330-349): f64 dot with the dequantized weights, to f32."""
    return (np.asarray(x, np.float64) @ _dq(*w).T).astype(np.float32)


def _rope_ref(v, p, hd, theta):
    half = hd // 2
    j = np.arange(half)
    ang = p * theta ** (-(2.0 * j) / hd)
    c, s = np.cos(ang), np.sin(ang)
    a, b = v[:half].copy(), v[half:].copy()
    v[:half], v[half:] = a * c - b * s, b * c + a * s


def _attention_ref(x, wq, wk, wv, wo, nh, nkv, hd, theta):
    """Attention::forward_ref (attention.rs:603-663): float q / k / v, RoPE, causal softmax, o."""
    seq = x.shape[0]
    q = _lin_ref(x, wq).astype(np.float64).reshape(seq, nh, hd)
    k = _lin_ref(x, wk).astype(np.float64).reshape(seq, nkv, hd)
    v = _lin_ref(x, wv).astype(np.float64).reshape(seq, nkv, hd)
    for i in range(seq):
        for h in range(nh):
            _rope_ref(q[i, h], i, hd, theta)
        for h in range(nkv):
            _rope_ref(k[i, h], i, hd, theta)
    out = np.zeros((seq, nh * hd), np.float32)
    for h in range(nh):
        kv = h // (nh // nkv)
        for i in range(seq):
            sc = np.array([q[i, h] @ k[j, kv] for j in range(i + 1)]) / np.sqrt(hd)
            e = np.exp(sc - sc.max())
            out[i, h * hd:(h + 1) * hd] = ((e / e.sum()) @ v[:i + 1, kv]).astype(np.float32)
    return _lin_ref(out, wo)


def test_attention_gqa_causal_tracks_float():
    """attention_gqa_causal_tracks_float_and_is_deterministic (tests.rs:184-198): seed 0x4242, dim 32, 4 / 2 heads
    of 8, 5 rows, max_seq 16, theta 1e4; the integer attention within 3% of its float twin's peak."""
    dim, nh, nkv, hd, seq = 32, 4, 2, 8, 5
    qd, kvd = nh * hd, nkv * hd
    s = 0x4242
    ws = {}
    for name, n in (("wq", qd * dim), ("wk", kvd * dim), ("wv", kvd * dim), ("wo", dim * qd)):
        f, s = O.vecf(s, n)
        ws[name] = O.quant_weights(f)
    xf, s = O.vecf(s, seq * dim)
    x, xs = O.from_reals(xf.astype(np.float64))
    m = O.RefModel.from_weights(dict(dim=dim, layers=1, nh=nh, nkv=nkv, hd=hd, hidden=8, vocab=2, eps=1e-6,
                                     theta=10000.0, max_seq=16),
                                (np.zeros((2, dim), np.int32), (0, 0)), (np.zeros(dim, np.int32), (0, 0)),
                                (np.zeros((2, dim), np.int32), (0, 0)), [])
    shapes = {"wq": qd, "wk": kvd, "wv": kvd}
    proj = {n: O.quant_linear_forward(x, seq, dim, xs, ws[n][0], shapes[n], ws[n][1])[:2] for n in shapes}
    runs = []
    for _ in range(2):
        o, os_ = m.attention_prefill(seq, proj["wq"][0], proj["wq"][1], proj["wk"][0], proj["wk"][1],
                                     proj["wv"][0], proj["wv"][1])
        y, ys, _, _ = O.quant_linear_forward(o, seq, qd, os_, ws["wo"][0], dim, ws["wo"][1])
        runs.append((y.copy(), ys))
    assert np.array_equal(runs[0][0], runs[1][0]) and runs[0][1] == runs[1][1], "not deterministic"
    w = {n: (ws[n][0].reshape(-1, dim if n != "wo" else qd), ws[n][1]) for n in ws}
    r = _attention_ref(_dq(x, xs).astype(np.float32).reshape(seq, dim), w["wq"], w["wk"], w["wv"], w["wo"], nh,
                       nkv, hd, 10000.0)
    got = _dq(runs[0][0], runs[0][1]).reshape(seq, dim)
    assert np.abs(got - r.astype(np.float64)).max() <= 3e-2 * np.abs(r).max()


def test_full_decoder_forward_tracks_float():
    """full_decoder_forward_tracks_float_and_is_deterministic (tests.rs:262-323): seed 0xD00D, dim 16, 2 layers,
    4 / 2 heads of 4, hidden 32, vocab 20, max_seq 8, tokens [5, 6, 7, 8]: logits within 10% of the float twin's
    peak and the same argmax at every position."""
    cfg = dict(dim=16, layers=2, nh=4, nkv=2, hd=4, hidden=32, vocab=20, eps=1e-6, theta=10000.0, max_seq=8)
    m = O.RefModel(0xD00D, cfg)
    toks = [5, 6, 7, 8]
    lg, ls = m.forward(toks)
    lg2, ls2 = m.forward(toks)
    assert np.array_equal(lg, lg2) and ls == ls2
    # the float twin (model.rs:369-384) over the same quantized weights; the norms' own float gammas
    d, qd, kvd, hid, voc = 16, 16, 8, 32, 20
    s = 0xD00D
    gam = []
    for _ in range(2):
        g_in, s = O.vecf(s, d)
        for n in (qd * d, kvd * d, kvd * d, d * qd):
            _, s = O.vecf(s, n)
        g_post, s = O.vecf(s, d)
        for n in (hid * d, hid * d, d * hid):
            _, s = O.vecf(s, n)
        gam.append((g_in.astype(np.float64), g_post.astype(np.float64)))
    _, s = O.vecf(s, voc * d)
    g_fin, s = O.vecf(s, d)

    def rms(x, g):
        ms = (x.astype(np.float64) ** 2).mean(axis=1, keepdims=True)
        return (x.astype(np.float64) / np.sqrt(ms + 1e-6) * g).astype(np.float32)

    emb = m.emb()
    x = _dq(emb[0][toks], emb[1]).astype(np.float32)
    for l in range(2):
        a = _attention_ref(rms(x, gam[l][0]), m.ql(l, "wq"), m.ql(l, "wk"), m.ql(l, "wv"), m.ql(l, "wo"), 4, 2, 4,
                           10000.0)
        x = (x + a).astype(np.float32)
        h = rms(x, gam[l][1])
        g, u = _lin_ref(h, m.ql(l, "gate")).astype(np.float64), _lin_ref(h, m.ql(l, "up")).astype(np.float64)
        x = (x + _lin_ref((g / (1.0 + np.exp(-g)) * u).astype(np.float32), m.ql(l, "down"))).astype(np.float32)
    lr = _lin_ref(rms(x, g_fin.astype(np.float64)), m.ql(0, "lm_head")).astype(np.float64)
    li = _dq(lg, ls)
    assert np.abs(li - lr).max() <= 0.1 * np.abs(lr).max()
    assert (np.argmax(li, axis=1) == np.argmax(lr, axis=1)).all()


# Exact cases of the batched forward (CausalLM::forward_int, Attention::forward_int over a sequence). The v scale is
# a power of two (2^31, s) = 2^(31 - s), so every Scale product, reciprocal and ratio of the attention's close is
# exact (kt-int/src/lib.rs:191-300) and the outputs follow from integer arithmetic: requant_dyn(v, 2^28, g) is
# round(v 2^28 / g) half away from zero.

def _rha(n, d):
    q = (2 * abs(n) + d) // (2 * d)
    return q if n >= 0 else -q


def _sval(sc):
    from fractions import Fraction

    return Fraction(sc[0]) / Fraction(2) ** sc[1]


PREFILL_CFG = dict(dim=16, layers=1, nh=4, nkv=2, hd=8, hidden=16, vocab=8, eps=1e-6, theta=1.0e6, max_seq=16)


def test_prefill_attention_one_hot_returns_the_attended_v_row_in_every_row():
    """Only k_0 is nonzero and every q row meets it with a score far past the exp table's -30 cutoff: every row's
    softmax is one-hot on step 0 (attention.rs:506-530), every row and head returns v_0 of its kv head; with v's
    largest |code| 2^28 the output codes are v_0 exactly and the scale is v's (2^20 / 2^20 cancels)."""
    m = O.RefModel(3, PREFILL_CFG)
    T, nh, nkv, hd = 9, 4, 2, 8
    rng = np.random.default_rng(31)
    q = np.zeros((T, nh, hd), np.int64)
    k = np.zeros((T, nkv, hd), np.int64)
    v = rng.integers(-(2**28), 2**28, size=(T, nkv, hd))
    k[0] = 2**20
    q[:] = 2**20  # rotated by position i, q_i . k_0 = 2^41 sum_j cos(i theta_j) > 2^42 for i < 9 (hd 8): at q and
    v[0, 0, 0] = 2**28  # k scales of 1 that is far past 30 real units ahead of the zero scores of steps 1..i
    qs, ks, vs = (1 << 31, 31), (1 << 31, 31), (1 << 31, 44)
    o, os_ = m.attention_prefill(T, q.astype(np.int32).ravel(), qs, k.astype(np.int32).ravel(), ks,
                                 v.astype(np.int32).ravel(), vs)
    o = o.reshape(T, nh, hd)
    for i in range(T):
        for h in range(nh):
            assert np.array_equal(o[i, h], v[0, h // 2]), (i, h)
    assert _sval(os_) == _sval(vs)


def test_prefill_attention_two_rows_uniform_softmax_is_exact():
    """k = 0: every score is 0, every numerator exp(0) = 2^20; row 0 returns v_0, row 1 the mean (v_0 + v_1) / 2
    (sumc 2^21: the scale v / 2^21 brought to the common v / 2^20 by an exact 1/2, attention.rs:560-590). A code of
    2^29 in row 0 sets the requant's divisor: out = round(2^20 v_0 / 2^21) and round(2^19 (v_0 + v_1) / 2^21),
    half away from zero, with values of both signs on the halves."""
    m = O.RefModel(3, PREFILL_CFG)
    T, nh, nkv, hd = 2, 4, 2, 8
    rng = np.random.default_rng(32)
    q = rng.integers(-(2**28), 2**28, size=(T, nh, hd))
    k = np.zeros((T, nkv, hd), np.int64)
    v = rng.integers(-(2**27), 2**27, size=(T, nkv, hd))
    v[0, 0, 0], v[1, 0, 0] = 2**29, 0
    # row 0 halves 1, -1 (v_0 / 2); row 1's sums 2, -2, 6, -6 land on halves of the quarter 2^19 s / 2^21
    v[0, 1, :4], v[1, 1, :4] = [1, -1, 2, -2], [1, -1, 4, -4]
    vs = (1 << 31, 50)
    o, os_ = m.attention_prefill(T, q.astype(np.int32).ravel(), (1 << 30, 40), k.astype(np.int32).ravel(),
                                 (1 << 30, 40), v.astype(np.int32).ravel(), vs)
    o = o.reshape(T, nh, hd)
    vv0 = [[2**20 * int(v[0, h // 2, d]) for d in range(hd)] for h in range(nh)]
    vv1 = [[(2**20 * (int(v[0, h // 2, d]) + int(v[1, h // 2, d]))) // 2 for d in range(hd)] for h in range(nh)]
    g = max(abs(x) for r in vv0 + vv1 for x in r)
    assert g == 2**49
    for h in range(nh):
        assert o[0, h].tolist() == [_rha(x * 2**28, g) for x in vv0[h]]
        assert o[1, h].tolist() == [_rha(x * 2**28, g) for x in vv1[h]]
    assert o[0, 2, :4].tolist() == [1, -1, 1, -1] and o[1, 2, :4].tolist() == [1, -1, 2, -2]
    from fractions import Fraction

    assert _sval(os_) == Fraction(g, 2**28) * _sval(vs) / 2**20


def test_prefill_attention_thirds_round_half_away_per_row():
    """k = 0 over three rows: row r averages its r + 1 positions (sumc = (r + 1) 2^20). Every row's sum is brought
    to the common scale v / 2^20 by f = 1, 1/2 and, for row 2, the Scale nearest 1/3 (attention.rs:560-590); with
    v in {-1, 0, 1} the products 2^20 S / 3 sit at a third or two thirds past an integer, far from any half, so
    Scale::apply's round-half-away gives rha(2^20 S, 3) (a truncating apply, or one rounding the wrong way, differs
    on every S = 2 mod 3). One code of 1 in row 0 makes the largest |value| 2^20, so requant_dyn multiplies by 2^8
    exactly and no later rounding hides a unit of the per-row step."""
    m = O.RefModel(3, PREFILL_CFG)
    T, nh, nkv, hd = 3, 4, 2, 8
    rng = np.random.default_rng(33)
    q = rng.integers(-(2**28), 2**28, size=(T, nh, hd))
    k = np.zeros((T, nkv, hd), np.int64)
    v = rng.integers(-1, 2, size=(T, nkv, hd))
    v[0, 0, 0] = 1
    v[:, 1, :6] = [[1, 1, 1, -1, -1, -1], [1, 0, 1, -1, 0, -1], [0, 0, 1, 0, 0, -1]]  # S_2 = 2, 1, 3, -2, -1, -3
    vs = (1 << 31, 50)
    o, os_ = m.attention_prefill(T, q.astype(np.int32).ravel(), (1 << 30, 40), k.astype(np.int32).ravel(),
                                 (1 << 30, 40), v.astype(np.int32).ravel(), vs)
    o = o.reshape(T, nh, hd)
    for h in range(nh):
        g = h // 2
        for d in range(hd):
            s0 = int(v[0, g, d])
            s1 = s0 + int(v[1, g, d])
            s2 = s1 + int(v[2, g, d])
            assert int(o[0, h, d]) == 2**8 * 2**20 * s0, (h, d)
            assert int(o[1, h, d]) == 2**8 * 2**19 * s1, (h, d)
            assert int(o[2, h, d]) == 2**8 * _rha(2**20 * s2, 3), (h, d, s2)
    assert o[2, 2, :6].tolist() == [2**8 * x for x in (699051, 349525, 2**20, -699051, -349525, -(2**20))]
    assert _sval(os_) == _sval(vs) / 2**28


def test_batched_forward_is_the_composition_of_its_pinned_ops():
    """CausalLM::forward_int over T tokens (model.rs:361-367: embed_int, blocks_int, head_int; each block x + attn
    (input_norm(x)), then + ffn(post_norm(x)), model.rs:175-183; SwiGluMlp layers.rs:609-640) composed here from the
    oracle's separately pinned ops -- the Embedding rows at the embedding's scale, RmsNorm over T rows,
    QuantLinear over T rows, the prefill attention core, add, the SwiGLU activation over the T x hidden tensor --
    equals the oracle's batched forward, logits and scale, bit for bit, at T = 1, 2, 5 and 11."""
    cfg = dict(dim=32, layers=2, nh=4, nkv=2, hd=8, hidden=48, vocab=37, eps=1e-6, theta=1.0e6, max_seq=16)
    m = O.RefModel(0xC0FFEE, cfg)
    emb, es = m.emb()
    dim, hid, qd, kvd = cfg["dim"], cfg["hidden"], cfg["nh"] * cfg["hd"], cfg["nkv"] * cfg["hd"]

    def ql(x, xs, rows, which, layer=0):
        w, ws = m.ql(layer, which)
        y, ys, _, _ = O.quant_linear_forward(x, rows, w.shape[1], xs, w, w.shape[0], ws)
        return y.ravel(), ys

    def norm(x, xs, rows, layer, which):
        g, gs, eps = m.norm(layer, which)
        return O.rd_rmsnorm(x, rows, dim, xs, g, gs, eps)

    for T in (1, 2, 5, 11):
        toks = [(7 * i + 3) % cfg["vocab"] for i in range(T)]
        x, xs = emb[toks].ravel().astype(np.int32), es
        for l in range(cfg["layers"]):
            h, hs = norm(x, xs, T, l, "in_norm")
            q, qs = ql(h, hs, T, "wq", l)
            k, ks = ql(h, hs, T, "wk", l)
            v, vs = ql(h, hs, T, "wv", l)
            o, os_ = m.attention_prefill(T, q, qs, k, ks, v, vs)
            a, as_ = ql(o, os_, T, "wo", l)
            x, xs = O.rd_add(x, xs, a, as_)
            h, hs = norm(x, xs, T, l, "post_norm")
            g, gs = ql(h, hs, T, "gate", l)
            u, us = ql(h, hs, T, "up", l)
            hh, hhs = O.rd_swiglu_act(m, g, gs, u, us)
            d, ds = ql(hh, hhs, T, "down", l)
            x, xs = O.rd_add(x, xs, d, ds)
        h, hs = norm(x, xs, T, 0, "final_norm")
        lg, ls = ql(h, hs, T, "lm_head")
        want, wls = m.forward(toks)
        assert np.array_equal(lg.reshape(T, cfg["vocab"]), want) and ls == wls, T
