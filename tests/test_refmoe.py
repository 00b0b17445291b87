"""The reference's MoeMlp at its own semantics, on the CPU: the oracle's restatement (route / route_sigmoid, combine,
merge_rows, the shared expert; oracle/kt_oracle_refdec.c) pinned by the reference's own MoE tests
(crates/01-engine/kt-core/src/tests.rs:113-180, tests_glm.rs:139-259) -- the integer layer tracks its float twin
within 3% of the output's peak with no routing flip, the sigmoid codes sit within one table step, a zero bias
selects the softmax router's experts, the bias moves the choice but not the weights, the shared expert is added
unweighted -- and by closed forms of combine and merge_rows. The float twin is numpy over the dequantized weights,
as the reference's forward_ref is. No GPU call."""
import numpy as np
import pytest

from oracle import oracle as O


def dq(codes, sc):
    return np.asarray(codes, dtype=np.float64) * (sc[0] * 2.0 ** -sc[1])


def lin_ref(m, e, which, x):
    """QuantLinear::forward_ref (layers.rs:330-348): f64 dot of x with the dequantized weights, to f32."""
    w, ws = m.ql(e, which)
    return (np.asarray(x, np.float64) @ dq(w, ws).T).astype(np.float32)


def mlp_ref(m, e, x):
    """SwiGluMlp::forward_ref (layers.rs:642-648)."""
    g = lin_ref(m, e, "gate", x).astype(np.float64)
    u = lin_ref(m, e, "up", x).astype(np.float64)
    return lin_ref(m, e, "down", (g / (1.0 + np.exp(-g)) * u).astype(np.float32))


def bias_ref(seed, n):
    """vecf(seed, n) * 0.05 in f32 (tests_glm.rs:40-43)."""
    s, out = seed, []
    for _ in range(n):
        s = (s * 6364136223846793005 + 1442695040888963407) % 2**64
        u = np.float32((s >> 40) / float(1 << 24) * 2.0 - 1.0)
        out.append(np.float32(u * np.float32(0.05)))
    return np.array(out, np.float32)


def topk_ref(keys, k):
    return sorted(range(len(keys)), key=lambda j: (-keys[j], j))[:k]


def moe_ref(m, x, bias=None):
    """MoeMlp::forward_ref (layers.rs:1036-1088): per token the float router, softmax or sigmoid weights, the
    top-k experts' weighted sum, plus the shared expert unweighted."""
    rows = x.reshape(-1, m.dim)
    out = np.zeros(rows.shape, np.float64)
    for t, xr in enumerate(rows):
        logits = lin_ref(m, 0, "router", xr[None])[0]
        if m.sigmoid:
            w = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
            top = topk_ref(w + bias.astype(np.float64), m.top_k)
            total = w[top].sum() if m.norm_topk else 1.0
        else:
            lmax = logits.max()
            w = np.exp((logits - lmax).astype(np.float64))
            top = topk_ref(logits, m.top_k)
            total = w[top].sum() if m.norm_topk else w.sum()
        for ex in top:
            out[t] += w[ex] / total * mlp_ref(m, ex, xr[None])[0].astype(np.float64)
    if m.shared_hidden:
        out += mlp_ref(m, m.E, rows).astype(np.float64)
    return out.astype(np.float32).reshape(-1)


def check_tracks_float(m, T, seed, bias=None):
    x, xs, _ = O.rm_probe(seed, T * m.dim)
    got, gs = m.forward(x, T, xs)
    again = m.forward(x, T, xs)
    assert np.array_equal(again[0], got) and again[1] == gs, "not deterministic"
    ref = moe_ref(m, dq(x, xs).astype(np.float32), bias)
    err = np.abs(dq(got, gs).astype(np.float32).astype(np.float64) - ref).max()
    peak = np.abs(ref).max()
    assert err <= 3e-2 * peak, f"drifted from float: {err} against peak {peak}"
    return x, xs


def test_softmax_moe_tracks_float_with_no_routing_flip():
    """tests.rs:113-150: 8 experts of hidden 96 over dim 64, top-2, normalized over all experts."""
    m = O.RefMoe(0x30E1, 64, 8, 2, 96)
    for T, seed in ((1, 0x30E2), (5, 0x30E3)):
        x, xs = check_tracks_float(m, T, seed)
        for t in range(T):
            sel, ec, sumc, lg, ls = m.route(x[t * 64:(t + 1) * 64], xs)
            lf = lin_ref(m, 0, "router", dq(x[t * 64:(t + 1) * 64], xs)[None].astype(np.float32))[0]
            assert sel == topk_ref(lg.astype(np.float64), 2) == topk_ref(lf.astype(np.float64), 2)
            assert sumc >= ec.sum() > 0 and (ec <= 1 << 20).all()


def test_sigmoid_codes_within_one_table_step_and_clamped():
    """tests_glm.rs:139-156."""
    m = O.RefMoe(0x51, 32, 16, 4, 24, True, 2)
    k, step = float(1 << 20), 32.0 / 65535
    scale = O.from_f64(1.0 / 4096.0)
    for l in range(-80_000, 80_001, 997):
        vals = np.array([l, -l, 0, l // 3], np.int32)
        codes = m.sigmoid_codes(vals, (scale.mant, scale.shift))
        real = vals / 4096.0
        want = k / (1.0 + np.exp(-real))
        assert (np.abs(codes - want) <= step / 4.0 * k + 1.0).all()
        assert ((codes >= 0) & (codes <= 1 << 20)).all()
    ends = m.sigmoid_codes(np.array([-(1 << 20), 1 << 20, 0, 0], np.int32), (1 << 30, 30))
    assert ends[0] == 0 and ends[1] == 1 << 20


def test_a_zero_bias_selects_the_softmax_routers_experts():
    """tests_glm.rs:159-180: where the sigma codes separate the k-th and (k+1)-th logit, a zero-bias sigmoid router
    picks the softmax router's experts."""
    soft = O.RefMoe(0x51, 32, 16, 4, 24, True, 0)
    sig = O.RefMoe(0x51, 32, 16, 4, 24, True, 2)
    x, xs, _ = O.rm_probe(0x52, 64 * 32)
    compared = 0
    for t in range(64):
        row = x[t * 32:(t + 1) * 32]
        _, _, _, lg, ls = sig.route(row, xs)
        codes = np.sort(sig.sigmoid_codes(lg, ls))[::-1]
        if codes[3] == codes[4]:
            continue
        compared += 1
        assert sorted(soft.route(row, xs)[0]) == sorted(sig.route(row, xs)[0])
    assert compared * 10 >= 64 * 9


def test_the_bias_moves_the_choice_but_not_the_weights():
    """tests_glm.rs:183-200."""
    x, xs, _ = O.rm_probe(0x54, 32)
    plain = O.RefMoe(0x53, 32, 16, 4, 24, True, 2)
    sel0 = plain.route(x, xs)[0]
    outsider = next(e for e in range(16) if e not in sel0)
    biased = O.RefMoe(0x53, 32, 16, 4, 24, True, 2)
    biased.set_bias(outsider, 1.5)
    sel, ec, sumc, lg, ls = biased.route(x, xs)
    assert outsider in sel
    codes = plain.sigmoid_codes(lg, ls)
    assert all(c == codes[e] for e, c in zip(sel, ec))
    assert sumc == int(ec.sum())
    raw = O.RefMoe(0x53, 32, 16, 4, 24, False, 2)
    raw.set_bias(outsider, 1.5)
    assert raw.route(x, xs)[2] == 1 << 20


def test_the_sigmoid_moe_tracks_float_with_no_routing_flip():
    """tests_glm.rs:203-220: bias(0x55) on moe(0x56)."""
    m = O.RefMoe(0x56, 32, 16, 4, 24, True, 1, 0x55)
    b = bias_ref(0x55, 16)
    assert np.array_equal(m.bias(), np.round(b.astype(np.float64) * (1 << 20)).astype(np.int64))
    x, xs = check_tracks_float(m, 8, 0x57, b)
    for t in range(8):
        row = x[t * 32:(t + 1) * 32]
        lf = lin_ref(m, 0, "router", dq(row, xs)[None].astype(np.float32))[0].astype(np.float64)
        want = topk_ref(1.0 / (1.0 + np.exp(-lf)) + b.astype(np.float64), 4)
        assert m.route(row, xs)[0] == want


def test_the_shared_expert_is_added_unweighted_and_tracks_float():
    """tests_glm.rs:244-259: glm_like(0x5C) -- sigmoid router, bias(0x5C), shared expert of hidden 40."""
    with_ = O.RefMoe(0x5C, 32, 16, 4, 24, True, 1, 0x5C, 40)
    without = O.RefMoe(0x5C, 32, 16, 4, 24, True, 1, 0x5C, 0)
    b = bias_ref(0x5C, 16)
    x, xs = check_tracks_float(with_, 6, 0x5D, b)
    assert not np.array_equal(with_.forward(x, 6, xs)[0], without.forward(x, 6, xs)[0])


def test_combine_and_merge_closed_forms():
    """combine of one expert with its own numerator as the normalizer is that expert's output requantized; the
    weighted sum equals the real ec-weighted mean within one output unit; merge_rows keeps every row's real values
    within one unit of the common scale, and a zero-scale row merges as zeros."""
    rng = np.random.default_rng(8)
    y = rng.integers(-(2**28), 2**28, size=(3, 40)).astype(np.int32)
    y[0, 0] = 2**28
    ss = [(1610612736, 61), (1288490189, 60), (1073741824, 62)]
    out, os_ = O.rm_combine(y[:1].ravel(), ss[:1], 40, [777], 777)
    assert np.abs(dq(out, os_) - dq(y[0], ss[0])).max() <= os_[0] * 2.0 ** -os_[1]
    ec = np.array([300000, 500000, 248576], np.int64)
    out, os_ = O.rm_combine(y.ravel(), ss, 40, ec, int(ec.sum()))
    want = sum(ec[i] * dq(y[i], ss[i]) for i in range(3)) / ec.sum()
    assert np.abs(dq(out, os_) - want).max() <= 2 * os_[0] * 2.0 ** -os_[1]
    rows = y.copy()
    rs = [ss[0], (0, 0), ss[2]]
    out, os_ = O.rm_merge_rows(rows.ravel(), rs, 3, 40)
    got = dq(out, os_).reshape(3, 40)
    assert not out.reshape(3, 40)[1].any()
    for t in (0, 2):
        assert np.abs(got[t] - dq(rows[t], rs[t])).max() <= os_[0] * 2.0 ** -os_[1]


# Exact cases. A Scale (2^31, s) is the power of two 2^(31 - s); products, reciprocals and from_ratio of powers of
# two are exact in kt-int (crates/00-kernels/kt-int/src/lib.rs:191-300), so with such scales every factor combine
# and merge_rows form is exact and their outputs follow from integer arithmetic alone: f.apply(v) for f = 2^-e is
# round(v / 2^e) half away from zero, requant_dyn(v, 2^28, g) is round(v 2^28 / g) half away from zero. The inputs
# put values on exact halves, where a truncating, flooring or half-even rounding gives another answer.


def p2(s):
    return (1 << 31, s)


def rha(n, d):
    """round(n / d) half away from zero, Python integers, d > 0."""
    q = (2 * abs(n) + d) // (2 * d)
    return q if n >= 0 else -q


def sval(sc):
    from fractions import Fraction

    return Fraction(sc[0]) / Fraction(2) ** sc[1]


def test_combine_of_one_expert_with_its_own_numerator_returns_its_codes():
    """ec = sumc = 2^19, the expert's largest |code| 2^28, its scale a power of two: the codes come back unchanged
    and the scale equals the expert's (layers.rs:893-923)."""
    rng = np.random.default_rng(21)
    y = rng.integers(-(2**28), 2**28, size=57).astype(np.int32)
    y[13] = -(2**28)
    out, os_ = O.rm_combine(y, [p2(44)], 57, [2**19], 2**19)
    assert np.array_equal(out, y)
    assert sval(os_) == sval(p2(44))


def test_combine_rounds_half_away_from_zero_at_both_steps():
    """Two experts at 2^-9 and 2^-10 (the second brought to the first's scale: round(v / 2) on odd codes, exact
    halves of both signs), ec = [1, 1], sumc = 2, and one sum of exactly 2^29 so requant_dyn halves every sum:
    out = round(round(y1 / 2) + y0) / 2), all half away from zero; the output scale is the common scale."""
    rng = np.random.default_rng(22)
    n = 64
    y0 = rng.integers(-(2**26), 2**26, size=n).astype(np.int64)
    y1 = (rng.integers(-(2**26), 2**26, size=n) | 1).astype(np.int64)  # odd: y1 / 2 on a half
    y0[0], y1[0] = 2**29, 0
    y0[1:9] = [1, -1, 2, -2, 0, 0, 5, -5]
    y1[1:9] = [1, -1, 1, -1, 3, -3, -1, 1]
    ys = np.concatenate([y0, y1]).astype(np.int32)
    out, os_ = O.rm_combine(ys, [p2(40), p2(41)], n, [1, 1], 2)
    acc = [int(a) + rha(int(b), 2) for a, b in zip(y0, y1)]
    assert max(abs(a) for a in acc) == 2**29
    want = [rha(a * 2**28, 2**29) for a in acc]
    assert out.tolist() == want
    # the planted halves: 1 + round(1/2) = 2 -> 1; -1 + round(-1/2) = -2 -> -1; 2 + 1 = 3 -> 2 (half away);
    # -2 - 1 = -3 -> -2; round(3/2) = 2 -> 1; round(-3/2) = -2 -> -1; 5 - 1 = 4 -> 2; -5 + 1 = -4 -> -2
    assert out[1:9].tolist() == [1, -1, 2, -2, 1, -1, 2, -2]
    assert sval(os_) == sval(p2(40))


def test_combine_weighted_sum_is_exact_at_power_of_two_numerators():
    """ec = [2^19, 2^19], sumc = 2^20, experts at 2^-9 and 2^-10, one sum exactly 2^47: every code is
    y0 + round(y1 / 2) with nothing lost, and the scale is 2^-9 (2^47 / 2^28) / 2^20."""
    rng = np.random.default_rng(23)
    n = 50
    y0 = rng.integers(-(2**27) + 1, 2**27, size=n).astype(np.int64)
    y1 = rng.integers(-(2**27), 2**27, size=n).astype(np.int64)
    y0[0], y1[0] = 2**28, 0
    out, os_ = O.rm_combine(np.concatenate([y0, y1]).astype(np.int32), [p2(40), p2(41)], n, [2**19, 2**19], 2**20)
    assert out.tolist() == [int(a) + rha(int(b), 2) for a, b in zip(y0, y1)]
    from fractions import Fraction

    assert sval(os_) == sval(p2(40)) * Fraction(2**47, 2**28) / 2**20


def test_merge_rows_at_one_scale_is_requant_dyn_of_the_concatenation():
    """Rows that share one power-of-two scale merge as requant_dyn of their concatenation by its largest |code|
    (layers.rs:866-891); the scale is that maximum over 2^28 times the rows' scale."""
    rng = np.random.default_rng(24)
    T, d = 5, 33
    rows = rng.integers(-(2**30), 2**30, size=T * d).astype(np.int32)
    out, os_ = O.rm_merge_rows(rows, [p2(47)] * T, T, d)
    g = int(np.abs(rows.astype(np.int64)).max())
    assert out.tolist() == [rha(int(v) * 2**28, g) for v in rows]
    from fractions import Fraction

    assert sval(os_) == Fraction(g, 2**28) * sval(p2(47))


def test_merge_rows_brings_rows_to_the_largest_scale_with_exact_halves():
    """Rows at 2^-9, 2^-11 and zero: the second brought to the first by round(v / 4) (v = 2 mod 4: exact halves),
    the third all zeros; one code of exactly 2^29 makes requant_dyn halve every value: round(a / 2), half away from
    zero throughout."""
    rng = np.random.default_rng(25)
    d = 40
    r0 = rng.integers(-(2**27), 2**27, size=d).astype(np.int64)
    r1 = (rng.integers(-(2**26), 2**26, size=d) * 4 + 2).astype(np.int64)
    r1[1::2] = -r1[1::2]
    r2 = rng.integers(-(2**30), 2**30, size=d).astype(np.int64)
    r0[0] = 2**29
    r0[1:5], r1[1:5] = [1, -1, 3, -3], [2, -2, 6, -6]
    rows = np.concatenate([r0, r1, r2]).astype(np.int32)
    out, os_ = O.rm_merge_rows(rows, [p2(40), p2(42), (0, 0)], 3, d)
    a = [int(v) for v in r0] + [rha(int(v), 4) for v in r1] + [0] * d
    assert max(abs(x) for x in a) == 2**29
    assert out.tolist() == [rha(x * 2**28, 2**29) for x in a]
    # 1 -> round(1/2) = 1; -1 -> -1; 3 -> 2; -3 -> -2; round(2/4) = 1 -> 1; -1 -> -1; round(6/4) = 2 -> 1; -> -1
    assert out[1:5].tolist() == [1, -1, 2, -2] and out[d + 1:d + 5].tolist() == [1, -1, 1, -1]
    assert not out[2 * d:].any()
    assert sval(os_) == 2 * sval(p2(40))


def test_softmax_route_exact_identities():
    """MoeMlp::route (layers.rs:826-851): the selected experts are the top-k logits with ties to the lower index;
    the strongest one's numerator is exp(0) = 2^20 exactly (the table's last entry); numerators fall with the logit;
    normalized over the top k, sumc is their sum; normalized over all E, sumc is the sum of every expert's numerator,
    which a top-E route of the same layer lists."""
    for norm in (False, True):
        m = O.RefMoe(0x30E1, 64, 8, 2, 96, norm)
        full = O.RefMoe(0x30E1, 64, 8, 8, 96, norm)
        x, xs, _ = O.rm_probe(0x30E4, 9 * 64)
        for t in range(9):
            row = x[t * 64:(t + 1) * 64]
            sel, ec, sumc, lg, ls = m.route(row, xs)
            fsel, fec, fsumc, flg, _ = full.route(row, xs)
            assert np.array_equal(lg, flg)
            assert sel == topk_ref(lg.astype(np.int64), 2) and fsel == topk_ref(lg.astype(np.int64), 8)
            assert ec[0] == 1 << 20 and fec[0] == 1 << 20
            assert all(fec[i] >= fec[i + 1] for i in range(7))
            assert np.array_equal(ec, fec[:2])
            assert sumc == (int(ec.sum()) if norm else int(fec.sum()))
            assert fsumc == int(fec.sum())


def test_sigmoid_route_exact_identities():
    """route_sigmoid (router.rs:29-79): the score of a zero logit at any scale is the table entry at index 32768 (
    = -round(-16 * 65535 / 32)), round(2^20 sigma(-16 + 32 * 32768 / 65535)) by math.exp; the choice is the
    top-k of score plus coded bias with ties to the lower index; the numerators are the chosen scores and sumc their
    sum (norm_topk_prob) or 2^20."""
    import math

    m = O.RefMoe(0x53, 32, 16, 4, 24, True, 1, 0x55)
    for sc in ((1 << 30, 30), (1234567890, 45), (1 << 31, 80)):
        c = m.sigmoid_codes(np.zeros(4, np.int32), sc)
        xg = -16.0 + 32.0 * 32768 / 65535
        assert (c == round((1 << 20) / (1.0 + math.exp(-xg)))).all()
    bias = m.bias()
    x, xs, _ = O.rm_probe(0x58, 6 * 32)
    for t in range(6):
        sel, ec, sumc, lg, ls = m.route(x[t * 32:(t + 1) * 32], xs)
        codes = m.sigmoid_codes(lg, ls)
        assert sel == topk_ref((codes + bias).astype(np.int64), 4)
        assert ec.tolist() == [int(codes[e]) for e in sel] and sumc == int(ec.sum())


@pytest.mark.parametrize("sig", [0, 1])
def test_a_layer_built_from_given_weights_equals_the_seeded_one(sig):
    """RefMoe.from_weights (kt_rm_empty / kt_rm_set_ql / kt_rm_set_bias_code) over the QuantLinears and coded bias of
    a seeded layer routes and forwards exactly as that layer does, shared expert included; a layer built from the
    same weights with one expert's scale changed does not."""
    m = O.RefMoe(0x5C, 32, 16, 4, 24, True, sig, 0x5C, 40)
    experts = [{n: m.ql(e, n) for n in ("gate", "up", "down")} for e in range(16)]
    shared = {n: m.ql(16, n) for n in ("gate", "up", "down")}
    g = O.RefMoe.from_weights(32, m.ql(0, "router"), experts, 4, True, m.bias() if sig else None, shared)
    x, xs, _ = O.rm_probe(0x5E, 7 * 32)
    for t in range(7):
        (gs_, ge, gc, gl, gls), (ms_, me, mc, ml, mls) = g.route(x[t * 32:(t + 1) * 32], xs), \
            m.route(x[t * 32:(t + 1) * 32], xs)
        assert gs_ == ms_ and np.array_equal(ge, me) and gc == mc and np.array_equal(gl, ml) and gls == mls
    want, ws = m.forward(x, 7, xs)
    got, gs = g.forward(x, 7, xs)
    assert np.array_equal(got, want) and gs == ws
    sel = m.route(x[:32], xs)[0]
    codes, (mant, shift) = experts[sel[0]]["down"]
    experts[sel[0]]["down"] = (codes, (mant, shift + 1))
    h = O.RefMoe.from_weights(32, m.ql(0, "router"), experts, 4, True, m.bias() if sig else None, shared)
    assert not np.array_equal(h.forward(x, 7, xs)[0], want)
