"""CPU tests: the oracle of the layers around the 12-bit GEMM (oracle/kt_oracle_layers.c) pinned against brute
force and closed forms, and the product's host-side workload generators against the oracle's. No GPU needed.

What pins what:
  - gemm_i8w16 (the blocked dot of every dense W12 check) equals kt_linear_cpu, the restated reference linear_cpu;
  - moe_route equals a Python sort with the reference's tie rule (MoeMlp::topk, layers.rs:800-805);
  - moe_bucket equals a Python loop;
  - the expert-major MoE layer equals the per-token loop order of the reference (layers.rs:928-936, 988-1020), and
    on a tiny case both equal a pure-Python restatement with Python integers (requant of kt-int lib.rs:78-86);
  - the SiLU / sigmoid code tables satisfy the identities of the closed forms they come from.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O


def py_requant(acc: int, mant: int, shift: int) -> int:
    """kt-int requant (crates/00-kernels/kt-int/src/lib.rs:78-86) in Python integers: round(acc * mant / 2^shift)
    half away from zero."""
    p = acc * mant
    if shift <= 0:
        return p << (-shift)
    q = (abs(p) + (1 << (shift - 1))) >> shift
    return q if p >= 0 else -q


def clamp(v, lo=-127, hi=127):
    return max(lo, min(hi, v))


def test_gemm_i8w16_equals_linear_cpu():
    rng = np.random.default_rng(1)
    for m, n, k in [(1, 1, 1), (3, 70, 129), (33, 64, 512), (65, 5, 4096)]:
        x = rng.integers(-128, 128, size=m * k).astype(np.int8)
        w = rng.integers(-2048, 2048, size=n * k).astype(np.int16)
        acc, _ = O.gemm_i8w16(x, w, m, n, k)
        assert np.array_equal(acc, O.linear_cpu(x.astype(np.int32), w.astype(np.int32), m, n, k))
        mant = rng.integers(-(2**31), 2**31, size=n).astype(np.int32)
        shift = rng.integers(-3, 64, size=n).astype(np.int32)
        _, y8 = O.gemm_i8w16(x, w, m, n, k, mant, shift)
        want = O.requant_channels(acc, m, n, mant, shift, -127, 127)
        assert np.array_equal(y8.astype(np.int32), want)


def test_gemm_i8w16_extremes_fit_int32():
    """|x| = 128, |w| = 2048 at k = 8128: every partial sum of the int32 dot stays exact."""
    k = 8128
    x = np.full(k, -128, np.int8)
    w = np.full(2 * k, -2048, np.int16)
    acc, _ = O.gemm_i8w16(x, w, 1, 2, k)
    assert acc.tolist() == [k * 128 * 2048] * 2
    with pytest.raises(ValueError):
        O.gemm_i8w16(np.zeros(8192, np.int8), np.zeros(8192, np.int16), 1, 1, 8192)


def route_py(r, E, K, sig):
    out = []
    for t in range(len(r) // E):
        row = [int(v) for v in r[t * E:(t + 1) * E]]
        top = sorted(range(E), key=lambda e: (-row[e], e))[:K]
        cws = []
        for e in top:
            a = abs(row[e])
            q = min((a + 8) >> 4, 127)
            idx = q if row[e] >= 0 else -q
            cws.append(int(sig[idx + 127]))
        out.append((top, cws))
    return out


def test_moe_route_equals_python_sort():
    from tritify_amd import workloads as W

    sig = W.sigmoid_table()
    rng = np.random.default_rng(2)
    for T, E, K in [(50, 16, 4), (20, 128, 8), (5, 3, 3)]:
        r = O.gen_gauss_i32(T + E, 1024, T * E)
        r[: E] = 5  # one token of ties
        r[E: E + 3] = 10**7  # far outside the table
        r[E + 3: E + 6] = -(10**7)
        sel, cw = O.moe_route(r, T, E, K, sig)
        want = route_py(r, E, K, sig)
        assert sel.reshape(T, K).tolist() == [w[0] for w in want]
        assert cw.reshape(T, K).tolist() == [w[1] for w in want]


def test_moe_bucket_equals_python():
    rng = np.random.default_rng(3)
    T, E, K = 97, 10, 3
    sel = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32).reshape(-1)
    lst, pos, count = O.moe_bucket(sel, T, E, K)
    groups = {g: [] for g in range(E + 1)}
    for t in range(T):
        for i in range(K):
            g = int(sel[t * K + i])
            assert pos[t * K + i] == len(groups[g])
            groups[g].append(t)
        groups[E].append(t)
    assert count.tolist() == [len(groups[g]) for g in range(E + 1)]
    for g in range(E + 1):
        assert lst[g * T: g * T + count[g]].tolist() == groups[g]


def moe_case(T, H, F, E, K, seed, logits=None):
    from tritify_amd import workloads as W

    x = O.gen_act_gauss(seed, 40, T * H)
    r = O.gen_gauss_i32(seed + 1, 1024, T * E) if logits is None else logits
    G = E + 1
    wgu = np.stack([O.gen_w12_i16(seed + 10 + 2 * g, 2 * F * H) for g in range(G)])
    wd = np.stack([O.gen_w12_i16(seed + 11 + 2 * g, H * F) for g in range(G)])
    gm, gs = zip(*[O.channel_scales_i16(wgu[g], 2 * F, H, 40) for g in range(G)])
    dm, ds = zip(*[O.channel_scales_i16(wd[g], H, F, 16) for g in range(G)])
    return dict(x=x, r=r, wgu=wgu, wd=wd, gm=np.stack(gm), gs=np.stack(gs), dm=np.stack(dm), ds=np.stack(ds),
                silu=W.silu_table(), sig=W.sigmoid_table())


@pytest.mark.parametrize("T,H,F,E,K", [(64, 64, 32, 8, 2), (130, 128, 64, 6, 6), (1, 64, 32, 4, 1)])
def test_moe_expert_major_equals_token_order(T, H, F, E, K):
    c = moe_case(T, H, F, E, K, 17 * T + E)
    res = O.moe_layer(c["x"], c["r"], T, H, F, E, K, c["wgu"], c["wd"], c["gm"], c["gs"], c["dm"], c["ds"],
                      c["silu"], c["sig"], 8, 13)
    tok = O.moe_forward_token(c["x"], c["r"], T, H, F, E, K, c["wgu"], c["wd"], c["gm"], c["gs"], c["dm"], c["ds"],
                              c["silu"], c["sig"], 8, 13)
    assert np.array_equal(res["out"], tok)
    assert int(res["count"].sum()) == T * (K + 1)


def test_moe_layer_equals_python_restatement():
    """A tiny layer evaluated with Python integers only (route, SwiGLU, down, combine) equals the C oracle."""
    T, H, F, E, K = 3, 64, 32, 4, 2
    c = moe_case(T, H, F, E, K, 5)
    res = O.moe_layer(c["x"], c["r"], T, H, F, E, K, c["wgu"], c["wd"], c["gm"], c["gs"], c["dm"], c["ds"],
                      c["silu"], c["sig"], 8, 13)
    routes = route_py(c["r"], E, K, c["sig"])
    x = c["x"].reshape(T, H).astype(object)
    for t in range(T):
        y = [0] * H
        top, cws = routes[t]
        for g, wgt in list(zip(top, cws)) + [(E, 4096)]:
            wgu = c["wgu"][g].reshape(2 * F, H).astype(object)
            wd = c["wd"][g].reshape(H, F).astype(object)
            h = []
            for ch in range(F):
                gq = clamp(py_requant(int(np.dot(x[t], wgu[ch])), int(c["gm"][g][ch]), int(c["gs"][g][ch])))
                uq = clamp(py_requant(int(np.dot(x[t], wgu[F + ch])), int(c["gm"][g][F + ch]),
                                      int(c["gs"][g][F + ch])))
                h.append(clamp(py_requant(int(c["silu"][gq + 127]) * uq, 1, 8)))
            d = [clamp(py_requant(int(np.dot(np.array(h, dtype=object), wd[o])), int(c["dm"][g][o]),
                                  int(c["ds"][g][o]))) for o in range(H)]
            y = [a + wgt * b for a, b in zip(y, d)]
        want = [clamp(py_requant(v, 1, 13)) for v in y]
        assert res["out"].reshape(T, H)[t].tolist() == want


def test_code_tables_closed_forms():
    """sigmoid(v) + sigmoid(-v) = 1 and silu(v) - silu(-v) = v, at the tables' scales and resolution."""
    from tritify_amd import workloads as W

    sig, silu = W.sigmoid_table().astype(int), W.silu_table().astype(int)
    assert sig[127] == 2048 and silu[127] == 0
    for i in range(1, 128):
        assert sig[127 + i] + sig[127 - i] == 4096
        assert abs((silu[127 + i] - silu[127 - i]) - 8 * i) <= 1  # 256 * (i / 32)
    assert (np.diff(sig) >= 0).all()
    assert silu.min() >= -72 and silu.max() <= 1000


def test_product_generators_equal_the_oracle():
    """The product's multithreaded host generators (libkt_hip.so) draw the same streams as the oracle's."""
    import tritify_amd as TA

    for seed in (0, 3, 2**63 + 5):
        n = 3_000_001
        assert np.array_equal(TA.gen_w12_fast(seed, n), O.gen_w12(seed, n))
        assert np.array_equal(TA.gen_gauss_fast(seed, 40, n, clip=127), O.gen_act_gauss(seed, 40, n))
        assert np.array_equal(TA.gen_gauss_fast(seed, 1024, n // 7), O.gen_gauss_i32(seed, 1024, n // 7))
        assert np.array_equal(TA.gen_uniform_fast(seed, -127, 127, n), O.gen_act_uniform(seed, n))
    w = O.gen_w12(9, 300 * 517)
    m1, s1 = TA.channel_scales_fast(w, 300, 517, 40)
    m2, s2 = O.channel_scales(w, 300, 517, 40)
    assert np.array_equal(m1, m2) and np.array_equal(s1, s2)
    m3, s3 = O.channel_scales_i16(w.astype(np.int16), 300, 517, 40)
    assert np.array_equal(m1, m3) and np.array_equal(s1, s3)


def conv_numpy(q, ci, h, w, wt, co, kh, kw, s, p, bias):
    """The reference's direct loop (conv.rs:68-130) as a zero-padded numpy convolution: skipping a tap outside the
    image equals multiplying a zero."""
    x = np.zeros((ci, h + 2 * p, w + 2 * p), np.int64)
    x[:, p:p + h, p:p + w] = q.reshape(ci, h, w)
    oh, ow = (h + 2 * p - kh) // s + 1, (w + 2 * p - kw) // s + 1
    wt = wt.reshape(co, ci, kh, kw).astype(np.int64)
    acc = np.zeros((co, oh, ow), np.int64)
    for ky in range(kh):
        for kx in range(kw):
            patch = x[:, ky:ky + s * (oh - 1) + 1:s, kx:kx + s * (ow - 1) + 1:s]  # ci x oh x ow
            acc += np.einsum("cij,oc->oij", patch, wt[:, :, ky, kx])
    if bias is not None:
        acc += bias.astype(np.int64)[:, None, None]
    return acc.reshape(-1)


@pytest.mark.parametrize("ci,h,w,co,kh,kw,s,p", [(3, 30, 41, 7, 7, 7, 4, 3), (2, 9, 9, 3, 3, 3, 1, 1),
                                                 (1, 5, 12, 2, 5, 2, 2, 0)])
def test_conv_oracle_equals_padded_convolution(ci, h, w, co, kh, kw, s, p):
    rng = np.random.default_rng(ci * h + w)
    q = rng.integers(-127, 128, size=ci * h * w).astype(np.int8)
    wt = rng.integers(-2048, 2048, size=co * ci * kh * kw).astype(np.int16)
    bias = rng.integers(-(2**20), 2**20, size=co).astype(np.int32)
    mant = rng.integers(1, 2**31, size=co).astype(np.int32)
    shift = rng.integers(10, 40, size=co).astype(np.int32)
    out, acc = O.conv2d(q, ci, h, w, wt, co, kh, kw, s, p, bias, mant, shift, want_acc=True)
    want = conv_numpy(q, ci, h, w, wt, co, kh, kw, s, p, bias)
    assert np.array_equal(acc, want)
    oh, ow = (h + 2 * p - kh) // s + 1, (w + 2 * p - kw) // s + 1
    chan = np.repeat(np.arange(co), oh * ow)
    rq = [max(-127, min(127, py_requant(int(a), int(mant[c]), int(shift[c])))) for a, c in zip(want, chan)]
    assert out.tolist() == rq


def test_entry_and_gelu_tables_closed_forms():
    """The entry table is the ImageNet normalization at scale 48 (monotone, within int8, zero crossing at the mean);
    the GELU table is gelu on the int8 grid (gelu(v) - gelu(-v) = v, gelu(0) = 0)."""
    from tritify_amd import workloads as W

    t = W.sam_entry_table().astype(int)
    for c, (mu, sd) in enumerate(zip(W.IMAGENET_MEAN, W.IMAGENET_STD)):
        assert (np.diff(t[c]) >= 0).all() and abs(t[c]).max() <= 127
        p0 = int(round(mu * 255))
        assert abs(t[c][p0]) <= 1
        assert abs(t[c][255] - 48 * (1 - mu) / sd) <= 0.5 + 1e-9
    g = W.gelu_table().astype(int)
    assert g[127] == 0
    for i in range(1, 128):
        assert abs((g[127 + i] - g[127 - i]) - i) <= 1


def test_uniform_pixels_generator():
    import tritify_amd as TA

    assert np.array_equal(TA.gen_uniform_fast(51, 0, 255, 1_000_003), O.gen_uniform(51, 0, 255, 1_000_003))


# ---------------------------------------------------------------------------------------------------------------
# config 3: the decoder oracle


def dec_arrays(cfg, w_seed, max_pos):
    """Oracle-side model arrays (the oracle's own generators)."""
    from tritify_amd import workloads as W

    d, ffn, nh, nkv, hd, L, V = (cfg[k] for k in ("d", "ffn", "nh", "nkv", "hd", "layers", "vocab"))
    nq, nhd = (nh + 2 * nkv) * hd, nh * hd
    a = {k: [] for k in ("wqkv", "qkv_mant", "qkv_shift", "wo", "o_mant", "o_shift", "wgu", "gu_mant", "gu_shift",
                         "wd", "d_mant", "d_shift")}
    for l in range(L):
        for j, (name, n, k, key) in enumerate((("qkv", nq, d, "qkv"), ("o", d, nhd, "o"), ("gu", 2 * ffn, d, "gu"),
                                               ("dn", d, ffn, "d"))):
            w = O.gen_quant_rows(w_seed + 8 * l + j, n, k)
            sig, tgt = W.DEC_SCALES[name]
            m, s = O.channel_scales_target(w, n, k, sig, tgt)
            a[{"qkv": "wqkv", "o": "wo", "gu": "wgu", "d": "wd"}[key]].append(w)
            a[key + "_mant"].append(m)
            a[key + "_shift"].append(s)
    arrays = {k: np.concatenate(v) for k, v in a.items()}
    emb = O.gen_quant_rows(w_seed - 1, V, d)
    sig, tgt = W.DEC_SCALES["lm"]
    arrays["emb"] = emb
    arrays["lm_mant"], arrays["lm_shift"] = O.channel_scales_target(emb, V, d, sig, tgt)
    arrays["rope_cos"], arrays["rope_sin"] = W.rope_tables(max_pos, hd)
    arrays["exp_tab"] = W.exp_table()
    arrays["silu"] = W.silu_table()
    return arrays


TINY = dict(d=64, ffn=128, nh=2, nkv=1, hd=64, layers=2, vocab=53)


def test_decoder_batched_prefill_equals_position_by_position():
    """The prompt as one batch equals the reference's position-by-position feed (generate_greedy_by,
    generate.rs:82-111): every op is per row except attention, which is causal."""
    cfg = dict(TINY, max_pos=40, h_shift=8)
    arrays = dec_arrays(cfg, 700, 40)
    prompt = O.gen_uniform(701, 0, cfg["vocab"] - 1, 23)
    t1, l1 = O.dec_generate(cfg, arrays, prompt, 9, batched=True)
    t2, l2 = O.dec_generate(cfg, arrays, prompt, 9, batched=False)
    assert np.array_equal(l1, l2) and np.array_equal(t1, t2)
    assert np.array_equal(t1, l1.reshape(9, -1).argmax(axis=1))  # np.argmax is the first maximum too
    assert len(set(l1.tolist())) > 100


def py_decoder(cfg, a, prompt, max_new):
    """The decoder rules in Python integers, position by position (a second statement of the oracle's definition)."""
    d, ffn, nh, nkv, hd, L, V = (cfg[k] for k in ("d", "ffn", "nh", "nkv", "hd", "layers", "vocab"))
    nq, hh, rep = (nh + 2 * nkv) * hd, hd // 2, nh // nkv

    def dr(x, y):
        q = (2 * abs(x) + y) // (2 * y)
        return q if x >= 0 else -q

    def sr(v, s):
        q = (abs(v) + (1 << (s - 1))) >> s
        return q if v >= 0 else -q

    def c127(v):
        return max(-127, min(127, v))

    def s32(v):
        return max(-(2**31), min(2**31 - 1, v))

    def norm(r):
        ss = sum(v * v for v in r)
        import math as m_
        rms = m_.isqrt(ss // d)
        return [0 if rms == 0 else c127(dr(32 * v, rms)) for v in r]

    def mat(name, l, n, k):
        w = a[name].reshape(L if name != "emb" else 1, n, k)[l] if name != "emb" else a["emb"].reshape(n, k)
        return w.astype(np.int64)

    def lin(x, w, mant, shift):
        acc = w @ np.array(x, dtype=np.int64)
        return [py_requant(int(v), int(m), int(s)) for v, m, s in zip(acc, mant, shift)]

    kc = [[None] * (len(prompt) + max_new) for _ in range(L)]
    vc = [[None] * (len(prompt) + max_new) for _ in range(L)]

    def step(tok, p):
        r = [int(v) for v in a["emb"].reshape(V, d)[tok]]
        for l in range(L):
            x = norm(r)
            qkv = [c127(v) for v in lin(x, mat("wqkv", l, nq, d), a["qkv_mant"][l * nq:(l + 1) * nq],
                                        a["qkv_shift"][l * nq:(l + 1) * nq])]
            for hv in range(nh + nkv):
                seg = qkv[hv * hd:(hv + 1) * hd]
                for i in range(hh):
                    A, Bv = seg[i], seg[i + hh]
                    C, S = int(a["rope_cos"][p][i]), int(a["rope_sin"][p][i])
                    seg[i], seg[i + hh] = c127(sr(A * C - Bv * S, 14)), c127(sr(Bv * C + A * S, 14))
                qkv[hv * hd:(hv + 1) * hd] = seg
            kc[l][p] = qkv[nh * hd:(nh + nkv) * hd]
            vc[l][p] = qkv[(nh + nkv) * hd:]
            o = []
            for h in range(nh):
                g = h // rep
                q = qkv[h * hd:(h + 1) * hd]
                s = [sum(qi * ki for qi, ki in zip(q, kc[l][j][g * hd:(g + 1) * hd])) for j in range(p + 1)]
                m = max(s)
                e = [int(a["exp_tab"][(m - sj + 64) >> 7]) if (m - sj + 64) >> 7 < 1024 else 0 for sj in s]
                den = sum(e)
                for i in range(hd):
                    o.append(c127(dr(sum(e[j] * vc[l][j][g * hd + i] for j in range(p + 1)), den)))
            add = lin(o, mat("wo", l, d, nh * hd), a["o_mant"][l * d:(l + 1) * d], a["o_shift"][l * d:(l + 1) * d])
            r = [s32(x_ + s32(y_)) for x_, y_ in zip(r, add)]
            x = norm(r)
            gu = [c127(v) for v in lin(x, mat("wgu", l, 2 * ffn, d), a["gu_mant"][l * 2 * ffn:(l + 1) * 2 * ffn],
                                       a["gu_shift"][l * 2 * ffn:(l + 1) * 2 * ffn])]
            hv_ = [c127(sr(int(a["silu"][gu[c] + 127]) * gu[ffn + c], cfg["h_shift"])) for c in range(ffn)]
            add = lin(hv_, mat("wd", l, d, ffn), a["d_mant"][l * d:(l + 1) * d], a["d_shift"][l * d:(l + 1) * d])
            r = [s32(x_ + s32(y_)) for x_, y_ in zip(r, add)]
        lg = lin(norm(r), a["emb"].reshape(V, d).astype(np.int64), a["lm_mant"], a["lm_shift"])
        return [s32(v) for v in lg]

    for p, t in enumerate(prompt):
        lg = step(int(t), p)
    toks, logs = [], []
    pos = len(prompt)
    for n in range(max_new):
        logs.append(lg)
        nxt = max(range(V), key=lambda i: (lg[i], -i))
        toks.append(nxt)
        if n + 1 < max_new:
            lg = step(nxt, pos)
            pos += 1
    return toks, logs


def test_decoder_oracle_equals_python_restatement():
    cfg = dict(TINY, layers=1, vocab=37, max_pos=12, h_shift=8)
    arrays = dec_arrays(cfg, 900, 12)
    prompt = O.gen_uniform(901, 0, cfg["vocab"] - 1, 6)
    toks, logits = O.dec_generate(cfg, arrays, prompt, 4)
    pt, pl = py_decoder(cfg, arrays, prompt, 4)
    assert toks.tolist() == pt
    assert logits.reshape(4, -1).tolist() == pl


def test_decoder_generators_equal_the_product():
    import tritify_amd as TA

    assert np.array_equal(TA.gen_quant_rows_fast(5, 37, 300), O.gen_quant_rows(5, 37, 300).astype(np.int32))
    w = O.gen_quant_rows(6, 50, 200)
    assert np.abs(w.reshape(50, 200)).max(axis=1).tolist() == [2047] * 50
    m1, s1 = TA.channel_scales_fast(w.astype(np.int32), 50, 200, 16, 2048)
    m2, s2 = O.channel_scales_target(w, 50, 200, 16, 2048)
    assert np.array_equal(m1, m2) and np.array_equal(s1, s2)


# ---------------------------------------------------------------------------------------------------------------
# config 3: each rule of the W12 decoder oracle pinned by what the mathematics fixes (not by a second statement of
# the same formula)


def test_w12_rmsnorm_pins():
    """A constant row normalizes to +-32 everywhere (rms = |c|); a zero row gives 0; one nonzero value c in a row
    of d gives 32 sqrt(d) when c^2 / d is a perfect square (64 for d = 4), clamped to 127 from d = 16."""
    for c in (1, -7, 2**15 - 1, -(2**20), 2**31 - 1):
        q = O.dec_rmsnorm(np.full(896, c, dtype=np.int32), 1, 896)
        assert (q == (32 if c > 0 else -32)).all()
    assert not O.dec_rmsnorm(np.zeros((3, 64), dtype=np.int32), 3, 64).any()
    q = O.dec_rmsnorm(np.array([100, 0, 0, 0], dtype=np.int32), 1, 4)
    assert q.tolist() == [64, 0, 0, 0]
    q = O.dec_rmsnorm(np.array([-400] + [0] * 15, dtype=np.int32), 1, 16)
    assert q.tolist() == [-127] + [0] * 15
    # the sum of squares is exact: 896 values of 2^31 - 1 sum past 2^64 and still give rms = 2^31 - 1 (a wrapping
    # 64-bit sum would not)
    big = np.full(896, 2**31 - 1, dtype=np.int32)
    big[::2] = -(2**31 - 1)
    q = O.dec_rmsnorm(big, 1, 896)
    assert (q == np.where(big > 0, 32, -32)).all()


def test_w12_rope_pins():
    """RoPE at position 0 is the identity on every int8 pair (cos 0 = 1, sin 0 = 0 in the real table); a quarter
    turn (C = 0, S = 2^14) maps (a, b) to (-b, a) and a half turn to (-a, -b), clamped to +-127; at every position of
    the real table the rotation is the float rotation within its rounding."""
    from tritify_amd import workloads as W

    cos_t, sin_t = W.rope_tables(64, 64)
    a, b = np.meshgrid(np.arange(-127, 128), np.arange(-127, 128))
    pairs = np.stack([a.ravel(), b.ravel()], axis=1).astype(np.int8)  # (a, b) as one 2-wide head each
    one = np.array([[16384]], dtype=np.int16), np.array([[0]], dtype=np.int16)
    assert np.array_equal(O.dec_rope(pairs, len(pairs), 2, 0, cos_t[:, :1].copy(), sin_t[:, :1].copy()), pairs)
    quarter = O.dec_rope(pairs, len(pairs), 2, 0, np.array([0], dtype=np.int16), np.array([16384], dtype=np.int16))
    want = np.stack([np.clip(-pairs[:, 1].astype(int), -127, 127), pairs[:, 0]], axis=1)
    assert np.array_equal(quarter.reshape(-1, 2), want)
    half = O.dec_rope(pairs, len(pairs), 2, 0, np.array([-16384], dtype=np.int16), np.array([0], dtype=np.int16))
    assert np.array_equal(half.reshape(-1, 2), np.clip(-pairs.astype(int), -127, 127))
    assert one[0][0, 0] == cos_t[0, 0] and one[1][0, 0] == sin_t[0, 0]
    rng = np.random.default_rng(2)
    x = rng.integers(-90, 91, size=64).astype(np.int8)  # |rotated| < 128: no clamp
    for p in (1, 7, 63):
        y = O.dec_rope(x, 1, 64, p, cos_t, sin_t).astype(float)
        th = 1.0e6 ** (-2.0 * np.arange(32) / 64) * p
        xa, xb = x[:32].astype(float), x[32:].astype(float)
        fa, fb = xa * np.cos(th) - xb * np.sin(th), xb * np.cos(th) + xa * np.sin(th)
        tol = 0.5 + (np.abs(xa) + np.abs(xb)) / 32768 + 1e-9
        assert (np.abs(y[:32] - fa) <= tol).all() and (np.abs(y[32:] - fb) <= tol).all(), p


def test_w12_attention_pins():
    """At position 0 a head returns v_0 exactly; equal scores give the rounded mean of the v rows; one score ahead of
    every other by at least 1024 * 128 returns that row's v; the exp table starts at 2^15, falls monotonically and
    reads round(2^15 / e) at 64."""
    from tritify_amd import workloads as W

    E = W.exp_table()
    assert E[0] == 2**15 and E[64] == round(2**15 / math.e) and (np.diff(E) <= 0).all() and E[-1] >= 0
    rng = np.random.default_rng(12)
    hd, nkv = 64, 2
    q = rng.integers(-127, 128, size=hd).astype(np.int8)
    kl = rng.integers(-127, 128, size=(40, nkv, hd)).astype(np.int8)
    vl = rng.integers(-127, 128, size=(40, nkv, hd)).astype(np.int8)
    for g in range(nkv):
        assert np.array_equal(O.dec_attend(q, kl, vl, 0, nkv, g, hd, E), vl[0, g])
    flat_k = np.repeat(kl[:1], 40, axis=0)  # every key equal: every score equal
    o = O.dec_attend(q, flat_k, vl, 39, nkv, 1, hd, E)
    s = vl[:, 1].astype(np.int64).sum(axis=0)
    want = np.sign(s) * ((2 * np.abs(s) + 40) // 80)  # round half away from zero of s / 40
    assert np.array_equal(o, want.astype(np.int8))
    qd = np.full(hd, 127, dtype=np.int8)
    dom = np.full((40, nkv, hd), -127, dtype=np.int8)
    dom[17] = 127  # q . k = 64 * 127^2 there and -64 * 127^2 elsewhere: a gap of 2 064 512 > 1024 * 128
    assert np.array_equal(O.dec_attend(qd, dom, vl, 39, nkv, 0, hd, E), vl[17, 0])


def test_greedy_takes_the_first_maximum():
    """argmax_codes (generate.rs:48-56; the reference's own test cases, tests_generate.rs:46-50)."""
    for v, want in (([3, 7, 7, 1], 1), ([-5, -2, -9], 1), ([4], 0), ([0, 0, 0], 0)):
        a = np.array(v, dtype=np.int32)
        assert O.lib().kt_argmax_i32(a.ctypes.data, a.size) == want
