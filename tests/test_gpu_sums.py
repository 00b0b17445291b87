"""The decode row's QuantLinear stopped at its exact sums (kt_hip_quant_linear_multi_sums) and requantized by the op
that reads it (kt_hip_ref_add_rmsnorm_sums, kt_hip_ref_swiglu_sums, kt_hip_ref_attention_step_sums): every reader's
codes, Scale records and cache rows equal the two-launch path's -- the QuantLinear's own requant_dyn followed by the
plain reader, both pinned against the oracle in test_gpu_quant.py and test_gpu_refdec.py -- on live inputs, an
all-zero x (mode 1: zeros at Scale::ZERO) and a zero weight scale (mode 2: c == 0)."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

WLEVELS = 265720


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def rec(torch, sc):
    w = np.zeros(4, dtype=np.int64)
    w[0] = sc[0]
    w.view(np.int32)[2] = sc[1]
    return torch.from_numpy(w).cuda()


def words(r):
    """A record's four words (mant, shift + pad, xmax, ymax) as the host sees them."""
    return r.cpu().numpy().tolist()


def codes(torch, rng, n, mag=2**27, zero=False):
    a = np.zeros(n, np.int32) if zero else rng.integers(-mag, mag, size=n).astype(np.int32)
    return torch.from_numpy(a).cuda()


def wscale(rng, zero=False):
    return (0, 0) if zero else (int(rng.integers(2**30, 2**31)), int(rng.integers(40, 50)))


@pytest.mark.parametrize("mode", ["live", "zero_x", "zero_c"])
@pytest.mark.parametrize("n_in,n", [(896, 896), (4864, 896), (200, 4096)])
def test_add_rmsnorm_sums_equals_requant_then_add_rmsnorm(torch_dev, mode, n_in, n):
    """o / down -> the residual add and the next norm: the sums path against quant_linear + ref_add_rmsnorm."""
    torch = torch_dev
    import tritify_amd as TA
    from tritify_amd import backend as B

    say(f"case: add_rmsnorm sums in={n_in} n={n} mode={mode}")
    rng = np.random.default_rng(n_in + n)
    w = rng.integers(-WLEVELS, WLEVELS + 1, size=(n, n_in)).astype(np.int32)
    ql = TA.QuantLinear("o", w, n, n_in, wscale(rng, mode == "zero_c"))
    assert ql.sums_ok()
    c, cs = codes(torch, rng, n_in, zero=mode == "zero_x"), rec(torch, (1509949440, 58))
    x = codes(torch, rng, n, 2**28)
    xs = (int(rng.integers(2**30, 2**31)), 60)
    g = codes(torch, rng, n, 2**20)
    gs, eps = (1 << 30, 50), B.ref_scale_from_f64(1e-6)
    out = {}
    for path in ("requant", "sums"):
        y, ys = x.clone(), rec(torch, xs)
        h, hs = torch.zeros(n, dtype=torch.int32, device="cuda"), rec(torch, (0, 0))
        if path == "requant":
            b, bs = ql.forward_int(c, cs, 1)
            B.ref_add_rmsnorm(y, ys, b, bs, n, y, ys, g, gs, eps, h, hs)
        else:
            bs = rec(torch, (7, 7))
            B.ref_add_rmsnorm_sums(y, ys, ql.forward_sums(c, cs, rec=bs), n, y, ys, g, gs, eps, h, hs)
        torch.cuda.synchronize()
        out[path] = (y.cpu().numpy(), words(ys), h.cpu().numpy(), words(hs), words(bs))
    a, s = out["requant"], out["sums"]
    assert np.array_equal(a[0], s[0]) and a[1] == s[1], "the sum"
    assert np.array_equal(a[2], s[2]) and a[3] == s[3], "the norm"
    assert a[4] == s[4], "the projection's record"
    if mode != "live":
        assert a[4][0] == 0


@pytest.mark.parametrize("mode", ["live", "zero_x", "zero_c"])
@pytest.mark.parametrize("inp,n", [(896, 4864), (64, 128), (300, 8192)])
def test_swiglu_sums_equals_requant_then_swiglu(torch_dev, mode, inp, n):
    """gate / up -> SwiGLU: the sums path against the group's quant_linear_multi + ref_swiglu (zero_c: the up
    member at a zero weight scale)."""
    torch = torch_dev
    import tritify_amd as TA
    from tritify_amd import backend as B

    say(f"case: swiglu sums in={inp} n={n} mode={mode}")
    rng = np.random.default_rng(inp + n)
    members = [(nm, rng.integers(-WLEVELS, WLEVELS + 1, size=(n, inp)).astype(np.int32),
                wscale(rng, mode == "zero_c" and nm == "u"), None) for nm in ("g", "u")]
    grp = TA.QuantLinearGroup("gu", members, inp)
    assert grp.sums_ok()
    x, xs = codes(torch, rng, inp, zero=mode == "zero_x"), rec(torch, (1509949440, 58))
    silu_codes, silu = B.ref_codelut(B.LUT_SILU, -30.0, 30.0, 16, 20, True)
    sc = torch.from_numpy(silu_codes).cuda()
    out = {}
    for path in ("requant", "sums"):
        h, hs = torch.zeros(n, dtype=torch.int32, device="cuda"), rec(torch, (0, 0))
        recs = torch.full((8,), 5, dtype=torch.int64, device="cuda")
        if path == "requant":
            (gt, gr), (up, ur) = grp.forward_int(x, xs, 1, os_dev=recs)
            B.ref_swiglu(gt, gr, up, ur, n, sc, silu, h, hs)
        else:
            gt, up = grp.forward_sums(x, xs, os_dev=recs)
            B.ref_swiglu_sums(gt, up, n, sc, silu, h, hs)
        torch.cuda.synchronize()
        out[path] = (h.cpu().numpy(), words(hs), words(recs))
    a, s = out["requant"], out["sums"]
    assert np.array_equal(a[0], s[0]) and a[1] == s[1], "the activation"
    assert a[2] == s[2], "the gate / up records"


@pytest.mark.parametrize("max_seq,steps", [(48, 48), (4096, 24)])
@pytest.mark.parametrize("mode", ["live", "zero_c"])
def test_attention_step_sums_equals_requant_then_attention(torch_dev, max_seq, steps, mode):
    """q / k / v -> the attention step over a growing cache (two caches, one per path): output codes and record,
    the q / k / v records and every cache row and step scale equal at every step. Steps 3 and 10 take an all-zero x
    (mode 1: q, k and v zero at Scale::ZERO); zero_c puts the v member at a zero weight scale. max_seq 4096 keeps
    the per-step arrays in the workspace, 48 in LDS."""
    torch = torch_dev
    import tritify_amd as TA
    from tritify_amd import backend as B

    nh, nkv, hd, inp = 14, 2, 64, 896
    say(f"case: attention sums max_seq={max_seq} steps={steps} mode={mode}")
    rng = np.random.default_rng(max_seq)
    members = [(nm, rng.integers(-WLEVELS, WLEVELS + 1, size=(o, inp)).astype(np.int32),
                wscale(rng, mode == "zero_c" and nm == "v"), None)
               for nm, o in (("q", nh * hd), ("k", nkv * hd), ("v", nkv * hd))]
    grp = TA.QuantLinearGroup("qkv", members, inp)
    assert grp.sums_ok()
    cos_t, sin_t = B.ref_rope_tables(max_seq, hd, 1.0e6)
    cos_d, sin_d = (torch.from_numpy(t.view(np.uint8)).cuda() for t in (cos_t, sin_t))
    exp_codes, exp_lut = B.ref_codelut(B.LUT_EXP, -30.0, 0.0, 16, 20, False)
    exp_d = torch.from_numpy(exp_codes).cuda()
    isq = B.ref_scale_from_f64(1.0 / np.sqrt(hd))
    kvd = nkv * hd
    st = {}
    for path in ("requant", "sums"):
        st[path] = dict(kc=torch.zeros(max_seq * kvd, dtype=torch.int32, device="cuda"),
                        vc=torch.zeros(max_seq * kvd, dtype=torch.int32, device="cuda"),
                        ks=torch.zeros(max_seq * 16, dtype=torch.uint8, device="cuda"),
                        vs=torch.zeros(max_seq * 16, dtype=torch.uint8, device="cuda"),
                        ws=torch.full((B.ref_attention_step_workspace(max_seq, nh, hd),), 0x77, dtype=torch.uint8,
                                      device="cuda"))
    pos = torch.zeros(1, dtype=torch.int32, device="cuda")
    for p in range(steps):
        x = codes(torch, rng, inp, zero=p in (3, 10))
        xs = rec(torch, (int(rng.integers(2**30, 2**31)), int(rng.integers(56, 60))))
        pos.fill_(p)
        out = {}
        for path in ("requant", "sums"):
            S = st[path]
            o, os_ = torch.zeros(nh * hd, dtype=torch.int32, device="cuda"), rec(torch, (0, 0))
            recs = torch.full((12,), 9, dtype=torch.int64, device="cuda")
            if path == "requant":
                (q, qr), (k, kr), (v, vr) = grp.forward_int(x, xs, 1, os_dev=recs)
                B.ref_attention_step(q, qr, k, kr, v, vr, pos, nh, nkv, hd, max_seq, S["kc"], S["vc"], S["ks"],
                                     S["vs"], cos_d, sin_d, isq, exp_d, exp_lut, o, os_, ws_dev=S["ws"])
            else:
                q, k, v = grp.forward_sums(x, xs, os_dev=recs)
                B.ref_attention_step_sums(q, k, v, pos, nh, nkv, hd, max_seq, S["kc"], S["vc"], S["ks"], S["vs"],
                                          cos_d, sin_d, isq, exp_d, exp_lut, o, os_, S["ws"])
            torch.cuda.synchronize()
            out[path] = (o.cpu().numpy(), words(os_), words(recs))
        a, s = out["requant"], out["sums"]
        assert np.array_equal(a[0], s[0]), f"step {p}: output codes"
        assert a[1] == s[1], f"step {p}: output record"
        assert a[2] == s[2], f"step {p}: q / k / v records"
    for t in ("kc", "vc", "ks", "vs"):
        assert torch.equal(st["requant"][t], st["sums"][t]), t


def test_sums_entries_refuse_what_they_cannot_take(torch_dev):
    """A bias, a shape past the one-launch product, a misaligned boundary and a reader of the wrong width are
    refused before any device work."""
    torch = torch_dev
    import tritify_amd as TA
    from tritify_amd import backend as B

    rng = np.random.default_rng(1)
    w = rng.integers(-WLEVELS, WLEVELS + 1, size=(64, 32)).astype(np.int32)
    assert not TA.QuantLinear("b", w, 64, 32, (1 << 30, 40), (np.zeros(64, np.int64), (1 << 30, 40))).sums_ok()
    ql = TA.QuantLinear("o", w, 64, 32, (1 << 30, 40))
    ws, nb = ql.workspace(1)
    x, xs = codes(torch, rng, 32), rec(torch, (1 << 30, 58))
    with pytest.raises(B.HipError):  # a boundary at 60 columns
        B.quant_linear_multi_sums(x, 32, xs, [60, 4], ql.w_planes, ql.pw, [(1 << 30, 40)] * 2, ws, nb)
    s = ql.forward_sums(x, xs)
    y, ys = torch.zeros(63, dtype=torch.int32, device="cuda"), rec(torch, (1 << 30, 40))
    h, hs = torch.zeros(63, dtype=torch.int32, device="cuda"), rec(torch, (0, 0))
    with pytest.raises(B.HipError):  # 63 values against a 64-value output
        B.ref_add_rmsnorm_sums(y, ys, s, 63, y, ys, h, (1, 0), (1, 0), h, hs)
    torch.cuda.synchronize()
