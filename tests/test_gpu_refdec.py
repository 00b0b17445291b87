"""The reference decoder at its own semantics on the GPU, through the C ABI, against the oracle
(oracle/kt_oracle_refdec.c): every op on random inputs and scales (codes and Scale records bit for bit), the
attention step over a growing cache, the reference's synthetic decoder reproducing verify_repro's golden
8109ebad... at every position, and a Qwen2.5-shaped two-layer model against the oracle position by position."""
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def rec(torch, sc):
    w = np.zeros(4, dtype=np.int64)
    w[0] = sc[0]
    w.view(np.int32)[2] = sc[1]
    return torch.from_numpy(w).cuda()


def rd(r):
    w = r.cpu().numpy()
    return int(w[0]), int(w.view(np.int32)[2])


def dev_i32(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32).reshape(-1)).cuda()


def rand_scale(rng):
    return int(rng.integers(2**30, 2**31)), int(rng.integers(40, 62))


@pytest.mark.parametrize("rows,dim,mag", [(1, 32, 2**28), (1, 896, 2**14), (1, 896, 2**28), (3, 200, 2**20),
                                          (1, 5000, 2**27)])
def test_ref_rmsnorm(torch_dev, rows, dim, mag):
    torch = torch_dev
    from tritify_amd import backend as B

    say(f"case: ref_rmsnorm rows={rows} dim={dim} mag={mag}")
    rng = np.random.default_rng(rows * 7 + dim)
    x = rng.integers(-mag, mag, size=rows * dim).astype(np.int32)
    g = rng.integers(-O.WLEVELS, O.WLEVELS + 1, size=dim).astype(np.int32)
    if rows > 1:
        x[dim:2 * dim] = 0  # a zero row among others
    xs, gs, eps = rand_scale(rng), rand_scale(rng), B.ref_scale_from_f64(1e-6)
    y, ys = torch.zeros(rows * dim, dtype=torch.int32, device="cuda"), rec(torch, (0, 0))
    B.ref_rmsnorm(dev_i32(torch, x), rec(torch, xs), rows, dim, dev_i32(torch, g), gs, eps, y, ys)
    yo, so = O.rd_rmsnorm(x, rows, dim, xs, g, gs, eps)
    assert np.array_equal(y.cpu().numpy(), yo) and rd(ys) == so
    # a zero input scale gives zeros at Scale::ZERO
    B.ref_rmsnorm(dev_i32(torch, x), rec(torch, (0, 0)), rows, dim, dev_i32(torch, g), gs, eps, y, ys)
    assert not y.cpu().numpy().any() and rd(ys) == (0, 0)


@pytest.mark.parametrize("n", [32, 896, 4864])
def test_ref_add(torch_dev, n):
    torch = torch_dev
    from tritify_amd import backend as B

    say(f"case: ref_add n={n}")
    rng = np.random.default_rng(n)
    for trial in range(4):
        a = rng.integers(-(2**28), 2**28 + 1, size=n).astype(np.int32)
        b = rng.integers(-(2**28), 2**28 + 1, size=n).astype(np.int32)
        sa, sb = rand_scale(rng), rand_scale(rng)
        if trial == 2:
            sb = (0, 0)
        if trial == 3:
            b = -a
            sb = sa  # cancels exactly: zeros at Scale::ZERO
        yo, so = O.rd_add(a, sa, b, sb)
        ad, ar = dev_i32(torch, a), rec(torch, sa)
        B.ref_add(ad, ar, dev_i32(torch, b), rec(torch, sb), n, ad, ar)  # in place, as the residual add runs
        assert np.array_equal(ad.cpu().numpy(), yo) and rd(ar) == so, trial


@pytest.mark.parametrize("n", [1, 32, 896, 4096])
def test_ref_add_rmsnorm(torch_dev, n):
    """The residual add and the next norm in one launch: the oracle's add, then its RmsNorm of the sum (in place
    on a, as the decode step runs it), including a zero branch scale and an exact cancellation."""
    torch = torch_dev
    from tritify_amd import backend as B

    say(f"case: ref_add_rmsnorm n={n}")
    rng = np.random.default_rng(n + 11)
    g = rng.integers(-O.WLEVELS, O.WLEVELS + 1, size=n).astype(np.int32)
    gs, eps = rand_scale(rng), B.ref_scale_from_f64(1e-6)
    gd = dev_i32(torch, g)
    for trial in range(4):
        a = rng.integers(-(2**28), 2**28 + 1, size=n).astype(np.int32)
        b = rng.integers(-(2**28), 2**28 + 1, size=n).astype(np.int32)
        sa, sb = rand_scale(rng), rand_scale(rng)
        if trial == 2:
            sb = (0, 0)
        if trial == 3:
            b, sb = -a, sa  # cancels exactly: zeros at Scale::ZERO, then a zero norm
        yo, so = O.rd_add(a, sa, b, sb)
        ho, hso = O.rd_rmsnorm(yo, 1, n, so, g, gs, eps)
        ad, ar = dev_i32(torch, a), rec(torch, sa)
        h, hs = torch.zeros(n, dtype=torch.int32, device="cuda"), rec(torch, (0, 0))
        B.ref_add_rmsnorm(ad, ar, dev_i32(torch, b), rec(torch, sb), n, ad, ar, gd, gs, eps, h, hs)
        assert np.array_equal(ad.cpu().numpy(), yo) and rd(ar) == so, trial
        assert np.array_equal(h.cpu().numpy(), ho) and rd(hs) == hso, trial
    with pytest.raises(B.HipError):  # a row past the one-CTA bound, and h over y, are refused
        B.ref_add_rmsnorm(ad, ar, ad, ar, B.REF_ADD_NORM_MAX + 1, ad, ar, gd, gs, eps, h, hs)
    with pytest.raises(B.HipError):
        B.ref_add_rmsnorm(ad, ar, ad, ar, n, h, ar, gd, gs, eps, h, hs)


@pytest.mark.parametrize("n,gshift", [(64, 53), (4864, 53), (4864, 60), (777, 48)])
def test_ref_swiglu(torch_dev, n, gshift):
    torch = torch_dev
    from tritify_amd import backend as B

    say(f"case: ref_swiglu n={n} gshift={gshift}")
    model = O.RefModel(7)
    rng = np.random.default_rng(n + gshift)
    g = rng.integers(-(2**28), 2**28, size=n).astype(np.int32)
    u = rng.integers(-(2**28), 2**28, size=n).astype(np.int32)
    gs, us = (int(rng.integers(2**30, 2**31)), gshift), rand_scale(rng)
    codes, lut = B.ref_codelut(B.LUT_SILU, -30.0, 30.0, 16, 20, True)
    h, hs = torch.zeros(n, dtype=torch.int32, device="cuda"), rec(torch, (0, 0))
    B.ref_swiglu(dev_i32(torch, g), rec(torch, gs), dev_i32(torch, u), rec(torch, us), n,
                 torch.from_numpy(codes).cuda(), lut, h, hs)
    ho, so = O.rd_swiglu_act(model, g, gs, u, us)
    assert np.array_equal(h.cpu().numpy(), ho) and rd(hs) == so


def test_ref_embed_and_argmax(torch_dev):
    torch = torch_dev
    from tritify_amd import backend as B

    say("case: ref_embed / ref_argmax")
    rng = np.random.default_rng(1)
    vocab, dim = 50, 24
    emb = rng.integers(-O.WLEVELS, O.WLEVELS + 1, size=vocab * dim).astype(np.int32)
    ed = dev_i32(torch, emb)
    y, ys = torch.zeros(dim, dtype=torch.int32, device="cuda"), rec(torch, (0, 0))
    for t in (0, 17, 49, 50, -1):
        B.ref_embed(ed, (1234567890, 50), dev_i32(torch, [t]), vocab, dim, y, ys)
        if 0 <= t < vocab:
            assert np.array_equal(y.cpu().numpy(), emb[t * dim:(t + 1) * dim]) and rd(ys) == (1234567890, 50)
        else:
            assert not y.cpu().numpy().any() and rd(ys) == (0, 0)
    n = 151936
    logits = rng.integers(-(2**28), 2**28, size=n).astype(np.int32)
    logits[[5, 700, 150000]] = 2**28 + 7  # three equal maxima: the first wins
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    record = torch.zeros(2 * n, dtype=torch.int32, device="cuda")
    rscale = torch.zeros(2 * 16, dtype=torch.uint8, device="cuda")
    step = torch.zeros(1, dtype=torch.int32, device="cuda")
    ld = dev_i32(torch, logits)
    for s in range(2):
        B.ref_argmax(ld, n, rec(torch, (999, 9 + s)), tok, record, rscale, step)
        assert int(tok.item()) == 5
    assert int(step.item()) == 2
    rs = rscale.cpu().numpy().view(B.SSCALE)
    assert (rs["mant"] == 999).all() and rs["shift"].tolist() == [9, 10]
    assert np.array_equal(record.cpu().numpy().reshape(2, n)[1], logits)
    # ties inside one 16-byte group and in its neighbour; a length that is not a multiple of 4 (the scalar path),
    # with and without the record; a maximum at the last code
    for n2, at, want in ((4096, [9, 8, 4000], 8), (1001, [1000], 1000), (1001, [3, 2, 999], 2)):
        lg = rng.integers(-(2**30), 2**30, size=n2).astype(np.int32)
        lg[at] = 2**31 - 1
        ld2 = dev_i32(torch, lg)
        B.ref_argmax(ld2, n2, rec(torch, (1, 1)), tok, None, None, None)
        assert int(tok.item()) == want, (n2, at)
        rec2, st2 = torch.zeros(n2, dtype=torch.int32, device="cuda"), torch.zeros(1, dtype=torch.int32, device="cuda")
        B.ref_argmax(ld2, n2, rec(torch, (1, 1)), tok, rec2, torch.zeros(16, dtype=torch.uint8, device="cuda"), st2)
        assert int(tok.item()) == want and np.array_equal(rec2.cpu().numpy(), lg) and int(st2.item()) == 1


def test_ref_argmax_record_stops_at_its_last_row(torch_dev):
    """A step at or past the record's rows (replays of a captured greedy step beyond max_seq) or below zero records
    nothing and does not advance: the guard rows after the record stay untouched."""
    torch = torch_dev
    from tritify_amd import backend as B

    say("case: ref_argmax record capacity")
    rng = np.random.default_rng(5)
    n, cap, guard = 1000, 3, 2
    lg = rng.integers(-(2**30), 2**30, size=n).astype(np.int32)
    lg[417] = 2**31 - 1
    ld = dev_i32(torch, lg)
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    record = torch.full(((cap + guard) * n,), 0x5A5A5A5A, dtype=torch.int32, device="cuda")
    rscale = torch.full(((cap + guard) * 16,), 0xA5, dtype=torch.uint8, device="cuda")
    step = torch.tensor([cap - 1], dtype=torch.int32, device="cuda")
    for _ in range(cap + 2):
        B.ref_argmax(ld, n, rec(torch, (7, 3)), tok, record, rscale, step, record_rows=cap)
        assert int(tok.item()) == 417
    assert int(step.item()) == cap
    r = record.cpu().numpy().reshape(cap + guard, n)
    assert np.array_equal(r[cap - 1], lg) and (r[cap:] == 0x5A5A5A5A).all() and (r[:cap - 1] == 0x5A5A5A5A).all()
    rs = rscale.cpu().numpy().reshape(cap + guard, 16)
    assert (rs[cap:] == 0xA5).all() and (rs[:cap - 1] == 0xA5).all()
    step.fill_(-1)
    B.ref_argmax(ld, n, rec(torch, (7, 3)), tok, record, rscale, step, record_rows=cap)
    assert int(step.item()) == -1 and int(tok.item()) == 417
    assert (record.cpu().numpy().reshape(cap + guard, n)[:cap - 1] == 0x5A5A5A5A).all()
    with pytest.raises(RuntimeError):
        B.ref_argmax(ld, n, rec(torch, (7, 3)), tok, record, rscale, step, record_rows=0)


@pytest.mark.parametrize("cfg", [dict(O.SYNTH_CFG, max_seq=48),
                                 dict(dim=64, layers=1, nh=14, nkv=2, hd=64, hidden=64, vocab=8, eps=1e-6,
                                      theta=1.0e6, max_seq=80),
                                 dict(dim=64, layers=1, nh=12, nkv=1, hd=32, hidden=64, vocab=8, eps=1e-6,
                                      theta=1.0e6, max_seq=40),
                                 dict(dim=64, layers=1, nh=14, nkv=2, hd=128, hidden=64, vocab=8, eps=1e-6,
                                      theta=1.0e6, max_seq=512)])
@pytest.mark.parametrize("heads", [False, True])
def test_ref_attention_steps(torch_dev, cfg, heads):
    """Steps 0..max_seq-1 of Attention::decode_step's core on random q/k/v codes and scales (some steps with a zero k
    or v scale), the device cache against the oracle's, output codes and scale at every step. The configurations
    reach both P.V layouts of the one-CTA kernel: by kv head (groups of up to 8 q heads; at max_seq 512 with head_dim
    128 the heads' scores fit 5 at a time, so batches split the groups) and by (head, dim) for a 12-head group.
    heads: the same steps on the one-CTA-per-head kernels (a workspace given), head_dim 8 to 128."""
    torch = torch_dev
    from tritify_amd import backend as B

    say(f"case: ref_attention_steps nh={cfg['nh']} nkv={cfg['nkv']} hd={cfg['hd']} steps={cfg['max_seq']} "
        f"heads={heads}")
    model = O.RefModel(11, cfg)
    cache = O.RefCache(model)
    nh, nkv, hd, ms = cfg["nh"], cfg["nkv"], cfg["hd"], cfg["max_seq"]
    qd, kvd = nh * hd, nkv * hd
    cos_t, sin_t = B.ref_rope_tables(ms, hd, cfg["theta"])
    cos_d, sin_d = (torch.from_numpy(t.view(np.uint8)).cuda() for t in (cos_t, sin_t))
    exp_codes, exp_lut = B.ref_codelut(B.LUT_EXP, -30.0, 0.0, 16, 20, False)
    exp_d = torch.from_numpy(exp_codes).cuda()
    isq = B.ref_scale_from_f64(1.0 / np.sqrt(hd))
    kc = torch.zeros(ms * kvd, dtype=torch.int32, device="cuda")
    vc = torch.zeros(ms * kvd, dtype=torch.int32, device="cuda")
    ks_d = torch.zeros(ms * 16, dtype=torch.uint8, device="cuda")
    vs_d = torch.zeros(ms * 16, dtype=torch.uint8, device="cuda")
    o, os_ = torch.zeros(qd, dtype=torch.int32, device="cuda"), rec(torch, (0, 0))
    pos_d = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws = torch.full((B.ref_attention_step_workspace(ms, nh, hd),), 0x77, dtype=torch.uint8, device="cuda") \
        if heads else None
    rng = np.random.default_rng(nh)
    for p in range(ms):
        q = rng.integers(-(2**28), 2**28, size=qd).astype(np.int32)
        k = rng.integers(-(2**28), 2**28, size=kvd).astype(np.int32)
        v = rng.integers(-(2**28), 2**28, size=kvd).astype(np.int32)
        # scales spread over 2^6 so the softmax is neither flat nor one-hot
        qs, ks, vs = (int(rng.integers(2**30, 2**31)), int(rng.integers(78, 84))), rand_scale(rng), rand_scale(rng)
        if p % 7 == 3:
            ks = (0, 0)
        if p % 11 == 5:
            vs = (0, 0)
        pos_d.fill_(p)
        B.ref_attention_step(dev_i32(torch, q), rec(torch, qs), dev_i32(torch, k), rec(torch, ks), dev_i32(torch, v),
                             rec(torch, vs), pos_d, nh, nkv, hd, ms, kc, vc, ks_d, vs_d, cos_d, sin_d, isq, exp_d,
                             exp_lut, o, os_, ws_dev=ws)
        oo, so = O.rd_attention_core(cache, q, qs, k, ks, v, vs, p)
        got = o.cpu().numpy()
        assert np.array_equal(got, oo), f"step {p}: {np.argwhere(got != oo)[:5].tolist()}"
        assert rd(os_) == so, p


@pytest.mark.parametrize("max_seq,heads", [(1369, False), (1369, True), (4096, True)])
def test_ref_attention_steps_long_cache(torch_dev, max_seq, heads):
    """Attention::decode_step's core at the Qwen2.5-0.5B heads (14 / 2 of 64) over every position of a long cache:
    1369 positions, the most the one-CTA kernel's LDS holds (one head's scores at a time), and on the one-CTA-per-head
    kernels 1369 and 4096, the reference's MAX_SEQ_CAP (crates/03-models/kt-model-decoder/src/lib.rs:46). The device
    runs every step; the oracle
    checks the output codes and scale at spread positions (the first steps, every 97th, around 1369 and the last)
    and only appends to its cache in between."""
    torch = torch_dev
    from tritify_amd import backend as B

    nh, nkv, hd = 14, 2, 64
    say(f"case: ref_attention_steps long cache max_seq={max_seq} heads={heads}")
    cfg = dict(dim=64, layers=1, nh=nh, nkv=nkv, hd=hd, hidden=64, vocab=8, eps=1e-6, theta=1.0e6, max_seq=max_seq)
    assert B.ref_attention_step_fits_lds(max_seq, nh, hd) == (max_seq <= 1369)
    model = O.RefModel(11, cfg)
    cache = O.RefCache(model)
    qd, kvd, ms = nh * hd, nkv * hd, max_seq
    cos_t, sin_t = B.ref_rope_tables(ms, hd, cfg["theta"])
    cos_d, sin_d = (torch.from_numpy(t.view(np.uint8)).cuda() for t in (cos_t, sin_t))
    exp_codes, exp_lut = B.ref_codelut(B.LUT_EXP, -30.0, 0.0, 16, 20, False)
    exp_d = torch.from_numpy(exp_codes).cuda()
    isq = B.ref_scale_from_f64(1.0 / np.sqrt(hd))
    kc = torch.zeros(ms * kvd, dtype=torch.int32, device="cuda")
    vc = torch.zeros(ms * kvd, dtype=torch.int32, device="cuda")
    ks_d = torch.zeros(ms * 16, dtype=torch.uint8, device="cuda")
    vs_d = torch.zeros(ms * 16, dtype=torch.uint8, device="cuda")
    o, os_ = torch.zeros(qd, dtype=torch.int32, device="cuda"), rec(torch, (0, 0))
    pos_d = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws = torch.empty(B.ref_attention_step_workspace(ms, nh, hd), dtype=torch.uint8, device="cuda") if heads else None
    check = set(range(8)) | set(range(0, ms, 97)) | {1367, 1368, 1369, 1370} | set(range(ms - 3, ms))
    rng = np.random.default_rng(4096 + ms)
    qb = rng.integers(-(2**28), 2**28, size=(ms, qd)).astype(np.int32)
    kb = rng.integers(-(2**28), 2**28, size=(ms, kvd)).astype(np.int32)
    vb = rng.integers(-(2**28), 2**28, size=(ms, kvd)).astype(np.int32)
    qdv, kdv, vdv = (torch.from_numpy(a).cuda() for a in (qb, kb, vb))
    scl = [((int(rng.integers(2**30, 2**31)), int(rng.integers(78, 84))), rand_scale(rng), rand_scale(rng))
           for _ in range(ms)]
    srec = torch.from_numpy(np.array([[m, sh] for t in scl for (m, sh) in t], dtype=np.int64)).cuda()
    recs = torch.zeros((ms * 3, 4), dtype=torch.int64, device="cuda")
    recs[:, 0] = srec[:, 0]
    recs[:, 1] = srec[:, 1]  # the shift in the low word of the second int64 (little endian)
    checked = 0
    for p in range(ms):
        (qs, ks, vs) = scl[p]
        pos_d.fill_(p)
        B.ref_attention_step(qdv[p], recs[3 * p], kdv[p], recs[3 * p + 1], vdv[p], recs[3 * p + 2], pos_d, nh, nkv,
                             hd, ms, kc, vc, ks_d, vs_d, cos_d, sin_d, isq, exp_d, exp_lut, o, os_, ws_dev=ws)
        if p in check:
            oo, so = O.rd_attention_core(cache, qb[p], qs, kb[p], ks, vb[p], vs, p)
            got = o.cpu().numpy()
            assert np.array_equal(got, oo), f"step {p}: {np.argwhere(got != oo)[:5].tolist()}"
            assert rd(os_) == so, p
            checked += 1
        else:
            O.rd_attention_append(cache, kb[p], ks, vb[p], vs, p)
    assert checked == len([c for c in check if c < ms])
    # a cache past the one-CTA kernel's LDS is refused without a workspace
    if max_seq > 1369:
        with pytest.raises(RuntimeError):
            B.ref_attention_step(qdv[0], recs[0], kdv[0], recs[1], vdv[0], recs[2], pos_d, nh, nkv, hd, ms, kc, vc,
                                 ks_d, vs_d, cos_d, sin_d, isq, exp_d, exp_lut, o, os_)


def test_synthetic_decoder_reproduces_the_golden(torch_dev):
    """verify_repro --synthetic on the device: RefDecoder over the seed-7 model gives logits_hash 8109ebad...
    (REPRODUCE.md:17) and the oracle's hash at every position."""
    from tritify_amd.refdecoder import RefDecoder

    say("case: synthetic decoder seed 7, 12-token prompt, 32 greedy tokens")
    model = O.RefModel(7)
    toks_o, run_o, pos_o = model.generate(O.SYNTH_PROMPT, 32)
    dec = RefDecoder(O.SYNTH_CFG, *model.weights())
    toks, run, hashes = dec.generate_greedy(O.SYNTH_PROMPT, 32)
    first = next((i for i, (a, b) in enumerate(zip(hashes, pos_o)) if a != b), None)
    assert first is None, f"first differing position {first}"
    assert toks == toks_o and run == run_o == O.SYNTH_HASH


def test_graph_replayed_greedy_steps_reproduce_the_golden(torch_dev):
    """The same generation as replays of one captured greedy step (decode step + argmax_codes, the position advanced
    and the logits recorded on the device): every recorded position's hash equals the oracle's and the run's hash is
    8109ebad..."""
    import hashlib

    from tritify_amd.refdecoder import RefDecoder, logits_hash_bytes

    say("case: synthetic decoder seed 7 as graph replays")
    model = O.RefModel(7)
    toks_o, run_o, pos_o = model.generate(O.SYNTH_PROMPT, 32)
    dec = RefDecoder(O.SYNTH_CFG, *model.weights())
    dec.decode_step(O.SYNTH_PROMPT[0], 0)  # workspaces exist before the capture
    g = dec.capture_greedy_step()
    dec.new_cache()
    dec.pos.zero_()
    for t in O.SYNTH_PROMPT:
        dec.token.fill_(t)
        g.replay()
    for _ in range(31):
        g.replay()
    torch_dev.cuda.synchronize()
    P = len(O.SYNTH_PROMPT)
    rec = [dec.recorded(p) for p in range(P + 31)]
    hashes = [hashlib.sha256(logits_hash_bytes(*r)).hexdigest() for r in rec]
    assert hashes == pos_o
    run = hashlib.sha256(b"".join(logits_hash_bytes(*r) for r in rec[P - 1:])).hexdigest()
    assert run == run_o == O.SYNTH_HASH
    assert [int(np.argmax(r[0])) for r in rec[P - 1:]] == toks_o
    assert int(dec.pos.item()) == P + 31


def test_qwen_shaped_decoder_against_the_oracle(torch_dev):
    """Two layers of the Qwen2.5-0.5B shape (dim 896, 14 / 2 heads of 64, SwiGLU 4864, theta 1e6) with a short
    vocabulary, seeded float weights quantized as the engine does: every position's logits hash equals the
    oracle's."""
    from tritify_amd.refdecoder import RefDecoder

    cfg = dict(dim=896, layers=2, nh=14, nkv=2, hd=64, hidden=4864, vocab=512, eps=1e-6, theta=1.0e6, max_seq=64)
    say("case: qwen-shaped reference decoder, 2 layers, 6-token prompt, 8 greedy tokens")
    model = O.RefModel(5, cfg)
    prompt = [1, 100, 200, 300, 400, 511]
    toks_o, run_o, pos_o = model.generate(prompt, 8)
    dec = RefDecoder(cfg, *model.weights())
    toks, run, hashes = dec.generate_greedy(prompt, 8)
    first = next((i for i, (a, b) in enumerate(zip(hashes, pos_o)) if a != b), None)
    assert first is None, f"first differing position {first}"
    assert toks == toks_o and run == run_o


_C3_WEIGHTS: dict = {}


def _c3_weights():
    """Config 3's reference-decoder weights (generated once per session: 494 M codes)."""
    from tritify_amd import workloads as W

    if not _C3_WEIGHTS:
        _C3_WEIGHTS["w"] = W.ref_decoder_weights(W.REF_QWEN, W.REF_C3["w_seed"])
    return _C3_WEIGHTS["w"]


@pytest.mark.parametrize("max_seq,heads", [(640, False), (640, True), (4096, True)])
def test_config3_at_the_reference_semantics_full_size(torch_dev, max_seq, heads):
    """Config 3's workload at the reference's own semantics on the device: the Qwen2.5-0.5B-shape DecoderModel
    (24 layers, vocab 151936), a 512-token prompt through decode_step and 128 greedy steps as replays of one
    captured greedy step. Every one of the 640 positions' logits hash, the run's hash and the chosen tokens equal the
    committed fixture (the oracle's repro::run, tests/golden/make_goldens.py config3_ref): on the one-CTA attention
    step (max_seq 640 in its LDS) and on the one-CTA-per-head step at max_seq 640 and 4096 (the reference's
    MAX_SEQ_CAP)."""
    import hashlib
    import json
    import os

    from tritify_amd import workloads as W
    from tritify_amd.refdecoder import RefDecoder, logits_hash_bytes

    torch = torch_dev
    fx = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "goldens.json")))["config3_ref"]
    cfg = dict(W.REF_QWEN, max_seq=max_seq, attn_heads=heads)
    assert fx["cfg"] == W.REF_QWEN
    prompt = W.ref_c3_prompt(W.REF_QWEN)
    assert hashlib.sha256(np.asarray(prompt, dtype=np.int32).tobytes()).hexdigest() == fx["prompt_sha256"]
    say(f"case: config 3 at the reference semantics, 512 + 128 positions, max_seq {max_seq} heads={heads}")
    dec = RefDecoder(cfg, *_c3_weights())
    assert (dec.attn_ws is None) == (not heads)
    dec.decode_step(prompt[0], 0)
    g = dec.capture_greedy_step()
    dec.new_cache()
    dec.pos.zero_()
    for t in prompt:
        dec.token.fill_(t)
        g.replay()
    for _ in range(W.REF_C3["decode"]):
        g.replay()
    torch.cuda.synchronize()
    P, npos = len(prompt), len(prompt) + W.REF_C3["decode"]
    rec = [dec.recorded(p) for p in range(npos)]
    hashes = [hashlib.sha256(logits_hash_bytes(*r)).hexdigest() for r in rec]
    first = next((i for i, (a, b) in enumerate(zip(hashes, fx["position_sha256"])) if a != b), None)
    assert first is None, f"first differing position {first}"
    assert len(hashes) == len(fx["position_sha256"]) == 640
    run = hashlib.sha256(b"".join(logits_hash_bytes(*r) for r in rec[P - 1:])).hexdigest()
    assert run == fx["run_sha256"]
    assert [int(np.argmax(r[0])) for r in rec[P - 1:]] == fx["tokens"]
    assert int(dec.pos.item()) == npos
    del dec, g, rec
    torch.cuda.empty_cache()
    if max_seq == 4096:
        _C3_WEIGHTS.clear()


@pytest.mark.parametrize("rows,dim", [(65, 896), (300, 64), (1024, 96)])
def test_ref_rmsnorm_many_rows(torch_dev, rows, dim):
    """RMSNorm over a sequence (the batched forward's norms): every row's factor, their largest, one requant."""
    torch = torch_dev
    from tritify_amd import backend as B

    say(f"case: ref_rmsnorm rows={rows} dim={dim}")
    rng = np.random.default_rng(rows + dim)
    x = rng.integers(-(2**28), 2**28, size=rows * dim).astype(np.int32)
    x[dim:2 * dim] = 0
    x[5 * dim:6 * dim] = x[:dim]  # a row equal to row 0: equal factors, the later one is kept
    g = rng.integers(-O.WLEVELS, O.WLEVELS + 1, size=dim).astype(np.int32)
    xs, gs, eps = rand_scale(rng), rand_scale(rng), B.ref_scale_from_f64(1e-6)
    y, ys = torch.zeros(rows * dim, dtype=torch.int32, device="cuda"), rec(torch, (0, 0))
    B.ref_rmsnorm(dev_i32(torch, x), rec(torch, xs), rows, dim, dev_i32(torch, g), gs, eps, y, ys)
    yo, so = O.rd_rmsnorm(x, rows, dim, xs, g, gs, eps)
    assert np.array_equal(y.cpu().numpy(), yo) and rd(ys) == so


@pytest.mark.parametrize("nh,nkv,hd,T,max_seq", [(4, 2, 8, 5, 16), (14, 2, 64, 1, 64), (14, 2, 64, 37, 64),
                                                 (14, 2, 64, 64, 64), (8, 8, 32, 200, 256)])
def test_ref_attention_prefill_against_the_oracle(torch_dev, nh, nkv, hd, T, max_seq):
    torch = torch_dev
    from tritify_amd import backend as B

    say(f"case: ref attention prefill nh={nh} nkv={nkv} hd={hd} T={T}")
    cfg = dict(dim=nh * hd, layers=1, nh=nh, nkv=nkv, hd=hd, hidden=8, vocab=2, eps=1e-6, theta=10000.0,
               max_seq=max_seq)
    m = O.RefModel(3, cfg)
    rng = np.random.default_rng(T + nh)
    q = rng.integers(-(2**28), 2**28, size=T * nh * hd).astype(np.int32)
    k = rng.integers(-(2**28), 2**28, size=T * nkv * hd).astype(np.int32)
    v = rng.integers(-(2**28), 2**28, size=T * nkv * hd).astype(np.int32)
    # score scales spread so the softmax is neither flat nor one-hot
    qs, ks, vs = (int(rng.integers(2**30, 2**31)), 81), rand_scale(rng), rand_scale(rng)
    o_want, os_want = m.attention_prefill(T, q, qs, k, ks, v, vs)
    cos_t, sin_t = B.ref_rope_tables(max_seq, hd, 10000.0)
    exp_codes, exp_lut = B.ref_codelut(B.LUT_EXP, -30.0, 0.0, 16, 20, False)
    n = B.ref_attention_prefill_workspace(T, nh, nkv, hd)
    ws = torch.empty(n, dtype=torch.uint8, device="cuda")
    o, os_ = torch.zeros(T * nh * hd, dtype=torch.int32, device="cuda"), rec(torch, (0, 0))
    B.ref_attention_prefill(dev_i32(torch, q), rec(torch, qs), dev_i32(torch, k), rec(torch, ks), dev_i32(torch, v),
                            rec(torch, vs), T, nh, nkv, hd, max_seq,
                            torch.from_numpy(cos_t.view(np.uint8)).cuda(),
                            torch.from_numpy(sin_t.view(np.uint8)).cuda(), B.ref_scale_from_f64(1.0 / np.sqrt(hd)),
                            torch.from_numpy(exp_codes).cuda(), exp_lut, ws, n, o, os_)
    got = o.cpu().numpy()
    assert np.array_equal(got, o_want), f"codes differ at {np.argwhere(got != o_want)[:5].tolist()}"
    assert rd(os_) == os_want


def test_ref_attention_prefill_thirds_closed_form(torch_dev):
    """The device prefill attention on the closed-form case of the oracle's pin (k = 0, v in {-1, 0, 1}, three
    rows: row r averages r + 1 positions, row 2 brought to the common scale by the Scale nearest 1/3): out =
    2^8 * (2^20 S_0, 2^19 S_1, rha(2^20 S_2, 3)), every unit of the per-row rounding visible."""
    torch = torch_dev
    from tritify_amd import backend as B

    nh, nkv, hd, T, max_seq = 4, 2, 8, 3, 16
    say(f"case: ref attention prefill thirds T={T}")
    rng = np.random.default_rng(33)
    q = rng.integers(-(2**28), 2**28, size=(T, nh, hd)).astype(np.int32)
    k = np.zeros((T, nkv, hd), np.int32)
    v = rng.integers(-1, 2, size=(T, nkv, hd)).astype(np.int32)
    v[0, 0, 0] = 1
    v[:, 1, :6] = [[1, 1, 1, -1, -1, -1], [1, 0, 1, -1, 0, -1], [0, 0, 1, 0, 0, -1]]
    qs, ks, vs = (1 << 30, 40), (1 << 30, 40), (1 << 31, 50)
    cos_t, sin_t = B.ref_rope_tables(max_seq, hd, 1.0e6)
    exp_codes, exp_lut = B.ref_codelut(B.LUT_EXP, -30.0, 0.0, 16, 20, False)
    n = B.ref_attention_prefill_workspace(T, nh, nkv, hd)
    ws = torch.empty(n, dtype=torch.uint8, device="cuda")
    o, os_ = torch.zeros(T * nh * hd, dtype=torch.int32, device="cuda"), rec(torch, (0, 0))
    B.ref_attention_prefill(dev_i32(torch, q.ravel()), rec(torch, qs), dev_i32(torch, k.ravel()), rec(torch, ks),
                            dev_i32(torch, v.ravel()), rec(torch, vs), T, nh, nkv, hd, max_seq,
                            torch.from_numpy(cos_t.view(np.uint8)).cuda(),
                            torch.from_numpy(sin_t.view(np.uint8)).cuda(), B.ref_scale_from_f64(1.0 / np.sqrt(hd)),
                            torch.from_numpy(exp_codes).cuda(), exp_lut, ws, n, o, os_)
    got = o.cpu().numpy().reshape(T, nh, hd)

    def rha(a, b):
        r = (2 * abs(a) + b) // (2 * b)
        return r if a >= 0 else -r

    for h in range(nh):
        for d in range(hd):
            s0 = int(v[0, h // 2, d])
            s1, s2 = s0 + int(v[1, h // 2, d]), s0 + int(v[1, h // 2, d]) + int(v[2, h // 2, d])
            assert [int(got[r, h, d]) for r in range(3)] == [2**28 * s0, 2**27 * s1, 2**8 * rha(2**20 * s2, 3)], (h, d)
    m = O.RefModel(3, dict(dim=nh * hd, layers=1, nh=nh, nkv=nkv, hd=hd, hidden=16, vocab=8, eps=1e-6, theta=1.0e6,
                           max_seq=max_seq))
    o_want, os_want = m.attention_prefill(T, q.ravel(), qs, k.ravel(), ks, v.ravel(), vs)
    assert np.array_equal(got.ravel(), o_want) and rd(os_) == os_want


@pytest.mark.parametrize("case", ["synthetic", "d00d", "qwen2"])
def test_ref_forward_against_the_oracle(torch_dev, case):
    """CausalLM::forward_int of whole sequences on the device against the oracle's restatement: the seed-7
    synthetic model over verify_repro's 12-token prompt, the reference test's 0xD00D model over [5, 6, 7, 8], a
    Qwen2.5-shaped 2-layer model over 20 tokens -- logits codes and scale bit for bit."""
    from tritify_amd.refdecoder import RefDecoder

    if case == "synthetic":
        cfg, seed, toks = O.SYNTH_CFG, 7, O.SYNTH_PROMPT
    elif case == "d00d":
        cfg = dict(dim=16, layers=2, nh=4, nkv=2, hd=4, hidden=32, vocab=20, eps=1e-6, theta=10000.0, max_seq=8)
        seed, toks = 0xD00D, [5, 6, 7, 8]
    else:
        cfg = dict(dim=896, layers=2, nh=14, nkv=2, hd=64, hidden=4864, vocab=512, eps=1e-6, theta=1.0e6,
                   max_seq=64)
        seed, toks = 5, [1, 100, 200, 300, 400, 511, 7, 9, 11, 13, 17, 19, 23, 29, 31, 37, 41, 43, 47, 53]
    say(f"case: ref forward {case} T={len(toks)}")
    m = O.RefModel(seed, cfg)
    want, ws_ = m.forward(toks)
    dec = RefDecoder(cfg, *m.weights())
    y, yr = dec.forward(toks)
    got = y.cpu().numpy().reshape(want.shape)
    assert np.array_equal(got, want), f"codes differ at {np.argwhere(got != want)[:5].tolist()}"
    assert rd(yr) == ws_


@pytest.mark.parametrize("rows,dim", [(1, 896), (64, 896), (300, 64), (2048, 40)])
def test_ref_seq_ops_equal_the_one_cta_ops_and_the_oracle(torch_dev, rows, dim):
    """The many-CTA RMSNorm, add (in place) and SwiGLU give the integers of the one-CTA kernels and the oracle."""
    torch = torch_dev
    from tritify_amd import backend as B

    say(f"case: ref seq ops rows={rows} dim={dim}")
    rng = np.random.default_rng(rows * 3 + dim)
    n = rows * dim
    x = rng.integers(-(2**28), 2**28, size=n).astype(np.int32)
    x[:dim] = 0
    g = rng.integers(-O.WLEVELS, O.WLEVELS + 1, size=dim).astype(np.int32)
    xs, gs, eps = rand_scale(rng), rand_scale(rng), B.ref_scale_from_f64(1e-6)
    nws = B.ref_seq_workspace(rows)
    ws = torch.empty(nws, dtype=torch.uint8, device="cuda")
    y, ys = torch.zeros(n, dtype=torch.int32, device="cuda"), rec(torch, (0, 0))
    B.ref_rmsnorm_seq(dev_i32(torch, x), rec(torch, xs), rows, dim, dev_i32(torch, g), gs, eps, ws, nws, y, ys)
    yo, so = O.rd_rmsnorm(x, rows, dim, xs, g, gs, eps)
    assert np.array_equal(y.cpu().numpy(), yo) and rd(ys) == so
    b = rng.integers(-(2**28), 2**28, size=n).astype(np.int32)
    sb = rand_scale(rng)
    ad, ar = dev_i32(torch, x), rec(torch, xs)
    B.ref_add_seq(ad, ar, dev_i32(torch, b), rec(torch, sb), n, ws, nws, ad, ar)
    wo, wso = O.rd_add(x, xs, b, sb)
    assert np.array_equal(ad.cpu().numpy(), wo) and rd(ar) == wso
    model = O.RefModel(7)
    codes, lut = B.ref_codelut(B.LUT_SILU, -30.0, 30.0, 16, 20, True)
    us = rand_scale(rng)
    gsw = (int(rng.integers(2**30, 2**31)), 55)
    h, hs = torch.zeros(n, dtype=torch.int32, device="cuda"), rec(torch, (0, 0))
    B.ref_swiglu_seq(dev_i32(torch, x), rec(torch, gsw), dev_i32(torch, b), rec(torch, us), n,
                     torch.from_numpy(codes).cuda(), lut, ws, nws, h, hs)
    ho, hso = O.rd_swiglu_act(model, x, gsw, b, us)
    assert np.array_equal(h.cpu().numpy(), ho) and rd(hs) == hso
