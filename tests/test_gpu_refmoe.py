"""The reference's MoeMlp at its own semantics on the GPU, through the C ABI, against the oracle's restatement
(oracle/kt_oracle_refdec.c, pinned by the reference's own MoE tests in tests/test_refmoe.py): the row-wise grouped
QuantLinear against per-row forward_int calls, route and combine per token, merge_rows, and whole layers -- the
reference tests' softmax MoE (one token and a sequence), the GLM-like sigmoid MoE with its bias and shared expert,
and a larger GLM-shaped layer -- codes and Scales bit for bit."""
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

WL = 265720


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def recs(torch, scales):
    w = np.zeros((len(scales), 4), dtype=np.int64)
    for i, (m, s) in enumerate(scales):
        w[i, 0] = m
        w[i].view(np.int32)[2] = s
    return torch.from_numpy(w.reshape(-1)).cuda()


def read_recs(t, n):
    w = t.cpu().numpy().reshape(n, 4)
    return [(int(r[0]), int(r.view(np.int32)[2])) for r in w]


def i32(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32).reshape(-1)).cuda()


def test_quant_linear_rows_grouped(torch_dev):
    """Each output row is forward_int of its own input row (own xmax, own ymax) against its group's weights; rows
    picked by index (one past the input reads as zeros), per-row input scales, an empty group, a zero row."""
    torch = torch_dev
    import tritify_amd as T
    from tritify_amd import backend as B

    say("case: quant_linear_rows G=4 rows=37 in=300 out=70")
    rng = np.random.default_rng(5)
    G, inp, out, x_rows = 4, 300, 70, 12
    counts = [10, 0, 20, 7]
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    P = int(off[-1])
    x = rng.integers(-(2**28), 2**28, size=(x_rows, inp)).astype(np.int32)
    x[3] = 0
    xidx = rng.integers(0, x_rows, size=P).astype(np.int32)
    xidx[5] = x_rows  # outside x: a zero row
    xs = [(int(rng.integers(2**30, 2**31)), int(rng.integers(50, 60))) for _ in range(P)]
    ws = [(int(rng.integers(2**30, 2**31)), int(rng.integers(40, 50))) for _ in range(G)]
    w = rng.integers(-WL, WL + 1, size=(G, out, inp)).astype(np.int32)
    pw = 3
    gbytes = B.pack_planes_tiled_bytes(out, inp, pw)
    planes = torch.empty(G * gbytes, dtype=torch.int8, device="cuda")
    for g in range(G):
        B.pack_planes_tiled(i32(torch, w[g]), out, inp, pw, planes[g * gbytes:])
    n = B.quant_linear_rows_workspace(P, inp, out, G)
    wsb = torch.empty(n, dtype=torch.uint8, device="cuda")
    y = torch.empty(P * out, dtype=torch.int32, device="cuda")
    ys = torch.zeros(P * 4, dtype=torch.int64, device="cuda")
    B.quant_linear_rows(i32(torch, x), i32(torch, xidx), x_rows, P, inp, recs(torch, xs), 1, off,
                        torch.from_numpy(off).cuda(), planes, gbytes, pw, out,
                        torch.from_numpy(np.array([a for a, _ in ws], np.int64)).cuda(),
                        torch.from_numpy(np.array([b for _, b in ws], np.int32)).cuda(), wsb, n, y, ys)
    got, got_s = y.cpu().numpy().reshape(P, out), read_recs(ys, P)
    for r in range(P):
        g = int(np.searchsorted(off, r, side="right") - 1)
        xr = x[xidx[r]] if xidx[r] < x_rows else np.zeros(inp, np.int32)
        yo, so, _, _ = O.quant_linear_forward(xr, 1, inp, xs[r], w[g].reshape(-1), out, ws[g])
        assert np.array_equal(got[r], yo.reshape(-1)), r
        assert got_s[r] == so, r


def rows_ql_case(torch, rng, counts, inp, out, pw, wmax, x_rows=9, off_dev_override=None, host_off=True):
    """quant_linear_rows over groups of the given row counts against per-row oracle forward_int calls; returns
    (got codes, got records, want codes, want records)."""
    import tritify_amd as T
    from tritify_amd import backend as B

    G = len(counts)
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    P = int(off[-1])
    x = rng.integers(-(2**28), 2**28, size=(x_rows, inp)).astype(np.int32)
    xidx = rng.integers(0, x_rows, size=P).astype(np.int32)
    xs = [(int(rng.integers(2**30, 2**31)), int(rng.integers(50, 60))) for _ in range(P)]
    ws = [(int(rng.integers(2**30, 2**31)), int(rng.integers(40, 50))) for _ in range(G)]
    w = rng.integers(-wmax, wmax + 1, size=(G, out, inp)).astype(np.int32)
    gbytes = B.pack_planes_tiled_bytes(out, inp, pw)
    planes = torch.empty(G * gbytes, dtype=torch.int8, device="cuda")
    for g in range(G):
        B.pack_planes_tiled(i32(torch, w[g]), out, inp, pw, planes[g * gbytes:])
    n = B.quant_linear_rows_workspace(P, inp, out, G)
    wsb = torch.empty(n, dtype=torch.uint8, device="cuda")
    y = torch.empty(P * out, dtype=torch.int32, device="cuda")
    ys = torch.empty(P * 4, dtype=torch.int64, device="cuda")
    off_dev = torch.from_numpy(off if off_dev_override is None else off_dev_override).cuda()
    B.quant_linear_rows(i32(torch, x), i32(torch, xidx), x_rows, P, inp, recs(torch, xs), 1,
                        off if host_off else None, off_dev, planes, gbytes, pw, out,
                        torch.from_numpy(np.array([a for a, _ in ws], np.int64)).cuda(),
                        torch.from_numpy(np.array([b for _, b in ws], np.int32)).cuda(), wsb, n, y, ys, groups=G)
    got, got_s = y.cpu().numpy().reshape(P, out), read_recs(ys, P)
    want, want_s = np.zeros((P, out), np.int32), []
    for r in range(P):
        g = int(np.searchsorted(off, r, side="right") - 1)
        yo, so, _, _ = O.quant_linear_forward(x[xidx[r]], 1, inp, xs[r], w[g].reshape(-1), out, ws[g])
        want[r] = yo.reshape(-1)
        want_s.append(so)
    return got, got_s, want, want_s


@pytest.mark.parametrize("pw,wmax", [(1, 127), (3, WL), (5, 2**30)])
def test_quant_linear_rows_every_group_size(torch_dev, pw, wmax):
    """Groups of every size the grouped products treat apart -- empty, 1 row (the one-row skinny list), 2-4 rows
    (the few-row list), 5-32 rows (one MFMA tile), several tiles with a ragged last one -- over 1, 3 and 5 weight
    planes, offsets on the device only: each row bit-exact against its own forward_int."""
    counts = [0, 1, 2, 3, 4, 5, 31, 0, 32, 33, 70, 1]
    say(f"case: quant_linear_rows every group size pw={pw}")
    got, got_s, want, want_s = rows_ql_case(torch_dev, np.random.default_rng(pw), counts, 200, 150, pw, wmax,
                                            host_off=False)
    assert np.array_equal(got, want), f"rows differ: {np.unique(np.argwhere(got != want)[:, 0]).tolist()[:10]}"
    assert got_s == want_s


def test_quant_linear_rows_long_k_and_wide_out(torch_dev):
    """K = 2100 (33 k-steps, kp padded) and 300 outputs (three 128-column tiles, the last ragged), groups of 1, 3, 9
    and 40 rows."""
    say("case: quant_linear_rows in=2100 out=300")
    got, got_s, want, want_s = rows_ql_case(torch_dev, np.random.default_rng(11), [1, 3, 9, 40], 2100, 300, 3, WL)
    assert np.array_equal(got, want) and got_s == want_s


def test_quant_linear_rows_clamps_device_offsets(torch_dev):
    """Offsets on the device that fall back or overshoot are taken as their running maximum clamped to [0, rows]
    (a valid split, no access outside the buffers): the rows then follow that split's groups."""
    torch = torch_dev
    say("case: quant_linear_rows clamped offsets")
    counts = [4, 6, 3, 7]  # the split the clamped offsets describe
    bad = np.array([0, 4, 2, 10, 99], np.int64)  # falls back at 2, overshoots rows (20) at the end
    # running max clamped: [0, 4, 4, 10, 20] -> groups of 4, 0, 6, 10 rows; the wanted rows use that split
    got, got_s, _, _ = rows_ql_case(torch, np.random.default_rng(3), counts, 96, 40, 3, WL, off_dev_override=bad,
                                    host_off=False)
    want, want_s, _, _ = rows_ql_case(torch, np.random.default_rng(3), counts, 96, 40, 3, WL,
                                      off_dev_override=np.array([0, 4, 4, 10, 20], np.int64), host_off=False)
    assert np.array_equal(got, want) and got_s == want_s


@pytest.mark.parametrize("rows,k,pw", [(128, 64, 3), (200, 150, 1), (300, 1000, 5)])
def test_tiled_planes_are_the_row_major_digits_rearranged(torch_dev, rows, k, pw):
    """kt_hip_pack_planes_tiled holds kt_hip_pack_planes' digits: byte t of chunk position s of row r in plane q of
    k-step kt of row block nb is digit q of code (128 nb + r, 64 kt + 16 (s ^ (r / 4) % 4) + t); rows and k past the
    matrix are zero."""
    torch = torch_dev
    import tritify_amd as T
    from tritify_amd import backend as B

    rng = np.random.default_rng(rows + k)
    lim = {1: 127, 3: WL, 5: 2**30}[pw]
    w = rng.integers(-lim, lim + 1, size=(rows, k)).astype(np.int32)
    kp = T.kp(k)
    flat = torch.empty(pw * rows * kp, dtype=torch.int8, device="cuda")
    T.pack_planes(i32(torch, w), rows, k, pw, flat)
    tiled = torch.empty(B.pack_planes_tiled_bytes(rows, k, pw), dtype=torch.int8, device="cuda")
    B.pack_planes_tiled(i32(torch, w), rows, k, pw, tiled)
    rm = flat.cpu().numpy().reshape(pw, rows, kp)
    nblk = (rows + 127) // 128
    pad = np.zeros((pw, nblk * 128, kp), np.int8)
    pad[:, :rows] = rm
    # [q][nb][r][kt][c][t] -> [nb][kt][q][r][slot][t] with slot = c ^ swz(r)
    v = pad.reshape(pw, nblk, 128, kp // 64, 4, 16)
    swz = (np.arange(128) >> 2) & 3
    slots = np.arange(4)[None, :] ^ swz[:, None]  # (r, slot) -> the chunk stored there
    gathered = np.take_along_axis(v, slots[None, None, :, None, :, None], axis=4)
    want = gathered.transpose(1, 3, 0, 2, 4, 5).reshape(-1)
    assert np.array_equal(tiled.cpu().numpy(), want)


def test_bucket_groups_the_pairs_by_expert(torch_dev):
    """kt_hip_ref_moe_bucket: the offsets are the experts' pair counts summed; every pair's row lies in its expert's
    group and points back at its token; the rows are a permutation; an id outside [0, E) gets no row."""
    torch = torch_dev
    from tritify_amd import backend as B

    rng = np.random.default_rng(21)
    for T_, K, E in ((1, 8, 128), (37, 4, 16), (300, 8, 128), (5, 2, 3000)):
        say(f"case: bucket T={T_} k={K} E={E}")
        sel = np.stack([rng.choice(E, K, replace=False) for _ in range(T_)]).astype(np.int32).reshape(-1)
        P = T_ * K
        off = torch.empty(E + 1, dtype=torch.int64, device="cuda")
        xidx = torch.empty(P, dtype=torch.int32, device="cuda")
        pos = torch.empty(P, dtype=torch.int32, device="cuda")
        B.ref_moe_bucket(i32(torch, sel), T_, K, E, off, xidx, pos)
        o, xi, po = off.cpu().numpy(), xidx.cpu().numpy(), pos.cpu().numpy()
        assert np.array_equal(o, np.concatenate([[0], np.cumsum(np.bincount(sel, minlength=E))]))
        assert np.array_equal(np.sort(po), np.arange(P))
        for p in range(P):
            assert o[sel[p]] <= po[p] < o[sel[p] + 1] and xi[po[p]] == p // K
    sel = np.array([0, 5, 1, -1, 2, 9], np.int32)  # E = 3: ids 5, -1, 9 get no row
    off = torch.empty(4, dtype=torch.int64, device="cuda")
    xidx = torch.empty(6, dtype=torch.int32, device="cuda")
    pos = torch.empty(6, dtype=torch.int32, device="cuda")
    B.ref_moe_bucket(i32(torch, sel), 3, 2, 3, off, xidx, pos)
    o, xi, po = off.cpu().numpy(), xidx.cpu().numpy(), pos.cpu().numpy()
    assert o.tolist() == [0, 1, 2, 3] and po[1] == po[3] == po[5] == -1 and (xi[3:] == -1).all()
    assert [xi[po[p]] for p in (0, 2, 4)] == [0, 1, 2]


def layer_from(m: O.RefMoe, dev_sigmoid: bool):
    from tritify_amd.refmoe import RefMoeLayer

    experts = [{n: m.ql(e, n) for n in ("gate", "up", "down")} for e in range(m.E)]
    shared = {n: m.ql(m.E, n) for n in ("gate", "up", "down")} if m.shared_hidden else None
    return RefMoeLayer(m.dim, m.ql(0, "router"), experts, m.top_k, m.norm_topk,
                       m.bias() if dev_sigmoid else None, shared)


@pytest.mark.parametrize("case", [
    dict(seed=0x30E1, dim=64, E=8, k=2, hidden=96, norm=False, sig=0, bseed=0, shared=0, T=1),
    dict(seed=0x30E1, dim=64, E=8, k=2, hidden=96, norm=False, sig=0, bseed=0, shared=0, T=5),
    dict(seed=0x5C, dim=32, E=16, k=4, hidden=24, norm=True, sig=1, bseed=0x5C, shared=40, T=6),
    dict(seed=0x91, dim=256, E=32, k=4, hidden=128, norm=True, sig=1, bseed=0x92, shared=192, T=40),
    dict(seed=0x93, dim=128, E=16, k=2, hidden=64, norm=False, sig=1, bseed=0x94, shared=0, T=9),
    dict(seed=0x97, dim=128, E=16, k=4, hidden=64, norm=True, sig=1, bseed=0x98, shared=256, T=7),  # grouped gate/up
])
def test_moe_layer_against_the_oracle(torch_dev, case):
    torch = torch_dev
    c = case
    say(f"case: ref moe {c}")
    m = O.RefMoe(c["seed"], c["dim"], c["E"], c["k"], c["hidden"], c["norm"], c["sig"], c["bseed"], c["shared"])
    layer = layer_from(m, c["sig"] == 1)
    x, xs, _ = O.rm_probe(c["seed"] + 1, c["T"] * c["dim"])
    xd, xr = i32(torch, x), recs(torch, [xs])
    # route, token by token
    sel, ec, sumc, logits, ls = layer.route(xd, xr, c["T"])
    sel, ec, sumc = sel.cpu().numpy().reshape(c["T"], c["k"]), ec.cpu().numpy().reshape(c["T"], c["k"]), \
        sumc.cpu().numpy()
    lg, lsr = logits.cpu().numpy().reshape(c["T"], c["E"]), read_recs(ls, c["T"])
    for t in range(c["T"]):
        so, eo, sumo, lo, lso = m.route(x[t * c["dim"]:(t + 1) * c["dim"]], xs)
        assert np.array_equal(lg[t], lo) and lsr[t] == lso, f"logits of token {t}"
        assert sel[t].tolist() == so and np.array_equal(ec[t], eo) and sumc[t] == sumo, f"route of token {t}"
    out, orec = layer.forward(xd, xr, c["T"])
    want, ws = m.forward(x, c["T"], xs)
    got = out.cpu().numpy()
    assert np.array_equal(got, want), f"codes differ at {np.argwhere(got != want)[:5].tolist()}"
    assert read_recs(orec, 1)[0] == ws


def test_moe_layer_graph_replays_equal_eager(torch_dev):
    """The whole layer captured as one HIP graph (no host round trip in forward): three replays, each after eager
    work of the program's own on the same buffers and a synchronization, over two inputs, every replay bit-exact
    against the eager forward and the oracle."""
    torch = torch_dev
    say("case: ref moe graph replays")
    m = O.RefMoe(0x91, 256, 32, 4, 128, True, 1, 0x92, 192)
    layer = layer_from(m, True)
    T_ = 40
    x0, xs0, _ = O.rm_probe(0x95, T_ * 256)
    x1, xs1, _ = O.rm_probe(0x96, T_ * 256)
    xd, xr = i32(torch, x0), recs(torch, [xs0])
    layer.forward(xd, xr, T_)
    g, gout, grec = layer.capture(xd, xr, T_)
    for rep, (x, xs) in enumerate(((x1, xs1), (x0, xs0), (x1, xs1))):
        xd.copy_(i32(torch, x))
        xr.copy_(recs(torch, [xs]))
        eager, erec = layer.forward(xd, xr, T_)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want, ws = m.forward(x, T_, xs)
        assert np.array_equal(gout.cpu().numpy(), eager.cpu().numpy()), f"replay {rep} differs from eager"
        assert np.array_equal(gout.cpu().numpy(), want) and read_recs(grec, 1)[0] == ws, f"replay {rep}"


def test_combine_and_merge_against_the_oracle(torch_dev):
    torch = torch_dev
    from tritify_amd import backend as B

    say("case: ref moe combine / merge_rows")
    rng = np.random.default_rng(21)
    T, K, dim = 7, 3, 50
    P = T * K
    y = rng.integers(-(2**28), 2**28 + 1, size=(P, dim)).astype(np.int32)
    ys = [(int(rng.integers(2**30, 2**31)), int(rng.integers(55, 62))) for _ in range(P)]
    ys[4] = (0, 0)
    ys[7] = (ys[8][0] * 2 if ys[8][0] < 2**31 else ys[8][0], ys[8][1] + (1 if ys[8][0] < 2**31 else 0))  # equal values
    pos = rng.permutation(P).astype(np.int32)
    ec = rng.integers(0, 1 << 20, size=P).astype(np.int64)
    sumc = np.array([int(ec[t * K:(t + 1) * K].sum()) for t in range(T)], np.int64)
    sumc[2] = 0  # the zero path
    out = torch.empty(T * dim, dtype=torch.int32, device="cuda")
    os_ = torch.zeros(T * 4, dtype=torch.int64, device="cuda")
    B.ref_moe_combine(i32(torch, y), recs(torch, ys), P, dim, i32(torch, pos), torch.from_numpy(ec).cuda(),
                      torch.from_numpy(sumc).cuda(), T, K, out, os_)
    got, got_s = out.cpu().numpy().reshape(T, dim), read_recs(os_, T)
    for t in range(T):
        rows = [pos[t * K + i] for i in range(K)]
        wo, wso = O.rm_combine(y[rows].reshape(-1), [ys[r] for r in rows], dim, ec[t * K:(t + 1) * K], int(sumc[t]))
        assert np.array_equal(got[t], wo) and got_s[t] == wso, t
    rs = [ys[i] for i in range(T)]
    n = B.ref_merge_rows_workspace(T)
    wsb = torch.empty(n, dtype=torch.uint8, device="cuda")
    mo = torch.empty(T * dim, dtype=torch.int32, device="cuda")
    mrec = torch.zeros(4, dtype=torch.int64, device="cuda")
    B.ref_merge_rows(i32(torch, y[:T]), recs(torch, rs), T, dim, wsb, n, mo, mrec)
    wo, wso = O.rm_merge_rows(y[:T].reshape(-1), rs, T, dim)
    assert np.array_equal(mo.cpu().numpy(), wo) and read_recs(mrec, 1)[0] == wso
