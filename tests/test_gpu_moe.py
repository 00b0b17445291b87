"""Parity of the config-4 MoE layer (route, bucket, ragged grouped W12 GEMM, SwiGLU, combine) on the MI355X with the
CPU oracle, through the C ABI. Run on a GPU box with -m gpu.

The oracle evaluates the layer two ways: expert-major (kt_moe_layer: the order the GPU uses) and token by token
(kt_moe_forward_token: the reference's MoeMlp loop, crates/01-engine/kt-core/src/layers.rs:928-936, 988-1020).
Small shapes are checked against both, every intermediate byte for byte; the full GLM-4.5-Air shape against the
committed fixture hashes (tests/golden/goldens.json, written by tests/golden/make_goldens.py). Edge cases follow the
reference's routing rules: experts nobody chooses, experts everybody chooses, ties (lower index wins, layers.rs:800-805),
a single token, groups longer than one row tile.
"""
import hashlib
import json
import os
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "goldens.json")))


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def make_case(torch, T, H, F, E, K, w_seed, x_seed, r_seed, logits=None, h_shift=8, out_shift=13):
    """Generate a layer and its inputs; return (layer, device inputs, host arrays for the oracle)."""
    import tritify_amd as TA
    from tritify_amd import workloads as W
    from tritify_amd.moe import MoeLayer

    x, r = W.moe_inputs(T, H, E, x_seed, r_seed)
    if logits is not None:
        r = np.ascontiguousarray(logits, dtype=np.int32)
    silu, sig = W.silu_table(), W.sigmoid_table()
    layer = MoeLayer(H, F, E, K, silu, sig, h_shift, out_shift)
    G = E + 1
    host = dict(wgu=np.empty((G, 2 * F * H), np.int16), wd=np.empty((G, H * F), np.int16),
                gm=np.empty((G, 2 * F), np.int32), gs=np.empty((G, 2 * F), np.int32),
                dm=np.empty((G, H), np.int32), ds=np.empty((G, H), np.int32))
    for g in range(G):
        gu, dn, gm, gs, dm, ds = W.moe_expert(g, H, F, w_seed)
        layer.set_expert(g, gu, dn, gm, gs, dm, ds)
        host["wgu"][g], host["wd"][g], host["gm"][g], host["gs"][g], host["dm"][g], host["ds"][g] = gu, dn, gm, gs, dm, ds
    xd = torch.from_numpy(x.astype(np.int8)).cuda()
    rd = torch.from_numpy(r).cuda()
    host.update(x=x, r=r, silu=silu, sig=sig, h_shift=h_shift, out_shift=out_shift)
    return layer, xd, rd, host


def oracle_layer(host, T, H, F, E, K):
    return O.moe_layer(host["x"], host["r"], T, H, F, E, K, host["wgu"], host["wd"], host["gm"], host["gs"],
                       host["dm"], host["ds"], host["silu"], host["sig"], host["h_shift"], host["out_shift"])


def run_and_compare(torch, T, H, F, E, K, logits=None, token_order=True, seeds=(700, 71, 72)):
    say(f"case: moe T={T} H={H} F={F} E={E} top_k={K} seeds={seeds} custom_logits={logits is not None}")
    layer, xd, rd, host = make_case(torch, T, H, F, E, K, *seeds, logits=logits)
    out = torch.empty(T * H, dtype=torch.int8, device="cuda")
    v = layer.forward(xd, rd, T, out)
    torch.cuda.synchronize()
    ref = oracle_layer(host, T, H, F, E, K)
    P = T * (K + 1)
    got = {k: v[k].cpu().numpy() for k in ("sel", "cw", "pos", "count")}
    for k in ("sel", "cw", "pos", "count"):
        assert np.array_equal(got[k], ref[k]), f"{k} differs"
    lst = v["list"].cpu().numpy().reshape(E + 1, T)
    for g in range(E + 1):
        c = int(ref["count"][g])
        assert np.array_equal(lst[g, :c], ref["list"].reshape(E + 1, T)[g, :c]), f"list of group {g} differs"
    off = v["off"].cpu().numpy()[: E + 2]
    assert np.array_equal(off, np.concatenate([[0], np.cumsum(ref["count"])]).astype(np.int32))
    assert np.array_equal(v["h"].cpu().numpy()[: P * F], ref["h"]), "h (gate/up + SwiGLU) differs"
    assert np.array_equal(v["d"].cpu().numpy()[: P * H], ref["d"]), "d (down) differs"
    o = out.cpu().numpy()
    assert np.array_equal(o, ref["out"]), "combined output differs"
    if token_order:
        tok = O.moe_forward_token(host["x"], host["r"], T, H, F, E, K, host["wgu"], host["wd"], host["gm"],
                                  host["gs"], host["dm"], host["ds"], host["silu"], host["sig"], host["h_shift"],
                                  host["out_shift"])
        assert np.array_equal(o, tok), "differs from the reference's per-token loop order"
    return ref


def test_moe_small_layer(torch_dev):
    ref = run_and_compare(torch_dev, 300, 256, 128, 16, 4)
    assert (ref["count"][:16] > 0).all()


def test_moe_unchosen_and_always_chosen_experts(torch_dev):
    """Expert 3 is never chosen (an empty group), expert 5 always (a group of every token, > 2 row tiles)."""
    from tritify_amd import workloads as W

    T, H, F, E, K = 257, 192, 64, 8, 2
    _, r = W.moe_inputs(T, H, E, 81, 82)
    r = r.reshape(T, E).copy()
    r[:, 3] = -(10**6)
    r[:, 5] = 10**6
    ref = run_and_compare(torch_dev, T, H, F, E, K, logits=r.reshape(-1), seeds=(800, 81, 82))
    assert ref["count"][3] == 0 and ref["count"][5] == T


def test_moe_ties_take_the_lower_index(torch_dev):
    """Tokens whose router codes tie: the lower expert index wins (MoeMlp::topk, layers.rs:800-805)."""
    from tritify_amd import workloads as W

    T, H, F, E, K = 40, 128, 64, 16, 4
    _, r = W.moe_inputs(T, H, E, 91, 92)
    r = r.reshape(T, E).copy()
    r[:10, :] = 7  # all equal: experts 0..3
    r[10:20, 8:12] = 10**5  # a 4-way tie at the top
    ref = run_and_compare(torch_dev, T, H, F, E, K, logits=r.reshape(-1), seeds=(900, 91, 92))
    assert np.array_equal(ref["sel"].reshape(T, K)[:10], np.tile(np.arange(4), (10, 1)))
    assert np.array_equal(ref["sel"].reshape(T, K)[10:20], np.tile(np.arange(8, 12), (10, 1)))


def test_moe_every_expert_every_token(torch_dev):
    """top_k = E: every group holds every token (groups of 300 rows: three row tiles, the last partial)."""
    run_and_compare(torch_dev, 300, 128, 64, 4, 4, seeds=(1000, 101, 102))


def test_moe_one_token(torch_dev):
    run_and_compare(torch_dev, 1, 256, 128, 8, 2, seeds=(1100, 111, 112))


@pytest.mark.parametrize("T,E,K", [(1, 4, 2), (4096, 64, 8), (5000, 64, 8), (300, 40, 12), (9000, 16, 16)])
def test_moe_bucket_against_the_oracle(torch_dev, T, E, K):
    """kt_hip_moe_bucket's lists (each group's tokens in increasing order), positions and counts equal the oracle's;
    T past one 4096-token pass and ragged, top_k past the unrolled 8."""
    from tritify_amd import backend as B

    torch = torch_dev
    rng = np.random.default_rng(T * 131 + E * 7 + K)
    sel = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32).ravel()
    lst, pos, count = O.moe_bucket(sel, T, E, K)
    say(f"case: moe bucket T={T} E={E} top_k={K}")
    d_lst = torch.full(((E + 1) * T,), -7, dtype=torch.int32, device="cuda")
    d_pos = torch.full((T * K,), -7, dtype=torch.int32, device="cuda")
    d_cnt = torch.full((E + 1,), -7, dtype=torch.int32, device="cuda")
    B.moe_bucket(torch.from_numpy(sel).cuda(), T, E, K, d_lst, d_pos, d_cnt)
    torch.cuda.synchronize()
    got_cnt, got_lst = d_cnt.cpu().numpy(), d_lst.cpu().numpy()
    assert np.array_equal(got_cnt, count)
    for g in range(E + 1):
        assert np.array_equal(got_lst[g * T:g * T + count[g]], lst[g * T:g * T + count[g]]), g
    assert np.array_equal(d_pos.cpu().numpy(), pos)


def test_grouped_linear_ragged_gather(torch_dev):
    """The grouped W12 GEMM alone, int8 epilogue: ragged counts (0, 1, one row tile + 2, two + 1, 64), rows gathered
    through a list with repeats, n not a multiple of the tile, k not a multiple of 64."""
    import tritify_amd as TA
    from tritify_amd import workloads as W

    torch = torch_dev
    counts = np.array([0, 1, 130, 257, 64], dtype=np.int32)
    G, n, k, xrows = len(counts), 200, 300, 97
    kp = (k + 63) // 64 * 64
    say(f"case: grouped linear counts={counts.tolist()} n={n} k={k}")
    rng = np.random.default_rng(5)
    x = rng.integers(-127, 128, size=(xrows, k), dtype=np.int8)
    xp = np.zeros((xrows, kp), np.int8)
    xp[:, :k] = x
    lst = np.full((G, 300), -1, np.int32)
    for g in range(G):
        lst[g, : counts[g]] = rng.integers(0, xrows, size=counts[g])
    lo_b, _ = TA.w12_bytes(n, k)
    lo = torch.zeros(G * lo_b, dtype=torch.int8, device="cuda")
    nib = torch.zeros(G * lo_b // 2, dtype=torch.uint8, device="cuda")
    ws, ms, ss = [], [], []
    for g in range(G):
        w = W.gen_w12(1200 + g, n * k)
        m_, s_ = W.channel_scales(w, n, k, 40)
        TA.w12_upload(w, n, k, lo[g * lo_b:(g + 1) * lo_b], nib[g * lo_b // 2:(g + 1) * lo_b // 2])
        ws.append(w), ms.append(m_), ss.append(s_)
    P = int(counts.sum())
    y = torch.full((P * n,), 99, dtype=torch.int8, device="cuda")
    off = torch.zeros(G + 1, dtype=torch.int32, device="cuda")
    TA.w12_grouped_linear(torch.from_numpy(xp).cuda(), xrows, torch.from_numpy(lst).cuda(), 300,
                          torch.from_numpy(counts).cuda(), G, P, lo, nib, n, k,
                          torch.from_numpy(np.concatenate(ms)).cuda(), torch.from_numpy(np.concatenate(ss)).cuda(),
                          TA.EPI_I8, y, n, off_dev=off)
    torch.cuda.synchronize()
    yh = y.cpu().numpy().reshape(P, n)
    assert np.array_equal(off.cpu().numpy(), np.concatenate([[0], np.cumsum(counts)]))
    at = 0
    for g in range(G):
        c = int(counts[g])
        if c == 0:
            continue
        rows = x[lst[g, :c]]
        _, y8 = O.gemm_i8w16(rows, ws[g].astype(np.int16), c, n, k, ms[g], ss[g])
        assert np.array_equal(yh[at:at + c], y8.reshape(c, n)), f"group {g} differs"
        at += c


@pytest.mark.parametrize("k,gathered", [(40, True), (100, True), (320, False)])
def test_grouped_dma_tiles(torch_dev, k, gathered):
    """Enough rows for the DMA-fed grouped kernel (256-row tiles, one CTA per CU), int8 epilogue: groups of 0, 1, 64,
    65, 128, 129, 256, 257, 288, 289, 300, 520, 544 and 700 rows (every tail class: the 64- and 128-row register
    tiles, the DMA tile, and the 288-row DMA tile that absorbs a tail of 1-32 rows: 257, 288, 520, 544; 289 keeps a
    33-row tail tile), n = 4000 (a partial last column tile), k of one, two and five 64-deep k-tiles; rows gathered
    through a list with repeats, or read in place from offset ranges."""
    import tritify_amd as TA
    from tritify_amd import workloads as W

    torch = torch_dev
    counts = np.array([0, 1, 64, 65, 128, 129, 256, 257, 288, 289, 300, 520, 544, 700], dtype=np.int32)
    G, n = len(counts), 4000
    P = int(counts.sum())
    kp = (k + 63) // 64 * 64
    xrows = 900 if gathered else P
    say(f"case: grouped dma tiles counts={counts.tolist()} n={n} k={k} gathered={gathered}")
    rng = np.random.default_rng(k)
    x = rng.integers(-127, 128, size=(xrows, k), dtype=np.int8)
    xp = np.zeros((xrows, kp), np.int8)
    xp[:, :k] = x
    off_h = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    lst = np.full((G, 1024), -1, np.int32)
    for g in range(G):
        lst[g, : counts[g]] = rng.integers(0, xrows, size=counts[g]) if gathered else np.arange(off_h[g], off_h[g + 1])
    lo_b, _ = TA.w12_bytes(n, k)
    lo = torch.zeros(G * lo_b, dtype=torch.int8, device="cuda")
    nib = torch.zeros(G * lo_b // 2, dtype=torch.uint8, device="cuda")
    ws, ms, ss = [], [], []
    for g in range(G):
        w = W.gen_w12(1300 + g, n * k)
        m_, s_ = W.channel_scales(w, n, k, 40)
        TA.w12_upload(w, n, k, lo[g * lo_b:(g + 1) * lo_b], nib[g * lo_b // 2:(g + 1) * lo_b // 2])
        ws.append(w), ms.append(m_), ss.append(s_)
    y = torch.full((P * n,), 99, dtype=torch.int8, device="cuda")
    off = torch.zeros(G + 1, dtype=torch.int32, device="cuda")
    TA.w12_grouped_linear(torch.from_numpy(xp).cuda(), xrows, torch.from_numpy(lst).cuda() if gathered else None,
                          1024, torch.from_numpy(counts).cuda(), G, P, lo, nib, n, k,
                          torch.from_numpy(np.concatenate(ms)).cuda(), torch.from_numpy(np.concatenate(ss)).cuda(),
                          TA.EPI_I8, y, n, off_dev=off)
    torch.cuda.synchronize()
    yh = y.cpu().numpy().reshape(P, n)
    assert np.array_equal(off.cpu().numpy(), off_h)
    for g in range(G):
        c = int(counts[g])
        if c == 0:
            continue
        rows = x[lst[g, :c]]
        _, y8 = O.gemm_i8w16(rows, ws[g].astype(np.int16), c, n, k, ms[g], ss[g])
        got = yh[off_h[g]:off_h[g + 1]]
        assert np.array_equal(got, y8.reshape(c, n)), f"group {g} ({c} rows) differs"


def test_moe_layer_on_dma_tiles(torch_dev):
    """A layer whose gate/up product takes the DMA-fed grouped kernel (T = 1024 tokens x 4 rows, 2F = 2048) with the
    SwiGLU epilogue, routed so the experts get 1024, 1024, 257, 256, 129, 128, 124, 65, 64, 1 and 0 rows (every
    tail class); every intermediate against the oracle."""
    T, H, F, E, K = 1024, 128, 1024, 16, 3
    want = [1024, 1024, 257, 256, 129, 128, 65, 64, 1, 0, 124, 0, 0, 0, 0, 0]
    assert sum(want) == T * K
    seq = np.repeat(np.arange(E), want)  # expert ids by position; token t takes positions t, t + T, t + 2T
    logits = np.full((T, E), 0, np.int64) - 1000 - np.arange(E)[None, :]
    for t in range(T):
        for r, e in enumerate(seq[[t, t + T, t + 2 * T]]):
            logits[t, e] = 3000 - 1000 * r
    ref = run_and_compare(torch_dev, T, H, F, E, K, logits=logits.astype(np.int32).ravel(), token_order=False)
    assert ref["count"][:E].tolist() == want


def test_moe_full_config4(torch_dev):
    """benchmark config 4 at full size (4096 tokens, H 4096, 128 experts + shared, F 1408, top-8) against the
    fixture hashes of the oracle's expert-major evaluation."""
    from tritify_amd import workloads as W

    torch = torch_dev
    g4 = GOLD["config4"]
    T, H, F, E, K = g4["T"], g4["H"], g4["F"], g4["E"], g4["top_k"]
    say(f"case: moe full config 4 T={T} H={H} F={F} E={E} top_k={K}")
    layer, xd, rd, host = make_case_full(torch, g4)
    assert sha(host["x"]) == g4["x_sha256"] and sha(host["r"]) == g4["logits_sha256"]
    assert sha(host["silu"]) == g4["silu_sha256"] and sha(host["sig"]) == g4["sig_sha256"]
    out = torch.empty(T * H, dtype=torch.int8, device="cuda")
    v = layer.forward(xd, rd, T, out)
    torch.cuda.synchronize()
    P = T * (K + 1)
    assert v["count"].cpu().numpy().tolist() == g4["count"]
    assert sha(v["sel"].cpu().numpy()) == g4["sel_sha256"]
    assert sha(v["cw"].cpu().numpy()) == g4["cw_sha256"]
    assert sha(v["h"].cpu().numpy()[: P * F]) == g4["h_sha256"], "h differs from the CPU fixture"
    assert sha(v["d"].cpu().numpy()[: P * H]) == g4["d_sha256"], "d differs from the CPU fixture"
    assert sha(out.cpu().numpy()) == g4["out_sha256"], "the layer output differs from the CPU fixture"


def make_case_full(torch, g4):
    """The full config-4 layer from the fixture's seeds (weights from the product's generators)."""
    from tritify_amd import workloads as W
    from tritify_amd.moe import MoeLayer

    T, H, F, E, K = g4["T"], g4["H"], g4["F"], g4["E"], g4["top_k"]
    x, r = W.moe_inputs(T, H, E, g4["x_seed"], g4["r_seed"], g4["sigma_x"], g4["sigma_r"])
    silu, sig = W.silu_table(), W.sigmoid_table()
    layer = MoeLayer(H, F, E, K, silu, sig, g4["h_shift"], g4["out_shift"])
    for g in range(E + 1):
        layer.set_expert(g, *W.moe_expert(g, H, F, g4["w_seed"], g4["sigma_x"], g4["sigma_h"]))
    xd = torch.from_numpy(x.astype(np.int8)).cuda()
    rd = torch.from_numpy(r).cuda()
    return layer, xd, rd, dict(x=x, r=r, silu=silu, sig=sig)
