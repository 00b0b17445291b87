"""The balanced two-plane 12-bit weights (W12B: hi = (v + 128) >> 8 in [-8, 8], lo = v - 256 hi in [-128, 127]) and
their DMA-fed 256 x 128 GEMM, through the C ABI, against the CPU oracle: the planes against the fragment layout built
here in numpy from the split rule, the product for every output kind over ragged shapes, k past the int32
recombination, every product at its largest magnitude, and config 2 at M = 2048 against the committed fixture hashes.
The integers are those of the W12 path (w12_linear): only the weights' digit split differs.
"""
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


def tb():
    import tritify_amd

    return tritify_amd


def split(v):
    """The balanced split of codes in [-2048, 2047]: (lo, hi) with v = lo + 256 hi."""
    v = np.asarray(v, np.int64)
    hi = (v + 128) >> 8
    return v - 256 * hi, hi


def layout(plane, n, k):
    """A plane of n x k digits in the fragment-tiled order of the W12 lo plane: per 32-row column block and k32 block,
    64 lanes x 16 bytes, lane l = row % 32 + 32 * ((k % 32) // 16), byte k % 16; rows padded to 32, k to 64."""
    npad, kp = (n + 31) // 32 * 32, (k + 63) // 64 * 64
    full = np.zeros((npad, kp), np.int8)
    full[:n, :k] = plane.reshape(n, k)
    KB = kp // 32
    # [nb][r32][kb][h][t] -> [nb][kb][h][r32][t]
    return full.reshape(npad // 32, 32, KB, 2, 16).transpose(0, 2, 3, 1, 4).reshape(-1)


def _w12b_device(torch, w, n, k):
    T = tb()
    nb = T.w12b_bytes(n, k)
    lo = torch.empty(nb, dtype=torch.int8, device="cuda")
    hi = torch.empty(nb, dtype=torch.int8, device="cuda")
    T.w12b_pack(torch.from_numpy(np.ascontiguousarray(w, np.int32)).cuda(), n, k, lo, hi)
    return lo, hi


def _x_device(torch, x, m, k):
    kp = tb().kp(k)
    xp = np.zeros((m, kp), np.int8)
    xp[:, :k] = x.reshape(m, k)
    return torch.from_numpy(xp).cuda()


def test_w12b_planes_match_the_split_and_the_fragment_layout(torch_dev):
    torch = torch_dev
    rng = np.random.default_rng(7)
    for n, k in [(1, 1), (3, 33), (64, 64), (101, 200), (37, 4100)]:
        w = rng.integers(-2048, 2048, size=n * k).astype(np.int32)
        w[: min(n * k, 4096)] = np.arange(-2048, 2048, dtype=np.int32)[: min(n * k, 4096)]  # every code once
        say(f"case: w12b pack n={n} k={k}")
        lo, hi = _w12b_device(torch, w, n, k)
        wl, wh = split(w)
        assert np.array_equal(lo.cpu().numpy(), layout(wl, n, k)), (n, k)
        assert np.array_equal(hi.cpu().numpy(), layout(wh, n, k)), (n, k)


def _check(torch, m, n, k, rng, kinds=None):
    T = tb()
    x = rng.integers(-128, 128, size=m * k).astype(np.int32)
    w = rng.integers(-2048, 2048, size=n * k).astype(np.int32)
    mant, shift = O.channel_scales(w, n, k, 40)
    lo, hi = _w12b_device(torch, w, n, k)
    xd = _x_device(torch, x, m, k)
    md, sd = torch.from_numpy(mant).cuda(), torch.from_numpy(shift).cuda()
    acc = O.linear_threads(x, w, m, n, k, 16, O.lib().kt_cpu_auto_variant())
    q32 = O.requant_channels(acc, m, n, mant, shift, -(2**31), 2**31 - 1)
    res = rng.integers(-(2**31), 2**31, size=m * n, dtype=np.int64).astype(np.int32)
    res[:2] = [2**31 - 1, -(2**31)][:res.size]
    wants = {T.OUT_I64: acc, T.OUT_I32: q32,
             T.OUT_I8: O.requant_channels(acc, m, n, mant, shift, -127, 127).astype(np.int8),
             T.OUT_I32_ADD: np.clip(res.astype(np.int64) + q32, -(2**31), 2**31 - 1).astype(np.int32)}
    for kind, want in wants.items():
        if kinds is not None and kind not in kinds:
            continue
        say(f"case: w12b linear {m}x{n}x{k} out_kind={kind}")
        y = torch.from_numpy(res.copy()).cuda() if kind == T.OUT_I32_ADD else \
            torch.empty(m * n, dtype={T.OUT_I64: torch.int64, T.OUT_I32: torch.int32, T.OUT_I8: torch.int8}[kind],
                        device="cuda")
        T.w12b_linear(xd, lo, hi, m, n, k, y, kind, md, sd)
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        assert np.array_equal(got, want), (m, n, k, kind, np.argwhere(got != want)[:5].tolist())


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (5, 33, 100), (300, 257, 448), (2048, 4096, 64), (2100, 3900, 100),
                                   (2305, 4000, 704), (257, 130, 8200)])
def test_w12b_linear_against_the_oracle(torch_dev, m, n, k):
    """Ragged rows (a one-row last tile) and columns (a partial column block), k of one and two k-tiles and longer,
    k = 8200 past the int32 recombination (the i64 epilogue); every output kind, the saturating residual add
    included."""
    _check(torch_dev, m, n, k, np.random.default_rng(m * 7 + n + k))


def test_w12b_extremes(torch_dev):
    """Every product at its largest magnitude (v = -2048: hi -8, lo 0; v = 2047: hi 8, lo -1) at k = 4096 and at
    k = 8200: each output is k * x * w exactly."""
    torch = torch_dev
    T = tb()
    m, n = 300, 160
    for k in (4096, 8200):
        for xv, wv in [(-128, -2048), (127, 2047), (-128, 2047), (127, -2048)]:
            lo, hi = _w12b_device(torch, np.full(n * k, wv, np.int32), n, k)
            xd = torch.full((m, T.kp(k)), xv, dtype=torch.int8, device="cuda")
            xd[:, k:] = 0
            y = torch.empty(m * n, dtype=torch.int64, device="cuda")
            say(f"case: w12b extremes k={k} x={xv} w={wv}")
            T.w12b_linear(xd, lo, hi, m, n, k, y)
            torch.cuda.synchronize()
            assert bool((y == k * xv * wv).all().item()), (k, xv, wv)


def test_w12b_config2_m2048_against_the_fixture(torch_dev):
    """benchmark config 2 at M = 2048 (N = K = 4096) on the balanced planes: the i64 accumulators and the int8
    outputs hash to the fixtures the CPU oracle produced, as the W12 path's do."""
    torch = torch_dev
    T = tb()
    g = GOLD["config2"]
    N, K, m = g["N"], g["K"], 2048
    w = O.gen_w12(g["w_seed"], N * K)
    x = O.gen_act_gauss(g["x_seed"], g["sigma"], m * K)
    mant, shift = O.channel_scales(w, N, K, g["sigma"])
    assert O.sha256_hex(w) == g["w_sha256"]
    lo, hi = _w12b_device(torch, w, N, K)
    md, sd = torch.from_numpy(mant).cuda(), torch.from_numpy(shift).cuda()
    xd = torch.from_numpy(x.astype(np.int8)).cuda()
    acc = torch.empty(m * N, dtype=torch.int64, device="cuda")
    q = torch.empty(m * N, dtype=torch.int8, device="cuda")
    say("case: w12b config2 M=2048")
    T.w12b_linear(xd, lo, hi, m, N, K, acc, T.OUT_I64)
    T.w12b_linear(xd, lo, hi, m, N, K, q, T.OUT_I8, md, sd)
    torch.cuda.synchronize()
    want = g["outputs"][str(m)]
    assert O.sha256_hex(acc.cpu().numpy()) == want["acc_i64_sha256"]
    assert O.sha256_hex(q.cpu().numpy()) == want["out_i8_sha256"]


def test_w12b_rejects_what_it_cannot_run(torch_dev):
    torch = torch_dev
    T = tb()
    lo = torch.zeros(T.w12b_bytes(64, 64), dtype=torch.int8, device="cuda")
    x = torch.zeros((8, 64), dtype=torch.int8, device="cuda")
    y = torch.zeros(8 * 64, dtype=torch.int32, device="cuda")
    with pytest.raises(T.HipError):
        T.w12b_linear(x, lo, lo, 8, 64, 64, y, T.OUT_I32)  # no scales for a requantized output
    with pytest.raises(T.HipError):
        T.w12b_linear(x, lo, lo, 8, 64, 0, y)  # k = 0
    with pytest.raises(T.HipError):
        T.w12b_linear(x, lo, lo, 8, 64, 131008 + 64, y)  # past KT_W12_GEMM_MAX_K
