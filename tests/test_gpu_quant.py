"""Parity of the device QuantLinear::forward_int (kt_hip_quant_linear) with the oracle's restatement of
crates/01-engine/kt-core/src/layers.rs:275-328, through the C ABI. Run on a GPU box with -m gpu.

Every case compares the output codes, the output Scale and both maxima bit for bit: the reference's own test case
(kt-core/src/tests.rs:34-46), ragged shapes with and without a bias, extreme input codes (+-(2^31 - 1), -2^31),
weights needing 1, 3 and 5 digit planes, the xmax == 0 and zero-scale paths, a config-3 projection shape, shapes
whose GEMM splits k across CTAs, a chain of two layers that passes the scale record on the device, and replays of a
captured HIP graph.
"""
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

WLEVELS = 265720


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def run(torch, x, rows, inp, xs, w, out, ws, bias=None, bs=None):
    import tritify_amd as TA

    say(f"case: quant_linear rows={rows} in={inp} out={out} bias={bias is not None}")
    ql = TA.QuantLinear("t", w, out, inp, ws, None if bias is None else (bias, bs))
    y, sc = ql.forward_int_host(x, xs)
    yo, so, xmax, ymax = O.quant_linear_forward(x, rows, inp, xs, w, out, ws, bias=bias,
                                                bs=bs if bs is not None else (0, 0))
    assert np.array_equal(y, yo), f"codes differ at {np.argwhere(y != yo)[:5].tolist()}"
    assert (sc["mant"], sc["shift"]) == so
    assert sc["xmax"] == xmax and sc["ymax"] == ymax
    return ql


def test_reference_case(torch_dev):
    sys.path.insert(0, __file__.rsplit("/", 1)[0])
    from test_quant_linear import reference_case

    codes, ws, x, xs = reference_case()
    run(torch_dev, x, 1, 128, xs, codes, 64, ws)


@pytest.mark.parametrize("rows,inp,out", [(1, 1, 1), (3, 63, 17), (67, 130, 65), (1, 896, 896), (200, 64, 300)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_shapes(torch_dev, rows, inp, out, with_bias):
    rng = np.random.default_rng(rows * 1000 + inp + out)
    x = rng.integers(-(2**27), 2**27, size=rows * inp).astype(np.int32)
    w = rng.integers(-WLEVELS, WLEVELS + 1, size=out * inp).astype(np.int32)
    bias = rng.integers(-(2**28), 2**28, size=out).astype(np.int64) if with_bias else None
    run(torch_dev, x, rows, inp, (1509949440, 58), w, out, (1657624235, 49), bias, (1318646415, 57))


def test_extreme_codes_and_plane_counts(torch_dev):
    rng = np.random.default_rng(11)
    rows, inp, out = 5, 100, 40
    x = rng.integers(-(2**31), 2**31, size=rows * inp, dtype=np.int64).astype(np.int32)
    x[:4] = [2**31 - 1, -(2**31), -(2**31) + 1, 0]
    for lim in (127, WLEVELS, 2**31 - 1):  # 1, 3 and 5 weight planes
        w = rng.integers(-lim, lim + 1, size=out * inp, dtype=np.int64).astype(np.int32)
        ql = run(torch_dev, x, rows, inp, (1 << 30, 30), w, out, (1 << 30, 40))
        assert ql.pw == {127: 1, WLEVELS: 3, 2**31 - 1: 5}[lim]


def test_zero_paths(torch_dev):
    rows, inp, out = 4, 33, 9
    w = (np.arange(out * inp, dtype=np.int32) % 201) - 100
    z = np.zeros(rows * inp, dtype=np.int32)
    b = np.arange(out, dtype=np.int64) * 1000003 - 4000000
    run(torch_dev, z, rows, inp, (1 << 30, 30), w, out, (1 << 30, 30), b, (777, 12))  # bias codes out
    run(torch_dev, z, rows, inp, (1 << 30, 30), w, out, (1 << 30, 30))  # zeros
    x = np.arange(rows * inp, dtype=np.int32) - 50
    run(torch_dev, x, rows, inp, (1 << 30, 30), w, out, (0, 0), b, (777, 12))  # c == 0
    run(torch_dev, x, rows, inp, (1 << 30, 30), np.zeros_like(w), out, (1 << 30, 30))  # ymax == 0


def test_config3_projection_shape(torch_dev):
    rng = np.random.default_rng(896)
    rows, inp, out = 512, 896, 4864
    x = rng.integers(-(2**28), 2**28, size=rows * inp).astype(np.int32)
    w = rng.integers(-WLEVELS, WLEVELS + 1, size=out * inp).astype(np.int32)
    run(torch_dev, x, rows, inp, (1509949440, 58), w, out, (1657624235, 49))


@pytest.mark.parametrize("rows,inp,out,with_bias", [(512, 4864, 896, True), (64, 2048, 1000, False),
                                                      (65, 1600, 300, True)])
def test_split_k_shapes(torch_dev, rows, inp, out, with_bias):
    """Shapes whose digit GEMM splits k across CTAs (few tiles: the config-3 down projection, one row tile, a ragged
    second row tile), partial sums added with atomics and the bias and maximum taken by each tile's last CTA."""
    rng = np.random.default_rng(rows + inp + out)
    x = rng.integers(-(2**28), 2**28, size=rows * inp).astype(np.int32)
    w = rng.integers(-WLEVELS, WLEVELS + 1, size=out * inp).astype(np.int32)
    bias = rng.integers(-(2**28), 2**28, size=out).astype(np.int64) if with_bias else None
    run(torch_dev, x, rows, inp, (1509949440, 58), w, out, (1657624235, 49), bias, (1318646415, 57))


def _two_layers(rng, d0=96, d1=80, d2=48):
    w1 = rng.integers(-WLEVELS, WLEVELS + 1, size=d1 * d0).astype(np.int32)
    w2 = rng.integers(-WLEVELS, WLEVELS + 1, size=d2 * d1).astype(np.int32)
    b2 = rng.integers(-(2**28), 2**28, size=d2).astype(np.int64)
    return (d0, d1, d2), w1, w2, b2


def test_chain_and_graph_replay(torch_dev):
    """Two layers (Sequential, tests.rs:48-62) with the scale record passed on the device, eager and as a captured
    graph replayed with fresh inputs between replays; every result against the oracle."""
    import tritify_amd as TA

    torch = torch_dev
    rng = np.random.default_rng(5)
    (d0, d1, d2), w1, w2, b2 = _two_layers(rng)
    ws1, ws2, bs2 = (1657624235, 49), (1200000000, 48), (1318646415, 57)
    l1 = TA.QuantLinear("l1", w1, d1, d0, ws1)
    l2 = TA.QuantLinear("l2", w2, d2, d1, ws2, (b2, bs2))
    rows = 7
    xd = torch.zeros(rows * d0, dtype=torch.int32, device="cuda")
    xs = TA.qscale_record(1509949440, 58)
    h = torch.zeros(rows * d1, dtype=torch.int32, device="cuda")
    hs = torch.zeros(4, dtype=torch.int64, device="cuda")
    y = torch.zeros(rows * d2, dtype=torch.int32, device="cuda")
    ys = torch.zeros(4, dtype=torch.int64, device="cuda")

    def expect(x):
        hh, hsc, _, _ = O.quant_linear_forward(x, rows, d0, (1509949440, 58), w1, d1, ws1)
        return O.quant_linear_forward(hh, rows, d1, hsc, w2, d2, ws2, bias=b2, bs=bs2)

    def check(x):
        yo, so, xmax, ymax = expect(x)
        got = y.cpu().numpy().reshape(rows, d2)
        sc = TA.read_qscale(ys)
        assert np.array_equal(got, yo) and (sc["mant"], sc["shift"]) == so and sc["ymax"] == ymax

    say("case: two-layer chain, eager")
    x = rng.integers(-(2**28), 2**28, size=rows * d0).astype(np.int32)
    xd.copy_(torch.from_numpy(x))
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        l1.forward_int(xd, xs, rows, h, hs, stream=s)
        l2.forward_int(h, hs, rows, y, ys, stream=s)
    s.synchronize()
    check(x)

    say("case: two-layer chain, graph replays")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        l1.forward_int(xd, xs, rows, h, hs, stream=s)
        l2.forward_int(h, hs, rows, y, ys, stream=s)
    torch.cuda.synchronize()
    for rep in range(3):
        x = rng.integers(-(2 ** (20 + 3 * rep)), 2 ** (20 + 3 * rep), size=rows * d0).astype(np.int32)
        if rep == 2:
            x[:] = 0  # the xmax == 0 path on a replay after two live ones
        xd.copy_(torch.from_numpy(x))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        check(x)


def group_case(torch, rng, rows, inp, outs, lims, biases, zero_x=False, w_zero_scale=()):
    """A QuantLinearGroup against each member's own QuantLinear and the oracle: codes and records."""
    import tritify_amd as TA

    say(f"case: quant_linear group rows={rows} in={inp} outs={outs} biases={biases}")
    x = np.zeros(rows * inp, np.int32) if zero_x else rng.integers(-(2**27), 2**27, size=rows * inp).astype(np.int32)
    xs = (1509949440, 58)
    members = []
    for g, (o, lim, hb) in enumerate(zip(outs, lims, biases)):
        w = rng.integers(-lim, lim + 1, size=o * inp, dtype=np.int64).astype(np.int32).reshape(o, inp)
        ws = (0, 0) if g in w_zero_scale else (int(rng.integers(2**30, 2**31)), int(rng.integers(40, 50)))
        b = (rng.integers(-(2**28), 2**28, size=o).astype(np.int64), (int(rng.integers(2**30, 2**31)), 57)) \
            if hb else None
        members.append((f"m{g}", w, ws, b))
    grp = TA.QuantLinearGroup("grp", members, inp)
    xd = torch.from_numpy(x).cuda()
    xr = TA.qscale_record(*xs)
    res = grp.forward_int(xd, xr, rows)
    torch.cuda.synchronize()
    for (name, w, ws, b), (y, rec) in zip(members, res):
        yo, so, xmax, ymax = O.quant_linear_forward(x, rows, inp, xs, w.reshape(-1), w.shape[0], ws,
                                                    bias=None if b is None else b[0],
                                                    bs=(0, 0) if b is None else b[1])
        got = y.cpu().numpy().reshape(rows, w.shape[0])
        assert np.array_equal(got, yo.reshape(rows, -1)), f"{name}: codes differ"
        r = TA.read_qscale(rec)
        assert (r["mant"], r["shift"]) == so and r["xmax"] == xmax and r["ymax"] == ymax, f"{name}: record"
    return grp


@pytest.mark.parametrize("rows", [1, 3, 64, 512])
def test_group_equals_separate_calls(torch_dev, rows):
    """q / k / v- and gate / up-shaped groups (decode rows on the skinny product, prefill rows on MFMA tiles, a
    split-k shape), biases on some members: every member's codes, Scale and maxima equal its own call's."""
    rng = np.random.default_rng(rows)
    group_case(torch_dev, rng, rows, 896, (896, 128, 128), (WLEVELS,) * 3, (True, False, True))
    group_case(torch_dev, rng, rows, 896, (1024, 1024), (WLEVELS, WLEVELS), (False, False))


def test_group_plane_counts_and_zero_paths(torch_dev):
    """Members of 1, 3 and 5 weight planes (the group packs at the largest), an all-zero x (bias codes or zeros),
    a member at a zero weight scale."""
    rng = np.random.default_rng(3)
    grp = group_case(torch_dev, rng, 2, 200, (128, 256, 128), (127, WLEVELS, 2**31 - 1), (True, False, False))
    assert grp.pw == 5
    group_case(torch_dev, rng, 2, 200, (128, 128), (WLEVELS, WLEVELS), (True, False), zero_x=True)
    group_case(torch_dev, rng, 5, 200, (256, 128), (WLEVELS, WLEVELS), (True, True), w_zero_scale=(1,))


def test_group_rejects_misaligned_boundaries(torch_dev):
    """A boundary that is not a multiple of the digit GEMM's column block is refused (the host then makes the calls
    one at a time), by the class and by the C entry."""
    torch = torch_dev
    import tritify_amd as TA
    from tritify_amd import backend as B

    assert not TA.QuantLinearGroup.fits((100, 28)) and TA.QuantLinearGroup.fits((128, 28))
    w = np.ones((136, 64), np.int32)
    planes = torch.zeros(3 * 136 * 64, dtype=torch.int8, device="cuda")
    n, _ = B.quant_linear_workspace(1, 64, 136)
    ws = torch.empty(n, dtype=torch.uint8, device="cuda")
    ys = [torch.empty(100, dtype=torch.int32, device="cuda"), torch.empty(36, dtype=torch.int32, device="cuda")]
    with pytest.raises(Exception):
        B.quant_linear_multi(torch.zeros(64, dtype=torch.int32, device="cuda"), 1, 64, TA.qscale_record(1 << 30, 30),
                             [100, 36], planes, 3, [(1 << 30, 40)] * 2, None, [None, None], ws, n, ys,
                             torch.empty(8, dtype=torch.int64, device="cuda"))
    del w
