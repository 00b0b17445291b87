"""kt_hip_quant_linear_noalloc (the QuantLinear entry point that allocates nothing: its workspace is the library's
per-GPU scratch array) against kt_hip_quant_linear with a caller workspace, through the C ABI: codes and the output
scale record bit for bit, on calls in a row whose later inputs are smaller (the scratch keeps the previous call's
contents), with and without a bias, including a shape whose digit GEMM splits k across CTAs (its accumulators and
tile counters live in the scratch and must start from zero on every call). Sizes past the scratch are refused
before any device work."""
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

WLEVELS = 265720


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def _case(rng, rows, inp, out, with_bias):
    x = rng.integers(-(2**27), 2**27, size=rows * inp).astype(np.int32)
    w = rng.integers(-WLEVELS, WLEVELS + 1, size=out * inp).astype(np.int32)
    bias = rng.integers(-(2**28), 2**28, size=out).astype(np.int64) if with_bias else None
    return x, w, bias


def test_noalloc_equals_the_workspace_entry_on_calls_in_a_row(torch_dev):
    torch = torch_dev
    import tritify_amd as TA
    from tritify_amd import backend as B
    from tritify_amd.quant import qscale_record, read_qscale

    rng = np.random.default_rng(2024)
    xs, wsc, bsc = (1509949440, 58), (1657624235, 49), (1318646415, 57)
    # the first call is the largest; each later one is smaller and finds the earlier call's bytes in the scratch
    shapes = [(512, 896, 896, True), (64, 896, 4864, False), (3, 130, 65, True), (1, 896, 896, False)]
    for rows, inp, out, with_bias in shapes:
        say(f"case: quant_linear_noalloc rows={rows} in={inp} out={out} bias={with_bias}")
        x, w, bias = _case(rng, rows, inp, out, with_bias)
        ql = TA.QuantLinear("t", w, out, inp, wsc, None if bias is None else (bias, bsc))
        xd = torch.from_numpy(x).cuda()
        xr = qscale_record(*xs)
        y_ws, os_ws = ql.forward_int(xd, xr, rows)
        y_na = torch.full((rows * out,), 0x5A5A5A5A, dtype=torch.int32, device="cuda")
        os_na = torch.full((4,), -1, dtype=torch.int64, device="cuda")
        B.quant_linear_noalloc(xd, rows, inp, xr, ql.w_planes, ql.pw, out, ql.w_scale, ql.bias, ql.b_scale, y_na,
                               os_na)
        torch.cuda.synchronize()
        a, b = y_ws.cpu().numpy(), y_na.cpu().numpy()
        assert np.array_equal(a, b), f"codes differ at {np.argwhere(a != b)[:5].tolist()}"
        assert read_qscale(os_ws) == read_qscale(os_na)
        # and both are the oracle's QuantLinear::forward_int
        yo, so, xmax, ymax = O.quant_linear_forward(x, rows, inp, xs, w, out, wsc, bias=bias,
                                                    bs=bsc if bias is not None else (0, 0))
        assert np.array_equal(b.reshape(rows, out), yo)
        r = read_qscale(os_na)
        assert (r["mant"], r["shift"]) == so and r["xmax"] == xmax and r["ymax"] == ymax
        del ql


def test_noalloc_captured_in_a_graph_and_replayed(torch_dev):
    """After one eager call on the GPU (the array's address is looked up there), the call captures into a HIP graph;
    replays with new inputs equal the oracle, for a shape whose digit GEMM splits k across CTAs and for a decode row,
    with eager work on the same scratch between the replays."""
    torch = torch_dev
    import tritify_amd as TA
    from tritify_amd import backend as B
    from tritify_amd.quant import qscale_record, read_qscale

    rng = np.random.default_rng(77)
    xs, wsc = (1509949440, 58), (1657624235, 49)
    for rows, inp, out in ((512, 896, 896), (1, 896, 4864)):
        say(f"case: quant_linear_noalloc graph rows={rows} in={inp} out={out}")
        x, w, _ = _case(rng, rows, inp, out, False)
        ql = TA.QuantLinear("g", w, out, inp, wsc, None)
        xd = torch.from_numpy(x).cuda()
        xr = qscale_record(*xs)
        y = torch.zeros(rows * out, dtype=torch.int32, device="cuda")
        osr = torch.zeros(4, dtype=torch.int64, device="cuda")
        B.quant_linear_noalloc(xd, rows, inp, xr, ql.w_planes, ql.pw, out, ql.w_scale, None, None, y, osr)
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            B.quant_linear_noalloc(xd, rows, inp, xr, ql.w_planes, ql.pw, out, ql.w_scale, None, None, y, osr,
                                   stream=s)
        torch.cuda.synchronize()
        other = _case(rng, 3, 130, 65, False)
        for rep in range(3):
            x = rng.integers(-(2 ** (22 + 2 * rep)), 2 ** (22 + 2 * rep), size=rows * inp).astype(np.int32)
            xd.copy_(torch.from_numpy(x))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            yo, so, xmax, ymax = O.quant_linear_forward(x, rows, inp, xs, w, out, wsc)
            assert np.array_equal(y.cpu().numpy().reshape(rows, out), yo), (rows, rep)
            r = read_qscale(osr)
            assert (r["mant"], r["shift"]) == so and r["xmax"] == xmax and r["ymax"] == ymax
            # an eager call of another shape between the replays overwrites the scratch
            ox, ow, _ = other
            q2 = TA.QuantLinear("o", ow, 65, 130, wsc, None)
            y2 = torch.zeros(3 * 65, dtype=torch.int32, device="cuda")
            B.quant_linear_noalloc(torch.from_numpy(ox).cuda(), 3, 130, xr, q2.w_planes, q2.pw, 65, q2.w_scale, None,
                                   None, y2, torch.zeros(4, dtype=torch.int64, device="cuda"))
            torch.cuda.synchronize()
            assert np.array_equal(y2.cpu().numpy().reshape(3, 65), O.quant_linear_forward(ox, 3, 130, xs, ow, 65,
                                                                                          wsc)[0])
        del g, ql


def test_noalloc_refuses_a_workspace_past_the_scratch(torch_dev):
    torch = torch_dev
    from tritify_amd import backend as B

    L = B.lib()
    rows, inp, out = 2048, 896, 4864  # 2048 * 4864 i64 accumulators alone are 76 MiB
    n, _ = B.quant_linear_workspace(rows, inp, out)
    assert n > B.QL_SCRATCH_BYTES
    x = torch.zeros(rows * inp, dtype=torch.int32, device="cuda")
    w = torch.zeros(out * 896, dtype=torch.int8, device="cuda")
    y = torch.zeros(rows * out, dtype=torch.int32, device="cuda")
    rec = torch.zeros(4, dtype=torch.int64, device="cuda")
    e = L.kt_hip_quant_linear_noalloc(0, x.data_ptr(), rows, inp, rec.data_ptr(), w.data_ptr(), 1, out, 1, 0, None,
                                      0, 0, y.data_ptr(), rec.data_ptr(), None)
    assert e == 1  # hipErrorInvalidValue, before any device work
    torch.cuda.synchronize()
    assert int(y.abs().sum().item()) == 0
