"""SAM's image path at the reference's semantics, on the CPU: the oracle's Conv2d, pixel entry, GELU CodeLut,
apply_gelu and FeedForward (oracle/kt_oracle_refdec.c) pinned by
  - the reference's own conv test (crates/01-engine/kt-core/src/conv.rs:479-500): seed 0xC0F, the integer conv
    tracks its float twin within 2% of the peak and is deterministic;
  - an independent lowering: Conv2d::forward_int equals QuantLinear::forward_int (pinned by the reference's golden
    vectors elsewhere) over numpy's zero-padded im2col rows, transposed -- over strides, paddings, kernels larger
    than the stride, 1x1 kernels, with and without bias;
  - the GELU table against the true GELU (math.erf) within the A&S 7.1.26 bound, and apply_gelu's closed forms:
    inside the table within one step of GELU, zero below it, the identity above it;
  - FeedForward tracking its float twin (hiera.rs:342-345) and composing proj_in, apply_gelu, proj_out.
The product's host-side builders (from_reals, the GELU CodeLut) are checked against the oracle bit for bit: they
need no GPU. No GPU call."""
import math

import numpy as np
import pytest

from oracle import oracle as O

STEP = 20.0 / 65535


def dq(codes, sc):
    return np.asarray(codes, dtype=np.float64) * (sc[0] * 2.0 ** -sc[1])


def gelu_true(x):
    return 0.5 * x * (1.0 + math.erf(x / math.sqrt(2.0)))


def conv_ref(xr, ci, h, w, wc, ws, co, k, stride, pad, bias):
    """Conv2d::forward_ref (conv.rs:133-163): f64 over the dequantized weights, (ic, ky, kx) order, to f32."""
    oh, ow = (h + 2 * pad - k) // stride + 1, (w + 2 * pad - k) // stride + 1
    wf = dq(wc, ws).reshape(co, ci, k, k)
    x = np.asarray(xr, np.float64).reshape(ci, h, w)
    out = np.zeros((co, oh, ow), np.float32)
    for oc in range(co):
        for oy in range(oh):
            for ox in range(ow):
                acc = 0.0
                for ic in range(ci):
                    for ky in range(k):
                        iy = oy * stride + ky - pad
                        if not 0 <= iy < h:
                            continue
                        for kx in range(k):
                            ix = ox * stride + kx - pad
                            if 0 <= ix < w:
                                acc += x[ic, iy, ix] * wf[oc, ic, ky, kx]
                out[oc, oy, ox] = acc + (0.0 if bias is None else bias[0][oc] * bias[1][0] * 2.0 ** -bias[1][1])
    return out


def test_conv2d_tracks_float_and_is_deterministic():
    """conv.rs:479-500, with its seed and draw order (weights, bias, image)."""
    ci, h, w, co, k, stride, pad = 3, 8, 8, 4, 3, 2, 1
    s = 0xC0F
    wt, s = O.vecf(s, co * ci * k * k)
    b, s = O.vecf(s, co)
    xf, s = O.vecf(s, ci * h * w)
    x, xs = O.from_reals(xf.astype(np.float64))
    wc, ws = O.quant_weights(wt)
    bq = O.quant_bias(b)
    oi, os_ = O.ref_conv2d(x, xs, ci, h, w, wc, ws, co, k, k, stride, pad, bq)
    assert oi.shape == (co, 4, 4)
    xr = dq(x, xs).astype(np.float32)  # IntTensor::to_f32
    r = conv_ref(xr, ci, h, w, wc, ws, co, k, stride, pad, bq)
    got = dq(oi, os_).astype(np.float32)
    mae = np.abs(got.astype(np.float64) - r.astype(np.float64)).max()
    peak = np.abs(r.astype(np.float64)).max()
    assert mae <= peak * 2e-2, f"conv2d drifted from float: {mae} against peak {peak}"
    again = O.ref_conv2d(x, xs, ci, h, w, wc, ws, co, k, k, stride, pad, bq)
    assert np.array_equal(again[0], oi) and again[1] == os_


def im2col(x, ci, h, w, k, stride, pad):
    xp = np.pad(np.asarray(x, np.int32).reshape(ci, h, w), ((0, 0), (pad, pad), (pad, pad)))
    oh, ow = (h + 2 * pad - k) // stride + 1, (w + 2 * pad - k) // stride + 1
    rows = np.empty((oh * ow, ci * k * k), np.int32)
    for oy in range(oh):
        for ox in range(ow):
            rows[oy * ow + ox] = xp[:, oy * stride:oy * stride + k, ox * stride:ox * stride + k].reshape(-1)
    return rows, oh, ow


@pytest.mark.parametrize("geom", [
    (3, 8, 8, 4, 3, 2, 1), (3, 29, 23, 7, 7, 4, 3), (5, 6, 9, 3, 1, 1, 0), (2, 5, 5, 2, 5, 1, 2), (4, 9, 7, 6, 2, 2, 0),
    (1, 3, 3, 1, 3, 1, 1),
])
@pytest.mark.parametrize("with_bias", [False, True])
def test_conv2d_equals_quantlinear_over_zero_padded_im2col(geom, with_bias):
    ci, h, w, co, k, stride, pad = geom
    rng = np.random.default_rng(hash(geom) & 0xFFFF)
    x = rng.integers(-(2**28), 2**28 + 1, size=ci * h * w).astype(np.int32)
    xs = (int(rng.integers(2**30, 2**31)), int(rng.integers(50, 60)))
    wc = rng.integers(-265720, 265721, size=co * ci * k * k).astype(np.int32)
    ws = (int(rng.integers(2**30, 2**31)), int(rng.integers(44, 50)))
    bias = None
    if with_bias:
        bias = (rng.integers(-(2**28), 2**28, size=co).astype(np.int64), (int(rng.integers(2**30, 2**31)), 58))
    y, ys = O.ref_conv2d(x, xs, ci, h, w, wc, ws, co, k, k, stride, pad, bias)
    rows, oh, ow = im2col(x, ci, h, w, k, stride, pad)
    yq, yqs, _, _ = O.quant_linear_forward(rows, oh * ow, ci * k * k, xs, wc, co, ws,
                                           None if bias is None else bias[0], (0, 0) if bias is None else bias[1])
    assert np.array_equal(y.reshape(co, oh * ow), yq.T) and ys == yqs


def test_conv2d_zero_image_gives_zeros_at_scale_zero_even_with_bias():
    """conv.rs:78-80: unlike QuantLinear (bias codes at the bias scale), an all-zero image closes at Scale::ZERO."""
    y, ys = O.ref_conv2d(np.zeros(2 * 4 * 4, np.int32), (1 << 30, 40), 2, 4, 4, np.ones(2 * 2 * 9, np.int32),
                     (1 << 30, 40), 2, 3, 3, 1, 1, (np.array([5, -7], np.int64), (1 << 30, 40)))
    assert not y.any() and ys == (0, 0)


def test_from_reals_closed_forms():
    """tensor.rs:106-117: the largest magnitude maps to +-levels, codes round half away from zero, zeros to ZERO."""
    real = np.array([0.0, -3.0, 1.5, 2.999999, -0.75, 3.0 / (1 << 28) * 0.5], np.float64)
    codes, sc = O.from_reals(real)
    assert codes[1] == -(1 << 28) and codes[0] == 0
    step = 3.0 / (1 << 28)
    for v, c in zip(real, codes):
        q = v / step
        assert c == int(math.floor(abs(q) + 0.5)) * (1 if q >= 0 else -1), (v, c)
    assert sc == (O.from_f64(step).mant, O.from_f64(step).shift)
    z, zs = O.from_reals(np.zeros(5))
    assert not z.any() and zs == (0, 0)


def test_gelu_table_matches_the_true_gelu():
    """nonlin.rs:7-26: every entry within the A&S 7.1.26 bound (|erf error| <= 1.5e-7, so |GELU error| <= 7.5e-7 on
    [-10, 10], 0.79 code units) plus rounding of the true GELU; the constants of CodeLut::build."""
    codes, inv, lo, cs = O.gelu_table()
    xs = -10.0 + 20.0 * (np.arange(1 << 16) / 65535.0)
    true = np.array([gelu_true(x) for x in xs]) * (1 << 20)
    assert np.abs(codes - true).max() <= 0.79 + 0.5
    assert lo == -32768  # round(-10 * 65535 / 20), half away from zero
    assert cs == (1 << 30, 50)  # 2^-20
    assert abs(inv[0] * 2.0 ** -inv[1] - 65535 / 20) < 1e-6
    assert codes[0] == 0 and codes[-1] == 10 << 20 and codes[32767] < 0 < codes[32768]


def test_apply_gelu_closed_forms():
    """nonlin.rs:30-45: inside the table within one step's worth of GELU's slope, zero below, identity above, at the
    table's code scale."""
    xs = O.from_f64(1.0 / (1 << 22))
    xsc = (xs.mant, xs.shift)
    reals = np.concatenate([np.linspace(-12, 12, 4001), [-10.0, 10.0, -10.0002, 10.0002, 0.0]])
    d = np.round(reals * (1 << 22)).astype(np.int32)
    y, ys = O.apply_gelu(d, xsc)
    assert ys == (1 << 30, 50)
    x = d.astype(np.float64) / (1 << 22)
    got = y.astype(np.float64) / (1 << 20)
    inside = np.abs(x) <= 10.0 - STEP
    want = np.array([gelu_true(v) for v in x[inside]])
    assert np.abs(got[inside] - want).max() <= 1.13 * STEP + 2.0 ** -19
    below, above = x < -10.0 - STEP, x > 10.0 + STEP
    assert not y[below].any()
    assert np.abs(got[above] - x[above]).max() <= 2.0 ** -20
    assert below.any() and above.any()


def test_feedforward_tracks_float_and_composes():
    """hiera.rs:336-345: proj_in (+bias) -> apply_gelu -> proj_out (+bias), against the float twin; and the
    composition of the oracle's own QuantLinear and apply_gelu."""
    dim, hidden, rows = 48, 192, 7
    s = 0xFF0
    wi, s = O.vecf(s, hidden * dim)
    bi, s = O.vecf(s, hidden)
    wo, s = O.vecf(s, dim * hidden)
    bo, s = O.vecf(s, dim)
    xf, s = O.vecf(s, rows * dim)
    wic, wis = O.quant_weights(wi * 0.2)
    woc, wos = O.quant_weights(wo * 0.1)
    biq, boq = O.quant_bias(bi * 0.1), O.quant_bias(bo * 0.1)
    x, xs = O.from_reals((xf * 3.0).astype(np.float64))
    y, ys = O.feedforward(x, rows, dim, xs, wic, wis, hidden, woc, wos, biq, boq)
    h, hs, _, _ = O.quant_linear_forward(x, rows, dim, xs, wic, hidden, wis, biq[0], biq[1])
    g, gs = O.apply_gelu(h.reshape(-1), hs)
    y2, ys2, _, _ = O.quant_linear_forward(g, rows, hidden, gs, woc, dim, wos, boq[0], boq[1])
    assert np.array_equal(y, y2) and ys == ys2
    xr = dq(x, xs).reshape(rows, dim)
    hr = xr @ dq(wic, wis).reshape(hidden, dim).T + dq(biq[0], biq[1])
    gr = np.vectorize(gelu_true)(hr.astype(np.float32).astype(np.float64))
    yr = gr.astype(np.float32).astype(np.float64) @ dq(woc, wos).reshape(dim, hidden).T + dq(boq[0], boq[1])
    err = np.abs(dq(y, ys) - yr).max()
    assert err <= 2e-2 * np.abs(yr).max(), f"drifted from float: {err}"


def test_product_host_builders_equal_the_oracle():
    """kt_hip_ref_from_reals and kt_hip_ref_codelut(KT_LUT_GELU) run on the host: bit for bit the oracle's."""
    from tritify_amd import backend as B

    rng = np.random.default_rng(3)
    real = rng.standard_normal(3 * 32 * 32) * 2.5
    real[5] = 0.5 * 2.5 * 4 / (1 << 28)  # a tie somewhere near the bottom
    assert all(np.array_equal(a, b) if isinstance(a, np.ndarray) else a == b
               for a, b in zip(B.ref_from_reals(real), O.from_reals(real)))
    z = B.ref_from_reals(np.zeros(4))
    assert not z[0].any() and z[1] == (0, 0)
    with pytest.raises(Exception):
        B.ref_from_reals(np.array([1.0, np.nan]))
    codes, lut = B.ref_codelut(B.LUT_GELU, -10.0, 10.0, 16, 20, True)
    oc, inv, lo, cs = O.gelu_table()
    assert np.array_equal(codes, oc)
    assert (lut.inv_mant, lut.inv_shift) == inv and lut.lo_index == lo and (lut.code_mant, lut.code_shift) == cs
    assert lut.n == 1 << 16 and lut.right_identity == 1


def test_conv_is_the_same_for_any_thread_count():
    """par_blocks (layers.rs:88-115) splits Conv2d::forward_int's output channels over workers: 1, 2, 3 and 8
    threads give the same codes and scale (the partition property of tests_partition.rs:43-58, for the conv)."""
    rng = np.random.default_rng(91)
    ci, h, w, co, k = 3, 64, 80, 13, 5
    x = rng.integers(-(2**28), 2**28, size=ci * h * w).astype(np.int32)
    wc = rng.integers(-O.WLEVELS, O.WLEVELS + 1, size=co * ci * k * k).astype(np.int32)
    bias = (rng.integers(-(2**40), 2**40, size=co).astype(np.int64), (1 << 30, 70))
    runs = []
    for t in (1, 2, 3, 8):
        O.set_max_threads(t)
        runs.append(O.ref_conv2d(x, (1 << 30, 40), ci, h, w, wc, (1 << 30, 50), co, k, k, 2, 2, bias))
    O.set_max_threads(0)
    for y, s in runs[1:]:
        assert np.array_equal(y, runs[0][0]) and s == runs[0][1]

