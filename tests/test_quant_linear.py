"""The oracle's restatement of QuantLinear::forward_int (crates/01-engine/kt-core/src/layers.rs:275-328), pinned on
the CPU, and the product's QuantLinear binding checked without a GPU.

Pins (each chosen so that a plausible slip fails one of them):
- the reference's own test `quantlinear_tracks_float_and_is_deterministic` (kt-core/src/tests.rs:34-46): the same
  generator, seed 0xBEEF, 64 x 128 weights from `QuantLinear::from_weights` and a `from_reals` probe; the dequantized
  output must track the float product (`forward_ref`, layers.rs:330-349) within the reference's 1% of the peak and,
  since the output level is 2^28, within 1e-5 of it; with a bias (`with_bias`, layers.rs:246-257) the same;
- exact invariants: doubling every input code leaves the output codes unchanged (quant_to normalizes by xmax);
  negating the input negates the output codes exactly without a bias (both roundings are half away from zero); the
  output's maximum code is exactly 2^28 (ymax maps to ACT_LEVELS); xmax == 0 gives the bias codes at the bias scale
  or zeros at Scale::ZERO (layers.rs:282-295); a zero weight scale gives zeros;
- rows are independent of each other only through the two maxima: the batch equals the per-row evaluation when
  every row has the same xmax and ymax (checked on a constructed case).
"""
import numpy as np
import pytest

from oracle import oracle as O

WLEVELS = 265720
ACT_LEVELS = 1 << 28


def lcg(s: int) -> int:
    return (s * 6364136223846793005 + 1442695040888963407) % 2**64


class Unif:
    """tests.rs:15-24: unif = ((lcg >> 40) / 2^24 * 2 - 1) as f32."""

    def __init__(self, seed: int):
        self.s = seed

    def vecf(self, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        for i in range(n):
            self.s = lcg(self.s)
            out[i] = np.float32((self.s >> 40) / float(1 << 24) * 2.0 - 1.0)
        return out


def round_away(v: np.ndarray) -> np.ndarray:
    return np.where(v >= 0, np.floor(v + 0.5), -np.floor(-v + 0.5))


def from_weights(w: np.ndarray):
    """QuantLinear::from_weights (layers.rs:225-244): codes round(w / step) clamped, scale from_f64(step)."""
    peak = float(np.max(np.abs(w.astype(np.float64))))
    step = peak / WLEVELS
    codes = np.clip(round_away(w.astype(np.float64) / step), -WLEVELS, WLEVELS).astype(np.int32)
    s = O.from_f64(step)
    return codes, (s.mant, s.shift)


def from_reals(real: np.ndarray, levels: int):
    """IntTensor::from_reals (tensor.rs:106-117)."""
    mx = float(np.max(np.abs(real)))
    step = mx / levels
    s = O.from_f64(step)
    return round_away(real * (levels / mx)).astype(np.int32), (s.mant, s.shift)


def to_f64(codes: np.ndarray, scale) -> np.ndarray:
    return codes.astype(np.float64) * (scale[0] * 2.0 ** (-scale[1]))


def reference_case(seed=0xBEEF, out=64, inp=128, rows=1):
    u = Unif(seed)
    w = u.vecf(out * inp)
    probe = u.vecf(rows * inp).astype(np.float64)
    codes, ws = from_weights(w)
    x, xs = from_reals(probe, ACT_LEVELS)
    return codes, ws, x, xs


def test_oracle_tracks_float_as_the_reference_test():
    out, inp = 64, 128
    codes, ws, x, xs = reference_case()
    y, os_, xmax, ymax = O.quant_linear_forward(x, 1, inp, xs, codes, out, ws)
    y2, os2, _, _ = O.quant_linear_forward(x, 1, inp, xs, codes, out, ws)
    assert np.array_equal(y, y2) and os_ == os2  # deterministic
    xr = to_f64(x, xs).astype(np.float32).astype(np.float64)  # probe.to_f32()
    ref = (to_f64(codes, ws).reshape(out, inp) @ xr.reshape(inp)).astype(np.float32)
    got = to_f64(y.reshape(out), os_).astype(np.float32)
    err = float(np.max(np.abs(got.astype(np.float64) - ref)))
    peak = float(np.max(np.abs(ref)))
    assert err <= peak * 1e-2
    assert err <= peak * 1e-5
    assert xmax == int(np.max(np.abs(x))) and ymax > 0
    assert int(np.max(np.abs(y))) == ACT_LEVELS


def test_oracle_bias_tracks_float():
    out, inp, rows = 48, 96, 5
    codes, ws, x, xs = reference_case(seed=0x5EED, out=out, inp=inp, rows=rows)
    b = Unif(99).vecf(out).astype(np.float64) * 0.3
    bcodes, bs = from_reals(b, ACT_LEVELS)  # with_bias: step = bmax / ACT_LEVELS
    y, os_, _, _ = O.quant_linear_forward(x, rows, inp, xs, codes, out, ws, bias=bcodes.astype(np.int64), bs=bs)
    xr = to_f64(x, xs).reshape(rows, inp)
    ref = xr @ to_f64(codes, ws).reshape(out, inp).T + to_f64(bcodes, bs)[None, :]
    err = float(np.max(np.abs(to_f64(y, os_) - ref)))
    assert err <= float(np.max(np.abs(ref))) * 1e-5


def test_oracle_invariants():
    rng = np.random.default_rng(7)
    rows, inp, out = 6, 70, 33
    x = rng.integers(-(2**20), 2**20, size=rows * inp).astype(np.int32)
    w = rng.integers(-WLEVELS, WLEVELS + 1, size=out * inp).astype(np.int32)
    xs, ws = (1 << 30, 40), (1 << 30, 50)
    y, os_, xmax, ymax = O.quant_linear_forward(x, rows, inp, xs, w, out, ws)
    # doubling the codes: same output codes
    y2, _, xmax2, _ = O.quant_linear_forward(2 * x, rows, inp, xs, w, out, ws)
    assert np.array_equal(y, y2) and xmax2 == 2 * xmax
    # negation
    yn, osn, _, ymaxn = O.quant_linear_forward(-x, rows, inp, xs, w, out, ws)
    assert np.array_equal(yn, -y) and osn == os_ and ymaxn == ymax
    # the largest |output| is the level
    assert int(np.max(np.abs(y))) == ACT_LEVELS
    # ymax is the largest |exact product|
    qx = O.quant_to(x, xmax).astype(np.int64).reshape(rows, inp)
    acc = qx @ w.astype(np.int64).reshape(out, inp).T
    assert ymax == int(np.max(np.abs(acc)))
    # every code is requant_dyn (pinned by brute force on its own) of that exact product
    assert all(int(y.flat[i]) == O.requant_dyn(int(acc.flat[i]), ACT_LEVELS, ymax) for i in range(0, acc.size, 7))


def test_oracle_zero_cases():
    rows, inp, out = 3, 10, 4
    w = np.arange(out * inp, dtype=np.int32) - 20
    b = np.array([5, -7, 0, 123456789], dtype=np.int64)
    z = np.zeros(rows * inp, dtype=np.int32)
    y, os_, xmax, ymax = O.quant_linear_forward(z, rows, inp, (1 << 30, 30), w, out, (1 << 30, 30), bias=b,
                                                bs=(12345, 20))
    assert (y == b[None, :].astype(np.int32)).all() and os_ == (12345, 20) and xmax == 0 and ymax == 0
    y, os_, _, _ = O.quant_linear_forward(z, rows, inp, (1 << 30, 30), w, out, (1 << 30, 30))
    assert (y == 0).all() and os_ == (0, 0)
    x = np.ones(rows * inp, dtype=np.int32)
    y, os_, xmax, _ = O.quant_linear_forward(x, rows, inp, (1 << 30, 30), w, out, (0, 0))
    assert (y == 0).all() and os_ == (0, 0) and xmax == 1
    y, os_, _, ymax = O.quant_linear_forward(x, rows, inp, (1 << 30, 30), np.zeros_like(w), out, (1 << 30, 30))
    assert (y == 0).all() and os_ == (0, 0) and ymax == 0


def test_oracle_rows_couple_only_through_the_maxima():
    inp, out = 40, 9
    rng = np.random.default_rng(3)
    w = rng.integers(-1000, 1000, size=out * inp).astype(np.int32)
    row = rng.integers(-500, 500, size=inp).astype(np.int32)
    x = np.concatenate([row, -row])  # same xmax; |acc| rows equal, so the same ymax
    y, _, _, _ = O.quant_linear_forward(x, 2, inp, (1 << 30, 30), w, out, (1 << 30, 30))
    y1, _, _, _ = O.quant_linear_forward(row, 1, inp, (1 << 30, 30), w, out, (1 << 30, 30))
    assert np.array_equal(y[0], y1[0]) and np.array_equal(y[1], -y1[0])


def test_quant_linear_workspace_sizes():
    """The product's workspace rule loads without a GPU and covers each part."""
    import tritify_amd as TA

    try:
        n, off = TA.quant_linear_workspace(5, 70, 33)
    except ImportError:
        pytest.skip("libkt_hip.so is not built here")
    kp = 128
    assert off[0] == 0 and off[1] >= 3 * 5 * kp and off[2] >= off[1] + 5 * 33 * 8
    assert off[3] >= off[2] + 1024 * 4 and off[4] >= off[3] + 1024 * 8 and n >= off[4] + 48
    assert all(o % 256 == 0 for o in off)
    with pytest.raises(ValueError):
        TA.quant_linear_workspace(0, 70, 33)
