"""SAM's image path at the reference's semantics on the GPU, through the C ABI, against the oracle's restatement
(oracle/kt_oracle_refdec.c, pinned in tests/test_refconv.py): Conv2d::forward_int over strides, paddings and
kernel sizes with and without bias, an all-zero image, and the full Hiera-B+ PatchEmbed (3 x 1024 x 1024 pixels
from from_reals, 112 channels, 7 x 7 / 4, pad 3); apply_gelu by the GELU CodeLut across both tails and in place;
FeedForward at a stage-3 shape -- codes and Scales bit for bit."""
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

WL = 265720


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def rec(torch, sc):
    w = np.zeros(4, dtype=np.int64)
    w[0] = sc[0]
    w.view(np.int32)[2] = sc[1]
    return torch.from_numpy(w).cuda()


def read_rec(t):
    w = t.cpu().numpy()
    return int(w[0]), int(w.view(np.int32)[2])


def i32(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32).reshape(-1)).cuda()


def conv_case(torch, ci, h, w, co, k, stride, pad, with_bias, seed, x=None, xs=None):
    from tritify_amd.refvision import RefConv2d

    rng = np.random.default_rng(seed)
    if x is None:
        x = rng.integers(-(2**28), 2**28 + 1, size=ci * h * w).astype(np.int32)
        xs = (int(rng.integers(2**30, 2**31)), int(rng.integers(50, 60)))
    wc = rng.integers(-WL, WL + 1, size=(co, ci, k, k)).astype(np.int32)
    ws = (int(rng.integers(2**30, 2**31)), int(rng.integers(44, 50)))
    bias = None
    if with_bias:
        bias = (rng.integers(-(2**28), 2**28, size=co).astype(np.int64), (int(rng.integers(2**30, 2**31)), 58))
    conv = RefConv2d(wc, ws, stride, pad, bias)
    y, os_ = conv.forward_int(i32(torch, x), rec(torch, xs), h, w)
    want, wso = O.ref_conv2d(x, xs, ci, h, w, wc.reshape(-1), ws, co, k, k, stride, pad, bias)
    got = y.cpu().numpy().reshape(want.shape)
    assert np.array_equal(got, want), f"codes differ at {np.argwhere(got != want)[:5].tolist()}"
    assert read_rec(os_) == wso


@pytest.mark.parametrize("geom", [
    (3, 8, 8, 4, 3, 2, 1), (3, 29, 23, 7, 7, 4, 3), (5, 6, 9, 3, 1, 1, 0), (2, 5, 5, 2, 5, 1, 2), (4, 9, 7, 6, 2, 2, 0),
    (1, 3, 3, 1, 3, 1, 1), (3, 130, 70, 112, 7, 4, 3), (64, 20, 20, 200, 3, 1, 1),
])
@pytest.mark.parametrize("with_bias", [False, True])
def test_conv2d_against_the_oracle(torch_dev, geom, with_bias):
    say(f"case: ref conv2d {geom} bias={with_bias}")
    conv_case(torch_dev, *geom, with_bias, seed=sum(geom) * 7 + with_bias)


def test_conv2d_zero_image(torch_dev):
    torch = torch_dev
    from tritify_amd.refvision import RefConv2d

    say("case: ref conv2d zero image")
    conv = RefConv2d(np.ones((2, 2, 3, 3), np.int32), (1 << 30, 40), 1, 1, (np.array([5, -7], np.int64), (1 << 30, 40)))
    y, os_ = conv.forward_int(torch.zeros(2 * 4 * 4, dtype=torch.int32, device="cuda"), rec(torch, (1 << 30, 40)), 4, 4)
    assert not y.cpu().numpy().any() and read_rec(os_) == (0, 0)


def test_patch_embed_full_image(torch_dev):
    """Hiera-B+ PatchEmbed (hiera.rs:133-190) on a 1024 x 1024 image brought in by from_reals at ACT_LEVELS."""
    torch = torch_dev
    from tritify_amd import backend as B

    say("case: ref patch embed 3x1024x1024 -> 112x256x256")
    rng = np.random.default_rng(0x5A)
    real = rng.standard_normal(3 * 1024 * 1024) * 1.7
    x, xs = B.ref_from_reals(real)
    assert np.array_equal(x, O.from_reals(real)[0])
    conv_case(torch, 3, 1024, 1024, 112, 7, 4, 3, True, seed=0x5B, x=x, xs=xs)


@pytest.mark.parametrize("scale_shift", [16, 22, 28, 34])
def test_gelu_against_the_oracle(torch_dev, scale_shift):
    torch = torch_dev
    from tritify_amd import backend as B
    from tritify_amd.refvision import gelu_table

    say(f"case: ref gelu shift {scale_shift}")
    rng = np.random.default_rng(scale_shift)
    n = 300_001
    x = rng.integers(-(2**31), 2**31, size=n, dtype=np.int64).astype(np.int32)
    x[::3] >>= 8
    x[::5] >>= 16
    xs = (int(rng.integers(2**30, 2**31)), scale_shift + 30)
    codes, lut = gelu_table()
    y = torch.empty(n, dtype=torch.int32, device="cuda")
    ys = torch.zeros(4, dtype=torch.int64, device="cuda")
    xd = i32(torch, x)
    B.ref_gelu(xd, rec(torch, xs), n, codes, lut, y, ys)
    want, wso = O.apply_gelu(x, xs)
    got = y.cpu().numpy()
    assert np.array_equal(got, want), f"codes differ at {np.argwhere(got != want)[:5].tolist()}"
    assert read_rec(ys) == wso
    B.ref_gelu(xd, rec(torch, xs), n, codes, lut, xd, ys)  # in place
    assert np.array_equal(xd.cpu().numpy(), want)


@pytest.mark.parametrize("rows,dim,hidden", [(7, 48, 192), (4096, 448, 1792)])
def test_feedforward_against_the_oracle(torch_dev, rows, dim, hidden):
    torch = torch_dev
    from tritify_amd.refvision import RefFeedForward

    say(f"case: ref feedforward rows={rows} dim={dim} hidden={hidden}")
    s = 0xFF0 + rows
    wi, s = O.vecf(s, hidden * dim)
    bi, s = O.vecf(s, hidden)
    wo, s = O.vecf(s, dim * hidden)
    bo, s = O.vecf(s, dim)
    wic, wis = O.quant_weights(wi * 0.2)
    woc, wos = O.quant_weights(wo * 0.1)
    biq, boq = O.quant_bias(bi * 0.1), O.quant_bias(bo * 0.1)
    rng = np.random.default_rng(rows)
    x, xs = O.from_reals(rng.standard_normal(rows * dim) * 3.0)
    ff = RefFeedForward(dim, hidden, (wic, wis, biq), (woc, wos, boq))
    y, ys = ff.forward_int(i32(torch, x), rec(torch, xs), rows)
    want, wso = O.feedforward(x, rows, dim, xs, wic, wis, hidden, woc, wos, biq, boq)
    got = y.cpu().numpy().reshape(want.shape)
    assert np.array_equal(got, want), f"codes differ at {np.argwhere(got != want)[:5].tolist()}"
    assert read_rec(ys) == wso
