"""Parity of config 5 (SAM 2.1 Hiera-B+ image-encoder GEMMs) on the MI355X with the CPU oracle, through the C ABI.
Run on a GPU box with -m gpu.

Patch embed: the im2col-fused W12 conv against the oracle's restatement of the reference's direct conv loop
(Conv2d::forward_int, crates/01-engine/kt-core/src/conv.rs:68-130: (ic, ky, kx) order, taps outside the image
skipped, bias in accumulator units, output [c_out, OH, OW]); on small and ragged shapes (partial row segments, more
than one channel tile, a 3x3 stride-1 kernel) against the oracle directly, at the full 1024 x 1024 image against the
fixture hashes. Stage-3 MLP: the dense W12 GEMM with the GELU code table in its epilogue, then the down projection.
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


def run_conv(torch, C, H, W, CO, KH, KW, S, P, seeds=(61, 62, 63), bias=True, scales=None):
    import tritify_amd as TA
    from tritify_amd import workloads as W_

    say(f"case: patch embed C={C} H={H} W={W} CO={CO} k={KH}x{KW} s={S} p={P}")
    img, w, b, mant, shift = W_.sam_patch_inputs(C, H, W, CO, KH, KW, *seeds)
    if scales is not None:
        mant, shift = scales(mant, shift)
    lut = np.concatenate([W_.sam_entry_table()] * 2)[:C]  # C <= 4 channels of entry codes
    lo_b, hi_b = TA.sam_patch_bytes(CO, C, KH, KW)
    lo = torch.empty(lo_b, dtype=torch.int8, device="cuda")
    hi = torch.empty(hi_b, dtype=torch.int8, device="cuda")
    TA.sam_patch_upload(w, CO, C, KH, KW, lo, hi)
    OH, OW = (H + 2 * P - KH) // S + 1, (W + 2 * P - KW) // S + 1
    out = torch.full((CO * OH * OW,), 77, dtype=torch.int8, device="cuda")
    bd = torch.from_numpy(b).cuda() if bias else None
    TA.sam_patch_embed(torch.from_numpy(img).cuda(), torch.from_numpy(np.ascontiguousarray(lut)).cuda(), C, H, W, lo,
                       hi, CO, KH, KW, S, P, bd, torch.from_numpy(mant).cuda(), torch.from_numpy(shift).cuda(), out)
    torch.cuda.synchronize()
    q = O.sam_entry(img, C, H * W, lut)
    want, _ = O.conv2d(q, C, H, W, w.astype(np.int16), CO, KH, KW, S, P, b if bias else None, mant, shift)
    got = out.cpu().numpy()
    assert np.array_equal(got, want), f"patch embed differs at {np.flatnonzero(got != want)[:5]}"
    return got


def test_patch_embed_small(torch_dev):
    run_conv(torch_dev, 3, 70, 70, 40, 7, 7, 4, 3)


def test_patch_embed_ragged_segments_and_channel_tiles(torch_dev):
    """OW = 130 (a full and a 2-wide row segment), 150 output channels (two channel tiles, the second partial)."""
    run_conv(torch_dev, 3, 33, 517, 150, 7, 7, 4, 3, seeds=(64, 65, 66))


def test_patch_embed_other_kernels(torch_dev):
    """A 3x3 stride-1 conv over 4 channels (k = 36, one k tile; four phase copies of each staged row) and a 5x5
    stride-2 conv without bias (k = 75; two copies)."""
    run_conv(torch_dev, 4, 20, 260, 24, 3, 3, 1, 1, seeds=(67, 68, 69))
    run_conv(torch_dev, 2, 31, 45, 8, 5, 5, 2, 0, seeds=(70, 71, 72), bias=False)


def test_patch_embed_wide_and_strided_kernels(torch_dev):
    """A 9x9 stride-3 conv (taps padded to 12: three dwords per kernel row, four copies; k = 162 over 2 channels,
    byte loads since w % 4 != 0) and a ViT-style 16x16 stride-16 patchify (one dword-aligned copy, k = 256)."""
    run_conv(torch_dev, 2, 40, 66, 20, 9, 9, 3, 4, seeds=(73, 74, 75))
    run_conv(torch_dev, 1, 64, 320, 36, 16, 16, 16, 0, seeds=(76, 77, 78))


def test_patch_embed_negative_and_edge_scales(torch_dev):
    """The requant epilogue's sign and clamp: every other channel's multiplier negated (the double path with both
    signs), then every pairing of edge multipliers and shifts, first those the double path takes (shift -200 .. 33,
    saturating ones included), then all of them (waves whose channels mix the double and the integer path)."""
    from test_oracle import EDGE_MANT, EDGE_SHIFT

    def negate_odd(mant, shift):
        mant = mant.copy()
        mant[1::2] = -mant[1::2]
        return mant, shift

    def edges(shifts):
        pairs = [(m, s) for m in EDGE_MANT for s in shifts]
        return len(pairs), lambda mant, shift: (np.array([p[0] for p in pairs], np.int32),
                                                np.array([p[1] for p in pairs], np.int32))

    run_conv(torch_dev, 3, 70, 70, 40, 7, 7, 4, 3, seeds=(79, 80, 81), scales=negate_odd)
    for shifts in ([s for s in EDGE_SHIFT if -512 <= s <= 46], EDGE_SHIFT):
        co, f = edges(shifts)
        run_conv(torch_dev, 3, 40, 64, co, 7, 7, 4, 3, seeds=(82, 83, 84), scales=f)


def test_patch_weights_device_pack_equals_upload(torch_dev):
    """kt_hip_sam_patch_pack (device codes) writes the same two planes as kt_hip_sam_patch_upload (host codes): codes
    at both ends of the range, tap widths padded by 1, 3 and 0, partial column blocks and k tiles."""
    import tritify_amd as TA

    torch = torch_dev
    rng = np.random.default_rng(91)
    for co, ci, kh, kw in [(40, 3, 7, 7), (20, 2, 9, 9), (8, 1, 16, 16), (33, 4, 3, 1)]:
        say(f"case: patch weight planes co={co} ci={ci} k={kh}x{kw}")
        w = rng.integers(-2048, 2048, size=co * ci * kh * kw).astype(np.int32)
        w[:4] = [-2048, 2047, 0, -1]
        lo_b, hi_b = TA.sam_patch_bytes(co, ci, kh, kw)
        planes = []
        for dev_pack in (False, True):
            lo = torch.full((lo_b,), 55, dtype=torch.int8, device="cuda")
            hi = torch.full((hi_b,), 55, dtype=torch.int8, device="cuda")
            if dev_pack:
                TA.sam_patch_pack(torch.from_numpy(w).cuda(), co, ci, kh, kw, lo, hi)
            else:
                TA.sam_patch_upload(w, co, ci, kh, kw, lo, hi)
            torch.cuda.synchronize()
            planes.append((lo.cpu().numpy(), hi.cpu().numpy()))
        assert np.array_equal(planes[0][0], planes[1][0]) and np.array_equal(planes[0][1], planes[1][1])
        # every code is lo + 256 hi with hi in [-8, 8]; the planes hold co * ci * kh * kw codes (the pad taps, rows
        # and k are zero) and their sum of codes equals the weights'
        lo8, hi8 = planes[0][0].astype(np.int64), planes[0][1].astype(np.int64)
        assert hi8.min() >= -8 and hi8.max() <= 8
        assert (lo8 + 256 * hi8).sum() == w.astype(np.int64).sum()
    with pytest.raises(RuntimeError):  # a code out of range: refused before any upload
        TA.sam_patch_upload(np.full(8 * 3 * 3 * 3, 2048, np.int32), 8, 3, 3, 3, lo, hi)


def test_patch_weight_layout_rejects_wide_kernels(torch_dev):
    """kw > 16 and ci * kh * kwp > 256 have no patch-embed layout; the entry rejects them before any launch."""
    import tritify_amd as TA

    with pytest.raises(ValueError):
        TA.sam_patch_bytes(8, 3, 3, 17)
    lo = torch_dev.zeros(1 << 16, dtype=torch_dev.int8, device="cuda")
    hi = torch_dev.zeros(1 << 16, dtype=torch_dev.int8, device="cuda")
    out = torch_dev.zeros(64, dtype=torch_dev.int8, device="cuda")
    img = torch_dev.zeros(3 * 32 * 32, dtype=torch_dev.uint8, device="cuda")
    lut = torch_dev.zeros(3 * 256, dtype=torch_dev.int8, device="cuda")
    sc = torch_dev.zeros(8, dtype=torch_dev.int32, device="cuda")
    with pytest.raises(RuntimeError):  # 3 * 9 * 12 = 324 > 256
        TA.sam_patch_embed(img, lut, 3, 32, 32, lo, hi, 8, 9, 9, 4, 0, None, sc, sc, out)


def run_mlp(torch, tokens, dim, hidden, seeds=(81, 82, 83)):
    import tritify_amd as TA
    from tritify_amd import workloads as W_

    say(f"case: sam mlp tokens={tokens} dim={dim} hidden={hidden}")
    x, wi, wo, im, is_, om, os_ = W_.sam_mlp_inputs(tokens, dim, hidden, *seeds)
    gelu = W_.gelu_table()
    lo_i = [torch.empty(n, dtype=dt, device="cuda") for n, dt in zip(TA.w12_bytes(hidden, dim), (torch.int8, torch.uint8))]
    lo_o = [torch.empty(n, dtype=dt, device="cuda") for n, dt in zip(TA.w12_bytes(dim, hidden), (torch.int8, torch.uint8))]
    TA.w12_upload(wi, hidden, dim, *lo_i)
    TA.w12_upload(wo, dim, hidden, *lo_o)
    kp_d, kp_h = TA.kp(dim), TA.kp(hidden)
    xp = np.zeros((tokens, kp_d), np.int8)
    xp[:, :dim] = x.reshape(tokens, dim)
    h = torch.zeros((tokens, kp_h), dtype=torch.int8, device="cuda")
    y = torch.empty(tokens * dim, dtype=torch.int8, device="cuda")
    hh = torch.empty(tokens * hidden, dtype=torch.int8, device="cuda")
    TA.w12_linear_lut(torch.from_numpy(xp).cuda(), *lo_i, tokens, hidden, dim, hh, torch.from_numpy(im).cuda(),
                      torch.from_numpy(is_).cuda(), torch.from_numpy(gelu).cuda())
    h[:, :hidden] = hh.view(tokens, hidden)
    TA.w12_linear(h, *lo_o, tokens, dim, hidden, y, TA.OUT_I8, torch.from_numpy(om).cuda(), torch.from_numpy(os_).cuda())
    torch.cuda.synchronize()
    return x, wi, wo, im, is_, om, os_, gelu, hh.cpu().numpy(), y.cpu().numpy()


@pytest.mark.parametrize("tokens,dim,hidden", [(300, 192, 320), (100, 448, 1792), (4, 64, 96)])
def test_sam_mlp_against_oracle(torch_dev, tokens, dim, hidden):
    """Both the GEMM path (M > 128) and the skinny path (M <= 128) with the GELU table in the epilogue."""
    x, wi, wo, im, is_, om, os_, gelu, h, y = run_mlp(torch_dev, tokens, dim, hidden)
    hw, yw = O.mlp_gelu(x, tokens, dim, hidden, wi, im, is_, gelu, wo, om, os_)
    assert np.array_equal(h, hw), "proj_in + GELU differs"
    assert np.array_equal(y, yw), "proj_out differs"


def test_sam_full_config5(torch_dev):
    """Config 5 at full size: the 1024 x 1024 x 3 patch embed (M = 65,536, K = 147, N = 112) and the stage-3 MLP
    (4096 tokens, 448 -> 1792 -> 448), against the fixture hashes."""
    import tritify_amd as TA
    from tritify_amd import workloads as W_

    torch = torch_dev
    g5 = GOLD["config5"]
    say("case: sam full config 5")
    img, w, b, mant, shift = W_.sam_patch_inputs(g5["C"], g5["H"], g5["W"], g5["CO"], g5["KH"], g5["KW"],
                                                 g5["img_seed"], g5["pe_seed"], g5["bias_seed"], g5["sigma_q"],
                                                 g5["bias_sigma"])
    lut = W_.sam_entry_table(g5["entry_scale"])
    assert sha(img) == g5["img_sha256"] and sha(lut) == g5["entry_sha256"] and sha(W_.gelu_table()) == g5["gelu_sha256"]
    lo_b, hi_b = TA.sam_patch_bytes(g5["CO"], g5["C"], g5["KH"], g5["KW"])
    lo = torch.empty(lo_b, dtype=torch.int8, device="cuda")
    hi = torch.empty(hi_b, dtype=torch.int8, device="cuda")
    TA.sam_patch_upload(w, g5["CO"], g5["C"], g5["KH"], g5["KW"], lo, hi)
    OH = (g5["H"] + 2 * g5["P"] - g5["KH"]) // g5["S"] + 1
    OW = (g5["W"] + 2 * g5["P"] - g5["KW"]) // g5["S"] + 1
    out = torch.empty(g5["CO"] * OH * OW, dtype=torch.int8, device="cuda")
    TA.sam_patch_embed(torch.from_numpy(img).cuda(), torch.from_numpy(lut).cuda(), g5["C"], g5["H"], g5["W"], lo, hi,
                       g5["CO"], g5["KH"], g5["KW"], g5["S"], g5["P"], torch.from_numpy(b).cuda(),
                       torch.from_numpy(mant).cuda(), torch.from_numpy(shift).cuda(), out)
    torch.cuda.synchronize()
    assert sha(out.cpu().numpy()) == g5["patch_sha256"], "patch embed differs from the CPU fixture"
    *_, h, y = run_mlp(torch, g5["tokens"], g5["dim"], g5["hidden"],
                       (g5["x_seed"], g5["wi_seed"], g5["wo_seed"]))
    assert sha(h) == g5["mlp_h_sha256"], "stage-3 proj_in + GELU differs from the CPU fixture"
    assert sha(y) == g5["mlp_y_sha256"], "stage-3 proj_out differs from the CPU fixture"
