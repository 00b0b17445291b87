"""Parity of the config-3 decoder (Qwen2.5-0.5B shape) on the MI355X with the CPU oracle, through the C ABI. Run on
a GPU box with -m gpu.

The GPU path (tritify_amd.decoder: embed, RmsNorm, q/k/v W12 GEMM, RoPE + KV cache, integer attention, o GEMM into
the residual, SwiGLU gate/up GEMM, down GEMM into the residual, lm_head, greedy argmax on the device) is compared
with the oracle's decoder (kt_dec_generate, the reference's DecoderModel / generate_greedy_by loop,
crates/01-engine/kt-core/src/model.rs:290-353, generate.rs:82-111): every step's logits and token byte for byte on
a small model, eager and as a replayed HIP graph, and at the full benchmark shape (512-token prefill, 128 greedy
decode steps) against the fixture's logits hash.
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


def build(cfg, w_seed, max_pos, max_rows, h_shift=8):
    """The GPU model from the product's generators, and the same arrays for the oracle."""
    from tritify_amd import workloads as W
    from tritify_amd.decoder import DecoderModel

    m = DecoderModel(cfg, max_pos, max_rows, h_shift)
    a = {k: [] for k in ("wqkv", "qkv_mant", "qkv_shift", "wo", "o_mant", "o_shift", "wgu", "gu_mant", "gu_shift",
                         "wd", "d_mant", "d_shift")}
    for l in range(cfg["layers"]):
        wqkv, qms, wo, oms, wgu, gms, wd, dms = W.decoder_layer_codes(l, cfg, w_seed)
        m.set_layer(l, wqkv, qms, wo, oms, wgu, gms, wd, dms)
        for key, w, ms in (("qkv", wqkv, qms), ("o", wo, oms), ("gu", wgu, gms), ("d", wd, dms)):
            a[{"qkv": "wqkv", "o": "wo", "gu": "wgu", "d": "wd"}[key]].append(w.astype(np.int16))
            a[key + "_mant"].append(ms[0])
            a[key + "_shift"].append(ms[1])
    arrays = {k: np.concatenate(v) for k, v in a.items()}
    emb, lms = W.decoder_embedding_codes(cfg, w_seed)
    m.set_embedding(emb, lms)
    cos, sin = W.rope_tables(max_pos, cfg["hd"])
    m.set_tables(cos, sin, W.exp_table(), W.silu_table())
    arrays.update(emb=emb.astype(np.int16), lm_mant=lms[0], lm_shift=lms[1], rope_cos=cos, rope_sin=sin,
                  exp_tab=W.exp_table(), silu=W.silu_table())
    return m, arrays


SMALL = dict(d=128, ffn=256, nh=4, nkv=2, hd=64, layers=2, vocab=1000)


@pytest.mark.parametrize("graph", [False, True])
def test_decoder_small_against_oracle(torch_dev, graph):
    from tritify_amd import workloads as W

    say(f"case: decoder small {SMALL} prompt 37, 9 tokens, graph={graph}")
    m, arrays = build(SMALL, 500, 64, 64)
    prompt = W.decoder_prompt(501, 37, SMALL["vocab"])
    toks, logits = m.generate(prompt, 9, graph=graph)
    shape = dict(SMALL, max_pos=64, h_shift=8)
    wt, wl = O.dec_generate(shape, arrays, prompt, 9)
    assert np.array_equal(logits.reshape(-1), wl), "logits differ from the oracle"
    assert np.array_equal(toks, wt)


def test_decoder_prompt_of_one_and_ragged_heads(torch_dev):
    """A one-token prompt (prefill is a decode step) and 6 query heads over 3 kv heads."""
    from tritify_amd import workloads as W

    cfg = dict(d=192, ffn=128, nh=6, nkv=3, hd=64, layers=1, vocab=300)
    say(f"case: decoder {cfg} prompt 1, 5 tokens")
    m, arrays = build(cfg, 600, 16, 8)
    prompt = W.decoder_prompt(601, 1, cfg["vocab"])
    toks, logits = m.generate(prompt, 5)
    wt, wl = O.dec_generate(dict(cfg, max_pos=16, h_shift=8), arrays, prompt, 5)
    assert np.array_equal(logits.reshape(-1), wl) and np.array_equal(toks, wt)


def test_decoder_full_config3(torch_dev):
    """benchmark config 3: Qwen2.5-0.5B shape, 512-token prefill, 128 greedy decode steps (129 hashed logit rows),
    decode steps replayed from one captured HIP graph."""
    from tritify_amd import workloads as W

    g3 = GOLD["config3"]
    cfg = {k: g3[k] for k in ("d", "ffn", "nh", "nkv", "hd", "layers", "vocab")}
    say(f"case: decoder full config 3 {cfg}")
    m, _ = build_full(cfg, g3)
    prompt = W.decoder_prompt(g3["prompt_seed"], g3["prompt"], cfg["vocab"])
    assert sha(prompt) == g3["prompt_sha256"]
    toks, logits = m.generate(prompt, g3["max_new"], graph=True)
    assert toks.tolist() == g3["tokens"], "generated tokens differ from the CPU fixture"
    assert sha(logits) == g3["logits_sha256"], "the logits hash differs from the CPU fixture"


def build_full(cfg, g3):
    from tritify_amd import workloads as W
    from tritify_amd.decoder import DecoderModel

    max_pos = g3["prompt"] + g3["max_new"]
    m = DecoderModel(cfg, max_pos, g3["prompt"], g3["h_shift"])
    for l in range(cfg["layers"]):
        m.set_layer(l, *W.decoder_layer_codes(l, cfg, g3["w_seed"]))
    m.set_embedding(*W.decoder_embedding_codes(cfg, g3["w_seed"]))
    cos, sin = W.rope_tables(max_pos, cfg["hd"])
    m.set_tables(cos, sin, W.exp_table(), W.silu_table())
    return m, None


@pytest.mark.parametrize("m", [1, 20, 50, 100, 129, 300])
def test_w12_swiglu_every_path(torch_dev, m):
    """The dense SwiGLU gate/up product on each skinny tile count (m <= 16, 32, 64, 128) and on the MFMA tile path,
    against the oracle's GEMM and the SwiGLU rule."""
    import tritify_amd as TA
    from tritify_amd import workloads as W

    torch = torch_dev
    ffn, k = 192, 320
    say(f"case: w12 swiglu m={m} ffn={ffn} k={k}")
    x = W.gen_act_gauss(1300 + m, 40, m * k)
    w = W.gen_w12(1301, 2 * ffn * k)
    mant, shift = W.channel_scales(w, 2 * ffn, k, 40)
    silu = W.silu_table()
    lo_b, nib_b = TA.w12_bytes(2 * ffn, k)
    lo = torch.empty(lo_b, dtype=torch.int8, device="cuda")
    nib = torch.empty(nib_b, dtype=torch.uint8, device="cuda")
    TA.w12_pack_gate_up(torch.from_numpy(w).cuda(), ffn, k, lo, nib)
    y = torch.full((m * (ffn + 16),), 55, dtype=torch.int8, device="cuda")
    TA.w12_swiglu(torch.from_numpy(W.pad_k(x, m, k)).cuda(), lo, nib, m, ffn, k, torch.from_numpy(mant).cuda(),
                  torch.from_numpy(shift).cuda(), torch.from_numpy(silu).cuda(), 8, y, ffn + 16)
    torch.cuda.synchronize()
    _, gu = O.gemm_i8w16(x.astype(np.int8), w.astype(np.int16), m, 2 * ffn, k, mant, shift)
    gu = gu.reshape(m, 2 * ffn).astype(np.int64)
    hv = silu.astype(np.int64)[gu[:, :ffn] + 127] * gu[:, ffn:]
    want = np.clip(np.sign(hv) * ((np.abs(hv) + 128) >> 8), -127, 127).astype(np.int8)
    got = y.cpu().numpy().reshape(m, ffn + 16)
    assert np.array_equal(got[:, :ffn], want), "swiglu differs"
    assert (got[:, ffn:] == 55).all(), "wrote past the row"


def rmsnorm_rows_py(r: np.ndarray, d: int) -> np.ndarray:
    """The decoder's RMSNorm in Python integers (the rule of kt_oracle_layers.c's kt_dec_rmsnorm_rows)."""
    import math

    out = np.zeros(r.shape, dtype=np.int8)
    for t, row in enumerate(r.astype(np.int64)):
        ss = int(sum(int(v) * int(v) for v in row))  # exact: the full-range row sums past 2^64
        rms = math.isqrt(ss // d)
        for i, v in enumerate(row):
            if rms:
                a = 32 * int(v)
                q = (2 * abs(a) + rms) // (2 * rms)
                out[t, i] = max(-127, min(127, -q if a < 0 else q))
    return out


@pytest.mark.parametrize("m,d", [(1, 896), (1, 200), (5, 64), (16, 320)])
def test_w12_norm_fused_products(torch_dev, m, d):
    """kt_hip_w12_linear_norm (I64, I32, I8) and kt_hip_w12_swiglu_norm against the RMSNorm rule in Python integers
    followed by the oracle's GEMM; residual rows with large, small and all-zero values."""
    import tritify_amd as TA
    from tritify_amd import workloads as W

    torch = torch_dev
    say(f"case: norm-fused products m={m} d={d}")
    rng = np.random.default_rng(m * 1000 + d)
    r = rng.integers(-(2**20), 2**20, size=(m, d)).astype(np.int32)
    if m > 1:
        r[1] = 0  # rms = 0: the row quantizes to zeros
    if m > 2:
        r[2] = rng.integers(-(2**31) + 1, 2**31 - 1, size=d).astype(np.int32)  # sum of squares past 2^64
    q = rmsnorm_rows_py(r, d)
    rd = torch.from_numpy(r.reshape(-1)).cuda()
    n = 200
    w = W.gen_w12(2000 + d, n * d)
    mant, shift = W.channel_scales(w, n, d, 40)
    lo_b, nib_b = TA.w12_bytes(n, d)
    lo = torch.empty(lo_b, dtype=torch.int8, device="cuda")
    nib = torch.empty(nib_b, dtype=torch.uint8, device="cuda")
    TA.w12_upload(w, n, d, lo, nib)
    md, sd = torch.from_numpy(mant).cuda(), torch.from_numpy(shift).cuda()
    acc, y8 = O.gemm_i8w16(q.reshape(-1), w.astype(np.int16), m, n, d, mant, shift)
    y64 = torch.empty(m * n, dtype=torch.int64, device="cuda")
    y32 = torch.empty(m * n, dtype=torch.int32, device="cuda")
    yi8 = torch.empty(m * n, dtype=torch.int8, device="cuda")
    TA.w12_linear_norm(rd, lo, nib, m, n, d, y64, TA.OUT_I64)
    TA.w12_linear_norm(rd, lo, nib, m, n, d, y32, TA.OUT_I32, md, sd)
    TA.w12_linear_norm(rd, lo, nib, m, n, d, yi8, TA.OUT_I8, md, sd)
    torch.cuda.synchronize()
    assert np.array_equal(y64.cpu().numpy(), acc), "i64 accumulators differ"
    assert np.array_equal(yi8.cpu().numpy(), y8), "int8 outputs differ"
    want32 = np.array([O.requant_sat(int(a), int(mant[i % n]), int(shift[i % n])) for i, a in enumerate(acc)])
    assert np.array_equal(y32.cpu().numpy().astype(np.int64), np.clip(want32, -(2**31), 2**31 - 1))

    ffn = 128
    wg = W.gen_w12(3000 + d, 2 * ffn * d)
    gm, gs = W.channel_scales(wg, 2 * ffn, d, 40)
    glo_b, gnib_b = TA.w12_bytes(2 * ffn, d)
    glo = torch.empty(glo_b, dtype=torch.int8, device="cuda")
    gnib = torch.empty(gnib_b, dtype=torch.uint8, device="cuda")
    TA.w12_pack_gate_up(torch.from_numpy(wg).cuda(), ffn, d, glo, gnib)
    silu = W.silu_table()
    h = torch.full((m * (ffn + 8),), 55, dtype=torch.int8, device="cuda")
    TA.w12_swiglu_norm(rd, glo, gnib, m, ffn, d, torch.from_numpy(gm).cuda(), torch.from_numpy(gs).cuda(),
                       torch.from_numpy(silu).cuda(), 8, h, ffn + 8)
    torch.cuda.synchronize()
    _, gu = O.gemm_i8w16(q.reshape(-1), wg.astype(np.int16), m, 2 * ffn, d, gm, gs)
    gu = gu.reshape(m, 2 * ffn).astype(np.int64)
    hv = silu.astype(np.int64)[gu[:, :ffn] + 127] * gu[:, ffn:]
    want = np.clip(np.sign(hv) * ((np.abs(hv) + 128) >> 8), -127, 127).astype(np.int8)
    got = h.cpu().numpy().reshape(m, ffn + 8)
    assert np.array_equal(got[:, :ffn], want), "swiglu (norm) differs"
    assert (got[:, ffn:] == 55).all(), "wrote past the row"


@pytest.mark.parametrize("fuse", [False, True])
def test_decoder_long_context_step(torch_dev, fuse):
    """Decode steps beyond the attention kernel's two prefetched chunks (positions past 1024, read in its loop),
    both RMSNorm placements and the output projection inside or after the attention kernel, against the oracle."""
    from tritify_amd import workloads as W

    cfg = dict(d=64, ffn=64, nh=2, nkv=1, hd=64, layers=1, vocab=97)
    say(f"case: decoder long context {cfg} prompt 1100, 4 tokens, fuse={fuse}")
    m, arrays = build(cfg, 700, 1104, 1100)
    m.fuse_norm = m.fuse_norm_head = m.fuse_o = fuse
    prompt = W.decoder_prompt(701, 1100, cfg["vocab"])
    toks, logits = m.generate(prompt, 4, graph=fuse)
    wt, wl = O.dec_generate(dict(cfg, max_pos=1104, h_shift=8), arrays, prompt, 4)
    assert np.array_equal(logits.reshape(-1), wl) and np.array_equal(toks, wt)


@pytest.mark.parametrize("ffn", [192, 1500, 4864])
def test_fold_o_entry_points_saturate(torch_dev, ffn):
    """The decode step's o-projection fold through the C ABI against the unfused integers: kt_hip_w12_linear_add_o
    adds the requantized o sums into the residual and then its own requantized product, each addition saturating
    (residual entries at the int32 limits, o sums at both signs), and clears the accumulator; twice in a row on
    one accumulator, the second call's sums added on the device to what the first call left (so the cleared state
    is what the next step starts from). ffn 192, 1500 and 4864 reach the kernel's three builds (8 waves x 2 pairs,
    x 4 pairs, 16 waves x 5 pairs). (The gate/up side of the fold is covered by the decoder runs against the
    oracle.)"""
    import tritify_amd as T

    torch = torch_dev
    lib, P = T.lib(), T.backend._ptr
    s = torch.cuda.current_stream().cuda_stream
    d = 128
    rng = np.random.default_rng(77 + ffn)
    w_dn = rng.integers(-2048, 2048, size=d * ffn).astype(np.int32)
    dm, dsh = O.channel_scales(w_dn, d, ffn, 40)
    om = rng.integers(1 << 29, 1 << 30, size=d).astype(np.int32)
    osh = rng.integers(20, 30, size=d).astype(np.int32)
    lo_dn, nib_dn = T.w12_bytes(d, ffn)
    lo_d = torch.empty(lo_dn, dtype=torch.int8, device="cuda")
    nib_d = torch.empty(nib_dn, dtype=torch.uint8, device="cuda")
    T.w12_upload(w_dn, d, ffn, lo_d, nib_d)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    acc_d = torch.zeros(d, dtype=torch.int32, device="cuda")
    for call in range(2):
        r = rng.integers(-(2**31), 2**31, size=d, dtype=np.int64).astype(np.int32)
        r[:4] = [2**31 - 1, -(2**31), 2**31 - 5, -(2**31) + 5]
        acc = rng.integers(-(2**28), 2**28, size=d).astype(np.int32)
        acc[:4] = [2**28, -(2**28), 2**28, -(2**28)]
        h = rng.integers(-127, 128, size=ffn).astype(np.int8)
        ro = np.clip(r.astype(np.int64) + O.requant_channels(acc, 1, d, om, osh, -(2**31), 2**31 - 1),
                     -(2**31), 2**31 - 1)
        dot = O.linear_threads(h.astype(np.int32), w_dn, 1, d, ffn, 1, O.lib().kt_cpu_auto_variant())
        want = np.clip(ro + O.requant_channels(dot, 1, d, dm, dsh, -(2**31), 2**31 - 1), -(2**31), 2**31 - 1)
        say(f"case: fold-o down d={d} ffn={ffn} call {call}")
        if call == 0:
            acc_d.copy_(dev(acc))
        else:  # onto what the first call left: equal to acc only if that is zero everywhere
            acc_d.add_(dev(acc))
        r_d = dev(r)
        h_d = torch.zeros(T.kp(ffn), dtype=torch.int8, device="cuda")
        h_d[:ffn] = dev(h)
        om_d, osh_d, dm_d, dsh_d = dev(om), dev(osh), dev(dm), dev(dsh)
        T.backend.check(lib.kt_hip_w12_linear_add_o(0, P(h_d), P(lo_d), P(nib_d), d, ffn, P(dm_d), P(dsh_d),
                                                    P(r_d),
                                                    P(acc_d), P(om_d), P(osh_d), s), "w12 linear add o")
        torch.cuda.synchronize()
        assert np.array_equal(r_d.cpu().numpy(), want.astype(np.int32)), call
        assert int(acc_d.count_nonzero().item()) == 0, "the accumulator is cleared"
