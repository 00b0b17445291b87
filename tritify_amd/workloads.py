"""Synthetic inputs of the benchmark workloads, integer-only and identical on every machine.

The stream is the reference's LCG, s <- s*6364136223846793005 + 1442695040888963407 mod 2^64
(apps/kt-demo/src/main.rs:19-22), drawn as (s >> 33). It is evaluated here in numpy: a first block step by step,
then the sequence doubles, each new half the affine map s -> A*s + C (mod 2^64) of the half before it.

- gen_demo: the kt-demo generator (main.rs:23-28), benchmark config 1.
- gen_w12 / gen_act_gauss / channel_scales: benchmark config 2 (this build's definitions): 12-bit weight codes
  uniform in [-2048, 2047]; activations round(N(0, sigma)) clipped to +-127, N(0,1) drawn as an Irwin-Hall sum of
  12 16-bit uniforms; per-channel int32 requant scales mapping 4 standard deviations of a channel's accumulator to
  127 (crates/00-kernels/kt-int/src/lib.rs:191-212 for the fixed-point ratio).
"""
from __future__ import annotations

import math

import numpy as np

LCG_A = 6364136223846793005
LCG_C = 1442695040888963407
M64 = (1 << 64) - 1
_BLOCK = 1 << 10


def lcg_states(seed: int, n: int) -> np.ndarray:
    """The n states after `seed` (the value lcg() returns on each of n calls). The first block is stepped; then,
    holding `have` states and the affine map (A, C) of `have` steps, the next `have` states are A*out[i] + C."""
    out = np.empty(n, dtype=np.uint64)
    if n == 0:
        return out
    first = min(n, _BLOCK)
    s, a, c = seed & M64, 1, 0
    head = []
    for _ in range(first):
        s = (s * LCG_A + LCG_C) & M64
        a, c = (a * LCG_A) & M64, (c * LCG_A + LCG_C) & M64
        head.append(s)
    out[:first] = np.array(head, dtype=np.uint64)
    have = first
    with np.errstate(over="ignore"):
        while have < n:
            take = min(have, n - have)
            dst = out[have:have + take]
            np.multiply(out[:take], np.uint64(a), out=dst)
            np.add(dst, np.uint64(c), out=dst)
            a, c = (a * a) & M64, (a * c + c) & M64
            have += take
    return out


def _draws(seed: int, n: int) -> np.ndarray:
    st = lcg_states(seed, n)
    np.right_shift(st, np.uint64(33), out=st)
    return st.view(np.int64)


def gen_demo(m: int, n: int, k: int, seed: int = 42):
    """kt-demo: qx (m*k in [-127,127]) then qw (n*k in {-1,0,1}) from one stream (main.rs:23-28)."""
    d = _draws(seed ^ 0x9E3779B97F4A7C15, m * k + n * k)
    qx = (d[: m * k] % 255 - 127).astype(np.int32)
    qw = (d[m * k:] % 3 - 1).astype(np.int32)
    return qx, qw


def gen_w12(seed: int, n: int) -> np.ndarray:
    """n codes uniform in [-2048, 2047] on the stream seed ^ 0x9E3779B97F4A7C15."""
    d = _draws(seed ^ 0x9E3779B97F4A7C15, n)
    np.bitwise_and(d, 4095, out=d)  # % 4096 of a non-negative draw
    np.subtract(d, 2048, out=d)
    return d.astype(np.int32)


def gen_act_gauss(seed: int, sigma: int, n: int) -> np.ndarray:
    """n activations round_half_away(N(0, sigma)) clipped to +-127 on the stream seed ^ 0xD1B54A32D192ED03:
    t = 2 * (sum of 12 draws & 0xFFFF) - 12 * 65535, x = sign(t) * ((|t| * sigma + 2^16) >> 17)."""
    out = np.empty(n, dtype=np.int32)
    chunk = 1 << 20
    s = (seed ^ 0xD1B54A32D192ED03) & M64
    done = 0
    while done < n:
        cnt = min(chunk, n - done)
        st = lcg_states(s, 12 * cnt)
        s = int(st[-1])
        np.right_shift(st, np.uint64(33), out=st)
        u = st.view(np.int64)
        np.bitwise_and(u, 0xFFFF, out=u)
        t = 2 * u.reshape(cnt, 12).sum(axis=1) - 12 * 65535
        mag = (np.abs(t) * sigma + 65536) >> 17
        v = np.where(t < 0, -mag, mag)
        out[done:done + cnt] = np.clip(v, -127, 127)
        done += cnt
    return out


def _bits(x: int) -> int:
    return x.bit_length()


def scale_from_ratio(num: int, den: int) -> tuple[int, int]:
    """kt_int::Scale::from_ratio (crates/00-kernels/kt-int/src/lib.rs:191-212): (mant, shift), mant ~31 bits."""
    if num == 0:
        return 0, 0
    while _bits(num) > 64 or _bits(den) > 64:
        num >>= 1
        den >>= 1
    den = max(den, 1)
    s = 31 - (_bits(num) - _bits(den))
    if s >= 0:
        mant = ((num << s) + den // 2) // den
    else:
        dd = den << (-s)
        mant = (num + dd // 2) // dd
    return mant, s


def scale_to_i32(mant: int, shift: int) -> tuple[int, int]:
    """An int32 multiplier: halve the mantissa with rounding (lowering the shift) until it is below 2^31."""
    while mant >= 1 << 31:
        mant = (mant + 1) >> 1
        shift -= 1
    return mant, shift


def channel_scales(w: np.ndarray, n: int, k: int, sigma: int = 40):
    """Per output channel: scale = to_i32(from_ratio(127, 4 * sigma * isqrt(sum_k w^2)))."""
    ss = (w.reshape(n, k).astype(np.int64) ** 2).sum(axis=1)
    mant = np.zeros(n, dtype=np.int32)
    shift = np.zeros(n, dtype=np.int32)
    for o in range(n):
        root = math.isqrt(int(ss[o]))
        if root == 0:
            continue
        m, s = scale_to_i32(*scale_from_ratio(127, 4 * sigma * root))
        mant[o], shift[o] = m, s
    return mant, shift


def pad_k(x: np.ndarray, m: int, k: int) -> np.ndarray:
    """int8 activations m x k -> m x kp (kp = k rounded up to 64), zero padded: the device operand layout."""
    kp = (k + 63) // 64 * 64
    out = np.zeros((m, kp), dtype=np.int8)
    out[:, :k] = x.reshape(m, k)
    return out


# ---------------------------------------------------------------------------------------------------------------
# Config 4: one MoE layer, GLM-4.5-Air shape (this build's integer definition; include/kt_hip.h states the rule)

MOE_FULL = dict(T=4096, H=4096, F=1408, E=128, top_k=8)
MOE_SEEDS = dict(x_seed=41, r_seed=42, w_seed=4000)
MOE_CONST = dict(sigma_x=40, sigma_r=1024, sigma_h=16, h_shift=8, out_shift=13)


def _round_half_away(v: float) -> int:
    return int(math.floor(abs(v) + 0.5)) * (1 if v >= 0 else -1)


def silu_table() -> np.ndarray:
    """255 int16 SiLU codes: t[i] = round(256 * v * sigmoid(v)), v = (i - 127) / 32 (int8 code q <-> q / 32), the
    integer-code SiLU of SwiGluMlp (crates/01-engine/kt-core/src/layers.rs:599) on this build's int8 grid."""
    return np.array([_round_half_away(256.0 * ((i - 127) / 32.0) / (1.0 + math.exp(-(i - 127) / 32.0)))
                     for i in range(255)], dtype=np.int16)


def sigmoid_table() -> np.ndarray:
    """255 int16 router weight codes: t[i] = round(4096 * sigmoid((i - 127) / 64)); a router code r (N(0,1) in units
    of 1/1024) reads entry clamp(round(r / 16), -127, 127) + 127 (GLM-4.5's sigmoid score, router.rs:29-79)."""
    return np.array([_round_half_away(4096.0 / (1.0 + math.exp(-(i - 127) / 64.0))) for i in range(255)],
                    dtype=np.int16)


def moe_inputs(T: int, H: int, E: int, x_seed: int, r_seed: int, sigma_x: int = 40, sigma_r: int = 1024):
    """x (T x H int8 as int32, round(N(0, sigma_x)) clipped to +-127) and router codes (T x E int32, round(N(0,
    sigma_r)) unclipped)."""
    from . import backend as B

    return B.gen_gauss_fast(x_seed, sigma_x, T * H, clip=127), B.gen_gauss_fast(r_seed, sigma_r, T * E)


def moe_expert(g: int, H: int, F: int, w_seed: int, sigma_x: int = 40, sigma_h: int = 16):
    """Expert g's codes and scales: gate/up (2F x H, gate rows first) from seed w_seed + 2g, down (H x F) from
    w_seed + 2g + 1; per-channel scales map 4 standard deviations of the accumulator to 127 (sigma_x for gate/up,
    sigma_h for down)."""
    from . import backend as B

    gu = B.gen_w12_fast(w_seed + 2 * g, 2 * F * H)
    dn = B.gen_w12_fast(w_seed + 2 * g + 1, H * F)
    gm, gs = B.channel_scales_fast(gu, 2 * F, H, sigma_x)
    dm, ds = B.channel_scales_fast(dn, H, F, sigma_h)
    return gu, dn, gm, gs, dm, ds


# ---------------------------------------------------------------------------------------------------------------
# Config 5: SAM 2.1 Hiera-B+ image-encoder GEMMs (this build's integer definition; include/kt_hip.h states the rule)

SAM_FULL = dict(C=3, H=1024, W=1024, CO=112, KH=7, KW=7, S=4, P=3, tokens=4096, dim=448, hidden=1792)
SAM_SEEDS = dict(img_seed=51, pe_seed=52, bias_seed=53, x_seed=54, wi_seed=55, wo_seed=56)
SAM_CONST = dict(entry_scale=48, sigma_q=61, bias_sigma=131072, sigma_x=40, sigma_h=24)
IMAGENET_MEAN = (0.485, 0.456, 0.406)  # crates/03-models/kt-model-vision/src/preprocess.rs:6-7
IMAGENET_STD = (0.229, 0.224, 0.225)


def sam_entry_table(scale: int = 48) -> np.ndarray:
    """3 x 256 int8 entry codes: t[c][p] = clamp(round(scale * (p / 255 - mean_c) / std_c), -127, 127), the ImageNet
    normalization of preprocess.rs and the entry quantization of plugin.rs:38 as one table per channel."""
    t = np.empty((3, 256), dtype=np.int8)
    for c in range(3):
        for p in range(256):
            v = _round_half_away(scale * (p / 255.0 - IMAGENET_MEAN[c]) / IMAGENET_STD[c])
            t[c, p] = max(-127, min(127, v))
    return t


def gelu_table() -> np.ndarray:
    """255 int8 GELU codes: t[i] = clamp(round(32 * gelu(v)), -127, 127), v = (i - 127) / 32, gelu(v) =
    v (1 + erf(v / sqrt 2)) / 2 (apply_gelu of crates/03-models/kt-model-vision/src/nonlin.rs:30-47 on the int8 grid)."""
    out = np.empty(255, dtype=np.int8)
    for i in range(255):
        v = (i - 127) / 32.0
        out[i] = max(-127, min(127, _round_half_away(32.0 * 0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0))))))
    return out


def sam_patch_inputs(C: int, H: int, W: int, CO: int, KH: int, KW: int, img_seed: int, pe_seed: int, bias_seed: int,
                     sigma_q: int = 61, bias_sigma: int = 131072):
    """The image (C x H x W u8, uniform), the patch-embed codes (CO x C*KH*KW, k ordered (ic, ky, kx)), its bias
    (CO int32, round(N(0, bias_sigma))) and per-channel scales (4 sigma of the accumulator at entry-code sigma_q)."""
    from . import backend as B

    img = B.gen_uniform_fast(img_seed, 0, 255, C * H * W).astype(np.uint8)
    k = C * KH * KW
    w = B.gen_w12_fast(pe_seed, CO * k)
    bias = B.gen_gauss_fast(bias_seed, bias_sigma, CO)
    mant, shift = B.channel_scales_fast(w, CO, k, sigma_q)
    return img, w, bias, mant, shift


def sam_mlp_inputs(tokens: int, dim: int, hidden: int, x_seed: int, wi_seed: int, wo_seed: int, sigma_x: int = 40,
                   sigma_h: int = 24):
    """Stage-3 MLP: tokens (tokens x dim int8, round(N(0, sigma_x)) clipped), proj_in (hidden x dim codes) and
    proj_out (dim x hidden codes) with their per-channel scales."""
    from . import backend as B

    x = B.gen_gauss_fast(x_seed, sigma_x, tokens * dim, clip=127)
    wi = B.gen_w12_fast(wi_seed, hidden * dim)
    wo = B.gen_w12_fast(wo_seed, dim * hidden)
    im, is_ = B.channel_scales_fast(wi, hidden, dim, sigma_x)
    om, os_ = B.channel_scales_fast(wo, dim, hidden, sigma_h)
    return x, wi, wo, im, is_, om, os_


# ---------------------------------------------------------------------------------------------------------------
# Config 3: a Qwen2.5-0.5B-shape decoder (this build's integer definition; include/kt_hip.h states the rules)

DEC_FULL = dict(d=896, ffn=4864, nh=14, nkv=2, hd=64, layers=24, vocab=151936)
DEC_RUN = dict(prompt=512, max_new=129, w_seed=3000, prompt_seed=3001, h_shift=8)
# per-channel scale rule of each projection: (sigma of its int8 input, the value 4 sigma of the accumulator maps to)
DEC_SCALES = dict(qkv=(32, 127), o=(16, 16384), gu=(32, 127), dn=(16, 16384), lm=(32, 1 << 20))


def rope_tables(max_pos: int, hd: int = 64, theta: float = 1.0e6):
    """int16 cos / sin tables [max_pos][hd / 2] at 2^14: round(2^14 cos(p theta^(-2i / hd))) (Qwen2's rotary
    embedding, rope_theta = 1e6)."""
    hh = hd // 2
    cos = np.empty((max_pos, hh), dtype=np.int16)
    sin = np.empty((max_pos, hh), dtype=np.int16)
    for i in range(hh):
        f = theta ** (-2.0 * i / hd)
        for p in range(max_pos):
            a = p * f
            cos[p, i] = _round_half_away(16384.0 * math.cos(a))
            sin[p, i] = _round_half_away(16384.0 * math.sin(a))
    return cos, sin


def exp_table() -> np.ndarray:
    """1024 int32 softmax weights: round(2^15 exp(-i / 64)); a score gap of m - s (q and k at 32 codes per unit, so
    m - s = 8192 per unit of logit / sqrt(64)) reads entry (m - s + 64) >> 7."""
    return np.array([_round_half_away(32768.0 * math.exp(-i / 64.0)) for i in range(1024)], dtype=np.int32)


def decoder_layer_codes(l: int, cfg: dict, w_seed: int):
    """Layer l's codes (per-row quantized Gaussians) and per-channel scales: qkv, o, gate/up (gate rows first), down."""
    from . import backend as B

    d, ffn, nq, nhd = cfg["d"], cfg["ffn"], (cfg["nh"] + 2 * cfg["nkv"]) * cfg["hd"], cfg["nh"] * cfg["hd"]
    out = []
    for j, (name, n, k) in enumerate((("qkv", nq, d), ("o", d, nhd), ("gu", 2 * ffn, d), ("dn", d, ffn))):
        w = B.gen_quant_rows_fast(w_seed + 8 * l + j, n, k)
        sig, tgt = DEC_SCALES[name]
        out += [w, B.channel_scales_fast(w, n, k, sig, tgt)]
    return out


def decoder_embedding_codes(cfg: dict, w_seed: int):
    """The tied embedding / lm_head codes (vocab x d) and the lm_head's per-row scales."""
    from . import backend as B

    w = B.gen_quant_rows_fast(w_seed - 1, cfg["vocab"], cfg["d"])
    sig, tgt = DEC_SCALES["lm"]
    return w, B.channel_scales_fast(w, cfg["vocab"], cfg["d"], sig, tgt)


def decoder_prompt(seed: int, n: int, vocab: int) -> np.ndarray:
    """n token ids uniform in [0, vocab)."""
    from . import backend as B

    return B.gen_uniform_fast(seed, 0, vocab - 1, n)


# The reference decoder at its own semantics (tritify_amd/refdecoder.py) at the Qwen2.5-0.5B shape: 12-trit weight
# codes, config 3's run (a 512-token prompt fed through decode_step, generate.rs:82-93, then 128 greedy steps:
# 640 positions).
WLEVELS = 265720
REF_QWEN = dict(dim=896, layers=24, nh=14, nkv=2, hd=64, hidden=4864, vocab=151936, eps=1e-6, theta=1.0e6,
                max_seq=640)
REF_C3 = dict(w_seed=0x5EED, prompt_seed=3001, prompt=512, decode=128)


def ref_decoder_weights(cfg: dict, seed: int):
    """Codes and Scales of a reference decoder of shape cfg, as RefDecoder's constructor takes them: every weight,
    gamma and embedding code uniform in +-WLEVELS at Scale(1 / WLEVELS) (floats of peak 1), from the LCG seeded
    seed + 1, seed + 2, ... in the order embedding-free layers first: per layer in_norm, post_norm, wq, wk, wv, wo,
    gate, up, down; then the embedding, the final norm and the lm_head."""
    from . import backend as B

    sc = B.ref_scale_from_f64(1.0 / WLEVELS)
    d, qd, kvd, h, V = cfg["dim"], cfg["nh"] * cfg["hd"], cfg["nkv"] * cfg["hd"], cfg["hidden"], cfg["vocab"]
    state = [seed]

    def codes(*shape):
        state[0] += 1
        return B.gen_uniform_fast(state[0], -WLEVELS, WLEVELS, int(np.prod(shape))).reshape(shape)

    layers = []
    for _ in range(cfg["layers"]):
        layers.append({"in_norm": (codes(d), sc), "post_norm": (codes(d), sc), "wq": (codes(qd, d), sc),
                       "wk": (codes(kvd, d), sc), "wv": (codes(kvd, d), sc), "wo": (codes(d, qd), sc),
                       "gate": (codes(h, d), sc), "up": (codes(h, d), sc), "down": (codes(d, h), sc)})
    return (codes(V, d), sc), (codes(d), sc), (codes(V, d), sc), layers


def ref_c3_prompt(cfg: dict = REF_QWEN) -> list:
    """Config 3's 512 prompt token ids (uniform over the vocabulary) for the reference-semantics decoder."""
    return decoder_prompt(REF_C3["prompt_seed"], REF_C3["prompt"], cfg["vocab"]).astype(int).tolist()

