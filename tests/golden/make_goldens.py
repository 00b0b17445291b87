"""Writes tests/golden/goldens.json: input and output hashes of the benchmark workloads, computed by the CPU oracle
(oracle/kt_oracle.c, the restated reference CPU path). The GPU tests compare the device results with these fixtures
at full size, where recomputing the CPU answer inside a test would take too long.

Run from the repository root:  python tests/golden/make_goldens.py [config1 config2 config3 config4 config5
config3_ref]  (config3_ref, the reference-semantics decoder over config 3's 640 positions, only when named)
"""
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import oracle as O  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "goldens.json")

# benchmark config 2 (this build's definitions; see oracle/kt_oracle.c kt_gen_w12 / kt_gen_act_gauss /
# kt_channel_scales): N = K = 4096, M in {1, 16, 128, 2048} taking the first M rows of one 2048-row activation draw.
C2 = {"w_seed": 2, "x_seed": 3, "sigma": 40, "N": 4096, "K": 4096, "Ms": [1, 16, 128, 2048]}

# benchmark config 4 (this build's integer MoE layer, include/kt_hip.h): GLM-4.5-Air shape.
C4 = {"T": 4096, "H": 4096, "F": 1408, "E": 128, "top_k": 8, "x_seed": 41, "r_seed": 42, "w_seed": 4000,
      "sigma_x": 40, "sigma_r": 1024, "sigma_h": 16, "h_shift": 8, "out_shift": 13}

# benchmark config 5 (this build's integer definition of the SAM 2.1 Hiera-B+ encoder GEMMs, include/kt_hip.h).
C5 = {"C": 3, "H": 1024, "W": 1024, "CO": 112, "KH": 7, "KW": 7, "S": 4, "P": 3, "tokens": 4096, "dim": 448,
      "hidden": 1792, "img_seed": 51, "pe_seed": 52, "bias_seed": 53, "x_seed": 54, "wi_seed": 55, "wo_seed": 56,
      "entry_scale": 48, "sigma_q": 61, "bias_sigma": 131072, "sigma_x": 40, "sigma_h": 24}


def config5() -> dict:
    """The oracle's direct conv (the reference's loop order) on the entry codes of the full image, and the stage-3
    MLP; inputs from the oracle's generators, tables from the workload definitions."""
    from tritify_amd import workloads as W

    c = dict(C5)
    C, H, Wd, CO, KH, KW = c["C"], c["H"], c["W"], c["CO"], c["KH"], c["KW"]
    img = O.gen_uniform(c["img_seed"], 0, 255, C * H * Wd).astype(np.uint8)
    lut = W.sam_entry_table(c["entry_scale"])
    k = C * KH * KW
    w = O.gen_w12_i16(c["pe_seed"], CO * k)
    b = O.gen_gauss_i32(c["bias_seed"], c["bias_sigma"], CO)
    mant, shift = O.channel_scales_i16(w, CO, k, c["sigma_q"])
    t = time.time()
    q = O.sam_entry(img, C, H * Wd, lut)
    out, _ = O.conv2d(q, C, H, Wd, w, CO, KH, KW, c["S"], c["P"], b, mant, shift)
    print(f"config5 patch embed: {time.time() - t:.1f}s", flush=True)
    T, D, Dh = c["tokens"], c["dim"], c["hidden"]
    x = O.gen_act_gauss(c["x_seed"], c["sigma_x"], T * D)
    wi = O.gen_w12_i16(c["wi_seed"], Dh * D)
    wo = O.gen_w12_i16(c["wo_seed"], D * Dh)
    im, is_ = O.channel_scales_i16(wi, Dh, D, c["sigma_x"])
    om, os_ = O.channel_scales_i16(wo, D, Dh, c["sigma_h"])
    h, y = O.mlp_gelu(x, T, D, Dh, wi, im, is_, W.gelu_table(), wo, om, os_)
    c.update({
        "img_sha256": O.sha256_hex(img), "entry_sha256": O.sha256_hex(lut), "gelu_sha256": O.sha256_hex(W.gelu_table()),
        "patch_sha256": O.sha256_hex(out), "mlp_h_sha256": O.sha256_hex(h), "mlp_y_sha256": O.sha256_hex(y),
        "patch_absmean": float(np.abs(out.astype(np.int32)).mean()),
        "mlp_y_absmean": float(np.abs(y.astype(np.int32)).mean()),
    })
    return c


# benchmark config 3 (this build's integer decoder, include/kt_hip.h): Qwen2.5-0.5B shape.
C3 = {"d": 896, "ffn": 4864, "nh": 14, "nkv": 2, "hd": 64, "layers": 24, "vocab": 151936, "prompt": 512,
      "max_new": 129, "w_seed": 3000, "prompt_seed": 3001, "h_shift": 8}


def config3() -> dict:
    """The oracle decoder (the reference's generate_greedy_by loop with a batched prefill) on the full shape: weights
    from the oracle's generators, tables from the workload definitions; the logits of all 129 steps hashed."""
    from tritify_amd import workloads as W

    c = dict(C3)
    d, ffn, nh, nkv, hd, L, V = (c[k] for k in ("d", "ffn", "nh", "nkv", "hd", "layers", "vocab"))
    nq, nhd, max_pos = (nh + 2 * nkv) * hd, nh * hd, c["prompt"] + c["max_new"]
    t = time.time()
    a = {k: [] for k in ("wqkv", "qkv_mant", "qkv_shift", "wo", "o_mant", "o_shift", "wgu", "gu_mant", "gu_shift",
                         "wd", "d_mant", "d_shift")}
    for l in range(L):
        for j, (name, n, k, key) in enumerate((("qkv", nq, d, "qkv"), ("o", d, nhd, "o"), ("gu", 2 * ffn, d, "gu"),
                                               ("dn", d, ffn, "d"))):
            w = O.gen_quant_rows(c["w_seed"] + 8 * l + j, n, k)
            sig, tgt = W.DEC_SCALES[name]
            ms = O.channel_scales_target(w, n, k, sig, tgt)
            a[{"qkv": "wqkv", "o": "wo", "gu": "wgu", "d": "wd"}[key]].append(w)
            a[key + "_mant"].append(ms[0])
            a[key + "_shift"].append(ms[1])
    arrays = {k: np.concatenate(v) for k, v in a.items()}
    emb = O.gen_quant_rows(c["w_seed"] - 1, V, d)
    sig, tgt = W.DEC_SCALES["lm"]
    arrays["emb"] = emb
    arrays["lm_mant"], arrays["lm_shift"] = O.channel_scales_target(emb, V, d, sig, tgt)
    arrays["rope_cos"], arrays["rope_sin"] = W.rope_tables(max_pos, hd)
    arrays["exp_tab"], arrays["silu"] = W.exp_table(), W.silu_table()
    print(f"config3 weights: {time.time() - t:.1f}s", flush=True)
    prompt = O.gen_uniform(c["prompt_seed"], 0, V - 1, c["prompt"])
    t = time.time()
    toks, logits = O.dec_generate(dict(c, max_pos=max_pos), arrays, prompt, c["max_new"])
    print(f"config3 generate: {time.time() - t:.1f}s", flush=True)
    c.update({"prompt_sha256": O.sha256_hex(prompt), "tokens": [int(v) for v in toks],
              "logits_sha256": O.sha256_hex(logits), "rope_sha256": O.sha256_hex(arrays["rope_cos"]),
              "exp_sha256": O.sha256_hex(arrays["exp_tab"])})
    return c


def config4() -> dict:
    """The expert-major oracle (kt_moe_layer) on the full config-4 layer: weights from the oracle's own generator
    (kt_gen_w12_i16, the kt_gen_w12 stream), tables from the workload definitions."""
    from tritify_amd import workloads as W

    c = dict(C4)
    T, H, F, E, K = c["T"], c["H"], c["F"], c["E"], c["top_k"]
    x = O.gen_act_gauss(c["x_seed"], c["sigma_x"], T * H)
    r = O.gen_gauss_i32(c["r_seed"], c["sigma_r"], T * E)
    silu, sig = W.silu_table(), W.sigmoid_table()
    G = E + 1
    wgu = np.empty((G, 2 * F * H), np.int16)
    wd = np.empty((G, H * F), np.int16)
    gm = np.empty((G, 2 * F), np.int32)
    gs = np.empty((G, 2 * F), np.int32)
    dm = np.empty((G, H), np.int32)
    ds = np.empty((G, H), np.int32)
    for g in range(G):
        wgu[g] = O.gen_w12_i16(c["w_seed"] + 2 * g, 2 * F * H)
        wd[g] = O.gen_w12_i16(c["w_seed"] + 2 * g + 1, H * F)
        gm[g], gs[g] = O.channel_scales_i16(wgu[g], 2 * F, H, c["sigma_x"])
        dm[g], ds[g] = O.channel_scales_i16(wd[g], H, F, c["sigma_h"])
    t = time.time()
    res = O.moe_layer(x, r, T, H, F, E, K, wgu, wd, gm, gs, dm, ds, silu, sig, c["h_shift"], c["out_shift"])
    print(f"config4 layer: {time.time() - t:.1f}s", flush=True)
    c.update({
        "x_sha256": O.sha256_hex(x), "logits_sha256": O.sha256_hex(r),
        "silu_sha256": O.sha256_hex(silu), "sig_sha256": O.sha256_hex(sig),
        "sel_sha256": O.sha256_hex(res["sel"]), "cw_sha256": O.sha256_hex(res["cw"]),
        "count": [int(v) for v in res["count"]],
        "h_sha256": O.sha256_hex(res["h"]), "d_sha256": O.sha256_hex(res["d"]), "out_sha256": O.sha256_hex(res["out"]),
        "out_absmean": float(np.abs(res["out"].astype(np.int32)).mean()),
        "out_saturated": int((np.abs(res["out"].astype(np.int32)) == 127).sum()),
    })
    return c


def main() -> None:
    """Recompute the configs named on the command line (config1 config2 config4 config5; none = all) and keep the
    other entries of the existing file."""
    t0 = time.time()
    want = set(sys.argv[1:]) or {"config1", "config2", "config3", "config4", "config5"}
    g = json.load(open(OUT)) if os.path.exists(OUT) else {}
    if "config1" in want:
        qx, qw = O.gen_demo(64, 1024, 1024, 42)
        y = O.linear_cpu(qx, qw, 64, 1024, 1024)
        g["config1"] = {
            "M": 64, "N": 1024, "K": 1024, "seed": 42,
            "x_sha256": O.sha256_hex(qx), "w_sha256": O.sha256_hex(qw),
            "y_i64_sha256": O.sha256_hex(y), "y_i32_sha256": O.sha256_hex(y.astype(np.int32)),
        }
        cs = O.corpus()
        g["corpus_sha256"] = O.sha256_hex(np.concatenate([O.linear_cpu(c.x, c.w, c.rows, c.out, c.k) for c in cs]))
    if "config2" in want:
        g["config2"] = config2()
    if "config3" in want:
        g["config3"] = config3()
    if "config4" in want:
        g["config4"] = config4()
    if "config5" in want:
        g["config5"] = config5()
    if "config3_ref" in want:
        g["config3_ref"] = config3_ref()
    json.dump(g, open(OUT, "w"), indent=1, sort_keys=True)
    print(f"wrote {OUT} in {time.time() - t0:.1f}s")


def config2() -> dict:
    N, K = C2["N"], C2["K"]
    w = O.gen_w12(C2["w_seed"], N * K)
    x = O.gen_act_gauss(C2["x_seed"], C2["sigma"], max(C2["Ms"]) * K)
    mant, shift = O.channel_scales(w, N, K, C2["sigma"])
    c2 = dict(C2)
    c2.update({
        "w_sha256": O.sha256_hex(w), "x_sha256": O.sha256_hex(x),
        "mant_sha256": O.sha256_hex(mant), "shift_sha256": O.sha256_hex(shift), "outputs": {},
    })
    for m in C2["Ms"]:
        t = time.time()
        acc = O.linear_cpu(x[: m * K], w, m, N, K)
        q = O.requant_channels(acc, m, N, mant, shift, -127, 127).astype(np.int8)
        c2["outputs"][str(m)] = {
            "x_sha256": O.sha256_hex(x[: m * K]),
            "acc_i64_sha256": O.sha256_hex(acc),
            "out_i8_sha256": O.sha256_hex(q),
            "acc_absmax": int(np.abs(acc).max()),
            "out_i8_saturated": int((np.abs(q.astype(np.int32)) == 127).sum()),
        }
        print(f"config2 M={m}: {time.time() - t:.1f}s", flush=True)
    return c2


def config3_ref() -> dict:
    """Config 3 at the reference's own semantics: the oracle's restatement of DecoderModel (kt_oracle_refdec.c) at
    the Qwen2.5-0.5B shape over the weights of tritify_amd.workloads.ref_decoder_weights, repro::run of a 512-token
    prompt (every prompt token through decode_step, generate.rs:82-93) and 128 greedy steps: the logits_hash of
    each of the 640 positions, the run's hash and the chosen tokens. Not in the default set (minutes of CPU)."""
    from tritify_amd import workloads as W

    cfg, rc = W.REF_QWEN, W.REF_C3
    t = time.time()
    model = O.RefModel.from_weights(cfg, *W.ref_decoder_weights(cfg, rc["w_seed"]))
    prompt = W.ref_c3_prompt(cfg)
    print(f"config3_ref: model built in {time.time() - t:.1f}s", flush=True)
    O.set_max_threads(0)
    t = time.time()
    toks, run, pos = model.generate(prompt, rc["decode"] + 1)
    print(f"config3_ref: {len(pos)} positions in {time.time() - t:.1f}s", flush=True)
    return {"cfg": cfg, "w_seed": rc["w_seed"], "prompt_seed": rc["prompt_seed"], "prompt": len(prompt),
            "decode": rc["decode"], "prompt_sha256": O.sha256_hex(np.asarray(prompt, dtype=np.int32)),
            "tokens": toks, "run_sha256": run, "position_sha256": pos}


if __name__ == "__main__":
    main()
