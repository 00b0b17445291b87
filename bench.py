#!/usr/bin/env python3
"""Benchmark of the MI355X exact-integer GEMM backend on the benchmark workloads, one GPU.

Headline (`value`): config 2, the exact 12-bit GEMM at M = 2048, N = K = 4096 -- int8 activations (round(N(0,40))
clipped to +-127) against 12-bit weight codes (as the benchmark describes them, two int8 digit planes: the balanced
W12B split, lo in [-128, 127] and hi in [-8, 8], 2 bytes per weight; the packed 1.5-byte W12 planes are timed
beside it), int32 accumulation per digit plane, exact recombination, then the per-channel integer requant (int32
multiplier + shift) to int8 outputs. A step is one launch. Inputs are resident in HBM before the timed region; the
weights rotate over 12 copies (> 256 MB) so no launch finds them in the Infinity Cache. Every configuration's result is checked byte for byte against the fixture
hashes the CPU oracle produced (tests/golden/goldens.json) before anything is timed.

Also measured, each under "configs" (skip with --configs):
  3  a Qwen2.5-0.5B-shape decoder: 512-token prefill, then 128 greedy decode steps replayed from one captured HIP
     graph -- decode tokens/s (the benchmark's second metric), prefill tokens/s, the weight bandwidth of a decode step.
  4  one MoE layer, GLM-4.5-Air shape (4096 tokens, H 4096, 128 experts top-8 + 1 shared, F 1408): route, bucket,
     the ragged grouped W12 GEMMs (gate/up with the SwiGLU epilogue, down), combine; per-stage times.
  5  SAM 2.1 Hiera-B+ encoder GEMMs: the 1024 x 1024 x 3 patch embed as an im2col-fused W12 GEMM (M 65,536, K 147,
     N 112) and the stage-3 MLP (4096 tokens, 448 -> 1792 with the GELU table -> 448).
  ql the reference's own QuantLinear::forward_int on the device (dynamic per-tensor quantization around the digit
     GEMM) at the config-3 projection shapes, with the digit GEMM timed alone beside it.
  lb the LinearBackend trait path (host buffers in, i64 out) on cuda_bench's shapes.
  ref the reference's own integer semantics end to end: its DecoderModel at the Qwen2.5-0.5B shape (decode tokens/s
     from one captured graph per position, every position's logits hash checked against the oracle, whose run is
     the CPU baseline), and SAM's PatchEmbed Conv2d and a stage-3 FeedForward.

Prints one JSON line on stdout (progress goes to stderr):
  value      logical effective TOPS = 2*M*N*K / time per step (one launch per step)
  roofline   the dominant kernel (w12_gemm_dma on the W12B planes at M = 2048) against the dense int8 MFMA peak
             (5.0 POPS)
  sweep      config 2, M in {1, 16, 128, 2048}: per-launch time, effective TOPS, algorithmic GB/s, roofline fractions
  cpu_baseline  the reference's multithreaded CPU integer path (the oracle's restatement of linear_cpu, AVX-512
             variant when the host has it) on the same M = 2048 workload, timed on this host's cores

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--configs 2,3,4,5,ql,lb,ref]
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA
ROTATE = 12  # weight copies cycled per launch: 12 x 25.2 MB > the 256 MB Infinity Cache


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def gold() -> dict:
    return json.load(open(os.path.join(ROOT, "tests", "golden", "goldens.json")))


def time_launches(torch, launch, n: int, warmup: int):
    """Time n back-to-back launches between two HIP events recorded on the launching stream (the stream the kernel
    runs on). Returns the mean launch duration (ms) and the host wall time of the n launches (s)."""
    stream = torch.cuda.current_stream()
    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(n):
        launch(i)
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return start.elapsed_time(end) / n, wall


def cpu_threads() -> int:
    cores = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    return max(1, min(cores, os.cpu_count() or 1))


def cpu_baseline(x32: np.ndarray, w32: np.ndarray, m: int, n: int, k: int) -> dict:
    """The reference's CPU path (crates/01-engine/kt-core/src/backend.rs:133-140 on the auto dot variant,
    kt-runtime/src/lib.rs:93-96), timed as cuda_bench does (one untimed call, then >= 2 calls and >= 5 s)."""
    from oracle import oracle as O

    cores = cpu_threads()
    O.set_max_threads(cores)
    variant = O.lib().kt_cpu_auto_variant()
    O.linear_cpu(x32, w32, m, n, k, variant)
    reps, t0 = 0, time.perf_counter()
    while reps < 2 or time.perf_counter() - t0 < 5.0:
        O.linear_cpu(x32, w32, m, n, k, variant)
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    return {
        "value": round(2.0 * m * n * k / dt / 1e12, 4),
        "unit": "TOPS",
        "cores": cores,
        "nproc": os.cpu_count(),
        "kind": "port",
        "sample": f"config 2 at M={m}, N={n}, K={k} (i32 codes in, i64 out; the whole workload), "
                  f"{reps} timed calls after one warm call, {dt * 1e3:.1f} ms/call, dot variant "
                  f"{['portable', 'avx2', 'avx512'][variant]}, threads capped at {cores}",
    }


# ---------------------------------------------------------------------------------------------------------------
# config 2: the 12-bit GEMM sweep


def bench_config2(torch, args) -> tuple[dict, tuple, np.ndarray, np.ndarray]:
    import tritify_amd as T
    from tritify_amd import workloads as W

    g2 = gold()["config2"]
    N, K, sigma = g2["N"], g2["K"], g2["sigma"]
    Ms = g2["Ms"]
    MH = max(Ms)
    if args.ms:
        Ms = [int(v) for v in args.ms.split(",")]
        assert all(str(m) in g2["outputs"] for m in Ms), "--ms takes values of the config-2 sweep"
    dev = torch.device("cuda:0")

    log("bench: generating config-2 inputs")
    w = W.gen_w12(g2["w_seed"], N * K)
    x = W.gen_act_gauss(g2["x_seed"], sigma, MH * K)
    mant, shift = W.channel_scales(w, N, K, sigma)
    assert sha(w) == g2["w_sha256"] and sha(x) == g2["x_sha256"], "synthetic inputs differ from the fixtures"
    assert sha(mant) == g2["mant_sha256"] and sha(shift) == g2["shift_sha256"]

    nlo, nnib = T.w12_bytes(N, K)
    lo0 = torch.empty(nlo, dtype=torch.int8, device=dev)
    nib0 = torch.empty(nnib, dtype=torch.uint8, device=dev)
    T.w12_upload(w, N, K, lo0, nib0)
    los = [lo0] + [lo0.clone() for _ in range(ROTATE - 1)]
    nibs = [nib0] + [nib0.clone() for _ in range(ROTATE - 1)]
    # the MFMA-bound M = 2048 product on the balanced two-plane weights (W12B: no nibble unpack, no row sums)
    nb = T.w12b_bytes(N, K)
    blo0 = torch.empty(nb, dtype=torch.int8, device=dev)
    bhi0 = torch.empty(nb, dtype=torch.int8, device=dev)
    T.w12b_pack(torch.from_numpy(w).to(dev), N, K, blo0, bhi0)
    blos = [blo0] + [blo0.clone() for _ in range(ROTATE - 1)]
    bhis = [bhi0] + [bhi0.clone() for _ in range(ROTATE - 1)]
    xd = torch.from_numpy(W.pad_k(x, MH, K)).to(dev)
    md, sd = torch.from_numpy(mant).to(dev), torch.from_numpy(shift).to(dev)
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()

    def big(m):  # the products timed on the W12B planes
        return m > 128

    # every M's result is checked first; the timings then run back to back with no host work between them, the
    # headline M last, so the GPU is busy (and its clocks up) when the headline's own warmup starts
    outs = {}
    for m in Ms:
        want = g2["outputs"][str(m)]
        y8 = torch.empty(m * N, dtype=torch.int8, device=dev)
        acc = torch.empty(m * N, dtype=torch.int64, device=dev)
        for planes in (("w12",) + (("w12b",) if big(m) else ())):
            acc.zero_(), y8.zero_()
            if planes == "w12":
                T.w12_linear(xd, lo0, nib0, m, N, K, acc, T.OUT_I64, stream=stream)
                T.w12_linear(xd, lo0, nib0, m, N, K, y8, T.OUT_I8, md, sd, stream=stream)
            else:
                T.w12b_linear(xd, blo0, bhi0, m, N, K, acc, T.OUT_I64, stream=stream)
                T.w12b_linear(xd, blo0, bhi0, m, N, K, y8, T.OUT_I8, md, sd, stream=stream)
            torch.cuda.synchronize()
            exact = sha(acc.cpu().numpy()) == want["acc_i64_sha256"] and sha(y8.cpu().numpy()) == want["out_i8_sha256"]
            if not exact:
                raise SystemExit(f"bench: config 2 M={m} ({planes}): the GPU result differs from the CPU fixture")
            log(f"bench: config 2 M={m} ({planes}): bit-exact vs the CPU fixture")
        del acc
        outs[m] = y8

    sweep = {}
    headline = None
    order = [m for m in Ms if m != MH] + ([MH] if MH in Ms else [])
    for m in order:
        y8 = outs[m]

        def launch(i, m=m, y8=y8):
            j = i % ROTATE
            if big(m):
                T.w12b_linear(xd, blos[j], bhis[j], m, N, K, y8, T.OUT_I8, md, sd, stream=stream)
            else:
                T.w12_linear(xd, los[j], nibs[j], m, N, K, y8, T.OUT_I8, md, sd, stream=stream)

        n_launch = args.steps if m == MH else max(args.steps, 1000)
        warm = args.warmup if m == MH else max(args.warmup, 100)
        log(f"bench: config 2 M={m}: timing {n_launch} launches after {warm} warmup launches")
        ms, wall = time_launches(torch, launch, n_launch, warm)
        us = ms * 1e3
        ops = 2.0 * m * N * K
        # weights as stored (1.5 B per weight packed W12; 2 B as the two W12B planes) + int8 activations + int8 out
        bytes_alg = (2.0 if big(m) else 1.5) * N * K + m * K + m * N * 1
        tops = ops / (us * 1e-6) / 1e12
        gbs = bytes_alg / (us * 1e-6) / 1e9
        sweep[str(m)] = {
            "us_per_launch": round(us, 3),
            "effective_tops": round(tops, 2),
            "executed_int8_tops": round(2 * tops, 2),
            "mfma_frac_logical": round(tops / INT8_PEAK_TOPS, 4),
            "alg_gbs": round(gbs, 1),
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "bit_exact": True,
            "kernel": "w12_skinny" if m <= 128 else "w12_gemm_dma on the W12B planes",
            "launches": n_launch, "warmup_launches": warm,
        }
        if m == 1:
            # the read floor of the same bytes: kt_hip_stream_read (the GEMV's 16-byte load form, no compute) over
            # each weight copy's two planes as one contiguous buffer, the same rotation and launch count
            flat = [torch.cat([los[j], nibs[j].view(torch.int8)]) for j in range(ROTATE)]
            xo = torch.empty(T.backend.STREAM_READ_CTAS, dtype=torch.int32, device=dev)
            ms_r, _ = time_launches(torch, lambda i: T.backend.stream_read(flat[i % ROTATE], flat[0].numel(), xo,
                                                                           stream=stream), n_launch, warm)
            sweep[str(m)]["read_floor_us"] = round(ms_r * 1e3, 3)
            sweep[str(m)]["read_floor"] = (f"kt_hip_stream_read of the {flat[0].numel() / 1e6:.1f} MB of one W12 "
                                           f"weight copy (both planes), {ROTATE} copies rotated, timed as this GEMV")
            del flat
        if m == MH:
            headline = (ms, wall, n_launch, warm, us, tops)
            # the same kernel once its clocks have settled under its own load (not the headline value)
            ms_s, _ = time_launches(torch, launch, 1000, 500)
            sweep[str(m)]["settled_us_per_launch"] = round(ms_s * 1e3, 3)
            sweep[str(m)]["settled_effective_tops"] = round(ops / (ms_s * 1e-3) / 1e12, 2)
            sweep[str(m)]["settled_launches"] = "1000 after 500 warmup launches, right after the headline timing"

            # the same product on the packed W12 planes (1.5 B per weight), for comparison
            def launch_w12(i, m=m, y8=y8):
                j = i % ROTATE
                T.w12_linear(xd, los[j], nibs[j], m, N, K, y8, T.OUT_I8, md, sd, stream=stream)

            ms_p, _ = time_launches(torch, launch_w12, 1000, 500)
            sweep[str(m)]["w12_planes_us_per_launch"] = round(ms_p * 1e3, 3)
            sweep[str(m)]["w12_planes_effective_tops"] = round(ops / (ms_p * 1e-3) / 1e12, 2)
    del los, nibs, blos, bhis
    return sweep, headline, x, w


# ---------------------------------------------------------------------------------------------------------------
# ql: the reference's own QuantLinear::forward_int (dynamic per-tensor quantization around the digit GEMM)

QL_SHAPES = [("prefill gate/up", 512, 896, 4864, False), ("prefill q (bias)", 512, 896, 896, True),
             ("prefill down", 512, 4864, 896, False), ("decode gate/up", 1, 896, 4864, False)]
QL_ROTATE = 24  # weight copies cycled per step: 24 x 13 MB of digit planes > the 256 MB Infinity Cache


def bench_quant_linear(torch, args) -> dict:
    """The device QuantLinear::forward_int (layers.rs:275-328) on the config-3 projection shapes, 12-trit codes:
    x at the 2^28 activation level, weights in +-WLEVELS (3 digit planes each), checked against the oracle's
    restatement before timing. The digit GEMM is timed beside it as the LinearBackend entry runs it (one k range per
    CTA); inside the call, shapes whose tiles leave CUs idle split k across CTAs instead, so for those the call can
    take less than this figure plus the passes around it."""
    import tritify_amd as T
    from oracle import oracle as O

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    xs, ws, bs = (1509949440, 58), (1657624235, 49), (1318646415, 57)
    res = {"workload": "QuantLinear::forward_int (xmax, quant_to, 3x3-plane digit GEMM, bias, ymax, requant_dyn), "
                       "config-3 projection shapes, 12-trit weights, 2^28-level activations", "shapes": {}}
    for idx, (name, rows, inp, out, with_bias) in enumerate(QL_SHAPES):
        x = T.gen_uniform_fast(700 + idx, -(1 << 28), 1 << 28, rows * inp)
        w = T.gen_uniform_fast(800 + idx, -265720, 265720, out * inp)
        b = T.gen_uniform_fast(900 + idx, -(1 << 28), 1 << 28, out).astype(np.int64) if with_bias else None
        ql = T.QuantLinear(name, w, out, inp, ws, None if b is None else (b, bs))
        y, sc = ql.forward_int_host(x, xs)
        yo, so, _, ymax = O.quant_linear_forward(x, rows, inp, xs, w, out, ws, bias=b, bs=bs)
        if not (np.array_equal(y, yo) and (sc["mant"], sc["shift"]) == so and sc["ymax"] == ymax):
            raise SystemExit(f"bench: quant_linear {name}: the GPU result differs from the CPU oracle")
        planes = [ql.w_planes] + [ql.w_planes.clone() for _ in range(QL_ROTATE - 1)]
        xd = torch.from_numpy(x).to(dev)
        xsd = T.qscale_record(*xs)
        yd = torch.empty(rows * out, dtype=torch.int32, device=dev)
        osd = torch.zeros(4, dtype=torch.int64, device=dev)
        wsb, n = ql.workspace(rows)
        _, off = T.quant_linear_workspace(rows, inp, out)
        torch.cuda.synchronize()

        def launch(i):
            T.quant_linear(xd, rows, inp, xsd, planes[i % QL_ROTATE], ql.pw, out, ws, ql.bias, ql.b_scale, wsb, n,
                           yd, osd, stream=stream)

        def gemm(i):
            T.digit_gemm(wsb[off[0]:], 3, planes[i % QL_ROTATE], ql.pw, wsb[off[1]:], rows, out, inp, stream=stream)

        steps = max(args.steps // 2, 50)
        log(f"bench: quant_linear {name}: bit-exact vs the CPU oracle; timing {steps} steps")
        ms, _ = time_launches(torch, launch, steps, 10)
        ms_g, _ = time_launches(torch, gemm, steps, 10)
        ops = 2.0 * rows * inp * out
        wbytes = 3 * out * T.kp(inp)
        res["shapes"][name] = {
            "rows": rows, "in": inp, "out": out, "bit_exact": True,
            "us": round(ms * 1e3, 2), "digit_gemm_alone_us": round(ms_g * 1e3, 2),
            "effective_tops": round(ops / (ms * 1e-3) / 1e12, 2),
            "gemm_executed_int8_tops": round(9 * ops / (ms_g * 1e-3) / 1e12, 2),
            "weight_plane_gbs": round(wbytes / (ms_g * 1e-3) / 1e9, 1),
        }
        del planes
        if name == QL_SHAPES[0][0] and not args.no_cpu:
            cores = cpu_threads()
            O.set_max_threads(cores)
            O.quant_linear_forward(x, rows, inp, xs, w, out, ws, threads=cores)
            reps, t0 = 0, time.perf_counter()
            while reps < 2 or time.perf_counter() - t0 < 3.0:
                O.quant_linear_forward(x, rows, inp, xs, w, out, ws, threads=cores)
                reps += 1
            dt = (time.perf_counter() - t0) / reps
            res["cpu_baseline"] = {
                "value": round(dt * 1e6, 1), "unit": "us per forward_int", "cores": cores, "kind": "port",
                "sample": f"the oracle's restatement of forward_int (host xmax, quant_to, threaded linear_cpu, "
                          f"ymax, requant_dyn) on {name} {rows}x{inp}->{out}, {reps} calls",
            }
    return res


# ---------------------------------------------------------------------------------------------------------------
# config 4: one MoE layer


def bench_config4(torch, args) -> dict:
    import tritify_amd as T
    from tritify_amd import workloads as W
    from tritify_amd.moe import MoeLayer

    g4 = gold()["config4"]
    Tk, H, F, E, K = g4["T"], g4["H"], g4["F"], g4["E"], g4["top_k"]
    log(f"bench: config 4: generating and packing {E} + 1 experts (H={H}, F={F})")
    t0 = time.perf_counter()
    x, r = W.moe_inputs(Tk, H, E, g4["x_seed"], g4["r_seed"], g4["sigma_x"], g4["sigma_r"])
    assert sha(x) == g4["x_sha256"] and sha(r) == g4["logits_sha256"]
    layer = MoeLayer(H, F, E, K, W.silu_table(), W.sigmoid_table(), g4["h_shift"], g4["out_shift"])
    for g in range(E + 1):
        layer.set_expert(g, *W.moe_expert(g, H, F, g4["w_seed"], g4["sigma_x"], g4["sigma_h"]))
    log(f"bench: config 4: weights resident in {time.perf_counter() - t0:.1f}s")
    xd = torch.from_numpy(x.astype(np.int8)).cuda()
    rd = torch.from_numpy(r).cuda()
    out = torch.empty(Tk * H, dtype=torch.int8, device="cuda")
    v = layer.forward(xd, rd, Tk, out)
    torch.cuda.synchronize()
    if sha(out.cpu().numpy()) != g4["out_sha256"] or sha(v["d"].cpu().numpy()[: Tk * (K + 1) * H]) != g4["d_sha256"]:
        raise SystemExit("bench: config 4: the GPU result differs from the CPU fixture")
    log("bench: config 4: bit-exact vs the CPU fixture; timing")

    stream = torch.cuda.current_stream()
    steps = max(5, args.steps // 10)
    ms_layer, _ = time_launches(torch, lambda i: layer.forward(xd, rd, Tk, out, stream=stream), steps, 2)
    # per stage: events between the stage launches of one pass
    P = Tk * (K + 1)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
    stage_ms = np.zeros(4)
    for _ in range(steps):
        ev[0].record(stream)
        layer.route(rd, Tk, v["sel"], v["cw"], stream=stream)
        layer.bucket(v["sel"], Tk, v["list"], v["pos"], v["count"], stream=stream)
        ev[1].record(stream)
        T.w12_grouped_linear(xd, Tk, v["list"], Tk, v["count"], E + 1, P, layer.gu_lo, layer.gu_nib, 2 * F, H,
                             layer.gu_mant, layer.gu_shift, T.EPI_SWIGLU, v["h"], F, silu_dev=layer.silu,
                             h_shift=layer.h_shift, off_dev=v["off"], stream=stream)
        ev[2].record(stream)
        T.w12_grouped_linear(v["h"], P, None, 0, v["count"], E + 1, P, layer.d_lo, layer.d_nib, H, F, layer.d_mant,
                             layer.d_shift, T.EPI_I8, v["d"], H, stream=stream)
        ev[3].record(stream)
        layer.combine(v["d"], v["off"], v["sel"], v["cw"], v["pos"], Tk, out, stream=stream)
        ev[4].record(stream)
        torch.cuda.synchronize()
        stage_ms += [ev[i].elapsed_time(ev[i + 1]) for i in range(4)]
    stage_ms /= steps
    if sha(out.cpu().numpy()) != g4["out_sha256"]:
        raise SystemExit("bench: config 4: the staged run differs from the CPU fixture")
    ops_gu, ops_dn = 2.0 * P * 2 * F * H, 2.0 * P * H * F
    w_gu, w_dn = 1.5 * (E + 1) * 2 * F * H, 1.5 * (E + 1) * H * F

    def kern(ms, ops, wbytes, xbytes, ybytes):
        s = ms * 1e-3
        return {"us": round(ms * 1e3, 1), "effective_tops": round(ops / s / 1e12, 1),
                "mfma_frac_logical": round(ops / s / 1e12 / INT8_PEAK_TOPS, 4),
                "alg_gbs": round((wbytes + xbytes + ybytes) / s / 1e9, 1),
                "hbm_frac": round((wbytes + xbytes + ybytes) / s / 1e9 / HBM_PEAK_GBS, 4)}

    res = {
        "workload": f"config 4: MoE layer, {Tk} tokens, H={H}, {E} experts top-{K} + 1 shared, F={F}, int8 "
                    f"activations, W12 weights ({(w_gu + w_dn) / 1e9:.2f} GB)",
        "bit_exact": True,
        "layer_us": round(ms_layer * 1e3, 1),
        "layer_effective_tops": round((ops_gu + ops_dn) / (ms_layer * 1e-3) / 1e12, 1),
        "tokens_per_s": round(Tk / (ms_layer * 1e-3), 0),
        "stages_us": {"route+bucket": round(stage_ms[0] * 1e3, 1), "gate_up_swiglu": round(stage_ms[1] * 1e3, 1),
                      "down": round(stage_ms[2] * 1e3, 1), "combine": round(stage_ms[3] * 1e3, 1)},
        "w12_grouped_gate_up": kern(stage_ms[1], ops_gu, w_gu, P * H, P * F),
        "w12_grouped_down": kern(stage_ms[2], ops_dn, w_dn, P * F, P * H),
    }
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline_moe(g4, x, r)
    return res


def bench_config5(torch, args) -> dict:
    import tritify_amd as T
    from tritify_amd import workloads as W

    g5 = gold()["config5"]
    C, H, Wd, CO, KH, KW, S, P = (g5[k] for k in ("C", "H", "W", "CO", "KH", "KW", "S", "P"))
    log("bench: config 5: generating the image, patch-embed and stage-3 MLP weights")
    img, w, b, mant, shift = W.sam_patch_inputs(C, H, Wd, CO, KH, KW, g5["img_seed"], g5["pe_seed"],
                                                g5["bias_seed"], g5["sigma_q"], g5["bias_sigma"])
    lut = W.sam_entry_table(g5["entry_scale"])
    assert sha(img) == g5["img_sha256"] and sha(lut) == g5["entry_sha256"]
    k = C * KH * KW
    lo_b, hi_b = T.sam_patch_bytes(CO, C, KH, KW)
    lo = torch.empty(lo_b, dtype=torch.int8, device="cuda")
    hi = torch.empty(hi_b, dtype=torch.int8, device="cuda")
    T.sam_patch_upload(w, CO, C, KH, KW, lo, hi)
    OH, OW = (H + 2 * P - KH) // S + 1, (Wd + 2 * P - KW) // S + 1
    out = torch.empty(CO * OH * OW, dtype=torch.int8, device="cuda")
    imgd, lutd = torch.from_numpy(img).cuda(), torch.from_numpy(lut).cuda()
    bd, md, sd = (torch.from_numpy(a).cuda() for a in (b, mant, shift))
    stream = torch.cuda.current_stream()

    def patch(i):
        T.sam_patch_embed(imgd, lutd, C, H, Wd, lo, hi, CO, KH, KW, S, P, bd, md, sd, out, stream=stream)

    patch(0)
    torch.cuda.synchronize()
    if sha(out.cpu().numpy()) != g5["patch_sha256"]:
        raise SystemExit("bench: config 5: the patch embed differs from the CPU fixture")

    Tk, D, Dh = g5["tokens"], g5["dim"], g5["hidden"]
    x, wi, wo, im, is_, om, os_ = W.sam_mlp_inputs(Tk, D, Dh, g5["x_seed"], g5["wi_seed"], g5["wo_seed"],
                                                   g5["sigma_x"], g5["sigma_h"])
    li = [torch.empty(n, dtype=dt, device="cuda") for n, dt in zip(T.w12_bytes(Dh, D), (torch.int8, torch.uint8))]
    lo_ = [torch.empty(n, dtype=dt, device="cuda") for n, dt in zip(T.w12_bytes(D, Dh), (torch.int8, torch.uint8))]
    T.w12_upload(wi, Dh, D, *li)
    T.w12_upload(wo, D, Dh, *lo_)
    xd = torch.from_numpy(W.pad_k(x, Tk, D)).cuda()
    hd = torch.zeros(Tk * Dh, dtype=torch.int8, device="cuda")
    yd = torch.empty(Tk * D, dtype=torch.int8, device="cuda")
    gelu = torch.from_numpy(W.gelu_table()).cuda()
    imd, isd, omd, osd = (torch.from_numpy(a).cuda() for a in (im, is_, om, os_))

    def mlp_in(i):
        T.w12_linear_lut(xd, *li, Tk, Dh, D, hd, imd, isd, gelu, stream=stream)

    def mlp_out(i):
        T.w12_linear(hd, *lo_, Tk, D, Dh, yd, T.OUT_I8, omd, osd, stream=stream)

    mlp_in(0)
    mlp_out(0)
    torch.cuda.synchronize()
    if sha(hd.cpu().numpy()) != g5["mlp_h_sha256"] or sha(yd.cpu().numpy()) != g5["mlp_y_sha256"]:
        raise SystemExit("bench: config 5: the stage-3 MLP differs from the CPU fixture")
    log("bench: config 5: bit-exact vs the CPU fixtures; timing")
    n = max(50, args.steps)
    ms_p, _ = time_launches(torch, patch, n, 5)
    ms_i, _ = time_launches(torch, mlp_in, n, 5)
    ms_o, _ = time_launches(torch, mlp_out, n, 5)
    M = OH * OW

    def kern(ms, ops, bytes_):
        s = ms * 1e-3
        return {"us": round(ms * 1e3, 2), "effective_tops": round(ops / s / 1e12, 1),
                "mfma_frac_logical": round(ops / s / 1e12 / INT8_PEAK_TOPS, 4),
                "alg_gbs": round(bytes_ / s / 1e9, 1), "hbm_frac": round(bytes_ / s / 1e9 / HBM_PEAK_GBS, 4)}

    return {
        "workload": f"config 5: SAM 2.1 Hiera-B+ encoder GEMMs: {H}x{Wd}x{C} image -> patch embed (im2col GEMM "
                    f"M={M}, K={k}, N={CO}); stage-3 MLP {Tk} tokens {D} -> {Dh} (GELU) -> {D}",
        "bit_exact": True,
        "patch_embed": kern(ms_p, 2.0 * M * k * CO, C * H * Wd + 1.5 * CO * k + CO * M),
        "mlp_in_gelu": kern(ms_i, 2.0 * Tk * D * Dh, Tk * D + 1.5 * D * Dh + Tk * Dh),
        "mlp_out": kern(ms_o, 2.0 * Tk * D * Dh, Tk * Dh + 1.5 * D * Dh + Tk * D),
        "total_us": round((ms_p + ms_i + ms_o) * 1e3, 2),
    }


def bench_config3(torch, args) -> dict:
    from tritify_amd import workloads as W
    from tritify_amd.decoder import DecoderModel

    g3 = gold()["config3"]
    cfg = {k: g3[k] for k in ("d", "ffn", "nh", "nkv", "hd", "layers", "vocab")}
    P, max_new = g3["prompt"], g3["max_new"]
    max_pos = P + max_new
    log(f"bench: config 3: generating and packing the decoder ({cfg['layers']} layers, vocab {cfg['vocab']})")
    t0 = time.perf_counter()
    m = DecoderModel(cfg, max_pos, P, g3["h_shift"])
    layers = []
    for l in range(cfg["layers"]):
        codes = W.decoder_layer_codes(l, cfg, g3["w_seed"])
        m.set_layer(l, *codes)
        layers.append(codes)
    emb = W.decoder_embedding_codes(cfg, g3["w_seed"])
    m.set_embedding(*emb)
    cos, sin = W.rope_tables(max_pos, cfg["hd"])
    m.set_tables(cos, sin, W.exp_table(), W.silu_table())
    prompt = W.decoder_prompt(g3["prompt_seed"], P, cfg["vocab"])
    log(f"bench: config 3: weights resident in {time.perf_counter() - t0:.1f}s")
    toks, logits = m.generate(prompt, max_new, graph=True)
    if toks.tolist() != g3["tokens"] or sha(logits) != g3["logits_sha256"]:
        raise SystemExit("bench: config 3: the generation differs from the CPU fixture")
    log("bench: config 3: bit-exact vs the CPU fixture (129 logit rows); timing")

    stream = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    graph = m.capture_decode_step()
    reps = 3
    pre_ms, dec_ms, eager_ms = [], [], []
    for _ in range(reps):
        m.pos.zero_()
        m.step.zero_()
        m.tok_in[:P] = torch.from_numpy(prompt).cuda()
        torch.cuda.synchronize()
        ev[0].record(stream)
        m.forward(m.tok_in, P, stream)
        ev[1].record(stream)
        for _ in range(max_new - 1):
            graph.replay()
        ev[2].record(stream)
        torch.cuda.synchronize()
        pre_ms.append(ev[0].elapsed_time(ev[1]))
        dec_ms.append(ev[1].elapsed_time(ev[2]))
    # eager decode (one launch per kernel from the host) for comparison
    m.pos.zero_()
    m.step.zero_()
    m.forward(m.tok_in, P, stream)
    torch.cuda.synchronize()
    ev[0].record(stream)
    for _ in range(max_new - 1):
        m.decode_step(stream)
    ev[1].record(stream)
    torch.cuda.synchronize()
    eager_ms = ev[0].elapsed_time(ev[1])
    # the lm_head alone: a batch-1 decode GEMV over 151,936 x 896 W12 weights (204 MB), cycling three copies so no
    # launch finds its weights in the 256 MB Infinity Cache (inside the decode step the layers evict them likewise)
    import tritify_amd.backend as TB
    lo_b, nib_b = m.sizes["emb"]
    lo0, nib0 = m.w["emb"]
    lo_c = [lo0[:lo_b]] + [lo0[:lo_b].clone() for _ in range(2)]
    nib_c = [nib0[:nib_b]] + [nib0[:nib_b].clone() for _ in range(2)]
    em, es = m.scale["emb"]
    V, d = cfg["vocab"], cfg["d"]

    def lm_head(i):
        TB.w12_linear(m.xn[:d], lo_c[i % 3], nib_c[i % 3], 1, V, d, m.logits, TB.OUT_I32, em, es, stream=stream)

    lm_ms, _ = time_launches(torch, lm_head, 300, 60)
    lm_bytes = 1.5 * V * d + d + 4 * V
    del lo_c, nib_c
    steps = max_new - 1
    dec = min(dec_ms)
    wbytes = 1.5 * (cfg["layers"] * (((cfg["nh"] + 2 * cfg["nkv"]) * cfg["hd"] + cfg["nh"] * cfg["hd"]) * cfg["d"] +
                                     3 * cfg["ffn"] * cfg["d"]) + cfg["vocab"] * cfg["d"])
    res = {
        "workload": f"config 3: Qwen2.5-0.5B-shape decoder (d {cfg['d']}, ffn {cfg['ffn']}, {cfg['nh']}/{cfg['nkv']} "
                    f"heads, {cfg['layers']} layers, vocab {cfg['vocab']}), W12 weights ({wbytes / 1e6:.0f} MB), "
                    f"{P}-token prefill then {steps} greedy decode steps",
        "bit_exact": True,
        "decode_tokens_per_s": round(steps / (dec * 1e-3), 1),
        "decode_us_per_token": round(dec * 1e3 / steps, 1),
        "decode_weight_gbs": round(wbytes / (dec * 1e-3 / steps) / 1e9, 1),
        "decode_hbm_frac": round(wbytes / (dec * 1e-3 / steps) / 1e9 / HBM_PEAK_GBS, 4),
        "decode_eager_tokens_per_s": round(steps / (eager_ms * 1e-3), 1),
        "prefill_ms": round(min(pre_ms), 3),
        "prefill_tokens_per_s": round(P / (min(pre_ms) * 1e-3), 0),
        "decode": "one captured HIP graph per step, replayed; positions and tokens stay on the device",
        "lm_head_gemv": {"us": round(lm_ms * 1e3, 2), "alg_gbs": round(lm_bytes / (lm_ms * 1e-3) / 1e9, 1),
                         "hbm_frac": round(lm_bytes / (lm_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                         "what": "the batch-1 decode GEMV of the 151,936 x 896 lm_head (w12_skinny, int32 logits), "
                                 "3 rotating weight copies"},
    }
    if not args.no_cpu:
        # the same semantics as this line's GPU figure (this build's int8 rules); the reference-semantics decoder
        # and its CPU pair are the `ref` entry's
        res["cpu_baseline"] = cpu_baseline_decoder(cfg, layers, emb, cos, sin, prompt, g3["h_shift"])
    return res


def cpu_baseline_decoder(cfg, layers, emb, cos, sin, prompt, h_shift) -> dict:
    """This build's W12 int8 decoder on the CPU (the oracle's restatement of it, in the reference's decoder loop,
    generate_greedy_by, generate.rs:82-111) on a bounded sample: a 32-token prompt and 4 greedy decode steps, on this
    host's cores. Reported beside the reference's own decoder, which is config 3's CPU baseline."""
    from oracle import oracle as O
    from tritify_amd import workloads as W

    a = {k: [] for k in ("wqkv", "qkv_mant", "qkv_shift", "wo", "o_mant", "o_shift", "wgu", "gu_mant", "gu_shift",
                         "wd", "d_mant", "d_shift")}
    for wqkv, qms, wo, oms, wgu, gms, wd, dms in layers:
        for key, w, ms in (("qkv", wqkv, qms), ("o", wo, oms), ("gu", wgu, gms), ("d", wd, dms)):
            a[{"qkv": "wqkv", "o": "wo", "gu": "wgu", "d": "wd"}[key]].append(w.astype(np.int16))
            a[key + "_mant"].append(ms[0])
            a[key + "_shift"].append(ms[1])
    arrays = {k: np.concatenate(v) for k, v in a.items()}
    arrays.update(emb=emb[0].astype(np.int16), lm_mant=emb[1][0], lm_shift=emb[1][1], rope_cos=cos, rope_sin=sin,
                  exp_tab=W.exp_table(), silu=W.silu_table())
    cores = cpu_threads()
    shape = dict(cfg, max_pos=cos.shape[0], h_shift=h_shift)
    O.dec_generate(shape, arrays, prompt[:32], 1, threads=cores)  # prefill only
    t0 = time.perf_counter()
    O.dec_generate(shape, arrays, prompt[:32], 5, threads=cores)
    t1 = time.perf_counter()
    O.dec_generate(shape, arrays, prompt[:32], 1, threads=cores)
    t2 = time.perf_counter()
    dt = (t1 - t0) - (t2 - t1)  # the 4 decode steps alone
    return {"value": round(4 / dt, 2), "unit": "tokens/s", "cores": cores, "nproc": os.cpu_count(), "kind": "port",
            "sample": f"4 greedy decode steps after a 32-token prompt through the oracle's restatement of this "
                      f"build's W12 int8 decoder (the reference's decoder loop with int8 activations and W12 weights, "
                      f"threaded GEMV), {dt * 1e3 / 4:.1f} ms/token"}


def cpu_baseline_moe(g4: dict, x: np.ndarray, r: np.ndarray) -> dict:
    """The reference's MoE on the CPU (MoeMlp::forward_routed, layers.rs:928-936, 988-1020): token by token, each of
    the top-k experts and the shared expert is a SwiGluMlp of one row whose three QuantLinear products go through
    linear_cpu with the workers plan_threads gives them (backend.rs:89-94, 133-140), on the auto dot variant. Timed on
    a bounded sample of tokens; the products dominate, the per-row quantization and SiLU passes (O(H + F)) are left
    out, so the figure bounds the reference's speed from above."""
    import tritify_amd as T
    from oracle import oracle as O

    H, F, E, K = g4["H"], g4["F"], g4["E"], g4["top_k"]
    n_tok = 8
    logits = r[: n_tok * E].reshape(n_tok, E)
    sel = [np.argsort(-logits[t].astype(np.int64), kind="stable")[:K].tolist() for t in range(n_tok)]  # ties: lower
    need = sorted({e for s_ in sel for e in s_} | {E})
    # i32 codes of the experts the sample uses (the dot's cost does not depend on the values)
    wgu = {g: T.gen_uniform_fast(50_000 + g, -2048, 2047, 2 * F * H) for g in need}
    wd = {g: T.gen_uniform_fast(60_000 + g, -2048, 2047, H * F) for g in need}
    hrow = T.gen_uniform_fast(3, -127, 127, F)
    xs = x.astype(np.int32)
    cores = cpu_threads()
    O.set_max_threads(cores)
    variant = O.lib().kt_cpu_auto_variant()

    def token(t):
        xr = xs[t * H:(t + 1) * H]
        for g in sel[t] + [E]:
            O.linear_cpu(xr, wgu[g][: F * H], 1, F, H, variant)
            O.linear_cpu(xr, wgu[g][F * H:], 1, F, H, variant)
            O.linear_cpu(hrow, wd[g], 1, H, F, variant)

    token(0)  # one untimed token
    t0 = time.perf_counter()
    for t in range(n_tok):
        token(t)
    dt = time.perf_counter() - t0
    ops = 2.0 * n_tok * (K + 1) * 3 * F * H
    workers = O.plan_threads(F, F * H)
    return {"value": round(n_tok / dt, 2), "unit": "tokens/s", "effective_tops": round(ops / dt / 1e12, 5),
            "cores": cores, "nproc": os.cpu_count(), "kind": "port",
            "sample": f"{n_tok} tokens of config 4, each through its {K} chosen experts and the shared expert as "
                      f"one-row QuantLinear products on the oracle's linear_cpu ({['portable', 'avx2', 'avx512'][variant]}"
                      f" dot, {workers} workers per product as plan_threads gives them), {dt * 1e3 / n_tok:.1f} ms/token"}


# ---------------------------------------------------------------------------------------------------------------
# the LinearBackend trait path, through the C ABI

CUDA_BENCH_SHAPES = ([(8, 2048, 2048, "prefill 8x2048x2048"), (1, 4864, 896, "decode 1x4864x896 (Qwen MLP)"),
                      (1, 151936, 896, "decode 1x151936x896 (Qwen LM head)")] +
                     [(r_, 2048, 2048, f"sweep {r_}x2048x2048") for r_ in (1, 2, 4, 8, 16, 32, 64)])


def bench_linear_backend(torch, args) -> dict:
    """LinearBackend::linear_weights through the C ABI (kt_hip_linear_weights: host i32 codes in, host i64 sums out,
    activations packed on the device, weights resident by WeightId after the first call) on the shapes of the
    reference's cuda_bench (crates/02-runtime/kt-runtime/examples/cuda_bench.rs:60-78), codes uniform in +-WLEVELS
    (3 digit planes each). Every answer equals the oracle's linear_cpu before it is timed; both are timed as
    cuda_bench times (one untimed call, then >= 2 calls and about 0.5 s, at most 200). The time includes the
    host-to-device copy of x, the packing, the product and the copy of the i64 result back (the trait's contract)."""
    import tritify_amd as T
    from oracle import oracle as O

    b = T.HipBackend(0)
    cores = cpu_threads()
    O.set_max_threads(cores)
    variant = O.lib().kt_cpu_auto_variant()
    WL = 265720

    def timeit(f):
        f()
        reps, t0 = 0, time.perf_counter()
        while reps < 2 or (time.perf_counter() - t0 < 0.5 and reps < 200):
            f()
            reps += 1
        return (time.perf_counter() - t0) / reps * 1e6

    res = {"what": "kt_hip_linear_weights (host buffers, PCIe included) against the oracle's linear_cpu on "
                   f"{cores} threads ({['portable', 'avx2', 'avx512'][variant]} dot)", "nproc": os.cpu_count(),
           "shapes": {}}
    for m, n, k, label in CUDA_BENCH_SHAPES:
        x = T.gen_uniform_fast(1 + m, -WL, WL, m * k)
        w = T.gen_uniform_fast(2 + n, -WL, WL, n * k)
        want = O.linear_cpu(x, w, m, n, k, variant)
        wts = T.Weights(T.weight_id_fresh(), w)
        if not np.array_equal(b.linear_weights(x, wts, m, n, k), want):
            raise SystemExit(f"bench: LinearBackend {label}: differs from the oracle")
        us_hip = timeit(lambda: b.linear_weights(x, wts, m, n, k))
        us_cpu = timeit(lambda: O.linear_cpu(x, w, m, n, k, variant))
        res["shapes"][label] = {"m": m, "n": n, "k": k, "bit_exact": True, "hip_us": round(us_hip, 1),
                                "hip_mmacs": round(m * n * k / us_hip, 1), "cpu_us": round(us_cpu, 1),
                                "cpu_mmacs": round(m * n * k / us_cpu, 1)}
        log(f"bench: LinearBackend {label}: hip {us_hip:.1f} us, cpu {us_cpu:.1f} us")
    res["fallbacks"] = T.fallbacks()
    b.close()
    return res


# ---------------------------------------------------------------------------------------------------------------


# ---------------------------------------------------------------------------------------------------------------
# the reference's own integer semantics on the device (RefDecoder, RefConv2d, RefFeedForward)

WL = 265720
REF_PROMPT, REF_NDEC = [9, 1000, 20000, 151935], 28
_ref_cpu: dict = {}


def _ref_qwen():
    from tritify_amd import workloads as W

    return W.REF_QWEN


def _ref_weights():
    from tritify_amd import workloads as W

    return W.ref_decoder_weights(W.REF_QWEN, W.REF_C3["w_seed"])


def ref_decoder_oracle() -> tuple:
    """The oracle's restatement of the reference decoder (the weights of config 3's reference-semantics run) over
    REF_PROMPT and REF_NDEC greedy steps: every position's logits hash, the seconds it took, the threads. The CPU
    baseline's bounded sample (32 positions)."""
    if "hashes" not in _ref_cpu:
        from oracle import oracle as O

        log("bench: the reference decoder on the CPU (the oracle), Qwen2.5-0.5B shape, 32 positions")
        model = O.RefModel.from_weights(_ref_qwen(), *_ref_weights())
        cores = cpu_threads()
        O.set_max_threads(cores)
        t0 = time.perf_counter()
        _, _, want = model.generate(REF_PROMPT, REF_NDEC + 1)
        _ref_cpu.update(hashes=want, seconds=time.perf_counter() - t0, cores=cores)
    return _ref_cpu["hashes"], _ref_cpu["seconds"], _ref_cpu["cores"]


REF_PREFILL_T = 64


def ref_forward_oracle() -> tuple:
    """The oracle's CausalLM::forward_int over REF_PREFILL_T tokens: (logits, scale, seconds, threads)."""
    if "fwd" not in _ref_cpu:
        from oracle import oracle as O

        model = O.RefModel.from_weights(_ref_qwen(), *_ref_weights())
        cores = cpu_threads()
        O.set_max_threads(cores)
        toks = [(7919 * i + 11) % _ref_qwen()["vocab"] for i in range(REF_PREFILL_T)]
        t0 = time.perf_counter()
        lg, ls = model.forward(toks)
        _ref_cpu["fwd"] = (toks, lg, ls, time.perf_counter() - t0, cores)
    return _ref_cpu["fwd"]


def ref_decoder_cpu_baseline() -> dict:
    hashes, secs, cores = ref_decoder_oracle()
    npos = len(hashes)
    return {"value": round(npos / secs, 2), "unit": "tokens/s", "cores": cores, "nproc": os.cpu_count(),
            "kind": "port",
            "sample": f"the reference's own decoder, same weights (the oracle's restatement: repro::run over "
                      f"{len(REF_PROMPT)} prompt and {REF_NDEC} greedy positions, every QuantLinear through the "
                      f"threaded linear_cpu restatement), {secs * 1e3 / npos:.0f} ms/position; positions 0-31, "
                      f"where its attention is cheaper than at the GPU figure's 512-639, so an upper bound on the "
                      f"CPU's rate there"}


def bench_ref_decoder(torch, args) -> dict:
    """The reference's DecoderModel (model.rs:290-353) at its own semantics on the device, config 3's workload:
    Qwen2.5-0.5B shape, a 512-token prompt fed through decode_step (generate.rs:82-93) then 128 greedy steps, one
    captured HIP graph per position (decode step + argmax_codes, the position advanced and the logits recorded on
    the device). Every run's 640 per-position logits hashes are checked against the committed fixture (the oracle's
    run, tests/golden/goldens.json config3_ref); the decode rate is over positions 512-639, the mean of the runs."""
    from tritify_amd import workloads as W
    from tritify_amd.refdecoder import RefDecoder, logits_hash_bytes

    cfg, rc = W.REF_QWEN, W.REF_C3
    fx = gold()["config3_ref"]
    prompt, n_dec = W.ref_c3_prompt(cfg), rc["decode"]
    t0 = time.perf_counter()
    w = _ref_weights()
    dec = RefDecoder(cfg, *w)
    log(f"bench: ref decoder: weights resident in {time.perf_counter() - t0:.1f}s")
    dec.decode_step(prompt[0], 0)
    g = dec.capture_greedy_step()
    stream = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    runs, pre = [], []
    npos = len(prompt) + n_dec
    for r in range(3):
        dec.new_cache()
        dec.pos.zero_()
        torch.cuda.synchronize()
        ev[2].record(stream)
        for t in prompt:
            dec.token.fill_(t)
            g.replay()
        ev[3].record(stream)
        torch.cuda.synchronize()
        ev[0].record(stream)
        for _ in range(n_dec):
            g.replay()
        ev[1].record(stream)
        torch.cuda.synchronize()
        runs.append(ev[0].elapsed_time(ev[1]) / n_dec)
        pre.append(ev[2].elapsed_time(ev[3]) / len(prompt))
        got = [hashlib.sha256(logits_hash_bytes(*dec.recorded(p))).hexdigest() for p in range(npos)]
        if got != fx["position_sha256"]:
            first = next(i for i, (a, b) in enumerate(zip(got, fx["position_sha256"])) if a != b)
            raise SystemExit(f"bench: ref decoder run {r}: position {first} differs from the CPU fixture")
    log(f"bench: ref decoder: {npos} positions bit-exact vs the CPU fixture in each of 3 runs")
    mean = sum(runs) / len(runs)
    del dec, g, w
    torch.cuda.empty_cache()
    wbytes = 3 * (cfg["layers"] * ((2 * cfg["nh"] + 2 * cfg["nkv"]) * cfg["hd"] * cfg["dim"] +
                                   3 * cfg["hidden"] * cfg["dim"]) + cfg["vocab"] * cfg["dim"])
    # the batched forward (prefill) of REF_PREFILL_T tokens, checked against the oracle's, then timed
    toks, lg_want, ls_want, cpu_fwd_s, cores = ref_forward_oracle()
    dec = RefDecoder(dict(cfg, max_seq=REF_PREFILL_T), *_ref_weights())
    y, yr = dec.forward(toks)
    ok = np.array_equal(y.cpu().numpy().reshape(lg_want.shape), lg_want)
    w_ = yr.cpu().numpy()
    if not (ok and (int(w_[0]), int(w_.view(np.int32)[2])) == ls_want):
        raise SystemExit("bench: ref forward differs from the CPU oracle")
    fwd_ms, _ = time_launches(torch, lambda i: dec.forward(toks, stream=stream), 5, 2)
    del dec, y
    torch.cuda.empty_cache()
    res = {
        "workload": "config 3 at the reference's own semantics: DecoderModel::decode_step (i32 codes at 2^28, "
                    "12-trit weights as 3 digit planes, per-tensor dynamic requant after every op, RmsNorm, RoPE "
                    "Scales, exp and SiLU CodeLuts), Qwen2.5-0.5B shape (24 layers, dim 896, 14/2 heads, 4864, "
                    "vocab 151936), a 512-token prompt through decode_step then 128 greedy steps, one HIP graph per "
                    "position",
        "bit_exact_positions": npos,
        "run_sha256": fx["run_sha256"],
        "decode_tokens_per_s": round(1e3 / mean, 1),
        "decode_us_per_token": round(mean * 1e3, 1),
        "decode_positions": f"{len(prompt)}-{npos - 1}",
        "decode_ms_runs": [round(x, 4) for x in runs],
        "prompt_us_per_position": round(sum(pre) / len(pre) * 1e3, 1),
        "weight_plane_gbs": round(wbytes / (mean * 1e-3) / 1e9, 1),
        "forward": {
            "what": f"CausalLM::forward_int over {REF_PREFILL_T} tokens (the batched prefill: every op over the "
                    f"{REF_PREFILL_T}-row tensors, the prefill attention at one score scale), logits bit-exact",
            "ms": round(fwd_ms, 3), "tokens_per_s": round(REF_PREFILL_T / (fwd_ms * 1e-3), 1),
            "cpu_baseline": {"value": round(REF_PREFILL_T / cpu_fwd_s, 1), "unit": "tokens/s", "cores": cores,
                             "nproc": os.cpu_count(), "kind": "port",
                             "sample": f"the oracle's forward of the same {REF_PREFILL_T} tokens, "
                                       f"{cpu_fwd_s * 1e3:.0f} ms"},
        },
    }
    if not args.no_cpu:
        res["cpu_baseline"] = ref_decoder_cpu_baseline()
    return res


def bench_ref_sam(torch, args) -> dict:
    """SAM 2.1 Hiera-B+ at the reference's semantics: the PatchEmbed Conv2d (conv.rs:68-130) on a 1024 x 1024 image
    entered by from_reals, and a stage-3 FeedForward (4096 tokens, 448 -> 1792 -> 448, GELU CodeLut), each checked
    against the oracle before timing; the oracle's direct conv is the CPU baseline."""
    import tritify_amd as T
    from oracle import oracle as O
    from tritify_amd import backend as B
    from tritify_amd.refvision import RefConv2d, RefFeedForward

    dev = torch.device("cuda:0")
    rng = np.random.default_rng(0x5A)
    real = rng.standard_normal(3 * 1024 * 1024) * 1.7
    x, xs = B.ref_from_reals(real)
    sc = B.ref_scale_from_f64(1.0 / WL)
    wc = T.gen_uniform_fast(0xC0, -WL, WL, 112 * 3 * 49).reshape(112, 3, 7, 7)
    bias = (T.gen_uniform_fast(0xC1, -(1 << 28), 1 << 28, 112).astype(np.int64), B.ref_scale_from_f64(1e-9))
    conv = RefConv2d(wc, sc, 4, 3, bias)
    xd = torch.from_numpy(x).to(dev)
    xr = T.qscale_record(*xs)
    y = torch.empty(112 * 256 * 256, dtype=torch.int32, device=dev)
    yr = torch.zeros(4, dtype=torch.int64, device=dev)
    conv.forward_int(xd, xr, 1024, 1024, y, yr)
    conv_cores = cpu_threads()
    O.set_max_threads(conv_cores)
    t0 = time.perf_counter()
    want, wso = O.ref_conv2d(x, xs, 3, 1024, 1024, wc.reshape(-1), sc, 112, 7, 7, 4, 3, bias)
    cpu_conv_s = time.perf_counter() - t0
    if not (np.array_equal(y.cpu().numpy(), want.reshape(-1)) and
            tuple(T.read_qscale(yr)[k] for k in ("mant", "shift")) == wso):
        raise SystemExit("bench: ref patch embed differs from the CPU oracle")
    stream = torch.cuda.current_stream()
    conv_ms, _ = time_launches(torch, lambda i: conv.forward_int(xd, xr, 1024, 1024, y, yr, stream=stream), 50, 10)
    rows, dim, hid = 4096, 448, 1792
    wi, wo = T.gen_uniform_fast(0xF1, -WL, WL, hid * dim), T.gen_uniform_fast(0xF2, -WL, WL, dim * hid)
    bi = (T.gen_uniform_fast(0xF3, -(1 << 28), 1 << 28, hid).astype(np.int64), B.ref_scale_from_f64(1e-9))
    bo = (T.gen_uniform_fast(0xF4, -(1 << 28), 1 << 28, dim).astype(np.int64), B.ref_scale_from_f64(1e-9))
    ff = RefFeedForward(dim, hid, (wi, sc, bi), (wo, sc, bo))
    fx = T.gen_uniform_fast(0xF5, -(1 << 28), 1 << 28, rows * dim)
    fxs = B.ref_scale_from_f64(3.0 / (1 << 28))
    fxd, fxr = torch.from_numpy(fx).to(dev), T.qscale_record(*fxs)
    fy, fyr = ff.forward_int(fxd, fxr, rows)
    fwant, fws = O.feedforward(fx, rows, dim, fxs, wi, sc, hid, wo, sc, bi, bo)
    if not (np.array_equal(fy.cpu().numpy(), fwant.reshape(-1)) and
            tuple(T.read_qscale(fyr)[k] for k in ("mant", "shift")) == fws):
        raise SystemExit("bench: ref feedforward differs from the CPU oracle")
    ff_ms, _ = time_launches(torch, lambda i: ff.forward_int(fxd, fxr, rows, stream=stream), 50, 10)
    conv_ops, ff_ops = 2.0 * 65536 * 147 * 112, 2.0 * 2 * rows * dim * hid
    return {
        "workload": "SAM 2.1 Hiera-B+ at the reference's semantics: PatchEmbed Conv2d::forward_int (3 x 1024 x 1024 "
                    "from_reals pixels, 112 channels, 7x7/4 pad 3: whole-image quant_to, im2col digit GEMM, bias, "
                    "whole-output requant_dyn) and a stage-3 FeedForward (4096 x 448 -> 1792 GELU CodeLut -> 448)",
        "bit_exact": True,
        "patch_embed_us": round(conv_ms * 1e3, 1),
        "patch_embed_effective_tops": round(conv_ops / (conv_ms * 1e-3) / 1e12, 2),
        "feedforward_us": round(ff_ms * 1e3, 1),
        "feedforward_effective_tops": round(ff_ops / (ff_ms * 1e-3) / 1e12, 2),
        "cpu_baseline": {
            "value": round(cpu_conv_s * 1e6, 0), "unit": "us per patch embed", "cores": conv_cores,
            "nproc": os.cpu_count(), "kind": "port",
            "sample": "the oracle's direct convolution (Conv2d::forward_int restated, the output channels split over "
                      "the threads as par_blocks does, conv.rs:123), one full image"},
    }


# GLM-4.5-Air's MoE layer: hidden 4096, 128 routed experts of 1408, 8 per token, the sigmoid router with its
# selection bias and norm_topk_prob, one shared expert of 1408
REF_GLM = dict(dim=4096, E=128, top_k=8, hidden=1408, shared=1408)
REF_MOE_T = (1, 256)


def ref_moe_weights(cfg: dict, seed: int):
    """(router, experts, coded bias, shared) of a REF_GLM layer: every code uniform in +-WLEVELS at the Scale
    from_weights gives floats of peak 1 (1 / WLEVELS), the router's of peak 0.1 (its logits then spread with a
    standard deviation near 2, so the sigmoid does not saturate and the tokens spread over about 122 of the 128
    experts; at peak 1 most scores tie at the top code and the bias alone picks the same few experts), the coded
    bias uniform in +-0.05 * 2^20; drawn on threads."""
    import tritify_amd as T
    from concurrent.futures import ThreadPoolExecutor
    from tritify_amd import backend as B

    sc = B.ref_scale_from_f64(1.0 / WL)
    d, E, h, hs = cfg["dim"], cfg["E"], cfg["hidden"], cfg["shared"]
    shapes = [(E, d)] + [sh for _ in range(E + 1) for sh in ((h, d), (h, d), (d, h))]
    shapes[-3:] = [(hs, d), (hs, d), (d, hs)]
    with ThreadPoolExecutor(max(1, min(8, cpu_threads()))) as ex:
        mats = list(ex.map(lambda i: T.gen_uniform_fast(seed + i, -WL, WL, shapes[i][0] * shapes[i][1])
                           .reshape(shapes[i]), range(len(shapes))))
    names = ("gate", "up", "down")
    experts = [{n: (mats[1 + 3 * e + j], sc) for j, n in enumerate(names)} for e in range(E + 1)]
    bias = T.gen_uniform_fast(seed - 1, -52429, 52429, E).astype(np.int64)
    return (mats[0], B.ref_scale_from_f64(0.1 / WL)), experts[:E], bias, experts[E]


def bench_ref_moe(torch, args) -> dict:
    """MoeMlp::forward_int (layers.rs:652-1034) at the reference's semantics, GLM-4.5-Air's layer shape: one decode
    token and a 256-token batch, each output checked against the oracle's token-by-token restatement before timing;
    the oracle's run of the batch is the CPU baseline."""
    from oracle import oracle as O
    from tritify_amd import backend as B
    from tritify_amd.refmoe import RefMoeLayer
    import tritify_amd as T

    cfg = REF_GLM
    t0 = time.perf_counter()
    router, experts, bias, shared = ref_moe_weights(cfg, 0x61A5)
    layer = RefMoeLayer(cfg["dim"], router, experts, cfg["top_k"], True, bias, shared)
    log(f"bench: ref moe: weights resident in {time.perf_counter() - t0:.1f}s")
    model = O.RefMoe.from_weights(cfg["dim"], router, experts, cfg["top_k"], True, bias, shared)
    del router, experts, shared
    cores = cpu_threads()
    O.set_max_threads(cores)
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    rng = np.random.default_rng(0x61A7)
    res = {"workload": "the reference's MoeMlp::forward_int at its own semantics (i32 codes, per-row dynamic "
                       "quantization of every QuantLinear row, sigmoid router with selection bias and norm_topk, "
                       "exp / sigmoid / SiLU CodeLuts, ec-weighted combine, merge_rows, shared expert), GLM-4.5-Air "
                       "MoE layer shape (dim 4096, 128 experts of 1408, top-8, shared 1408), 12-trit weights",
           "bit_exact": True}
    for T_ in REF_MOE_T:
        x, xs = B.ref_from_reals(rng.uniform(-1.0, 1.0, T_ * cfg["dim"]))
        xd, xr = torch.from_numpy(x).to(dev), T.qscale_record(*xs)
        out, orec = layer.forward(xd, xr, T_)
        off = layer.bucket(layer.route(xd, xr, T_)[0], T_)[0].cpu().numpy()
        cnt = np.diff(off)
        c0 = time.perf_counter()
        want, ws = model.forward(x, T_, xs)
        cpu_s = time.perf_counter() - c0
        if not (np.array_equal(out.cpu().numpy(), want) and
                tuple(T.read_qscale(orec)[k] for k in ("mant", "shift")) == ws):
            raise SystemExit(f"bench: ref moe T={T_}: differs from the CPU oracle")
        n = 200 if T_ == 1 else 20
        ms, _ = time_launches(torch, lambda i: layer.forward(xd, xr, T_, stream=stream), n, 5)
        # the same forward as one HIP graph (no host work between its launches), its output checked too
        g, gout, grec = layer.capture(xd, xr, T_)
        g.replay()
        torch.cuda.synchronize()
        if not (np.array_equal(gout.cpu().numpy(), want) and
                tuple(T.read_qscale(grec)[k] for k in ("mant", "shift")) == ws):
            raise SystemExit(f"bench: ref moe T={T_}: the graph replay differs from the CPU oracle")
        gms, _ = time_launches(torch, lambda i: g.replay(), n, 5)
        del g, gout, grec
        res[f"T{T_}"] = {"us_per_forward": round(ms * 1e3, 1), "tokens_per_s": round(T_ / (ms * 1e-3), 1),
                         "graph_us_per_forward": round(gms * 1e3, 1),
                         "graph_tokens_per_s": round(T_ / (gms * 1e-3), 1),
                         "experts_used": int((cnt > 0).sum()), "max_rows_per_expert": int(cnt.max())}
        log(f"bench: ref moe T={T_}: {ms * 1e3:.1f} us per forward ({gms * 1e3:.1f} us as a graph), bit-exact")
        if T_ == REF_MOE_T[-1]:
            res["cpu_baseline"] = {
                "value": round(T_ / cpu_s, 1), "unit": "tokens/s", "cores": cores, "nproc": os.cpu_count(),
                "kind": "port", "sample": f"the oracle's MoeMlp::forward_int of the same {T_} tokens (token by "
                                          f"token, QuantLinear rows on {cores} threads), {cpu_s * 1e3:.0f} ms"}
    del layer, model
    return res


def bench_ref(torch, args) -> dict:
    res = {"decoder": bench_ref_decoder(torch, args)}
    torch.cuda.empty_cache()
    res["sam"] = bench_ref_sam(torch, args)
    torch.cuda.empty_cache()
    res["moe"] = bench_ref_moe(torch, args)
    torch.cuda.empty_cache()
    return res


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    # 500 warmup launches (about 33 ms at M = 2048) let the GPU's clocks settle after the set-up's idle host work:
    # the first tens of milliseconds of a burst run at lower clocks (measured 76.6 us per launch with 20 warmup
    # launches and 200 timed against 65.6 us settled, on one box)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=500)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--configs", type=str, default="2,3,4,5,ql,lb,ref",
                    help="comma-separated configs to run (2 is the headline; ql = the reference's QuantLinear; "
                         "lb = the LinearBackend trait path on cuda_bench's shapes; ref = the reference-semantics "
                         "decoder, SAM image path and GLM MoE layer; refdec / refmoe = that decoder / MoE layer alone)")
    ap.add_argument("--ms", type=str, default="", help="comma-separated subset of config-2 M to run (profiling runs)")
    ap.add_argument("--copy-calib", action="store_true",
                    help="only run a plain 256 MiB device copy 10 times (scales the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (the 12-bit GEMM on one MI355X); "
              "multi-GPU sharding is designed, not built", file=sys.stderr)
        return 2

    import torch

    if args.copy_calib:
        src = torch.ones(256 << 20, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calib_bytes": 256 << 20, "copies": 10}), flush=True)
        return 0

    configs = [c.strip() for c in args.configs.split(",") if c.strip()]
    extra = {}
    headline = None
    if "2" in configs:
        sweep, headline, x, w = bench_config2(torch, args)
    for c in configs:
        if c == "4":
            extra["4"] = bench_config4(torch, args)
            torch.cuda.empty_cache()
        if c == "5":
            extra["5"] = bench_config5(torch, args)
            torch.cuda.empty_cache()
        if c == "3":
            extra["3"] = bench_config3(torch, args)
            torch.cuda.empty_cache()
        if c == "ql":
            extra["ql"] = bench_quant_linear(torch, args)
            torch.cuda.empty_cache()
        if c == "lb":
            extra["lb"] = bench_linear_backend(torch, args)
            torch.cuda.empty_cache()
        if c == "ref":
            extra["ref"] = bench_ref(torch, args)
        if c == "refdec":  # the reference decoder alone (profiling runs)
            extra["refdec"] = bench_ref_decoder(torch, args)
            torch.cuda.empty_cache()
        if c == "refmoe":  # the reference MoE layer alone (profiling runs)
            extra["refmoe"] = bench_ref_moe(torch, args)
            torch.cuda.empty_cache()

    if headline is None:
        print(json.dumps({"sweep": sweep if "2" in configs else None, "configs": extra}), flush=True)
        return 0
    ms_per_step, wall, n_launch, warm, us, tops = headline
    g2 = gold()["config2"]
    N, K, MH = g2["N"], g2["K"], max(g2["Ms"])
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "w12_gemm_m2048_traffic.json")
    if os.path.exists(tpath):
        traffic = json.load(open(tpath)).get("hbm_bytes_per_launch")

    out = {
        "metric": "bit-exact 12-bit int GEMM effective TOPS (M=2048, N=K=4096)",
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": n_launch,
        "warmup": warm,
        "ms_per_step": round(ms_per_step, 5),
        "wall_ms_per_step": round(wall / n_launch * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (LCG integer samplers; inputs and outputs hash-checked against the CPU oracle fixtures)",
        "config": {
            "workload": "config 2: exact 12-bit GEMM, int8 x 12-bit codes -> i64 -> per-channel requant -> int8",
            "M": MH, "N": N, "K": K, "weights": "two balanced int8 digit planes (W12B), 2 B/weight, 12 rotating copies",
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(tops, 2),
            "peak": INT8_PEAK_TOPS,
            "unit": "TOPS",
            "frac": round(tops / INT8_PEAK_TOPS, 4),
            "traffic": traffic,
            "traffic_source": "the committed rocprofv3 FETCH_SIZE + WRITE_SIZE figure of this kernel "
                              "(profiles/w12_gemm_m2048_traffic.json, copy-calibrated), not measured in this run",
            "kernel": "w12_gemm_dma_kernel<I8, SMALL, BAL> on the W12B planes (logical ops 2*M*N*K per launch; the 2 "
                      "digit planes execute twice that)",
        },
        "sweep": sweep,
        "configs": extra,
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        log("bench: timing the CPU baseline")
        out["cpu_baseline"] = cpu_baseline(x.astype(np.int32), w, MH, N, K)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
