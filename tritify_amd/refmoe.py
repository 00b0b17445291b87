"""The reference's MoeMlp at its own integer semantics on one MI355X: the host-side mirror of MoeMlp
(crates/01-engine/kt-core/src/layers.rs:652-1020, the sigmoid router of router.rs:29-79, GLM-4.5's shared expert of
layers.rs:757-780).

The reference routes and runs its experts token by token, each call a QuantLinear of one row with its own dynamic
quantization (per-row max |x|, per-(token, expert) max |acc|). `RefMoeLayer.forward` keeps every per-row step and
groups only the exact integer products:

  router                   kt_hip_quant_linear_rows (one group: every token row quantized on its own)
  route / route_sigmoid    kt_hip_ref_moe_route     (exp or sigmoid CodeLut numerators, top-k, sumc)
  bucket                   kt_hip_ref_moe_bucket    (the (token, expert) rows ordered by expert, on the device)
  experts gate / up        kt_hip_quant_linear_rows (E groups; x rows by index)
  SiLU * up                kt_hip_ref_swiglu        (one row per (token, expert))
  experts down             kt_hip_quant_linear_rows (E groups; per-row input scales)
  combine                  kt_hip_ref_moe_combine   (per token: common scale, ec-weighted sum, 1/sumc)
  merge_rows               kt_hip_ref_merge_rows    (a sequence: the tokens at one scale)
  shared expert + add      kt_hip_quant_linear(_multi), kt_hip_ref_swiglu_seq, kt_hip_ref_add_seq (the whole tensor, many
                           CTAs)

Nothing waits on the host: the group sizes stay on the device (the grouped products plan their tiles there), so a
forward is one stream of launches.

torch holds the device buffers; it computes nothing.
"""
from __future__ import annotations

import numpy as np

from . import backend as B
from .quant import QuantLinear, QuantLinearGroup


class RefMoeLayer:
    """MoeMlp { router, experts, top_k, norm_topk_prob, score, shared } resident on device `dev`.

    router: (codes E x dim, (mant, shift)); experts: one dict per expert with gate, up (codes hidden x dim, scale) and
    down (codes dim x hidden, scale); sigmoid_bias: None for the softmax router, else the sigmoid router's coded
    selection bias (E values round(b * 2^20), SigmoidScore::new); shared: None or a dict like an expert's.
    """

    def __init__(self, dim: int, router, experts, top_k: int, norm_topk: bool, sigmoid_bias=None, shared=None,
                 dev: int = 0):
        import torch

        self.torch = torch
        self.dev = dev
        self.device = torch.device("cuda", dev)
        self.dim, self.E, self.top_k, self.norm_topk = int(dim), len(experts), int(top_k), bool(norm_topk)
        if not 1 <= self.top_k <= min(self.E, B.REF_MOE_MAX_K):
            raise ValueError("RefMoeLayer: top_k out of range")
        self.hidden = int(np.asarray(experts[0]["gate"][0]).shape[0])
        d = self.device
        i64 = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.int64)).to(d)  # noqa: E731
        i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(d)  # noqa: E731
        self.router = self._pack_groups([router])
        self.w = {n: self._pack_groups([e[n] for e in experts]) for n in ("gate", "up", "down")}
        self.sigmoid = sigmoid_bias is not None
        if self.sigmoid:
            codes, self.route_lut = B.ref_codelut(B.LUT_SIGMOID, -16.0, 16.0, 16, 20, False)
            self.bias = i64(sigmoid_bias)
        else:
            codes, self.route_lut = B.ref_codelut(B.LUT_EXP, -30.0, 0.0, 16, 20, False)
            self.bias = None
        self.route_codes = i64(codes)
        silu_codes, self.silu_lut = B.ref_codelut(B.LUT_SILU, -30.0, 30.0, 16, 20, True)
        self.silu_codes = i64(silu_codes)
        self.shared = None
        if shared is not None:
            sh_hidden = int(np.asarray(shared["gate"][0]).shape[0])
            self.shared_hidden = sh_hidden
            # gate and up read the same x: one QuantLinearGroup where their boundary allows
            self.shared_grouped = QuantLinearGroup.fits((sh_hidden, sh_hidden))
            names = ("down",) if self.shared_grouped else ("gate", "up", "down")
            self.shared = {n: QuantLinear(f"shared.{n}", shared[n][0], *(
                (sh_hidden, self.dim) if n != "down" else (self.dim, sh_hidden)), shared[n][1], dev=dev)
                for n in names}
            if self.shared_grouped:
                self.shared["gu"] = QuantLinearGroup("shared.gu", [(n, shared[n][0], shared[n][1], None)
                                                                   for n in ("gate", "up")], self.dim, dev=dev)
        self._i32 = i32
        self._route_off = {}  # T -> the router's one-group offsets [0, T] on the device

    def _pack_groups(self, mats):
        """Digit planes of each (codes out x in, scale) in one buffer (all at the largest plane count, in the grouped
        product's tiled layout), with the per-group Scales on the device."""
        torch = self.torch
        codes = [np.ascontiguousarray(m[0], dtype=np.int32) for m in mats]
        out, inp = codes[0].shape
        pw = max(B.planes_for(c) for c in codes)
        gbytes = B.pack_planes_tiled_bytes(out, inp, pw)
        planes = torch.empty(len(codes) * gbytes, dtype=torch.int8, device=self.device)
        for g, c in enumerate(codes):
            B.pack_planes_tiled(torch.from_numpy(c.reshape(-1)).to(self.device), out, inp, pw, planes[g * gbytes:],
                                dev=self.dev)
        mant = torch.from_numpy(np.array([int(m[1][0]) for m in mats], np.int64)).to(self.device)
        shift = torch.from_numpy(np.array([int(m[1][1]) for m in mats], np.int32)).to(self.device)
        torch.cuda.synchronize(self.device)
        return {"planes": planes, "gbytes": gbytes, "pw": pw, "out": out, "in": inp, "mant": mant, "shift": shift}

    def _rows_ql(self, w, x, xidx, x_rows: int, rows: int, xs, xs_step: int, off_dev, groups: int, stream):
        torch = self.torch
        n = B.quant_linear_rows_workspace(rows, w["in"], w["out"], groups)
        ws = torch.empty(n, dtype=torch.uint8, device=self.device)
        y = torch.empty(rows * w["out"], dtype=torch.int32, device=self.device)
        ys = torch.empty(rows * 4, dtype=torch.int64, device=self.device)  # every row's record is written
        B.quant_linear_rows(x, xidx, x_rows, rows, w["in"], xs, xs_step, None, off_dev, w["planes"], w["gbytes"],
                            w["pw"], w["out"], w["mant"], w["shift"], ws, n, y, ys, stream=stream, dev=self.dev,
                            groups=groups)
        return y, ys

    def route(self, x_dev, xs_rec, T: int, stream=None):
        """MoeMlp::route of every token row: (sel T x k int32, ec T x k int64, sumc T int64, logits, logit records),
        device tensors."""
        torch = self.torch
        if T not in self._route_off:
            self._route_off[T] = torch.tensor([0, T], dtype=torch.int64, device=self.device)
        logits, ls = self._rows_ql(self.router, x_dev, None, T, T, xs_rec, 0, self._route_off[T], 1, stream)
        sel = torch.empty(T * self.top_k, dtype=torch.int32, device=self.device)
        ec = torch.empty(T * self.top_k, dtype=torch.int64, device=self.device)
        sumc = torch.empty(T, dtype=torch.int64, device=self.device)
        B.ref_moe_route(logits, T, self.E, self.top_k, ls, self.sigmoid, self.norm_topk, self.route_codes,
                        self.route_lut, self.bias, sel, ec, sumc, stream=stream, dev=self.dev)
        return sel, ec, sumc, logits, ls

    def bucket(self, sel, T: int, stream=None):
        """The (token, expert) rows grouped by expert, on the device: (off E + 1 int64, xidx P int32 row -> token,
        pos P int32 pair -> row)."""
        torch = self.torch
        P = T * self.top_k
        off = torch.empty(self.E + 1, dtype=torch.int64, device=self.device)
        xidx = torch.empty(P, dtype=torch.int32, device=self.device)
        pos = torch.empty(P, dtype=torch.int32, device=self.device)
        B.ref_moe_bucket(sel, T, self.top_k, self.E, off, xidx, pos, stream=stream, dev=self.dev)
        return off, xidx, pos

    def capture(self, x_dev, xs_rec, T: int):
        """forward of T rows of the buffers x_dev / xs_rec as one HIP graph: (graph, out, out record); each replay
        recomputes from what the buffers then hold, into the same out buffers. Call after one eager forward of T rows
        (its small device constants exist then)."""
        torch = self.torch
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            g.capture_begin()
            out, orec = self.forward(x_dev, xs_rec, T, stream=s)
            g.capture_end()
        torch.cuda.current_stream(self.device).wait_stream(s)
        return g, out, orec

    def forward(self, x_dev, xs_rec, T: int, stream=None):
        """MoeMlp::forward_int (layers.rs:1031-1034) of T token rows (x_dev: T x dim i32 codes at the record
        xs_rec): (out T x dim codes, its record), device tensors. Asynchronous on `stream`."""
        torch = self.torch
        dim, K, E = self.dim, self.top_k, self.E
        sel, ec, sumc, _, _ = self.route(x_dev, xs_rec, T, stream)
        P = T * K
        off_d, xidx_d, pos_d = self.bucket(sel, T, stream)
        g, gs = self._rows_ql(self.w["gate"], x_dev, xidx_d, T, P, xs_rec, 0, off_d, E, stream)
        u, us = self._rows_ql(self.w["up"], x_dev, xidx_d, T, P, xs_rec, 0, off_d, E, stream)
        h = torch.empty(P * self.hidden, dtype=torch.int32, device=self.device)
        hs = torch.empty(P * 4, dtype=torch.int64, device=self.device)  # (every record below is written whole)
        B.ref_swiglu(g, gs, u, us, self.hidden, self.silu_codes, self.silu_lut, h, hs, stream, self.dev, rows=P)
        y, ys = self._rows_ql(self.w["down"], h, None, P, P, hs, 1, off_d, E, stream)
        rows = torch.empty(T * dim, dtype=torch.int32, device=self.device)
        rs = torch.empty(T * 4, dtype=torch.int64, device=self.device)
        B.ref_moe_combine(y, ys, P, dim, pos_d, ec, sumc, T, K, rows, rs, stream=stream, dev=self.dev)
        if T > 1:
            routed = torch.empty(T * dim, dtype=torch.int32, device=self.device)
            rrec = torch.empty(4, dtype=torch.int64, device=self.device)
            n = B.ref_merge_rows_workspace(T)
            ws = torch.empty(n, dtype=torch.uint8, device=self.device)
            B.ref_merge_rows(rows, rs, T, dim, ws, n, routed, rrec, stream=stream, dev=self.dev)
        else:
            routed, rrec = rows, rs
        if self.shared is None:
            return routed, rrec
        rec = lambda: torch.empty(4, dtype=torch.int64, device=self.device)  # noqa: E731
        if self.shared_grouped:
            (sg, sgs), (su, sus) = self.shared["gu"].forward_int(x_dev, xs_rec, T, stream=stream)
        else:
            sg, sgs = self.shared["gate"].forward_int(x_dev, xs_rec, T, os_dev=rec(), stream=stream)
            su, sus = self.shared["up"].forward_int(x_dev, xs_rec, T, os_dev=rec(), stream=stream)
        sh = torch.empty(T * self.shared_hidden, dtype=torch.int32, device=self.device)
        shs = rec()
        nsq = B.ref_seq_workspace(1)  # whole-tensor SwiGLU and add on many CTAs
        wsq = torch.empty(nsq, dtype=torch.uint8, device=self.device)
        B.ref_swiglu_seq(sg, sgs, su, sus, T * self.shared_hidden, self.silu_codes, self.silu_lut, wsq, nsq, sh, shs,
                         stream, self.dev)
        sd, sds = self.shared["down"].forward_int(sh, shs, T, os_dev=rec(), stream=stream)
        out = torch.empty(T * dim, dtype=torch.int32, device=self.device)
        orec = rec()
        B.ref_add_seq(routed, rrec, sd, sds, T * dim, wsq, nsq, out, orec, stream, self.dev)
        return out, orec
