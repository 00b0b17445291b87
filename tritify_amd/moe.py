"""The config-4 MoE layer on one MI355X: the host-side mirror of the reference's MoeMlp
(crates/01-engine/kt-core/src/layers.rs:722-1020) over the C ABI's MoE entry points.

`MoeLayer` keeps every expert's weights resident in HBM as W12 planes (gate/up packed with the 32-row interleave the
SwiGLU epilogue reads) with their per-channel scales, and runs the layer as five asynchronous launches: route,
bucket, the gate/up grouped GEMM with the SwiGLU epilogue, the down grouped GEMM, combine. The stage methods
(`route`, `bucket`, `experts`, `combine`) are the reference's expert-parallel seam (route -> experts_fn -> combine,
layers.rs:826-986) one launch each. torch allocates the device buffers; it computes nothing.
"""
from __future__ import annotations

import numpy as np

from . import backend as B


class MoeLayer:
    def __init__(self, hidden: int, ffn: int, experts: int, top_k: int, silu: np.ndarray, sig: np.ndarray,
                 h_shift: int, out_shift: int, dev: int = 0):
        import torch

        if hidden % 64 or ffn % 64:
            raise ValueError("MoeLayer: hidden and ffn must be multiples of 64")
        if not (1 <= top_k <= min(experts, 32)) or experts + 1 > B.MAX_GROUPS:
            raise ValueError("MoeLayer: 1 <= top_k <= min(experts, 32) and experts + 1 <= MAX_GROUPS")
        self.H, self.F, self.E, self.K = hidden, ffn, experts, top_k
        self.h_shift, self.out_shift, self.dev = h_shift, out_shift, dev
        self.torch = torch
        d = torch.device("cuda", dev)
        self.device = d
        G = experts + 1
        self.gu_lo_bytes, _ = B.w12_bytes(2 * ffn, hidden)
        self.d_lo_bytes, _ = B.w12_bytes(hidden, ffn)
        self.gu_lo = torch.zeros(G * self.gu_lo_bytes, dtype=torch.int8, device=d)
        self.gu_nib = torch.zeros(G * self.gu_lo_bytes // 2, dtype=torch.uint8, device=d)
        self.d_lo = torch.zeros(G * self.d_lo_bytes, dtype=torch.int8, device=d)
        self.d_nib = torch.zeros(G * self.d_lo_bytes // 2, dtype=torch.uint8, device=d)
        self.gu_mant = torch.zeros(G * 2 * ffn, dtype=torch.int32, device=d)
        self.gu_shift = torch.zeros(G * 2 * ffn, dtype=torch.int32, device=d)
        self.d_mant = torch.zeros(G * hidden, dtype=torch.int32, device=d)
        self.d_shift = torch.zeros(G * hidden, dtype=torch.int32, device=d)
        self.silu = torch.from_numpy(np.ascontiguousarray(silu, dtype=np.int16)).to(d)
        self.sig = torch.from_numpy(np.ascontiguousarray(sig, dtype=np.int16)).to(d)
        self._ws = None
        self._ws_tokens = -1

    def set_expert(self, g: int, gate_up: np.ndarray, down: np.ndarray, gm, gs, dm, ds) -> None:
        """Expert g (g == experts: the shared expert): gate/up codes 2F x H (gate rows first), down codes H x F,
        all in [-2048, 2047], and their per-channel scales."""
        torch = self.torch
        H, F = self.H, self.F
        gate_up = np.ascontiguousarray(gate_up, dtype=np.int32)
        down = np.ascontiguousarray(down, dtype=np.int32)
        if gate_up.size != 2 * F * H or down.size != H * F:
            raise ValueError("set_expert: shapes")
        for a in (gate_up, down):
            if a.size and (a.min() < -2048 or a.max() > 2047):
                raise ValueError("set_expert: codes outside [-2048, 2047]")
        cg = torch.from_numpy(gate_up).to(self.device)
        cd = torch.from_numpy(down).to(self.device)
        a, b = g * self.gu_lo_bytes, (g + 1) * self.gu_lo_bytes
        B.w12_pack_gate_up(cg, F, H, self.gu_lo[a:b], self.gu_nib[a // 2:b // 2], dev=self.dev)
        a, b = g * self.d_lo_bytes, (g + 1) * self.d_lo_bytes
        B.w12_pack(cd, H, F, self.d_lo[a:b], self.d_nib[a // 2:b // 2], dev=self.dev)
        self.gu_mant[g * 2 * F:(g + 1) * 2 * F] = torch.from_numpy(np.ascontiguousarray(gm, dtype=np.int32))
        self.gu_shift[g * 2 * F:(g + 1) * 2 * F] = torch.from_numpy(np.ascontiguousarray(gs, dtype=np.int32))
        self.d_mant[g * H:(g + 1) * H] = torch.from_numpy(np.ascontiguousarray(dm, dtype=np.int32))
        self.d_shift[g * H:(g + 1) * H] = torch.from_numpy(np.ascontiguousarray(ds, dtype=np.int32))
        torch.cuda.synchronize(self.device)

    def workspace(self, tokens: int):
        """The device workspace for `tokens` tokens (grown on demand) and its parts as typed views."""
        torch = self.torch
        total, offs = B.moe_workspace(tokens, self.H, self.F, self.E, self.K)
        if self._ws is None or self._ws.numel() < total:
            self._ws = torch.empty(total, dtype=torch.uint8, device=self.device)
        T, K, E, P = tokens, self.K, self.E, tokens * (self.K + 1)
        ws = self._ws

        def part(name, n, dt):
            o = offs[name]
            return ws[o:o + n * torch.tensor([], dtype=dt).element_size()].view(dt)

        views = dict(sel=part("sel", T * K, torch.int32), cw=part("cw", T * K, torch.int32),
                     pos=part("pos", T * K, torch.int32), list=part("list", (E + 1) * T, torch.int32),
                     count=part("count", E + 1, torch.int32), off=part("off", E + 2, torch.int32),
                     h=part("h", P * self.F, torch.int8), d=part("d", P * self.H, torch.int8))
        return ws, views

    def forward(self, x_dev, logits_dev, tokens: int, out_dev, stream=None) -> dict:
        """out = the layer on x (T x H int8) and router codes (T x E int32). Returns the workspace views."""
        ws, views = self.workspace(tokens)
        B.moe_forward(x_dev, logits_dev, tokens, self.H, self.F, self.E, self.K, self.gu_lo, self.gu_nib,
                      self.gu_mant, self.gu_shift, self.d_lo, self.d_nib, self.d_mant, self.d_shift, self.silu,
                      self.sig, self.h_shift, self.out_shift, ws, out_dev, stream=stream, dev=self.dev)
        return views

    # the expert-parallel seam, one launch per stage ----------------------------------------------------------------

    def route(self, logits_dev, tokens: int, sel_dev, cw_dev, stream=None) -> None:
        B.moe_route(logits_dev, tokens, self.E, self.K, self.sig, sel_dev, cw_dev, stream=stream, dev=self.dev)

    def bucket(self, sel_dev, tokens: int, list_dev, pos_dev, count_dev, stream=None) -> None:
        B.moe_bucket(sel_dev, tokens, self.E, self.K, list_dev, pos_dev, count_dev, stream=stream, dev=self.dev)

    def experts(self, x_dev, tokens: int, list_dev, count_dev, h_dev, d_dev, off_dev, stream=None) -> None:
        """Every expert on its bucket: h (P x F) through the SwiGLU epilogue, then d (P x H)."""
        P = tokens * (self.K + 1)
        B.w12_grouped_linear(x_dev, tokens, list_dev, tokens, count_dev, self.E + 1, P, self.gu_lo, self.gu_nib,
                             2 * self.F, self.H, self.gu_mant, self.gu_shift, B.EPI_SWIGLU, h_dev, self.F,
                             silu_dev=self.silu, h_shift=self.h_shift, off_dev=off_dev, stream=stream, dev=self.dev)
        B.w12_grouped_linear(h_dev, P, None, 0, count_dev, self.E + 1, P, self.d_lo, self.d_nib, self.H, self.F,
                             self.d_mant, self.d_shift, B.EPI_I8, d_dev, self.H, stream=stream, dev=self.dev)

    def combine(self, d_dev, off_dev, sel_dev, cw_dev, pos_dev, tokens: int, out_dev, stream=None) -> None:
        B.moe_combine(d_dev, off_dev, sel_dev, cw_dev, pos_dev, tokens, self.H, self.E, self.K, self.out_shift,
                      out_dev, stream=stream, dev=self.dev)
