"""The config-3 decoder (Qwen2.5-0.5B shape) on one MI355X: the host-side mirror of the reference's DecoderModel
(crates/01-engine/kt-core/src/model.rs:168-188, 290-353) and generate_greedy_by (generate.rs:82-111) over the C ABI.

Every weight matrix is resident in HBM as W12 planes with per-channel scales (gate/up packed with the interleave
the SwiGLU epilogue reads; the embedding doubles as the lm_head, as Qwen2.5-0.5B ties them). A call runs T rows at the
device-held position: embed -> per layer (RmsNorm, q/k/v GEMM, RoPE + KV append, attention, o GEMM added into the
residual, RmsNorm, gate/up GEMM with SwiGLU, down GEMM added into the residual) -> final RmsNorm -> lm_head ->
argmax. For short calls (a decode step) each RmsNorm runs inside the prologue of the product that consumes it. Prefill is one call of T = prompt rows; each decode step is one call of T = 1 fed by the previous argmax on
the device, so a decode step can be captured once as a HIP graph and replayed. torch allocates the device buffers; it
computes nothing.
"""
from __future__ import annotations

import numpy as np

from . import backend as B

QWEN25_05B = dict(d=896, ffn=4864, nh=14, nkv=2, hd=64, layers=24, vocab=151936)


class DecoderModel:
    def __init__(self, cfg: dict, max_pos: int, max_rows: int, h_shift: int = 8, dev: int = 0):
        import torch

        self.torch = torch
        self.cfg = dict(cfg)
        d, ffn, nh, nkv, hd, L, V = (cfg[k] for k in ("d", "ffn", "nh", "nkv", "hd", "layers", "vocab"))
        if d % 64 or ffn % 64 or hd != 64 or nh % nkv:
            raise ValueError("DecoderModel: d and ffn multiples of 64, hd = 64, nh a multiple of nkv")
        self.d, self.ffn, self.nh, self.nkv, self.hd, self.L, self.V = d, ffn, nh, nkv, hd, L, V
        self.nq = (nh + 2 * nkv) * hd
        self.max_pos, self.max_rows, self.h_shift, self.dev = max_pos, max_rows, h_shift, dev
        # calls of at most NORM_MAX_M rows run the RMSNorm inside the qkv / gate-up products' prologue (one launch
        # instead of two); the lm_head's final norm likewise when fuse_norm_head is set (off: its 9,496 CTAs would
        # each repeat the norm, which costs more than the separate launch)
        self.fuse_norm, self.fuse_norm_head = True, False
        # decode steps fold the attention output projection into the calls around it (one launch fewer per layer):
        # each head's attention CTA adds its W_o dot products into o_acc; the gate/up product normalizes the residual
        # with their requantized sums added, and the down product adds them into the residual and clears o_acc
        self.fuse_o = True
        dv = torch.device("cuda", dev)
        self.device = dv

        def zeros(n, dt):
            return torch.zeros(n, dtype=dt, device=dv)

        self.sizes = {
            "qkv": B.w12_bytes(self.nq, d), "o": B.w12_bytes(d, nh * hd), "gu": B.w12_bytes(2 * ffn, d),
            "dn": B.w12_bytes(d, ffn), "emb": B.w12_bytes(V, d),
        }
        self.w = {}
        for name in ("qkv", "o", "gu", "dn"):
            lo, nib = self.sizes[name]
            self.w[name] = (zeros(L * lo, torch.int8), zeros(L * nib, torch.uint8))
        lo, nib = self.sizes["emb"]
        self.w["emb"] = (zeros(lo, torch.int8), zeros(nib, torch.uint8))
        self.emb16 = zeros(V * d, torch.int16)
        nch = {"qkv": self.nq, "o": d, "gu": 2 * ffn, "dn": d}
        self.scale = {k: (zeros(L * n, torch.int32), zeros(L * n, torch.int32)) for k, n in nch.items()}
        self.scale["emb"] = (zeros(V, torch.int32), zeros(V, torch.int32))
        # activations and caches
        R = max_rows
        self.r = zeros(R * d, torch.int32)
        self.xn = zeros(R * d, torch.int8)
        self.qkv = zeros(R * self.nq, torch.int8)
        self.o = zeros(R * nh * hd, torch.int8)
        self.o_acc = zeros(d, torch.int32)  # fuse_o: zero between decode steps (the down product clears it)
        self.h = zeros(R * ffn, torch.int8)
        self.logits = zeros(V, torch.int32)
        self.kc = zeros(L * max_pos * nkv * hd, torch.int8)
        self.vc = zeros(L * max_pos * nkv * hd, torch.int8)
        self.tok_in = zeros(R, torch.int32)
        self.token = zeros(1, torch.int32)
        self.pos = zeros(1, torch.int32)
        self.step = zeros(1, torch.int32)
        self.nparts = min(self.NPARTS, V)  # argmax first-stage CTAs, each with at least one logit
        self.part = torch.zeros(self.nparts, dtype=torch.int64, device=dv)
        self.record = None

    # weights -------------------------------------------------------------------------------------------------------

    def _put(self, name: str, l: int, codes: np.ndarray, n: int, k: int, mant, shift) -> None:
        torch = self.torch
        codes = np.ascontiguousarray(codes, dtype=np.int32)
        if codes.size != n * k or (codes.size and (codes.min() < -2048 or codes.max() > 2047)):
            raise ValueError(f"{name}: codes must be {n} x {k} in [-2048, 2047]")
        lo_b, nib_b = self.sizes[name]
        lo, nib = self.w[name]
        cd = torch.from_numpy(codes).to(self.device)
        if name == "gu":
            B.w12_pack_gate_up(cd, n // 2, k, lo[l * lo_b:(l + 1) * lo_b], nib[l * nib_b:(l + 1) * nib_b], dev=self.dev)
        else:
            B.w12_pack(cd, n, k, lo[l * lo_b:(l + 1) * lo_b], nib[l * nib_b:(l + 1) * nib_b], dev=self.dev)
        m, s = self.scale[name]
        m[l * n:(l + 1) * n] = torch.from_numpy(np.ascontiguousarray(mant, dtype=np.int32))
        s[l * n:(l + 1) * n] = torch.from_numpy(np.ascontiguousarray(shift, dtype=np.int32))
        torch.cuda.synchronize(self.device)

    def set_layer(self, l: int, wqkv, qkv_ms, wo, o_ms, wgu, gu_ms, wd, d_ms) -> None:
        """Layer l: q/k/v codes ((nh + 2 nkv) hd x d), o (d x nh hd), gate/up (2 ffn x d, gate rows first), down
        (d x ffn), each with its (mant, shift) per output channel."""
        d, ffn = self.d, self.ffn
        self._put("qkv", l, wqkv, self.nq, d, *qkv_ms)
        self._put("o", l, wo, d, self.nh * self.hd, *o_ms)
        self._put("gu", l, wgu, 2 * ffn, d, *gu_ms)
        self._put("dn", l, wd, d, ffn, *d_ms)

    def set_embedding(self, emb, lm_ms) -> None:
        """The tied embedding / lm_head codes (vocab x d) and the lm_head's per-row scales."""
        self._put("emb", 0, emb, self.V, self.d, *lm_ms)
        self.emb16.copy_(self.torch.from_numpy(np.ascontiguousarray(emb, dtype=np.int16)))

    def set_tables(self, rope_cos, rope_sin, exp_tab, silu) -> None:
        torch = self.torch
        self.rope_cos = torch.from_numpy(np.ascontiguousarray(rope_cos, dtype=np.int16)).to(self.device)
        self.rope_sin = torch.from_numpy(np.ascontiguousarray(rope_sin, dtype=np.int16)).to(self.device)
        self.exp_tab = torch.from_numpy(np.ascontiguousarray(exp_tab, dtype=np.int32)).to(self.device)
        self.silu = torch.from_numpy(np.ascontiguousarray(silu, dtype=np.int16)).to(self.device)

    # the forward ---------------------------------------------------------------------------------------------------

    NPARTS = 128  # argmax first-stage CTAs

    def forward(self, tokens_dev, T: int, stream=None) -> None:
        """Rows at positions pos .. pos + T - 1 (pos on the device) through every layer; the last row's logits go to
        self.logits and their argmax's first stage to self.part (with the logits recorded at self.record[step] when a
        record is set), and pos advances by T. tokens_dev None: one row, the token the previous call's argmax chose
        (a decode step; step advances by one). Asynchronous on `stream`."""
        if not 1 <= T <= self.max_rows or (tokens_dev is None and T != 1):
            raise ValueError("forward: 1 <= T <= max_rows, and T = 1 for a decode step")
        lib, dev, s = B.lib(), self.dev, B._stream(stream)
        P = B._ptr
        d, ffn, nh, nkv, hd, nq = self.d, self.ffn, self.nh, self.nkv, self.hd, self.nq
        cache = self.max_pos * nkv * hd
        if tokens_dev is None:
            B.check(lib.kt_hip_dec_embed_argmax(dev, P(self.part), self.nparts, P(self.emb16), d, P(self.r),
                                                P(self.token), P(self.step), s), "dec embed argmax")
        else:
            B.check(lib.kt_hip_dec_embed(dev, P(tokens_dev), T, P(self.emb16), d, P(self.r), s), "dec embed")
        fuse = self.fuse_norm and T <= B.NORM_MAX_M  # RMSNorm inside the skinny products' prologue
        # a decode step with the o projection spread over the attention, gate/up and down calls (o_acc between them)
        fold_o = tokens_dev is None and self.fuse_o and fuse and d <= 1024 and ffn <= 8128 and nh * hd <= 8128
        for l in range(self.L):
            kc, vc = P(self.kc) + l * cache, P(self.vc) + l * cache
            if fuse:
                self._gemm_norm("qkv", l, self.r, T, nq, d, self.qkv, B.OUT_I8, s)
            else:
                B.check(lib.kt_hip_dec_rmsnorm(dev, P(self.r), T, d, P(self.xn), d, s), "dec rmsnorm")
                self._gemm("qkv", l, self.xn, T, nq, d, self.qkv, B.OUT_I8, s)
            if fold_o:
                o_lo, o_nib, o_m, o_sh = self._layer_ptrs("o", l, d)
                B.check(lib.kt_hip_dec_attention_o_step(dev, P(self.qkv), P(self.pos), kc, vc, nh, nkv, hd,
                                                        P(self.rope_cos), P(self.rope_sin), P(self.exp_tab),
                                                        self.max_pos, o_lo, o_nib, d, P(self.o_acc), s),
                        "dec attention + o")
            else:
                if tokens_dev is None:
                    B.check(lib.kt_hip_dec_attention_step(dev, P(self.qkv), P(self.pos), kc, vc, nh, nkv, hd,
                                                          P(self.rope_cos), P(self.rope_sin), P(self.exp_tab),
                                                          P(self.o), self.max_pos, s), "dec attention step")
                else:
                    B.check(lib.kt_hip_dec_rope_kv(dev, P(self.qkv), T, nq, P(self.pos), nh, nkv, hd,
                                                   P(self.rope_cos), P(self.rope_sin), kc, vc, s), "dec rope")
                    B.check(lib.kt_hip_dec_attention(dev, P(self.qkv), T, nq, P(self.pos), kc, vc, nh, nkv, hd,
                                                      P(self.exp_tab), P(self.o), self.max_pos, s), "dec attention")
                self._gemm("o", l, self.o, T, d, nh * hd, self.r, B.OUT_I32_ADD, s)
            gu_lo, gu_nib, gu_m, gu_sh = self._layer_ptrs("gu", l, 2 * ffn)
            if fold_o:
                B.check(lib.kt_hip_w12_swiglu_norm_o(dev, P(self.r), gu_lo, gu_nib, ffn, d, gu_m, gu_sh, P(self.silu),
                                                     self.h_shift, P(self.h), P(self.o_acc), o_m, o_sh, s),
                        "dec gate/up + o")
            elif fuse:
                B.check(lib.kt_hip_w12_swiglu_norm(dev, P(self.r), gu_lo, gu_nib, T, ffn, d, gu_m, gu_sh,
                                                   P(self.silu), self.h_shift, P(self.h), ffn, s), "dec gate/up")
            else:
                B.check(lib.kt_hip_dec_rmsnorm(dev, P(self.r), T, d, P(self.xn), d, s), "dec rmsnorm")
                B.check(lib.kt_hip_w12_swiglu(dev, P(self.xn), gu_lo, gu_nib, T, ffn, d, gu_m, gu_sh, P(self.silu),
                                              self.h_shift, P(self.h), ffn, s), "dec gate/up")
            if fold_o:
                dn_lo, dn_nib, dn_m, dn_sh = self._layer_ptrs("dn", l, d)
                B.check(lib.kt_hip_w12_linear_add_o(dev, P(self.h), dn_lo, dn_nib, d, ffn, dn_m, dn_sh, P(self.r),
                                                    P(self.o_acc), o_m, o_sh, s), "dec down + o")
            else:
                self._gemm("dn", l, self.h, T, d, ffn, self.r, B.OUT_I32_ADD, s)
        last = P(self.r) + (T - 1) * d * 4
        if self.fuse_norm_head:
            self._gemm_norm("emb", 0, last, 1, self.V, d, self.logits, B.OUT_I32, s)
        else:
            B.check(lib.kt_hip_dec_rmsnorm(dev, last, 1, d, P(self.xn), d, s), "dec rmsnorm")
            self._gemm("emb", 0, self.xn, 1, self.V, d, self.logits, B.OUT_I32, s)
        rec = P(self.record) if self.record is not None else None
        B.check(lib.kt_hip_dec_argmax_part(dev, P(self.logits), self.V, P(self.part), self.nparts, rec,
                                           P(self.step), P(self.pos), T, s), "dec argmax")

    def _layer_ptrs(self, name, l, N):
        """Device addresses of layer l's lo plane, nib plane, and N per-channel multipliers and shifts."""
        lo_b, nib_b = self.sizes[name]
        lo, nib = self.w[name]
        m, sh = self.scale[name]
        P = B._ptr
        return P(lo) + l * lo_b, P(nib) + l * nib_b, P(m) + l * N * 4, P(sh) + l * N * 4

    def _gemm(self, name, l, x, M, N, K, y, out_kind, s) -> None:
        lo_b, nib_b = self.sizes[name]
        lo, nib = self.w[name]
        m, sh = self.scale[name]
        P = B._ptr
        B.check(B.lib().kt_hip_w12_linear(self.dev, P(x), P(lo) + l * lo_b, P(nib) + l * nib_b, M, N, K,
                                          P(m) + l * N * 4, P(sh) + l * N * 4, out_kind, P(y), s), f"dec {name}")

    def _gemm_norm(self, name, l, r, M, N, K, y, out_kind, s) -> None:
        lo_b, nib_b = self.sizes[name]
        lo, nib = self.w[name]
        m, sh = self.scale[name]
        P = B._ptr
        B.check(B.lib().kt_hip_w12_linear_norm(self.dev, P(r), P(lo) + l * lo_b, P(nib) + l * nib_b, M, N, K,
                                               P(m) + l * N * 4, P(sh) + l * N * 4, out_kind, P(y), s),
                f"dec {name} (norm)")

    def decode_step(self, stream=None) -> None:
        """DecoderModel::decode_step on the device: the previous argmax's token at the current position."""
        self.forward(None, 1, stream)

    def generate(self, prompt, max_new: int, graph: bool = False, stream=None):
        """generate_greedy_by with no stop tokens: prefill the prompt as one call, then max_new - 1 decode steps.
        Returns (tokens, logits) of every step (max_new x vocab int32), the rows the logits hash covers."""
        torch = self.torch
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        P = prompt.size
        if P < 1 or P > self.max_rows or P + max_new - 1 > self.max_pos:
            raise ValueError("generate: the prompt and the steps must fit max_rows / max_pos")
        self.record = torch.zeros(max_new * self.V, dtype=torch.int32, device=self.device)
        self.pos.zero_()
        self.step.zero_()
        self.tok_in[:P] = torch.from_numpy(prompt).to(self.device)
        self.forward(self.tok_in, P, stream)
        steps = max_new - 1
        if graph and steps > 0:
            g = self.capture_decode_step()
            for _ in range(steps):
                g.replay()
        else:
            for _ in range(steps):
                self.decode_step(stream)
        torch.cuda.synchronize(self.device)
        logits = self.record.cpu().numpy().reshape(max_new, self.V)
        return logits.argmax(axis=1).astype(np.int32), logits

    def capture_decode_step(self):
        """One decode step captured as a HIP graph (every position and token is read from device memory)."""
        torch = self.torch
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            g.capture_begin()
            self.decode_step(stream=s)
            g.capture_end()
        torch.cuda.current_stream(self.device).wait_stream(s)
        return g
