"""The reference's decoder at its own integer semantics on one MI355X: the host-side mirror of DecoderModel
(crates/01-engine/kt-core/src/model.rs) with every op of a decode step on the device.

The reference runs its decoder on 12-trit weight codes with per-tensor kt-int Scales; activations are i32 codes at
the 2^28 level, quantized dynamically per tensor after every op. `RefDecoder` keeps those integers exactly:

  embed                       kt_hip_ref_embed               Embedding::lookup          (layers.rs:1127-1140)
  input_norm / post_norm      kt_hip_ref_rmsnorm             RmsNorm::forward_int        (layers.rs:392-434)
  wq, wk, wv, wo, gate, up,   kt_hip_quant_linear            QuantLinear::forward_int    (layers.rs:275-328)
    down, lm_head             (digit-plane MFMA product)
  attention core              kt_hip_ref_attention_step      Attention::decode_step      (attention.rs:340-459)
  SiLU * up                   kt_hip_ref_swiglu              SwiGluMlp::forward_int      (layers.rs:609-640)
  residual adds               kt_hip_ref_add_rmsnorm         add, then the next RmsNorm  (layers.rs:121-136,
                              (one launch; kt_hip_ref_add)                               392-434)
  greedy choice               kt_hip_ref_argmax              argmax_codes                (generate.rs:48-56)
  sequence forward            kt_hip_ref_embed_seq,          CausalLM::forward_int       (model.rs:361-367,
    (prefill)                 kt_hip_ref_attention_prefill,  Attention::forward_int       168-189; attention.rs:
                              kt_hip_ref_*_seq (many CTAs)                                467-598)

The weights come in as the engine builds them (codes and Scales, `QuantLinear::from_weights` and its siblings);
the run-time tables (RoPE Scales, the exp and SiLU CodeLuts, 1/sqrt(head_dim)) are built here from the
configuration, as `Attention::new` and `SwiGluMlp::new` build them. `generate_greedy` follows generate_greedy_by
(generate.rs:82-111) and repro::run (crates/04-ingest/kt-convert/src/repro.rs:60-84): the prompt position by
position, then greedy tokens; every position's logits are hashed with the scale first (logits_hash, repro.rs:34-42)
and the run's hash covers every step that chose a token (hash_step, generate.rs:58-64).

torch holds the device buffers; it computes nothing.
"""
from __future__ import annotations

import hashlib
import math

import numpy as np

from . import backend as B
from .quant import QuantLinear, QuantLinearGroup

QL_NAMES = ("wq", "wk", "wv", "wo", "gate", "up", "down")


def logits_hash_bytes(codes: np.ndarray, scale) -> bytes:
    """The bytes one step adds to the generation hash: mant (i64 LE), shift (i32 LE), every code (i32 LE)."""
    return (np.int64(scale[0]).tobytes() + np.int32(scale[1]).tobytes() +
            np.ascontiguousarray(codes, dtype="<i4").tobytes())


class RefDecoder:
    """DecoderModel { emb, blocks, final_norm, lm_head } resident on device `dev`.

    cfg: dim, layers, nh, nkv, hd, hidden, vocab, eps, theta, max_seq (DecoderConfig, model.rs:17-29).
    emb, lm_head: (codes vocab x dim, (mant, shift)); final_norm: (codes dim, (mant, shift)); layers: one dict per
    block with in_norm, post_norm (codes dim, scale) and wq, wk, wv, wo, gate, up, down (codes out x in, scale).
    """

    def __init__(self, cfg: dict, emb, final_norm, lm_head, layers, dev: int = 0):
        import torch

        self.torch = torch
        self.dev = dev
        self.device = torch.device("cuda", dev)
        c = {k: cfg[k] for k in ("dim", "layers", "nh", "nkv", "hd", "hidden", "vocab", "max_seq")}
        self.dim, self.nl, self.nh, self.nkv, self.hd = c["dim"], c["layers"], c["nh"], c["nkv"], c["hd"]
        self.hidden, self.vocab, self.max_seq = c["hidden"], c["vocab"], c["max_seq"]
        if self.nh % self.nkv or self.hd % 2 or self.nh > B.REF_MAX_HEADS or len(layers) != self.nl:
            raise ValueError("RefDecoder: heads, head_dim or layer count out of range")
        dt = lambda a, t: torch.from_numpy(np.ascontiguousarray(a, dtype=t).reshape(-1)).to(self.device)  # noqa
        self.eps = B.ref_scale_from_f64(cfg["eps"])
        self.emb = dt(emb[0], np.int32)
        self.emb_scale = tuple(emb[1])
        self.final_norm = (dt(final_norm[0], np.int32), tuple(final_norm[1]))
        qd, kvd = self.nh * self.hd, self.nkv * self.hd
        shapes = {"wq": (qd, self.dim), "wk": (kvd, self.dim), "wv": (kvd, self.dim), "wo": (self.dim, qd),
                  "gate": (self.hidden, self.dim), "up": (self.hidden, self.dim), "down": (self.dim, self.hidden)}
        # q / k / v and gate / up each read one tensor: where their output boundaries allow, each trio / pair is one
        # QuantLinearGroup (one device call, the same integers as the separate QuantLinears)
        self.grouped = QuantLinearGroup.fits((qd, kvd, kvd)) and QuantLinearGroup.fits((self.hidden, self.hidden))
        self.blocks = []
        for i, lw in enumerate(layers):
            blk = {n: (dt(lw[n][0], np.int32), tuple(lw[n][1])) for n in ("in_norm", "post_norm")}
            for n in QL_NAMES:
                if self.grouped and n in ("wq", "wk", "wv", "gate", "up"):
                    continue
                out, inp = shapes[n]
                blk[n] = QuantLinear(f"{n}{i}", lw[n][0], out, inp, lw[n][1], dev=dev)
            if self.grouped:
                blk["qkv"] = QuantLinearGroup(f"qkv{i}", [(n, lw[n][0], lw[n][1], None) for n in ("wq", "wk", "wv")],
                                              self.dim, dev=dev)
                blk["gu"] = QuantLinearGroup(f"gu{i}", [(n, lw[n][0], lw[n][1], None) for n in ("gate", "up")],
                                             self.dim, dev=dev)
            self.blocks.append(blk)
        self.lm_head = QuantLinear("lm_head", lm_head[0], self.vocab, self.dim, lm_head[1], dev=dev)
        # the run-time tables of Attention::new and SwiGluMlp::new
        cos_t, sin_t = B.ref_rope_tables(self.max_seq, self.hd, float(cfg["theta"]))
        self.cos = torch.from_numpy(cos_t.view(np.uint8)).to(self.device)
        self.sin = torch.from_numpy(sin_t.view(np.uint8)).to(self.device)
        self.inv_sqrt = B.ref_scale_from_f64(1.0 / math.sqrt(self.hd))
        exp_codes, self.exp_lut = B.ref_codelut(B.LUT_EXP, -30.0, 0.0, 16, 20, False)
        silu_codes, self.silu_lut = B.ref_codelut(B.LUT_SILU, -30.0, 30.0, 16, 20, True)
        self.exp_codes, self.silu_codes = dt(exp_codes, np.int64), dt(silu_codes, np.int64)
        # one token's buffers and records
        z = lambda n: torch.zeros(n, dtype=torch.int32, device=self.device)  # noqa
        rec = lambda: torch.zeros(4, dtype=torch.int64, device=self.device)  # noqa
        self.buf = {n: z(sz) for n, sz in (("x", self.dim), ("h", self.dim), ("a", self.dim), ("m", self.dim),
                                           ("q", qd), ("k", kvd), ("v", kvd), ("cat", qd), ("g", self.hidden),
                                           ("u", self.hidden), ("hh", self.hidden), ("logits", self.vocab))}
        self.rec = {n: rec() for n in self.buf}
        # a group writes its members' records side by side: q / k / v and g / u as views of one buffer each
        qkv_rec, gu_rec = torch.zeros(12, dtype=torch.int64, device=self.device), torch.zeros(8, dtype=torch.int64,
                                                                                                device=self.device)
        self.rec.update(q=qkv_rec[0:4], k=qkv_rec[4:8], v=qkv_rec[8:12], g=gu_rec[0:4], u=gu_rec[4:8])
        self._rec_qkv, self._rec_gu = qkv_rec, gu_rec
        self.token = z(1)
        self.pos = z(1)
        # the attention step on several CTAs per head, its workspace shared by the layers (their steps run in order on
        # one stream); attn_heads=False keeps the one-CTA step where its LDS holds max_seq
        self.attn_ws = None
        if cfg.get("attn_heads", True) or not B.ref_attention_step_fits_lds(self.max_seq, self.nh, self.hd):
            n = B.ref_attention_step_workspace(self.max_seq, self.nh, self.hd)
            if n == 0:
                raise ValueError(f"max_seq {self.max_seq} beyond the attention step's limit")
            self.attn_ws = torch.empty((n + 15) // 16 * 16, dtype=torch.uint8, device=self.device)
        # each projection stops at its exact sums and the op reading its output applies requant_dyn (four launches
        # fewer per layer, the same integers); sums=False keeps the requant launches
        self.sums = (cfg.get("sums", True) and self.grouped and self.attn_ws is not None and
                     self.dim <= B.REF_ADD_NORM_MAX and self.hidden <= B.REF_SWIGLU_SUMS_MAX and
                     all(blk[n].sums_ok() for blk in self.blocks for n in ("qkv", "wo", "gu", "down")))
        self.new_cache()

    def new_cache(self) -> None:
        """A fresh KV cache (DecoderModel::new_cache, model.rs:280-284): per layer k and v codes and per-step scales."""
        torch = self.torch
        if hasattr(self, "kc"):  # in place: a captured step keeps these buffers' addresses
            for t in self.kc + self.vc + self.ks + self.vs:
                t.zero_()
            return
        kvd = self.nkv * self.hd
        self.kc = [torch.zeros(self.max_seq * kvd, dtype=torch.int32, device=self.device) for _ in range(self.nl)]
        self.vc = [torch.zeros(self.max_seq * kvd, dtype=torch.int32, device=self.device) for _ in range(self.nl)]
        self.ks = [torch.zeros(self.max_seq * 16, dtype=torch.uint8, device=self.device) for _ in range(self.nl)]
        self.vs = [torch.zeros(self.max_seq * 16, dtype=torch.uint8, device=self.device) for _ in range(self.nl)]

    def _ql(self, ql: QuantLinear, x: str, y: str, stream) -> None:
        ql.forward_int(self.buf[x], self.rec[x], 1, y_dev=self.buf[y], os_dev=self.rec[y], stream=stream)

    def step_launches(self, stream=None) -> None:
        """DecoderModel::decode_step (model.rs:290-294, 338-353) of the token at self.token, position self.pos (both
        device int32): every launch on `stream`, no host synchronization; the logits land in buf["logits"] with
        their scale in rec["logits"]."""
        b, r, dv = self.buf, self.rec, self.dev
        # a residual add and the norm after it are one launch where the row allows (the same integers)
        fuse = self.dim <= B.REF_ADD_NORM_MAX

        def add_norm(branch, norm):
            g_, gs_ = norm
            if fuse:
                B.ref_add_rmsnorm(b["x"], r["x"], b[branch], r[branch], self.dim, b["x"], r["x"], g_, gs_, self.eps,
                                  b["h"], r["h"], stream, dv)
            else:
                B.ref_add(b["x"], r["x"], b[branch], r[branch], self.dim, b["x"], r["x"], stream, dv)
                B.ref_rmsnorm(b["x"], r["x"], 1, self.dim, g_, gs_, self.eps, b["h"], r["h"], stream, dv)

        B.ref_embed(self.emb, self.emb_scale, self.token, self.vocab, self.dim, b["x"], r["x"], stream, dv)
        g, gs = self.blocks[0]["in_norm"] if self.blocks else self.final_norm
        B.ref_rmsnorm(b["x"], r["x"], 1, self.dim, g, gs, self.eps, b["h"], r["h"], stream, dv)
        for i, blk in enumerate(self.blocks):
            if self.sums:
                self._block_sums(i, blk, stream)
                continue
            if self.grouped:
                blk["qkv"].forward_int(b["h"], r["h"], 1, y_devs=[b["q"], b["k"], b["v"]], os_dev=self._rec_qkv,
                                       stream=stream)
            else:
                for n, out in (("wq", "q"), ("wk", "k"), ("wv", "v")):
                    self._ql(blk[n], "h", out, stream)
            B.ref_attention_step(b["q"], r["q"], b["k"], r["k"], b["v"], r["v"], self.pos, self.nh, self.nkv,
                                 self.hd, self.max_seq, self.kc[i], self.vc[i], self.ks[i], self.vs[i], self.cos,
                                 self.sin, self.inv_sqrt, self.exp_codes, self.exp_lut, b["cat"], r["cat"], stream,
                                 dv, ws_dev=self.attn_ws)
            self._ql(blk["wo"], "cat", "a", stream)
            add_norm("a", blk["post_norm"])
            if self.grouped:
                blk["gu"].forward_int(b["h"], r["h"], 1, y_devs=[b["g"], b["u"]], os_dev=self._rec_gu, stream=stream)
            else:
                self._ql(blk["gate"], "h", "g", stream)
                self._ql(blk["up"], "h", "u", stream)
            B.ref_swiglu(b["g"], r["g"], b["u"], r["u"], self.hidden, self.silu_codes, self.silu_lut, b["hh"],
                         r["hh"], stream, dv)  # one tensor (rows = 1)
            self._ql(blk["down"], "hh", "m", stream)
            # the next block's input norm, or the final norm after the last block
            add_norm("m", self.blocks[i + 1]["in_norm"] if i + 1 < len(self.blocks) else self.final_norm)
        self._ql(self.lm_head, "h", "logits", stream)

    def _block_sums(self, i: int, blk, stream) -> None:
        """One block of decode_step with each projection stopped at its sums and requantized by its reader: q / k / v
        -> attention, o -> add + post norm, gate / up -> SwiGLU, down -> add + the next norm (9 launches)."""
        b, r, dv = self.buf, self.rec, self.dev
        q, k, v = blk["qkv"].forward_sums(b["h"], r["h"], os_dev=self._rec_qkv, stream=stream)
        B.ref_attention_step_sums(q, k, v, self.pos, self.nh, self.nkv, self.hd, self.max_seq, self.kc[i], self.vc[i],
                                  self.ks[i], self.vs[i], self.cos, self.sin, self.inv_sqrt, self.exp_codes,
                                  self.exp_lut, b["cat"], r["cat"], self.attn_ws, stream, dv)
        a = blk["wo"].forward_sums(b["cat"], r["cat"], rec=r["a"], stream=stream)
        g_, gs_ = blk["post_norm"]
        B.ref_add_rmsnorm_sums(b["x"], r["x"], a, self.dim, b["x"], r["x"], g_, gs_, self.eps, b["h"], r["h"], stream,
                               dv)
        gt, up = blk["gu"].forward_sums(b["h"], r["h"], os_dev=self._rec_gu, stream=stream)
        B.ref_swiglu_sums(gt, up, self.hidden, self.silu_codes, self.silu_lut, b["hh"], r["hh"], stream, dv)
        m = blk["down"].forward_sums(b["hh"], r["hh"], rec=r["m"], stream=stream)
        g_, gs_ = self.blocks[i + 1]["in_norm"] if i + 1 < len(self.blocks) else self.final_norm
        B.ref_add_rmsnorm_sums(b["x"], r["x"], m, self.dim, b["x"], r["x"], g_, gs_, self.eps, b["h"], r["h"], stream,
                               dv)

    def capture_greedy_step(self):
        """One position of greedy decoding as a HIP graph: decode_step of the token at self.token and position
        self.pos, then argmax_codes into self.token, with the position's logits and scale recorded at
        self.record[pos] and self.rscale[pos] and self.pos advanced -- so replays run a greedy generation with no host
        work (a prompt position overwrites self.token before its replay). Call after one eager step (the launches'
        workspaces exist)."""
        torch = self.torch
        if not hasattr(self, "record"):
            self.record = torch.zeros(self.max_seq * self.vocab, dtype=torch.int32, device=self.device)
            self.rscale = torch.zeros(self.max_seq * 16, dtype=torch.uint8, device=self.device)
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            g.capture_begin()
            self.step_launches(stream=s)
            B.ref_argmax(self.buf["logits"], self.vocab, self.rec["logits"], self.token, self.record, self.rscale,
                         self.pos, s, self.dev, record_rows=self.max_seq)
            g.capture_end()
        torch.cuda.current_stream(self.device).wait_stream(s)
        return g

    def recorded(self, pos: int):
        """The logits and scale a captured greedy step recorded at position `pos`: (codes, (mant, shift))."""
        codes = self.record[pos * self.vocab:(pos + 1) * self.vocab].cpu().numpy()
        w = self.rscale[pos * 16:(pos + 1) * 16].cpu().numpy()
        return codes, (int(w.view(np.int64)[0]), int(w.view(np.int32)[2]))

    def forward(self, tokens, stream=None):
        """CausalLM::forward_int (model.rs:361-367 = embed_int, blocks_int, head_int): the T tokens as one sequence,
        every op over the whole T-row tensor (one dynamic quantization per tensor, the prefill attention at one
        score scale): (logits T x vocab codes, their record), device tensors. Independent of the KV cache."""
        torch = self.torch
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        T = int(toks.size)
        if not 1 <= T <= self.max_seq:
            raise ValueError(f"forward: {T} tokens, max_seq {self.max_seq}")
        if toks.min() < 0 or toks.max() >= self.vocab:
            raise ValueError("forward: a token outside the vocabulary")
        d, dv = self.device, self.dev
        z = lambda n: torch.empty(n, dtype=torch.int32, device=d)  # noqa: E731
        rec = lambda: torch.zeros(4, dtype=torch.int64, device=d)  # noqa: E731
        qd, kvd = self.nh * self.hd, self.nkv * self.hd
        x, xr, h, hr = z(T * self.dim), rec(), z(T * self.dim), rec()
        t_dev = torch.from_numpy(toks).to(d)
        B.ref_embed_seq(self.emb, self.emb_scale, t_dev, T, self.vocab, self.dim, x, xr, stream, dv)
        nws = B.ref_attention_prefill_workspace(T, self.nh, self.nkv, self.hd)
        ws = torch.empty(nws, dtype=torch.uint8, device=d)
        nsq = B.ref_seq_workspace(T)  # the many-CTA norm / add / SwiGLU over the T-row tensors
        wsq = torch.empty(nsq, dtype=torch.uint8, device=d)
        norm = lambda x_, xr_, g_, y_, yr_: B.ref_rmsnorm_seq(x_, xr_, T, self.dim, g_[0], g_[1], self.eps, wsq, nsq,  # noqa: E731
                                                                 y_, yr_, stream, dv)
        add = lambda y_, yr_, b_, br_: B.ref_add_seq(y_, yr_, b_, br_, T * self.dim, wsq, nsq, y_, yr_, stream, dv)  # noqa: E731
        cat, cr, a, ar, hh, hhr = z(T * qd), rec(), z(T * self.dim), rec(), z(T * self.hidden), rec()
        for blk in self.blocks:
            norm(x, xr, blk["in_norm"], h, hr)
            if self.grouped:
                (q, qr), (k, kr), (v, vr) = blk["qkv"].forward_int(h, hr, T, stream=stream)
            else:
                q, qr = blk["wq"].forward_int(h, hr, T, stream=stream)
                k, kr = blk["wk"].forward_int(h, hr, T, stream=stream)
                v, vr = blk["wv"].forward_int(h, hr, T, stream=stream)
            B.ref_attention_prefill(q, qr, k, kr, v, vr, T, self.nh, self.nkv, self.hd, self.max_seq, self.cos,
                                    self.sin, self.inv_sqrt, self.exp_codes, self.exp_lut, ws, nws, cat, cr, stream,
                                    dv)
            blk["wo"].forward_int(cat, cr, T, y_dev=a, os_dev=ar, stream=stream)
            add(x, xr, a, ar)
            norm(x, xr, blk["post_norm"], h, hr)
            if self.grouped:
                (gt, gtr), (up, upr) = blk["gu"].forward_int(h, hr, T, stream=stream)
            else:
                gt, gtr = blk["gate"].forward_int(h, hr, T, stream=stream)
                up, upr = blk["up"].forward_int(h, hr, T, stream=stream)
            B.ref_swiglu_seq(gt, gtr, up, upr, T * self.hidden, self.silu_codes, self.silu_lut, wsq, nsq, hh, hhr,
                             stream, dv)
            m, mr = blk["down"].forward_int(hh, hhr, T, stream=stream)
            add(x, xr, m, mr)
        norm(x, xr, self.final_norm, h, hr)
        return self.lm_head.forward_int(h, hr, T, stream=stream)

    def decode_step(self, token: int, pos: int):
        """The logits of `token` at `pos` against the cache: (codes, (mant, shift)) on the host."""
        if not 0 <= pos < self.max_seq:
            raise ValueError(f"position {pos} beyond the tables' {self.max_seq}")
        if not 0 <= token < self.vocab:
            raise ValueError(f"token {token} out of vocab {self.vocab}")
        self.token.fill_(int(token))
        self.pos.fill_(int(pos))
        self.step_launches()
        return self.read_logits()

    def read_logits(self):
        self.torch.cuda.synchronize(self.device)
        w = self.rec["logits"].cpu().numpy()
        return self.buf["logits"].cpu().numpy(), (int(w[0]), int(w.view(np.int32)[2]))

    def generate_greedy(self, prompt, max_new: int, stop=()):
        """generate_greedy_by as repro::run drives it: (tokens, run logits_hash hex, per-position hashes hex)."""
        if len(prompt) == 0:
            raise ValueError("generate: the prompt is empty")
        self.new_cache()
        hashes, run = [], hashlib.sha256()
        logits = None
        for pos, t in enumerate(prompt):
            logits = self.decode_step(int(t), pos)
            hashes.append(hashlib.sha256(logits_hash_bytes(*logits)).hexdigest())
        tokens, pos = [], len(prompt)
        while len(tokens) < max_new:
            codes, scale = logits
            run.update(logits_hash_bytes(codes, scale))
            nxt = int(np.argmax(codes))  # the first maximum, as argmax_codes
            if nxt in stop:
                break
            tokens.append(nxt)
            if len(tokens) < max_new:
                logits = self.decode_step(nxt, pos)
                hashes.append(hashlib.sha256(logits_hash_bytes(*logits)).hexdigest())
                pos += 1
        return tokens, run.hexdigest(), hashes
