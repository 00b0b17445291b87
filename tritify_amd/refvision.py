"""SAM 2.1's image path at the reference's own integer semantics on one MI355X: the host-side mirror of the Hiera
PatchEmbed and FeedForward (crates/03-models/kt-model-vision/src/hiera.rs:165-190, 321-345) over the reference's
Conv2d (crates/01-engine/kt-core/src/conv.rs:22-130) and GELU CodeLut (nonlin.rs:7-47).

  pixel entry        kt_hip_ref_from_reals   IntTensor::from_reals at ACT_LEVELS       (tensor.rs:106-117)
  patch embed        kt_hip_ref_conv2d       Conv2d::forward_int: whole-image quant_to, (conv.rs:68-130)
                                             the im2col rows through the digit-plane GEMM, bias, whole-output
                                             requant_dyn, stored [c_out][oh][ow]
  proj_in, proj_out  kt_hip_quant_linear     QuantLinear::forward_int (+ bias)          (layers.rs:275-328)
  GELU               kt_hip_ref_gelu         apply_gelu by the A&S-erf CodeLut          (nonlin.rs:24-45)

The weights come in as the engine builds them (codes and Scales, `Conv2d::from_weights` / `with_bias`); the GELU
table is built here as `build_gelu_lut` builds it. torch holds the device buffers; it computes nothing.
"""
from __future__ import annotations

import numpy as np

from . import backend as B
from .quant import QuantLinear

ACT_LEVELS = 1 << 28


def gelu_table(dev: int = 0):
    """build_gelu_lut (nonlin.rs:24-26): CodeLut(gelu, -10, 10, 2^16 entries, 2^20 code scale, identity right tail)
    as (device codes, constants)."""
    import torch

    codes, lut = B.ref_codelut(B.LUT_GELU, -10.0, 10.0, 16, 20, True)
    return torch.from_numpy(codes).to(torch.device("cuda", dev)), lut


class RefConv2d:
    """Conv2d { w_codes [c_out][c_in][kh][kw], w_scale, stride, pad, bias } with the weights resident on device
    `dev` as the digit planes of the c_out x (c_in kh kw) matrix."""

    def __init__(self, w_codes, w_scale, stride: int, pad: int, bias=None, dev: int = 0):
        import torch

        self.torch = torch
        self.dev = dev
        self.device = torch.device("cuda", dev)
        w = np.ascontiguousarray(w_codes, dtype=np.int32)
        if w.ndim != 4:
            raise ValueError("RefConv2d: weights are [c_out][c_in][kh][kw]")
        self.co, self.ci, self.kh, self.kw = (int(v) for v in w.shape)
        self.stride, self.pad = int(stride), int(pad)
        if self.stride < 1 or self.pad < 0:
            raise ValueError("RefConv2d: stride >= 1 and pad >= 0")
        self.w_scale = (int(w_scale[0]), int(w_scale[1]))
        k = self.ci * self.kh * self.kw
        flat = w.reshape(self.co, k)
        self.pw = B.planes_for(flat)
        self.w_planes = torch.empty(self.pw * self.co * B.kp(k), dtype=torch.int8, device=self.device)
        B.pack_planes(torch.from_numpy(flat.reshape(-1)).to(self.device), self.co, k, self.pw, self.w_planes, dev=dev)
        if bias is not None:
            b = np.ascontiguousarray(bias[0], dtype=np.int64)
            if b.size != self.co:
                raise ValueError("RefConv2d: bias len mismatch")
            self.bias, self.b_scale = torch.from_numpy(b).to(self.device), (int(bias[1][0]), int(bias[1][1]))
        else:
            self.bias, self.b_scale = None, None
        torch.cuda.synchronize(self.device)
        self._ws: dict[tuple, tuple] = {}

    def out_dims(self, h: int, w: int):
        return (h + 2 * self.pad - self.kh) // self.stride + 1, (w + 2 * self.pad - self.kw) // self.stride + 1

    def workspace(self, h: int, w: int):
        if (h, w) not in self._ws:
            n = B.ref_conv2d_workspace(self.ci, h, w, self.co, self.kh, self.kw, self.stride, self.pad)
            self._ws[(h, w)] = (self.torch.empty(n, dtype=self.torch.uint8, device=self.device), n)
        return self._ws[(h, w)]

    def forward_int(self, x_dev, xs_rec, h: int, w: int, y_dev=None, os_dev=None, stream=None):
        """Conv2d::forward_int of x_dev ([c_in][h][w] i32 codes at the record xs_rec): (y [c_out][oh][ow] codes,
        record), device tensors, no host synchronization."""
        torch = self.torch
        oh, ow = self.out_dims(h, w)
        if x_dev.numel() != self.ci * h * w:
            raise ValueError("RefConv2d: x is not [c_in][h][w]")
        if y_dev is None:
            y_dev = torch.empty(self.co * oh * ow, dtype=torch.int32, device=self.device)
        if os_dev is None:
            os_dev = torch.zeros(4, dtype=torch.int64, device=self.device)
        ws, n = self.workspace(h, w)
        B.ref_conv2d(x_dev, xs_rec, self.ci, h, w, self.w_planes, self.pw, self.co, self.kh, self.kw, self.stride,
                     self.pad, self.w_scale, self.bias, self.b_scale, ws, n, y_dev, os_dev, stream, self.dev)
        return y_dev, os_dev


class RefFeedForward:
    """FeedForward { proj_in, proj_out, gelu } (hiera.rs:321-345): proj_in and proj_out are (codes out x in,
    scale, bias) with bias None or (i64 codes, scale)."""

    def __init__(self, dim: int, hidden: int, proj_in, proj_out, dev: int = 0):
        import torch

        self.torch = torch
        self.dev = dev
        self.device = torch.device("cuda", dev)
        self.dim, self.hidden = int(dim), int(hidden)
        self.proj_in = QuantLinear("proj_in", proj_in[0], self.hidden, self.dim, proj_in[1],
                                   bias=proj_in[2] if len(proj_in) > 2 else None, dev=dev)
        self.proj_out = QuantLinear("proj_out", proj_out[0], self.dim, self.hidden, proj_out[1],
                                    bias=proj_out[2] if len(proj_out) > 2 else None, dev=dev)
        self.gelu_codes, self.gelu = gelu_table(dev)

    def forward_int(self, x_dev, xs_rec, rows: int, stream=None):
        """FeedForward::forward_int (hiera.rs:336-340) of rows x dim codes: (y rows x dim codes, record)."""
        torch = self.torch
        h, hs = self.proj_in.forward_int(x_dev, xs_rec, rows, stream=stream)
        g = torch.empty(rows * self.hidden, dtype=torch.int32, device=self.device)
        gs = torch.zeros(4, dtype=torch.int64, device=self.device)
        B.ref_gelu(h, hs, rows * self.hidden, self.gelu_codes, self.gelu, g, gs, stream, self.dev)
        return self.proj_out.forward_int(g, gs, rows, stream=stream)
