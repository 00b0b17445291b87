"""QuantLinear on one MI355X: the host-side mirror of the reference's QuantLinear
(crates/01-engine/kt-core/src/layers.rs:212-328) with all of `forward_int` on the device.

The reference runs `forward_int` as host passes around the LinearBackend seam: `xmax`, `quant_to` to the 12-trit
operand grid, the exact i32 x i32 -> i64 product, `+ bias`, `ymax` and `requant_dyn` to the 2^28 activation level,
with the output `Scale` built from the two maxima. Here the weights stay resident as base-256 digit planes, the
product is the digit-plane MFMA GEMM, and every pass before and after it is a kernel on the same stream
(`kt_hip_quant_linear`), so a chain of layers needs no host synchronization: each layer's output scale is a device
record that the next layer reads as its input scale.

A scale record is a 32-byte device buffer (`kt_hip_qscale`: i64 mant, i32 shift, i32 pad, i64 xmax, i64 ymax);
`qscale_record` makes one and `read_qscale` reads one back. torch allocates the device buffers; it computes
nothing.
"""
from __future__ import annotations

import numpy as np

from . import backend as B


def qscale_record(mant: int, shift: int, dev: int = 0):
    """A device scale record for an input tensor at Scale { mant, shift }."""
    import torch

    words = np.zeros(4, dtype=np.int64)
    words[0] = mant
    words.view(np.int32)[2] = shift
    return torch.from_numpy(words).to(torch.device("cuda", dev))


def read_qscale(rec) -> dict:
    """(mant, shift, xmax, ymax) of a device scale record (synchronizes with the device)."""
    words = rec.cpu().numpy().astype(np.int64)
    return {"mant": int(words[0]), "shift": int(words.view(np.int32)[2]), "xmax": int(words[2]),
            "ymax": int(words[3])}


class QuantLinear:
    """QuantLinear { w_codes, w_scale, bias } with weights resident on device `dev`.

    `w_codes` is out_features x in_features i32 (the reference clamps them to +-WLEVELS; any i32 works here),
    `w_scale` a (mant, shift) pair, `bias` None or (i64 codes of out_features, (mant, shift)).
    """

    def __init__(self, name: str, w_codes, out_features: int, in_features: int, w_scale, bias=None, dev: int = 0):
        import torch

        self.torch = torch
        self.name = name
        self.out_features, self.in_features = int(out_features), int(in_features)
        codes = np.ascontiguousarray(w_codes, dtype=np.int32).reshape(self.out_features, self.in_features)
        self._w_codes = codes
        self.w_scale = (int(w_scale[0]), int(w_scale[1]))
        self.dev = dev
        self.device = torch.device("cuda", dev)
        self.pw = B.planes_for(codes)
        kp = B.kp(self.in_features)
        cdev = torch.from_numpy(codes).to(self.device)
        self.w_planes = torch.empty(self.pw * self.out_features * kp, dtype=torch.int8, device=self.device)
        B.pack_planes(cdev, self.out_features, self.in_features, self.pw, self.w_planes, dev=dev)
        torch.cuda.synchronize(self.device)
        del cdev
        if bias is not None:
            bcodes, bscale = bias
            b = np.ascontiguousarray(bcodes, dtype=np.int64)
            if b.size != self.out_features:
                raise ValueError(f"{name}: bias len mismatch")
            self.bias = torch.from_numpy(b).to(self.device)
            self.b_scale = (int(bscale[0]), int(bscale[1]))
        else:
            self.bias, self.b_scale = None, None
        self._ws: dict[int, tuple] = {}

    def w_codes(self) -> np.ndarray:
        return self._w_codes

    def workspace(self, rows: int):
        if rows not in self._ws:
            n, _ = B.quant_linear_workspace(rows, self.in_features, self.out_features)
            self._ws[rows] = (self.torch.empty(n, dtype=self.torch.uint8, device=self.device), n)
        return self._ws[rows]

    def forward_int(self, x_dev, xs_dev, rows: int, y_dev=None, os_dev=None, stream=None):
        """y (rows x out_features i32 codes, device) and its scale record from x_dev (rows x in_features i32 codes)
        at the scale record xs_dev. Asynchronous on `stream`."""
        torch = self.torch
        if y_dev is None:
            y_dev = torch.empty(rows * self.out_features, dtype=torch.int32, device=self.device)
        if os_dev is None:
            os_dev = torch.zeros(4, dtype=torch.int64, device=self.device)
        ws, n = self.workspace(rows)
        B.quant_linear(x_dev, rows, self.in_features, xs_dev, self.w_planes, self.pw, self.out_features,
                       self.w_scale, self.bias, self.b_scale, ws, n, y_dev, os_dev, stream=stream, dev=self.dev)
        return y_dev, os_dev

    def sums_ok(self) -> bool:
        """Whether a one-row forward can stop at its exact sums (forward_sums): no bias, the one-launch product."""
        return self.bias is None and B.quant_linear_sums_ok(self.in_features, self.out_features, self.pw)

    def forward_sums(self, x_dev, xs_dev, rec=None, stream=None):
        """forward_int of one row stopped at its exact sums, left in this layer's one-row workspace: a B.QlSums for the
        op that reads the output next (B.ref_*_sums), which applies requant_dyn and writes the record to `rec` (or
        none). That op must run before this layer's next one-row call. Asynchronous on `stream`."""
        ws, n = self.workspace(1)
        return B.quant_linear_multi_sums(x_dev, self.in_features, xs_dev, [self.out_features], self.w_planes, self.pw,
                                         [self.w_scale], ws, n, recs=[rec], stream=stream, dev=self.dev)[0]

    def forward_int_host(self, x_codes, x_scale):
        """forward_int on host codes at Scale x_scale = (mant, shift): (y codes, dict of the output scale)."""
        torch = self.torch
        x = np.ascontiguousarray(x_codes, dtype=np.int32)
        if x.size % self.in_features:
            raise ValueError(f"{self.name}: input not a multiple of in_features")
        rows = x.size // self.in_features
        xd = torch.from_numpy(x.reshape(-1)).to(self.device)
        y, os_ = self.forward_int(xd, qscale_record(x_scale[0], x_scale[1], self.dev), rows)
        return y.cpu().numpy().reshape(rows, self.out_features), read_qscale(os_)


class QuantLinearGroup:
    """Several QuantLinears that read the same input (a tensor's projections: q / k / v, gate / up), each
    QuantLinear::forward_int called once by the reference (layers.rs:275-328), computed by one device call: one
    quantization of x, one digit GEMM over the members' weights stacked by rows, each member's own bias, output
    maximum, requant and record -- codes and records equal to its own QuantLinear's.

    members: (name, w_codes out x in, w_scale, bias or None) each, with one in_features. The boundaries between the
    members must be multiples of ALIGN (the widest column block of the digit GEMM, so any row count works):
    QuantLinearGroup.fits tells.
    """

    ALIGN = 128

    @staticmethod
    def fits(outs) -> bool:
        at = 0
        for o in list(outs)[:-1]:
            at += int(o)
            if at % QuantLinearGroup.ALIGN:
                return False
        return 1 <= len(list(outs)) <= 4

    def __init__(self, name: str, members, in_features: int, dev: int = 0):
        import torch

        self.torch = torch
        self.name = name
        self.in_features = int(in_features)
        self.outs = [int(np.asarray(m[1]).shape[0]) for m in members]
        if not QuantLinearGroup.fits(self.outs):
            raise ValueError(f"{name}: member boundaries not multiples of {QuantLinearGroup.ALIGN}")
        self.out_features = sum(self.outs)
        self.dev = dev
        self.device = torch.device("cuda", dev)
        codes = np.concatenate([np.ascontiguousarray(m[1], dtype=np.int32).reshape(o, self.in_features)
                                for m, o in zip(members, self.outs)])
        self.pw = B.planes_for(codes)
        kp = B.kp(self.in_features)
        cdev = torch.from_numpy(codes).to(self.device)
        self.w_planes = torch.empty(self.pw * self.out_features * kp, dtype=torch.int8, device=self.device)
        B.pack_planes(cdev, self.out_features, self.in_features, self.pw, self.w_planes, dev=dev)
        torch.cuda.synchronize(self.device)
        del cdev
        self.w_scales = [(int(m[2][0]), int(m[2][1])) for m in members]
        self.b_scales = [None if m[3] is None else (int(m[3][1][0]), int(m[3][1][1])) for m in members]
        if any(b is not None for b in self.b_scales):
            b = np.concatenate([np.zeros(o, np.int64) if m[3] is None else np.asarray(m[3][0], np.int64)
                                for m, o in zip(members, self.outs)])
            self.bias = torch.from_numpy(b).to(self.device)
        else:
            self.bias = None
        self._ws: dict[int, tuple] = {}

    def workspace(self, rows: int):
        if rows not in self._ws:
            n, _ = B.quant_linear_workspace(rows, self.in_features, self.out_features)
            self._ws[rows] = (self.torch.empty(n, dtype=self.torch.uint8, device=self.device), n)
        return self._ws[rows]

    def forward_int(self, x_dev, xs_dev, rows: int, y_devs=None, os_dev=None, stream=None):
        """Each member's (y rows x out i32 codes, its record): y_devs / os_dev given (os_dev: one record per member,
        consecutive) or allocated. Asynchronous on `stream`."""
        torch = self.torch
        if y_devs is None:
            y_devs = [torch.empty(rows * o, dtype=torch.int32, device=self.device) for o in self.outs]
        if os_dev is None:
            os_dev = torch.empty(4 * len(self.outs), dtype=torch.int64, device=self.device)
        ws, n = self.workspace(rows)
        B.quant_linear_multi(x_dev, rows, self.in_features, xs_dev, self.outs, self.w_planes, self.pw, self.w_scales,
                             self.bias, self.b_scales, ws, n, y_devs, os_dev, stream=stream, dev=self.dev)
        return [(y, os_dev[4 * g:4 * g + 4]) for g, y in enumerate(y_devs)]

    def sums_ok(self) -> bool:
        """Whether a one-row forward can stop at its members' exact sums (forward_sums)."""
        return (self.bias is None and all(o % 8 == 0 for o in self.outs[:-1]) and
                B.quant_linear_sums_ok(self.in_features, self.out_features, self.pw))

    def forward_sums(self, x_dev, xs_dev, os_dev=None, stream=None):
        """forward_int of one row stopped at the members' exact sums (QuantLinear.forward_sums for each member, one
        launch): a B.QlSums per member; their readers write the records to os_dev (one per member, consecutive) or
        none."""
        ws, n = self.workspace(1)
        recs = None if os_dev is None else [os_dev[4 * g:4 * g + 4] for g in range(len(self.outs))]
        return B.quant_linear_multi_sums(x_dev, self.in_features, xs_dev, self.outs, self.w_planes, self.pw,
                                         self.w_scales, ws, n, recs=recs, stream=stream, dev=self.dev)
