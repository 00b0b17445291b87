"""Python binding of the MI355X backend's C ABI (include/kt_hip.h).

`HipBackend` mirrors tritify's `LinearBackend` trait (crates/01-engine/kt-core/src/backend.rs:46-58) as the CUDA
digit backend exposes it (`kt_cuda::open`, `TcLinear`, crates/02-runtime/kt-cuda/src/lib.rs:252-279 and
backend.rs:77-192): `name`, `linear`, `linear_weights`, `resident_bytes`, and the process-wide `fallbacks` counter.
Errors raise `HipError` -- the reference panics there, because "a wrong answer is worse than a stop"
(crates/02-runtime/kt-cuda/src/device.rs:40-48).

The 12-bit-weight functions (`w12_*`) work on device-resident operands. torch tensors are accepted as plain device
buffers (their data_ptr is passed through the C ABI); torch never computes anything here.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(PKG, "libkt_hip.so")
LIB_PLANTED = os.path.join(PKG, "libkt_hip_planted.so")

OUT_I64, OUT_I32, OUT_I8, OUT_I32_ADD = 0, 1, 2, 3

# kt_cuda::Plant (crates/02-runtime/kt-cuda/src/backend.rs:31-40)
PLANT_DROP_TOP, PLANT_WRONG_CARRY, PLANT_NO_FLUSH, PLANT_CACHE_BY_SHAPE = 1, 2, 3, 4

_libs: dict[str, C.CDLL] = {}


class HipError(RuntimeError):
    pass


def _load(path: str) -> C.CDLL:
    if path not in _libs:
        if not os.path.exists(path):
            raise ImportError(f"the HIP backend is not built ({path} is missing): run __graft_entry__.build()")
        lib = C.CDLL(path)
        _declare(lib)
        _libs[path] = lib
    return _libs[path]


def lib(planted: bool = False) -> C.CDLL:
    return _load(LIB_PLANTED if planted else LIB)


_P, _SZ, _I, _I64, _U64 = C.c_void_p, C.c_size_t, C.c_int, C.c_int64, C.c_uint64


def _declare(L: C.CDLL) -> None:
    sig = {
        "kt_hip_device_count": (_I, [C.POINTER(_I)]),
        "kt_hip_device_info": (_I, [_I, C.c_char_p, _I, C.POINTER(_I), C.POINTER(_I), C.POINTER(_SZ)]),
        "kt_hip_alloc": (_I, [_I, _SZ, C.POINTER(_P)]),
        "kt_hip_free": (_I, [_I, _P]),
        "kt_hip_upload": (_I, [_I, _P, _P, _SZ]),
        "kt_hip_download": (_I, [_I, _P, _P, _SZ]),
        "kt_hip_error_string": (C.c_char_p, [_I]),
        "kt_hip_kp": (_I64, [_I64]),
        "kt_hip_planes_for": (_I, [_P, _SZ]),
        "kt_hip_pack_planes": (_I, [_I, _P, _I64, _I64, _I, _P, _P]),
        "kt_hip_flush_k": (_I64, [_I, _I]),
        "kt_hip_digit_gemm": (_I, [_I, _P, _I, _P, _I, _P, _I64, _I64, _I64, _I64, _I, _P]),
        "kt_hip_open": (_I, [_I, _U64, C.POINTER(_P)]),
        "kt_hip_open_planted": (_I, [_I, _I, C.POINTER(_P)]),
        "kt_hip_close": (None, [_P]),
        "kt_hip_name": (_I, [_P, C.c_char_p, _I]),
        "kt_hip_linear": (_I, [_P, _P, _P, _SZ, _SZ, _SZ, _P]),
        "kt_hip_linear_weights": (_I, [_P, _P, _U64, _P, _SZ, _SZ, _SZ, _P]),
        "kt_hip_weight_id_fresh": (_U64, []),
        "kt_hip_resident_bytes": (_U64, [_P]),
        "kt_hip_fallbacks": (_U64, []),
        "kt_hip_w12_bytes": (None, [_I64, _I64, C.POINTER(_SZ), C.POINTER(_SZ)]),
        "kt_hip_w12_pack": (_I, [_I, _P, _I64, _I64, _P, _P, _P]),
        "kt_hip_w12_upload": (_I, [_I, _P, _I64, _I64, _P, _P]),
        "kt_hip_w12_linear": (_I, [_I, _P, _P, _P, _I64, _I64, _I64, _P, _P, _I, _P, _P]),
        "kt_hip_w12b_bytes": (None, [_I64, _I64, C.POINTER(_SZ)]),
        "kt_hip_w12b_pack": (_I, [_I, _P, _I64, _I64, _P, _P, _P]),
        "kt_hip_w12b_linear": (_I, [_I, _P, _P, _P, _I64, _I64, _I64, _P, _P, _I, _P, _P]),
        "kt_hip_stream_read": (_I, [_I, _P, _I64, _P, _P]),
        "kt_hip_probe_mfma": (_I, [_I, _P, _P, _P, _P, _P]),
        "kt_hip_w12_linear_lut": (_I, [_I, _P, _P, _P, _I64, _I64, _I64, _P, _P, _P, _P, _P]),
        "kt_hip_w12_pack_gate_up": (_I, [_I, _P, _I64, _I64, _P, _P, _P]),
        "kt_hip_moe_route": (_I, [_I, _P, _I64, _I64, _I, _P, _P, _P, _P]),
        "kt_hip_moe_bucket": (_I, [_I, _P, _I64, _I64, _I, _P, _P, _P, _P]),
        "kt_hip_w12_grouped_linear": (_I, [_I, _P, _I64, _P, _I64, _P, _I64, _I64, _P, _P, _I64, _I64, _P, _P, _I,
                                           _P, _I, _P, _I64, _P, _P]),
        "kt_hip_w12_swiglu": (_I, [_I, _P, _P, _P, _I64, _I64, _I64, _P, _P, _P, _I, _P, _I64, _P]),
        "kt_hip_moe_combine": (_I, [_I, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _P, _P]),
        "kt_hip_moe_workspace": (_I, [_I64, _I64, _I64, _I64, _I, C.POINTER(_SZ), C.POINTER(_SZ)]),
        "kt_hip_moe_forward": (_I, [_I, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                    _I, _I, _P, _P, _P]),
        "kt_hip_sam_patch_embed": (_I, [_I, _P, _P, _I64, _I64, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P,
                                        _P, _P, _P]),
        "kt_hip_sam_patch_bytes": (None, [_I64, _I64, _I64, _I64, C.POINTER(_SZ), C.POINTER(_SZ)]),
        "kt_hip_sam_patch_pack": (_I, [_I, _P, _I64, _I64, _I64, _I64, _P, _P, _P]),
        "kt_hip_sam_patch_upload": (_I, [_I, _P, _I64, _I64, _I64, _I64, _P, _P]),
        "kt_hip_dec_embed": (_I, [_I, _P, _I64, _P, _I64, _P, _P]),
        "kt_hip_dec_rmsnorm": (_I, [_I, _P, _I64, _I64, _P, _I64, _P]),
        "kt_hip_dec_rope_kv": (_I, [_I, _P, _I64, _I64, _P, _I64, _I64, _I64, _P, _P, _P, _P, _P]),
        "kt_hip_dec_attention": (_I, [_I, _P, _I64, _I64, _P, _P, _P, _I64, _I64, _I64, _P, _P, _I64, _P]),
        "kt_hip_dec_argmax": (_I, [_I, _P, _I64, _P, _P, _P, _P]),
        "kt_hip_dec_advance": (_I, [_I, _P, _I64, _P]),
        "kt_hip_dec_attention_step": (_I, [_I, _P, _P, _P, _P, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _P]),
        "kt_hip_dec_attention_o_step": (_I, [_I, _P, _P, _P, _P, _I64, _I64, _I64, _P, _P, _P, _I64, _P, _P, _I64, _P, _P]),
        "kt_hip_w12_swiglu_norm_o": (_I, [_I, _P, _P, _P, _I64, _I64, _P, _P, _P, _I, _P, _P, _P, _P, _P]),
        "kt_hip_w12_linear_add_o": (_I, [_I, _P, _P, _P, _I64, _I64, _P, _P, _P, _P, _P, _P, _P]),
        "kt_hip_dec_argmax_part": (_I, [_I, _P, _I64, _P, _I64, _P, _P, _P, _I64, _P]),
        "kt_hip_dec_embed_argmax": (_I, [_I, _P, _I64, _P, _I64, _P, _P, _P, _P]),
        "kt_hip_w12_linear_norm": (_I, [_I, _P, _P, _P, _I64, _I64, _I64, _P, _P, _I, _P, _P]),
        "kt_hip_w12_swiglu_norm": (_I, [_I, _P, _P, _P, _I64, _I64, _I64, _P, _P, _P, _I, _P, _I64, _P]),
        "kt_hip_quant_linear_workspace": (_SZ, [_I64, _I64, _I64, _P]),
        "kt_hip_quant_linear": (_I, [_I, _P, _I64, _I64, _P, _P, _I, _I64, _I64, C.c_int32, _P, _I64, C.c_int32, _P,
                                     _SZ, _P, _P, _P]),
        "kt_hip_quant_linear_noalloc": (_I, [_I, _P, _I64, _I64, _P, _P, _I, _I64, _I64, C.c_int32, _P, _I64,
                                             C.c_int32, _P, _P, _P]),
        "kt_hip_ref_scale_from_f64": (None, [C.c_double, C.POINTER(_I64), C.POINTER(C.c_int32)]),
        "kt_hip_ref_codelut": (_I, [_I, C.c_double, C.c_double, _I, _I, _I, _P, _P]),
        "kt_hip_ref_rope_tables": (_I, [_I64, _I64, C.c_double, _P, _P]),
        "kt_hip_ref_embed": (_I, [_I, _P, _I64, C.c_int32, _P, _I64, _I64, _P, _P, _P]),
        "kt_hip_ref_rmsnorm": (_I, [_I, _P, _P, _I64, _I64, _P, _I64, C.c_int32, _I64, C.c_int32, _P, _P, _P]),
        "kt_hip_ref_add": (_I, [_I, _P, _P, _P, _P, _I64, _P, _P, _P]),
        "kt_hip_ref_add_rmsnorm": (_I, [_I, _P, _P, _P, _P, _I64, _P, _P, _P, _I64, C.c_int32, _I64, C.c_int32, _P,
                                        _P, _P]),
        "kt_hip_ref_swiglu": (_I, [_I, _P, _P, _P, _P, _I64, _I64, _P, _P, _P, _P, _P]),
        "kt_hip_ref_seq_workspace": (_SZ, [_I64]),
        "kt_hip_ref_rmsnorm_seq": (_I, [_I, _P, _P, _I64, _I64, _P, _I64, C.c_int32, _I64, C.c_int32, _P, _SZ, _P, _P,
                                        _P]),
        "kt_hip_ref_add_seq": (_I, [_I, _P, _P, _P, _P, _I64, _P, _SZ, _P, _P, _P]),
        "kt_hip_ref_swiglu_seq": (_I, [_I, _P, _P, _P, _P, _I64, _P, _P, _P, _SZ, _P, _P, _P]),
        "kt_hip_ref_embed_seq": (_I, [_I, _P, _I64, C.c_int32, _P, _I64, _I64, _I64, _P, _P, _P]),
        "kt_hip_ref_attention_prefill_workspace": (_SZ, [_I64, _I64, _I64, _I64]),
        "kt_hip_ref_attention_prefill": (_I, [_I, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _I64,
                                              C.c_int32, _P, _P, _P, _SZ, _P, _P, _P]),
        "kt_hip_ref_gelu": (_I, [_I, _P, _P, _I64, _P, _P, _P, _P, _P]),
        "kt_hip_ref_from_reals": (_I, [_P, _I64, _I64, _P, _P, _P]),
        "kt_hip_ref_conv2d_workspace": (_SZ, [_I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64]),
        "kt_hip_ref_conv2d": (_I, [_I, _P, _P, _I64, _I64, _I64, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64,
                                   C.c_int32, _P, _I64, C.c_int32, _P, _SZ, _P, _P, _P]),
        "kt_hip_quant_linear_rows_workspace": (_SZ, [_I64, _I64, _I64, _I64]),
        "kt_hip_quant_linear_rows": (_I, [_I, _P, _P, _I64, _I64, _I64, _P, _I, _I64, _P, _P, _P, _SZ, _I, _I64, _P,
                                          _P, _P, _SZ, _P, _P, _P]),
        "kt_hip_ref_moe_route": (_I, [_I, _P, _I64, _I64, _I, _P, _I, _I, _P, _P, _P, _P, _P, _P, _P]),
        "kt_hip_ref_moe_combine": (_I, [_I, _P, _P, _I64, _I64, _P, _P, _P, _I64, _I, _P, _P, _P]),
        "kt_hip_ref_moe_bucket": (_I, [_I, _P, _I64, _I, _I64, _P, _P, _P, _P]),
        "kt_hip_quant_linear_multi": (_I, [_I, _P, _I64, _I64, _P, _I, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P,
                                            _SZ, _P, _P, _P]),
        "kt_hip_quant_linear_multi_align": (_I64, [_I64, _I64, _I]),
        "kt_hip_quant_linear_sums_ok": (_I, [_I64, _I64, _I]),
        "kt_hip_quant_linear_multi_sums": (_I, [_I, _P, _I64, _P, _I, _P, _P, _I, _P, _P, _P, _SZ, _P]),
        "kt_hip_ref_add_rmsnorm_sums": (_I, [_I, _P, _P, _P, _I64, _P, _P, _P, _I64, C.c_int32, _I64, C.c_int32, _P,
                                             _P, _P]),
        "kt_hip_ref_swiglu_sums": (_I, [_I, _P, _P, _I64, _P, _P, _P, _P, _P]),
        "kt_hip_ref_attention_step_sums": (_I, [_I, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P,
                                                _I64, C.c_int32, _P, _P, _P, _P, _P, _SZ, _P]),
        "kt_hip_pack_planes_tiled_bytes": (_SZ, [_I64, _I64, _I]),
        "kt_hip_pack_planes_tiled": (_I, [_I, _P, _I64, _I64, _I, _P, _P]),
        "kt_hip_ref_merge_rows_workspace": (_SZ, [_I64]),
        "kt_hip_ref_merge_rows": (_I, [_I, _P, _P, _I64, _I64, _P, _SZ, _P, _P, _P]),
        "kt_hip_ref_attention_step": (_I, [_I, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _P,
                                           _P, _P, _I64, C.c_int32, _P, _P, _P, _P, _P]),
        "kt_hip_ref_attention_step_ws": (_I, [_I, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P,
                                              _P, _P, _P, _I64, C.c_int32, _P, _P, _P, _P, _P, _SZ, _P]),
        "kt_hip_ref_attention_step_workspace": (_SZ, [_I64, _I64, _I64]),
        "kt_hip_ref_argmax": (_I, [_I, _P, _I64, _P, _P, _P, _P, _P, _I64, _P]),
        "kt_hip_gen_w12": (None, [_U64, _SZ, _P]),
        "kt_hip_gen_gauss": (None, [_U64, _I64, _I64, _SZ, _P]),
        "kt_hip_gen_uniform": (None, [_U64, _I64, _I64, _SZ, _P]),
        "kt_hip_channel_scales": (None, [_P, _SZ, _SZ, _I64, _I64, _P, _P]),
        "kt_hip_gen_quant_rows": (None, [_U64, _SZ, _SZ, _P]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def check(e: int, what: str) -> None:
    if e != 0:
        msg = lib().kt_hip_error_string(e).decode()
        raise HipError(f"kt-hip: {what}: {msg} (hipError {e})")


def _i32(a) -> np.ndarray:
    a = np.ascontiguousarray(a)
    if a.dtype != np.int32:
        if a.size and (a.min() < -(2**31) or a.max() > 2**31 - 1):
            raise ValueError("codes must fit i32")
        a = a.astype(np.int32)
    return a


# ---------------------------------------------------------------------------------------------------------------
# device layer


def device_count() -> int:
    n = C.c_int(0)
    e = lib().kt_hip_device_count(C.byref(n))
    return n.value if e == 0 else 0


def device_info(dev: int = 0) -> dict:
    name = C.create_string_buffer(256)
    major, minor, free = C.c_int(), C.c_int(), C.c_size_t()
    check(lib().kt_hip_device_info(dev, name, 256, C.byref(major), C.byref(minor), C.byref(free)), "device info")
    return {"name": name.value.decode(), "major": major.value, "minor": minor.value, "free": free.value}


def kp(k: int) -> int:
    """k padded to the 64-value tile of the device layouts."""
    return (k + 63) // 64 * 64


def planes_for(codes) -> int:
    c = _i32(codes)
    return lib().kt_hip_planes_for(c.ctypes.data, c.size)


def flush_k(px: int, pw: int) -> int:
    return lib().kt_hip_flush_k(px, pw)


# ---------------------------------------------------------------------------------------------------------------
# backend layer


@dataclass(frozen=True)
class Weights:
    """kt_core::backend::Weights (backend.rs:37-42): codes behind an id never change."""

    id: int
    codes: np.ndarray


def weight_id_fresh() -> int:
    """WeightId::fresh (backend.rs:29-35)."""
    return lib().kt_hip_weight_id_fresh()


def fallbacks() -> int:
    """kt_cuda::fallbacks (backend.rs:42-48); this backend never falls back, so it stays 0."""
    return lib().kt_hip_fallbacks()


class HipBackend:
    """One LinearBackend on one MI355X (TcLinear<DeviceExec>)."""

    def __init__(self, dev: int = 0, budget: int | None = None, plant: int | None = None):
        self._planted = plant is not None
        self._lib = lib(self._planted)
        h = C.c_void_p()
        if plant is None:
            check(self._lib.kt_hip_open(dev, budget or 0, C.byref(h)), "open")
        else:
            if budget is not None:
                raise ValueError("a planted backend takes the default budget")
            check(self._lib.kt_hip_open_planted(dev, plant, C.byref(h)), "open planted")
        self._h = h

    def close(self) -> None:
        if self._h:
            self._lib.kt_hip_close(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def name(self) -> str:
        buf = C.create_string_buffer(512)
        check(self._lib.kt_hip_name(self._h, buf, 512), "name")
        return buf.value.decode()

    def _args(self, x, w, rows, out, k):
        x, w = _i32(x), _i32(w)
        if x.size != rows * k:
            raise ValueError("linear: x is not rows·k")
        if w.size != out * k:
            raise ValueError("linear: w is not out·k")
        return x, w, np.empty(rows * out, dtype=np.int64)

    def linear(self, x, w, rows: int, out: int, k: int) -> np.ndarray:
        x, w, y = self._args(x, w, rows, out, k)
        check(self._lib.kt_hip_linear(self._h, x.ctypes.data, w.ctypes.data, rows, out, k, y.ctypes.data), "linear")
        return y

    def linear_weights(self, x, weights: Weights, rows: int, out: int, k: int) -> np.ndarray:
        x, w, y = self._args(x, weights.codes, rows, out, k)
        check(
            self._lib.kt_hip_linear_weights(self._h, x.ctypes.data, weights.id, w.ctypes.data, rows, out, k,
                                            y.ctypes.data),
            "linear_weights",
        )
        return y

    def resident_bytes(self) -> int:
        return self._lib.kt_hip_resident_bytes(self._h)


# ---------------------------------------------------------------------------------------------------------------
# 12-bit-weight path (device-resident operands; torch tensors or raw device pointers)


def _ptr(t) -> int:
    if t is None:
        return 0
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(s) -> int:
    if s is None:
        return 0
    if isinstance(s, int):
        return s
    return s.cuda_stream


def w12_bytes(n: int, k: int) -> tuple[int, int]:
    """Bytes of the W12 lo and nib planes of an n x k weight matrix (rows padded to 32, k to 64)."""
    lo, nib = C.c_size_t(), C.c_size_t()
    lib().kt_hip_w12_bytes(n, k, C.byref(lo), C.byref(nib))
    return lo.value, nib.value


def w12_pack(codes_dev, n: int, k: int, lo_dev, nib_dev, stream=None, dev: int = 0) -> None:
    """Pack n x k codes in [-2048, 2047] (i32, device) into the W12 planes lo (n x kp) and nib (n x kp/2)."""
    check(lib().kt_hip_w12_pack(dev, _ptr(codes_dev), n, k, _ptr(lo_dev), _ptr(nib_dev), _stream(stream)), "w12 pack")


def w12_upload(codes, n: int, k: int, lo_dev, nib_dev, dev: int = 0) -> None:
    """Check host codes against [-2048, 2047], upload and pack them (synchronous)."""
    c = _i32(codes)
    if c.size != n * k:
        raise ValueError("codes are not n·k")
    check(lib().kt_hip_w12_upload(dev, c.ctypes.data, n, k, _ptr(lo_dev), _ptr(nib_dev)), "w12 upload")


def w12_linear(x_dev, lo_dev, nib_dev, m: int, n: int, k: int, y_dev, out_kind: int = OUT_I64, mant_dev=None,
               shift_dev=None, stream=None, dev: int = 0) -> None:
    """y = requant_or_identity(x · Wᵀ) with x int8 (m x kp, zero padded) and W12 weights (n x k). Asynchronous."""
    check(
        lib().kt_hip_w12_linear(dev, _ptr(x_dev), _ptr(lo_dev), _ptr(nib_dev), m, n, k, _ptr(mant_dev),
                                _ptr(shift_dev), out_kind, _ptr(y_dev), _stream(stream)),
        "w12 linear",
    )


def w12b_bytes(n: int, k: int) -> int:
    """Bytes of each of the two balanced W12B planes (lo, hi) of an n x k weight matrix."""
    b = C.c_size_t()
    lib().kt_hip_w12b_bytes(n, k, C.byref(b))
    return b.value


def w12b_pack(codes_dev, n: int, k: int, lo_dev, hi_dev, stream=None, dev: int = 0) -> None:
    """Pack n x k codes in [-2048, 2047] (i32, device) into the balanced planes: hi = (v + 128) >> 8, lo = v - 256 hi."""
    check(lib().kt_hip_w12b_pack(dev, _ptr(codes_dev), n, k, _ptr(lo_dev), _ptr(hi_dev), _stream(stream)),
          "w12b pack")


def w12b_linear(x_dev, lo_dev, hi_dev, m: int, n: int, k: int, y_dev, out_kind: int = OUT_I64, mant_dev=None,
                shift_dev=None, stream=None, dev: int = 0) -> None:
    """w12_linear's integers over the balanced W12B planes (the DMA-fed 256 x 128 GEMM). Asynchronous."""
    check(
        lib().kt_hip_w12b_linear(dev, _ptr(x_dev), _ptr(lo_dev), _ptr(hi_dev), m, n, k, _ptr(mant_dev),
                                 _ptr(shift_dev), out_kind, _ptr(y_dev), _stream(stream)),
        "w12b linear",
    )


STREAM_READ_CTAS = 256  # KT_STREAM_READ_CTAS


def stream_read(src_dev, nbytes: int, out_dev, stream=None, dev: int = 0) -> None:
    """A pure read of nbytes (a multiple of 16) of src_dev with the GEMV's load form; out_dev (STREAM_READ_CTAS
    uint32) receives each chunk's XOR of 32-bit words. A measurement aid. Asynchronous."""
    check(lib().kt_hip_stream_read(dev, _ptr(src_dev), nbytes, _ptr(out_dev), _stream(stream)), "stream read")


def digit_gemm(xa_dev, px: int, wb_dev, pw: int, y_dev, rows: int, out: int, k: int, flush: int = 0,
               drop_top: bool = False, stream=None, dev: int = 0) -> None:
    """The digit-plane product on device planes (kt_cuda_digit_gemm without the host copies)."""
    check(
        lib().kt_hip_digit_gemm(dev, _ptr(xa_dev), px, _ptr(wb_dev), pw, _ptr(y_dev), rows, out, k, flush,
                                int(drop_top), _stream(stream)),
        "digit gemm",
    )


def pack_planes(codes_dev, rows: int, k: int, planes: int, planes_dev, stream=None, dev: int = 0) -> None:
    check(lib().kt_hip_pack_planes(dev, _ptr(codes_dev), rows, k, planes, _ptr(planes_dev), _stream(stream)),
          "pack planes")


NORM_MAX_M = 16


def w12_linear_norm(r_dev, lo_dev, nib_dev, m: int, n: int, d: int, y_dev, out_kind: int, mant_dev=None,
                    shift_dev=None, stream=None, dev: int = 0) -> None:
    """The decoder's RMSNorm of m int32 residual rows (d values each) fused before w12_linear. Asynchronous."""
    check(lib().kt_hip_w12_linear_norm(dev, _ptr(r_dev), _ptr(lo_dev), _ptr(nib_dev), m, n, d, _ptr(mant_dev),
                                       _ptr(shift_dev), out_kind, _ptr(y_dev), _stream(stream)), "w12 linear norm")


def w12_swiglu_norm(r_dev, lo_dev, nib_dev, m: int, ffn: int, d: int, mant_dev, shift_dev, silu_dev, h_shift: int,
                    y_dev, y_stride: int, stream=None, dev: int = 0) -> None:
    """The decoder's RMSNorm of m int32 residual rows fused before w12_swiglu. Asynchronous."""
    check(lib().kt_hip_w12_swiglu_norm(dev, _ptr(r_dev), _ptr(lo_dev), _ptr(nib_dev), m, ffn, d, _ptr(mant_dev),
                                       _ptr(shift_dev), _ptr(silu_dev), h_shift, _ptr(y_dev), y_stride,
                                       _stream(stream)), "w12 swiglu norm")


QL_WS_PARTS = 5
QL_SCRATCH_BYTES = 32 << 20  # KT_QL_SCRATCH_BYTES: the no-allocation entry point's per-GPU scratch


def quant_linear_workspace(rows: int, in_f: int, out_f: int) -> tuple[int, list[int]]:
    """Workspace bytes of quant_linear for rows x in_f -> out_f, and the byte offsets of its parts."""
    off = (_SZ * QL_WS_PARTS)()
    n = lib().kt_hip_quant_linear_workspace(rows, in_f, out_f, off)
    if n == 0:
        raise ValueError("quant_linear: rows, in_f and out_f must be >= 1")
    return n, list(off)


def quant_linear(x_dev, rows: int, in_f: int, xs_dev, w_planes_dev, pw: int, out_f: int, w_scale, bias_dev,
                 b_scale, ws_dev, ws_bytes: int, y_dev, os_dev, stream=None, dev: int = 0) -> None:
    """QuantLinear::forward_int on the device (layers.rs:275-328): y_dev (rows x out_f i32 codes) and os_dev (their
    scale record) from x_dev at the scale record xs_dev. Scales are (mant, shift) pairs. Asynchronous."""
    bm, bs = b_scale if b_scale is not None else (0, 0)
    check(
        lib().kt_hip_quant_linear(dev, _ptr(x_dev), rows, in_f, _ptr(xs_dev), _ptr(w_planes_dev), pw, out_f,
                                  int(w_scale[0]), int(w_scale[1]), _ptr(bias_dev), int(bm), int(bs), _ptr(ws_dev),
                                  ws_bytes, _ptr(y_dev), _ptr(os_dev), _stream(stream)),
        "quant linear",
    )


def quant_linear_multi_align(rows: int, out_f: int, pw: int) -> int:
    """The multiple of which every boundary between the calls of quant_linear_multi must be."""
    return lib().kt_hip_quant_linear_multi_align(rows, out_f, pw)


def quant_linear_multi(x_dev, rows: int, in_f: int, xs_dev, seg_out, w_planes_dev, pw: int, w_scales, bias_dev,
                       b_scales, ws_dev, ws_bytes: int, y_devs, os_dev, stream=None, dev: int = 0) -> None:
    """Several QuantLinear::forward_int calls on one x, computed together (their weights stacked by rows in
    w_planes_dev): y_devs[g] and record os_dev[g] equal call g's own. b_scales[g]: None where call g has no bias
    (bias_dev: None, or the stacked bias codes with zeros there)."""
    n = len(seg_out)
    arr = lambda t, v: (t * n)(*v)  # noqa: E731
    hb = [0 if (bias_dev is None or b is None) else 1 for b in b_scales]
    check(lib().kt_hip_quant_linear_multi(
        dev, _ptr(x_dev), rows, in_f, _ptr(xs_dev), n, arr(C.c_int64, [int(v) for v in seg_out]), _ptr(w_planes_dev),
        pw, arr(C.c_int64, [int(w[0]) for w in w_scales]), arr(C.c_int32, [int(w[1]) for w in w_scales]),
        _ptr(bias_dev), arr(C.c_int, hb), arr(C.c_int64, [int(b[0]) if b else 0 for b in b_scales]),
        arr(C.c_int32, [int(b[1]) if b else 0 for b in b_scales]), _ptr(ws_dev), ws_bytes,
        arr(C.c_void_p, [_ptr(y) for y in y_devs]), _ptr(os_dev), _stream(stream)), "quant linear multi")


class QlSums(C.Structure):
    """kt_hip_ql_sums: one call's output of a quant_linear_multi_sums launch (its exact sums and state in that launch's
    workspace), as the op that reads it next takes it; rec: where that op writes the output's record, or 0."""
    _fields_ = [("ws", _P), ("in_f", _I64), ("out_f", _I64), ("col0", _I64), ("n", _I64), ("seg", C.c_int32),
                ("pad", C.c_int32), ("rec", _P)]


def quant_linear_sums_ok(in_f: int, out_f: int, pw: int) -> bool:
    """Whether a one-row QuantLinear of in_f -> out_f can stop at its sums (quant_linear_multi_sums)."""
    return bool(lib().kt_hip_quant_linear_sums_ok(in_f, out_f, pw))


def quant_linear_multi_sums(x_dev, in_f: int, xs_dev, seg_out, w_planes_dev, pw: int, w_scales, ws_dev,
                            ws_bytes: int, recs=None, stream=None, dev: int = 0) -> list:
    """quant_linear_multi of one row with no bias, stopped at the exact sums: the quantization and the digit product
    in one launch, each call's sums and state left in ws_dev for the op that reads the output next (ref_*_sums),
    which applies requant_dyn and writes the record (recs[g], or none). Returns one QlSums per call."""
    n = len(seg_out)
    arr = lambda t, v: (t * n)(*v)  # noqa: E731
    check(lib().kt_hip_quant_linear_multi_sums(
        dev, _ptr(x_dev), in_f, _ptr(xs_dev), n, arr(C.c_int64, [int(v) for v in seg_out]), _ptr(w_planes_dev), pw,
        arr(C.c_int64, [int(w[0]) for w in w_scales]), arr(C.c_int32, [int(w[1]) for w in w_scales]), _ptr(ws_dev),
        ws_bytes, _stream(stream)), "quant linear sums")
    out, col0 = [], 0
    for g, o in enumerate(seg_out):
        r = recs[g] if recs is not None else None
        out.append(QlSums(_ptr(ws_dev), in_f, sum(int(v) for v in seg_out), col0, int(o), g, 0,
                          _ptr(r) if r is not None else 0))
        col0 += int(o)
    return out


def quant_linear_noalloc(x_dev, rows: int, in_f: int, xs_dev, w_planes_dev, pw: int, out_f: int, w_scale,
                         bias_dev, b_scale, y_dev, os_dev, stream=None, dev: int = 0) -> None:
    """quant_linear with its workspace in the library's per-GPU scratch array: allocates nothing. Calls that overlap
    on one GPU race on that array."""
    bm, bs = b_scale if b_scale is not None else (0, 0)
    check(
        lib().kt_hip_quant_linear_noalloc(dev, _ptr(x_dev), rows, in_f, _ptr(xs_dev), _ptr(w_planes_dev), pw, out_f,
                                          int(w_scale[0]), int(w_scale[1]), _ptr(bias_dev), int(bm), int(bs),
                                          _ptr(y_dev), _ptr(os_dev), _stream(stream)),
        "quant linear (no allocation)",
    )


def probe_mfma(a_dev, b_dev, c32_dev, c16_dev, stream=None, dev: int = 0) -> None:
    check(lib().kt_hip_probe_mfma(dev, _ptr(a_dev), _ptr(b_dev), _ptr(c32_dev), _ptr(c16_dev), _stream(stream)),
          "mfma probe")


def w12_linear_lut(x_dev, lo_dev, nib_dev, m: int, n: int, k: int, y_dev, mant_dev, shift_dev, lut_dev, stream=None,
                   dev: int = 0) -> None:
    """y = lut[int8 requant(x · Wᵀ) + 127]: the dense W12 product with an activation-code table in the epilogue."""
    check(
        lib().kt_hip_w12_linear_lut(dev, _ptr(x_dev), _ptr(lo_dev), _ptr(nib_dev), m, n, k, _ptr(mant_dev),
                                    _ptr(shift_dev), _ptr(lut_dev), _ptr(y_dev), _stream(stream)),
        "w12 linear lut",
    )


# ---------------------------------------------------------------------------------------------------------------
# MoE layer (config 4): MoeMlp::route / experts / combine (crates/01-engine/kt-core/src/layers.rs:800-1020)

EPI_I8, EPI_SWIGLU = 0, 1
MAX_GROUPS = 1024


def w12_pack_gate_up(codes_dev, ffn: int, k: int, lo_dev, nib_dev, stream=None, dev: int = 0) -> None:
    """Pack a 2·ffn x k gate/up code matrix (gate rows first, device i32) with the 32-row gate/up interleave."""
    check(lib().kt_hip_w12_pack_gate_up(dev, _ptr(codes_dev), ffn, k, _ptr(lo_dev), _ptr(nib_dev), _stream(stream)),
          "w12 pack gate/up")


def moe_route(logits_dev, tokens: int, experts: int, top_k: int, sig_dev, sel_dev, cw_dev, stream=None,
              dev: int = 0) -> None:
    check(lib().kt_hip_moe_route(dev, _ptr(logits_dev), tokens, experts, top_k, _ptr(sig_dev), _ptr(sel_dev),
                                 _ptr(cw_dev), _stream(stream)), "moe route")


def moe_bucket(sel_dev, tokens: int, experts: int, top_k: int, list_dev, pos_dev, count_dev, stream=None,
               dev: int = 0) -> None:
    check(lib().kt_hip_moe_bucket(dev, _ptr(sel_dev), tokens, experts, top_k, _ptr(list_dev), _ptr(pos_dev),
                                  _ptr(count_dev), _stream(stream)), "moe bucket")


def w12_grouped_linear(x_dev, x_rows: int, list_dev, list_stride: int, count_dev, groups: int, max_rows: int, lo_dev,
                       nib_dev, n: int, k: int, mant_dev, shift_dev, epilogue: int, y_dev, y_stride: int,
                       silu_dev=None, h_shift: int = 0, off_dev=None, stream=None, dev: int = 0) -> None:
    """The ragged grouped W12 GEMM (one launch over every group; see include/kt_hip.h)."""
    check(
        lib().kt_hip_w12_grouped_linear(dev, _ptr(x_dev), x_rows, _ptr(list_dev), list_stride, _ptr(count_dev), groups,
                                        max_rows, _ptr(lo_dev), _ptr(nib_dev), n, k, _ptr(mant_dev), _ptr(shift_dev),
                                        epilogue, _ptr(silu_dev), h_shift, _ptr(y_dev), y_stride, _ptr(off_dev),
                                        _stream(stream)),
        "w12 grouped linear",
    )


def w12_swiglu(x_dev, lo_dev, nib_dev, m: int, ffn: int, k: int, mant_dev, shift_dev, silu_dev, h_shift: int, y_dev,
               y_stride: int, stream=None, dev: int = 0) -> None:
    """The dense SwiGLU gate/up product: int8 h = clamp(requant(silu[gq + 127] * uq, 1, h_shift))."""
    check(lib().kt_hip_w12_swiglu(dev, _ptr(x_dev), _ptr(lo_dev), _ptr(nib_dev), m, ffn, k, _ptr(mant_dev),
                                  _ptr(shift_dev), _ptr(silu_dev), h_shift, _ptr(y_dev), y_stride, _stream(stream)),
          "w12 swiglu")


def moe_combine(d_dev, off_dev, sel_dev, cw_dev, pos_dev, tokens: int, hidden: int, experts: int, top_k: int,
                out_shift: int, out_dev, stream=None, dev: int = 0) -> None:
    check(lib().kt_hip_moe_combine(dev, _ptr(d_dev), _ptr(off_dev), _ptr(sel_dev), _ptr(cw_dev), _ptr(pos_dev),
                                   tokens, hidden, experts, top_k, out_shift, _ptr(out_dev), _stream(stream)),
          "moe combine")


MOE_WS_PARTS = ("sel", "cw", "pos", "list", "count", "off", "h", "d")


def moe_workspace(tokens: int, hidden: int, ffn: int, experts: int, top_k: int) -> tuple[int, dict]:
    """Bytes of kt_hip_moe_forward's workspace and the byte offset of each part."""
    total = C.c_size_t()
    offs = (C.c_size_t * len(MOE_WS_PARTS))()
    check(lib().kt_hip_moe_workspace(tokens, hidden, ffn, experts, top_k, C.byref(total), offs), "moe workspace")
    return total.value, dict(zip(MOE_WS_PARTS, [o for o in offs]))


def moe_forward(x_dev, logits_dev, tokens: int, hidden: int, ffn: int, experts: int, top_k: int, gu_lo, gu_nib,
                gu_mant, gu_shift, d_lo, d_nib, d_mant, d_shift, silu_dev, sig_dev, h_shift: int, out_shift: int,
                workspace_dev, out_dev, stream=None, dev: int = 0) -> None:
    """The config-4 MoE layer: route, bucket, gate/up + SwiGLU, down, combine (five launches, asynchronous)."""
    check(
        lib().kt_hip_moe_forward(dev, _ptr(x_dev), _ptr(logits_dev), tokens, hidden, ffn, experts, top_k, _ptr(gu_lo),
                                 _ptr(gu_nib), _ptr(gu_mant), _ptr(gu_shift), _ptr(d_lo), _ptr(d_nib), _ptr(d_mant),
                                 _ptr(d_shift), _ptr(silu_dev), _ptr(sig_dev), h_shift, out_shift,
                                 _ptr(workspace_dev), _ptr(out_dev), _stream(stream)),
        "moe forward",
    )


# ---------------------------------------------------------------------------------------------------------------
# SAM image path (config 5)


def sam_patch_bytes(co: int, ci: int, kh: int, kw: int) -> tuple[int, int]:
    """Bytes of the two patch-embed weight planes (int8 lo and hi digits, co·ci·kh·kwp codes, kwp = kw rounded up
    to 4, in the W12 fragment tiling)."""
    lo, hi = C.c_size_t(), C.c_size_t()
    lib().kt_hip_sam_patch_bytes(co, ci, kh, kw, C.byref(lo), C.byref(hi))
    if lo.value == 0 and co > 0:
        raise ValueError(f"no patch-embed weight layout for ci={ci} kh={kh} kw={kw}")
    return lo.value, hi.value


def sam_patch_pack(codes_dev, co: int, ci: int, kh: int, kw: int, lo_dev, hi_dev, stream=None, dev: int = 0) -> None:
    """Pack co x (ci·kh·kw) codes (i32, device, [c_out][c_in][kh][kw]) into the patch-embed planes."""
    check(lib().kt_hip_sam_patch_pack(dev, _ptr(codes_dev), co, ci, kh, kw, _ptr(lo_dev), _ptr(hi_dev),
                                      _stream(stream)), "sam patch pack")


def sam_patch_upload(codes, co: int, ci: int, kh: int, kw: int, lo_dev, hi_dev, dev: int = 0) -> None:
    """Check host codes against [-2048, 2047], upload and pack them into the patch-embed planes (synchronous)."""
    c = _i32(codes)
    if c.size != co * ci * kh * kw:
        raise ValueError("codes are not co·ci·kh·kw")
    check(lib().kt_hip_sam_patch_upload(dev, c.ctypes.data, co, ci, kh, kw, _ptr(lo_dev), _ptr(hi_dev)),
          "sam patch upload")


def sam_patch_embed(img_dev, lut_dev, ci: int, h: int, w: int, lo_dev, hi_dev, co: int, kh: int, kw: int,
                    stride: int, pad: int, bias_dev, mant_dev, shift_dev, out_dev, stream=None, dev: int = 0) -> None:
    """The im2col-fused patch-embed conv: u8 pixels -> entry codes -> W12 GEMM -> +bias -> int8 [co][oh][ow]; the
    weights are the planes of sam_patch_pack / sam_patch_upload."""
    check(
        lib().kt_hip_sam_patch_embed(dev, _ptr(img_dev), _ptr(lut_dev), ci, h, w, _ptr(lo_dev), _ptr(hi_dev), co, kh,
                                     kw, stride, pad, _ptr(bias_dev), _ptr(mant_dev), _ptr(shift_dev), _ptr(out_dev),
                                     _stream(stream)),
        "sam patch embed",
    )


# ---------------------------------------------------------------------------------------------------------------
# host-side synthetic workload generators (no GPU)


def gen_w12_fast(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    lib().kt_hip_gen_w12(seed & (2**64 - 1), n, out.ctypes.data)
    return out


def gen_gauss_fast(seed: int, sigma: int, n: int, clip: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    lib().kt_hip_gen_gauss(seed & (2**64 - 1), sigma, clip, n, out.ctypes.data)
    return out


def gen_uniform_fast(seed: int, lo: int, hi: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    lib().kt_hip_gen_uniform(seed & (2**64 - 1), lo, hi, n, out.ctypes.data)
    return out


def channel_scales_fast(w: np.ndarray, n: int, k: int, sigma: int, target: int = 127) -> tuple[np.ndarray, np.ndarray]:
    w = _i32(w)
    mant = np.empty(n, dtype=np.int32)
    shift = np.empty(n, dtype=np.int32)
    lib().kt_hip_channel_scales(w.ctypes.data, n, k, sigma, target, mant.ctypes.data, shift.ctypes.data)
    return mant, shift


def gen_quant_rows_fast(seed: int, rows: int, cols: int) -> np.ndarray:
    out = np.empty(rows * cols, dtype=np.int32)
    lib().kt_hip_gen_quant_rows(seed & (2**64 - 1), rows, cols, out.ctypes.data)
    return out


# ---------------------------------------------------------------------------------------------------------------
# The reference decoder's layers at the reference's own semantics (crates/01-engine/kt-core/src/{layers,attention,
# model,generate}.rs): i32 codes at the 2^28 level with one kt-int Scale per tensor, in 32-byte device records.
# ---------------------------------------------------------------------------------------------------------------
LUT_EXP, LUT_SILU, LUT_SIGMOID, LUT_GELU = 0, 1, 2, 3
REF_MAX_HEADS = 64


class CodeLut(C.Structure):
    """kt_hip_codelut: a CodeLut's run-time constants (kt-int/src/lib.rs:346-396)."""

    _fields_ = [("inv_mant", C.c_int64), ("inv_shift", C.c_int32), ("n", C.c_int32), ("lo_index", C.c_int64),
                ("code_mant", C.c_int64), ("code_shift", C.c_int32), ("right_identity", C.c_int32)]


SSCALE = np.dtype([("mant", np.int64), ("shift", np.int32), ("sign", np.int32)])  # kt_hip_sscale


def ref_scale_from_f64(x: float) -> tuple[int, int]:
    """Scale::from_f64 (kt-int/src/lib.rs:215-222): (mant, shift) of a positive finite float, (0, 0) otherwise."""
    m, s = C.c_int64(), C.c_int32()
    lib().kt_hip_ref_scale_from_f64(float(x), C.byref(m), C.byref(s))
    return int(m.value), int(s.value)


def ref_codelut(kind: int, lo: float, hi: float, idx_bits: int, code_bits: int, right_identity: bool):
    """CodeLut::build (kt-int/src/lib.rs:359-379) of exp, SiLU, the router's sigmoid or SAM's GELU (LUT_*):
    (codes i64, constants)."""
    codes = np.zeros(1 << idx_bits, dtype=np.int64)
    lut = CodeLut()
    check(lib().kt_hip_ref_codelut(kind, lo, hi, idx_bits, code_bits, int(right_identity), codes.ctypes.data,
                                   C.byref(lut)), "codelut")
    return codes, lut


def ref_rope_tables(max_seq: int, rot_dim: int, theta: float):
    """The RoPE tables of Attention::new (attention.rs:64-90): (cos, sin) as max_seq x rot_dim/2 signed Scales."""
    n = max_seq * (rot_dim // 2)
    cos_t, sin_t = np.zeros(n, dtype=SSCALE), np.zeros(n, dtype=SSCALE)
    check(lib().kt_hip_ref_rope_tables(max_seq, rot_dim, theta, cos_t.ctypes.data, sin_t.ctypes.data), "rope tables")
    return cos_t, sin_t


def ref_embed(emb_dev, e_scale, token_dev, vocab: int, dim: int, y_dev, ys_dev, stream=None, dev: int = 0) -> None:
    check(lib().kt_hip_ref_embed(dev, _ptr(emb_dev), int(e_scale[0]), int(e_scale[1]), _ptr(token_dev), vocab, dim,
                                 _ptr(y_dev), _ptr(ys_dev), _stream(stream)), "ref embed")


def ref_rmsnorm(x_dev, xs_dev, rows: int, dim: int, g_dev, g_scale, eps_scale, y_dev, ys_dev, stream=None,
                dev: int = 0) -> None:
    check(lib().kt_hip_ref_rmsnorm(dev, _ptr(x_dev), _ptr(xs_dev), rows, dim, _ptr(g_dev), int(g_scale[0]),
                                   int(g_scale[1]), int(eps_scale[0]), int(eps_scale[1]), _ptr(y_dev), _ptr(ys_dev),
                                   _stream(stream)), "ref rmsnorm")


def ref_add(a_dev, as_dev, b_dev, bs_dev, n: int, y_dev, ys_dev, stream=None, dev: int = 0) -> None:
    check(lib().kt_hip_ref_add(dev, _ptr(a_dev), _ptr(as_dev), _ptr(b_dev), _ptr(bs_dev), n, _ptr(y_dev),
                               _ptr(ys_dev), _stream(stream)), "ref add")


REF_ADD_NORM_MAX = 4096  # kt_hip_ref_add_rmsnorm's longest row
REF_SWIGLU_SUMS_MAX = 8192  # kt_hip_ref_swiglu_sums's longest tensor


def ref_add_rmsnorm(a_dev, as_dev, b_dev, bs_dev, n: int, y_dev, ys_dev, g_dev, g_scale, eps_scale, h_dev, hs_dev,
                    stream=None, dev: int = 0) -> None:
    """add then RmsNorm of the sum in one launch (n <= REF_ADD_NORM_MAX): y = add(a, b), h = rmsnorm(y)."""
    check(lib().kt_hip_ref_add_rmsnorm(dev, _ptr(a_dev), _ptr(as_dev), _ptr(b_dev), _ptr(bs_dev), n, _ptr(y_dev),
                                       _ptr(ys_dev), _ptr(g_dev), int(g_scale[0]), int(g_scale[1]),
                                       int(eps_scale[0]), int(eps_scale[1]), _ptr(h_dev), _ptr(hs_dev),
                                       _stream(stream)), "ref add + rmsnorm")


def ref_add_rmsnorm_sums(a_dev, as_dev, b: QlSums, n: int, y_dev, ys_dev, g_dev, g_scale, eps_scale, h_dev, hs_dev,
                         stream=None, dev: int = 0) -> None:
    """ref_add_rmsnorm with b a QuantLinear's sums (quant_linear_multi_sums): its requant_dyn in the same launch."""
    check(lib().kt_hip_ref_add_rmsnorm_sums(dev, _ptr(a_dev), _ptr(as_dev), C.byref(b), n, _ptr(y_dev), _ptr(ys_dev),
                                            _ptr(g_dev), int(g_scale[0]), int(g_scale[1]), int(eps_scale[0]),
                                            int(eps_scale[1]), _ptr(h_dev), _ptr(hs_dev), _stream(stream)),
          "ref add + rmsnorm (sums)")


def ref_swiglu_sums(g: QlSums, u: QlSums, n: int, silu_codes_dev, silu: CodeLut, h_dev, hs_dev, stream=None,
                    dev: int = 0) -> None:
    """ref_swiglu of one tensor with g and u a gate / up product's sums: their requant_dyn in the same launch."""
    check(lib().kt_hip_ref_swiglu_sums(dev, C.byref(g), C.byref(u), n, _ptr(silu_codes_dev), C.byref(silu),
                                       _ptr(h_dev), _ptr(hs_dev), _stream(stream)), "ref swiglu (sums)")


def ref_swiglu(g_dev, gs_dev, u_dev, us_dev, n: int, silu_codes_dev, silu: CodeLut, h_dev, hs_dev, stream=None,
               dev: int = 0, rows: int = 1) -> None:
    """SwiGluMlp's activation of `rows` tensors of n values (row r with its own records at index r)."""
    check(lib().kt_hip_ref_swiglu(dev, _ptr(g_dev), _ptr(gs_dev), _ptr(u_dev), _ptr(us_dev), rows, n,
                                  _ptr(silu_codes_dev), C.byref(silu), _ptr(h_dev), _ptr(hs_dev), _stream(stream)),
          "ref swiglu")


def ref_gelu(x_dev, xs_dev, n: int, gelu_codes_dev, gelu: CodeLut, y_dev, ys_dev, stream=None, dev: int = 0) -> None:
    """apply_gelu (kt-model-vision/src/nonlin.rs:30-45) of n codes: y at the table's code scale."""
    check(lib().kt_hip_ref_gelu(dev, _ptr(x_dev), _ptr(xs_dev), n, _ptr(gelu_codes_dev), C.byref(gelu), _ptr(y_dev),
                                _ptr(ys_dev), _stream(stream)), "ref gelu")


def ref_from_reals(real, levels: int = 1 << 28):
    """IntTensor::from_reals (tensor.rs:106-117) on the host: (codes i32, (mant, shift))."""
    r = np.ascontiguousarray(real, dtype=np.float64).reshape(-1)
    codes = np.empty(r.size, dtype=np.int32)
    m, s = C.c_int64(), C.c_int32()
    check(lib().kt_hip_ref_from_reals(r.ctypes.data, r.size, levels, codes.ctypes.data, C.byref(m), C.byref(s)),
          "from_reals")
    return codes, (int(m.value), int(s.value))


def ref_conv2d_workspace(ci: int, h: int, w: int, co: int, kh: int, kw: int, stride: int, pad: int) -> int:
    n = lib().kt_hip_ref_conv2d_workspace(ci, h, w, co, kh, kw, stride, pad)
    if n == 0:
        raise ValueError("conv2d: shape out of range")
    return n


def ref_conv2d(x_dev, xs_dev, ci: int, h: int, w: int, w_planes_dev, pw: int, co: int, kh: int, kw: int, stride: int,
               pad: int, w_scale, bias_dev, b_scale, ws_dev, ws_bytes: int, y_dev, os_dev, stream=None,
               dev: int = 0) -> None:
    """Conv2d::forward_int (conv.rs:68-130): y [co][oh][ow] codes and its record."""
    bm, bsh = b_scale if b_scale is not None else (0, 0)
    check(lib().kt_hip_ref_conv2d(dev, _ptr(x_dev), _ptr(xs_dev), ci, h, w, _ptr(w_planes_dev), pw, co, kh, kw,
                                  stride, pad, int(w_scale[0]), int(w_scale[1]),
                                  0 if bias_dev is None else _ptr(bias_dev), int(bm), int(bsh), _ptr(ws_dev), ws_bytes,
                                  _ptr(y_dev), _ptr(os_dev), _stream(stream)), "ref conv2d")


def ref_seq_workspace(rows: int) -> int:
    return lib().kt_hip_ref_seq_workspace(rows)


def ref_rmsnorm_seq(x_dev, xs_dev, rows: int, dim: int, g_dev, g_scale, eps, ws_dev, ws_bytes: int, y_dev, ys_dev,
                    stream=None, dev: int = 0) -> None:
    """RmsNorm::forward_int of a whole-sequence tensor on many CTAs (the integers of ref_rmsnorm)."""
    check(lib().kt_hip_ref_rmsnorm_seq(dev, _ptr(x_dev), _ptr(xs_dev), rows, dim, _ptr(g_dev), int(g_scale[0]),
                                       int(g_scale[1]), int(eps[0]), int(eps[1]), _ptr(ws_dev), ws_bytes,
                                       _ptr(y_dev), _ptr(ys_dev), _stream(stream)), "ref rmsnorm seq")


def ref_add_seq(a_dev, as_dev, b_dev, bs_dev, n: int, ws_dev, ws_bytes: int, y_dev, ys_dev, stream=None,
                dev: int = 0) -> None:
    check(lib().kt_hip_ref_add_seq(dev, _ptr(a_dev), _ptr(as_dev), _ptr(b_dev), _ptr(bs_dev), n, _ptr(ws_dev),
                                   ws_bytes, _ptr(y_dev), _ptr(ys_dev), _stream(stream)), "ref add seq")


def ref_swiglu_seq(g_dev, gs_dev, u_dev, us_dev, n: int, silu_codes_dev, silu: CodeLut, ws_dev, ws_bytes: int, h_dev,
                   hs_dev, stream=None, dev: int = 0) -> None:
    check(lib().kt_hip_ref_swiglu_seq(dev, _ptr(g_dev), _ptr(gs_dev), _ptr(u_dev), _ptr(us_dev), n,
                                      _ptr(silu_codes_dev), C.byref(silu), _ptr(ws_dev), ws_bytes, _ptr(h_dev),
                                      _ptr(hs_dev), _stream(stream)), "ref swiglu seq")


def ref_embed_seq(emb_dev, e_scale, tokens_dev, T: int, vocab: int, dim: int, y_dev, ys_dev, stream=None,
                  dev: int = 0) -> None:
    """Embedding::lookup_seq (layers.rs:1138-1145) of T tokens in device memory."""
    check(lib().kt_hip_ref_embed_seq(dev, _ptr(emb_dev), int(e_scale[0]), int(e_scale[1]), _ptr(tokens_dev), T, vocab,
                                     dim, _ptr(y_dev), _ptr(ys_dev), _stream(stream)), "ref embed seq")


def ref_attention_prefill_workspace(T: int, nh: int, nkv: int, hd: int) -> int:
    n = lib().kt_hip_ref_attention_prefill_workspace(T, nh, nkv, hd)
    if n == 0:
        raise ValueError("attention prefill: shape out of range")
    return n


def ref_attention_prefill(q_dev, qs_dev, k_dev, ks_dev, v_dev, vs_dev, T: int, nh: int, nkv: int, hd: int,
                          max_seq: int, cos_dev, sin_dev, inv_sqrt, exp_codes_dev, exp_lut: CodeLut, ws_dev,
                          ws_bytes: int, o_dev, os_dev, stream=None, dev: int = 0) -> None:
    """Attention::forward_int between its projections over T rows (attention.rs:467-598)."""
    check(lib().kt_hip_ref_attention_prefill(dev, _ptr(q_dev), _ptr(qs_dev), _ptr(k_dev), _ptr(ks_dev), _ptr(v_dev),
                                             _ptr(vs_dev), T, nh, nkv, hd, max_seq, _ptr(cos_dev), _ptr(sin_dev),
                                             int(inv_sqrt[0]), int(inv_sqrt[1]), _ptr(exp_codes_dev),
                                             C.byref(exp_lut), _ptr(ws_dev), ws_bytes, _ptr(o_dev), _ptr(os_dev),
                                             _stream(stream)), "ref attention prefill")


def ref_attention_step_workspace(max_seq: int, nh: int, hd: int) -> int:
    """Bytes of the workspace of the several-CTAs-per-head attention step (kt_hip_ref_attention_step_ws)."""
    return lib().kt_hip_ref_attention_step_workspace(max_seq, nh, hd)


def ref_attention_step_fits_lds(max_seq: int, nh: int, hd: int) -> bool:
    """Whether the attention step holds a cache of max_seq positions in LDS alone (no workspace needed)."""
    return max_seq * (32 + 8) + nh * hd * 12 <= REF_ATTN_LDS


REF_ATTN_LDS = 65536  # KT_REF_ATTN_LDS


def ref_attention_step(q_dev, qs_dev, k_dev, ks_dev, v_dev, vs_dev, pos_dev, nh: int, nkv: int, hd: int,
                       max_seq: int, kc_dev, vc_dev, kscale_dev, vscale_dev, cos_dev, sin_dev, inv_sqrt,
                       exp_codes_dev, exp_lut: CodeLut, o_dev, os_dev, stream=None, dev: int = 0, ws_dev=None) -> None:
    """Attention::decode_step's core at position pos_dev[0]: with ws_dev (ref_attention_step_workspace bytes) several
    CTAs per head, any max_seq; without, one CTA whose LDS bounds max_seq (ref_attention_step_fits_lds)."""
    ws_bytes = 0 if ws_dev is None else ws_dev.numel() * ws_dev.element_size()
    check(lib().kt_hip_ref_attention_step_ws(dev, _ptr(q_dev), _ptr(qs_dev), _ptr(k_dev), _ptr(ks_dev),
                                             _ptr(v_dev), _ptr(vs_dev), _ptr(pos_dev), nh, nkv, hd, max_seq,
                                             _ptr(kc_dev), _ptr(vc_dev), _ptr(kscale_dev), _ptr(vscale_dev),
                                             _ptr(cos_dev), _ptr(sin_dev), int(inv_sqrt[0]), int(inv_sqrt[1]),
                                             _ptr(exp_codes_dev), C.byref(exp_lut), _ptr(o_dev), _ptr(os_dev),
                                             _ptr(ws_dev), ws_bytes, _stream(stream)),
          "ref attention step")


def ref_attention_step_sums(q: QlSums, k: QlSums, v: QlSums, pos_dev, nh: int, nkv: int, hd: int, max_seq: int,
                            kc_dev, vc_dev, kscale_dev, vscale_dev, cos_dev, sin_dev, inv_sqrt, exp_codes_dev,
                            exp_lut: CodeLut, o_dev, os_dev, ws_dev, stream=None, dev: int = 0) -> None:
    """ref_attention_step with a workspace and q, k, v a q / k / v product's sums: every CTA applies their
    requant_dyn itself."""
    ws_bytes = ws_dev.numel() * ws_dev.element_size()
    check(lib().kt_hip_ref_attention_step_sums(dev, C.byref(q), C.byref(k), C.byref(v), _ptr(pos_dev), nh, nkv, hd,
                                               max_seq, _ptr(kc_dev), _ptr(vc_dev), _ptr(kscale_dev),
                                               _ptr(vscale_dev), _ptr(cos_dev), _ptr(sin_dev), int(inv_sqrt[0]),
                                               int(inv_sqrt[1]), _ptr(exp_codes_dev), C.byref(exp_lut), _ptr(o_dev),
                                               _ptr(os_dev), _ptr(ws_dev), ws_bytes, _stream(stream)),
          "ref attention step (sums)")


def ref_argmax(logits_dev, n: int, ls_dev, token_dev, record_dev=None, rscale_dev=None, step_dev=None, stream=None,
               dev: int = 0, record_rows: int = None) -> None:
    """argmax_codes into token_dev; with a record, the codes and scale go to row step_dev[0] of record_dev /
    rscale_dev while that row exists (record_rows, by default as many rows of n codes as record_dev holds and as
    many 16-byte entries as rscale_dev holds), and the step advances; past the last row nothing is recorded."""
    if record_dev is not None and record_rows is None:
        record_rows = min(record_dev.numel() // n, rscale_dev.numel() * rscale_dev.element_size() // 16)
    check(lib().kt_hip_ref_argmax(dev, _ptr(logits_dev), n, _ptr(ls_dev), _ptr(token_dev), _ptr(record_dev),
                                  _ptr(rscale_dev), _ptr(step_dev), int(record_rows or 0), _stream(stream)),
          "ref argmax")


REF_MOE_MAX_K = 32


def quant_linear_rows_workspace(rows: int, in_f: int, out_f: int, groups: int) -> int:
    return lib().kt_hip_quant_linear_rows_workspace(rows, in_f, out_f, groups)


def quant_linear_rows(x_dev, xidx_dev, x_rows: int, rows: int, in_f: int, xs_dev, xs_step: int, off_host, off_dev,
                      w_planes_dev, w_group_bytes: int, pw: int, out_f: int, w_mant_dev, w_shift_dev, ws_dev,
                      ws_bytes: int, y_dev, ys_dev, stream=None, dev: int = 0, groups: int | None = None) -> None:
    """QuantLinear::forward_int on each row on its own, rows grouped by weights (off_dev: groups + 1 offsets on the
    device; off_host: None, or the same offsets on the host, checked; groups is then taken from them)."""
    if off_host is not None:
        off = np.ascontiguousarray(off_host, dtype=np.int64)
        groups, off_ptr = off.size - 1, off.ctypes.data
    else:
        off, off_ptr = None, None
        if groups is None:
            raise ValueError("quant_linear_rows: groups is needed without off_host")
    check(lib().kt_hip_quant_linear_rows(dev, _ptr(x_dev), _ptr(xidx_dev), x_rows, rows, in_f, _ptr(xs_dev), xs_step,
                                         groups, off_ptr, _ptr(off_dev), _ptr(w_planes_dev), w_group_bytes, pw, out_f,
                                         _ptr(w_mant_dev), _ptr(w_shift_dev), _ptr(ws_dev), ws_bytes, _ptr(y_dev),
                                         _ptr(ys_dev), _stream(stream)), "quant linear rows")


def pack_planes_tiled_bytes(rows: int, k: int, planes: int) -> int:
    n = lib().kt_hip_pack_planes_tiled_bytes(rows, k, planes)
    if n == 0:
        raise ValueError("pack_planes_tiled: no layout for this shape")
    return n


def pack_planes_tiled(codes_dev, rows: int, k: int, planes: int, planes_dev, stream=None, dev: int = 0) -> None:
    """The digit planes of rows x k codes in quant_linear_rows' tiled weight layout."""
    check(lib().kt_hip_pack_planes_tiled(dev, _ptr(codes_dev), rows, k, planes, _ptr(planes_dev), _stream(stream)),
          "pack planes tiled")


def ref_moe_bucket(sel_dev, tokens: int, top_k: int, experts: int, off_dev, xidx_dev, pos_dev, stream=None,
                   dev: int = 0) -> None:
    """MoeMlp's bucket on the device: sel (tokens x top_k expert ids) -> off (experts + 1), xidx (row -> token), pos
    (pair -> row)."""
    check(lib().kt_hip_ref_moe_bucket(dev, _ptr(sel_dev), tokens, top_k, experts, _ptr(off_dev), _ptr(xidx_dev),
                                      _ptr(pos_dev), _stream(stream)), "ref moe bucket")


def ref_moe_route(logits_dev, tokens: int, experts: int, top_k: int, ls_dev, sigmoid: bool, norm_topk: bool,
                  codes_dev, lut: CodeLut, bias_dev, sel_dev, ec_dev, sumc_dev, stream=None, dev: int = 0) -> None:
    check(lib().kt_hip_ref_moe_route(dev, _ptr(logits_dev), tokens, experts, top_k, _ptr(ls_dev), int(sigmoid),
                                     int(norm_topk), _ptr(codes_dev), C.byref(lut), _ptr(bias_dev), _ptr(sel_dev),
                                     _ptr(ec_dev), _ptr(sumc_dev), _stream(stream)), "ref moe route")


def ref_moe_combine(y_dev, ys_dev, y_rows: int, dim: int, pos_dev, ec_dev, sumc_dev, tokens: int, top_k: int, out_dev,
                    os_dev, stream=None, dev: int = 0) -> None:
    check(lib().kt_hip_ref_moe_combine(dev, _ptr(y_dev), _ptr(ys_dev), y_rows, dim, _ptr(pos_dev), _ptr(ec_dev),
                                       _ptr(sumc_dev), tokens, top_k, _ptr(out_dev), _ptr(os_dev), _stream(stream)),
          "ref moe combine")


def ref_merge_rows_workspace(tokens: int) -> int:
    return lib().kt_hip_ref_merge_rows_workspace(tokens)


def ref_merge_rows(rows_dev, rs_dev, tokens: int, dim: int, ws_dev, ws_bytes: int, out_dev, os_dev, stream=None,
                   dev: int = 0) -> None:
    check(lib().kt_hip_ref_merge_rows(dev, _ptr(rows_dev), _ptr(rs_dev), tokens, dim, _ptr(ws_dev), ws_bytes,
                                      _ptr(out_dev), _ptr(os_dev), _stream(stream)), "ref merge rows")
