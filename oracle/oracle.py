"""TEST INFRASTRUCTURE ONLY: numpy/ctypes access to the C oracle (oracle/kt_oracle.c).

The oracle is the CPU restatement of tritify's exact-integer path that the GPU backend is checked against, and the
timed CPU baseline. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module;
the product package (tritify_amd) never does.

Each wrapper names the reference function it restates (paths relative to the tritify repository root).
"""
from __future__ import annotations

import ctypes as C
import hashlib
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkt_oracle.so")

WLEVELS = 265_720  # crates/01-engine/kt-core/src/layers.rs:16
ACT_LEVELS = 1 << 28  # layers.rs:18
K_MAX = (2**63 - 1) // (WLEVELS * WLEVELS)  # kt-cuda/src/digits.rs:23
KT_FLUSH = (2**31 - 1) // (16 * 40 * 40)  # kt-cuda/src/digits.rs:20

_lib = None


def build() -> None:
    """Compile the oracle with its committed Makefile."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


class Scale(C.Structure):
    """kt_int::Scale (crates/00-kernels/kt-int/src/lib.rs:175-178)."""

    _fields_ = [("mant", C.c_int64), ("shift", C.c_int32)]

    def __repr__(self) -> str:
        return f"Scale(mant={self.mant}, shift={self.shift})"

    def __eq__(self, o) -> bool:
        return (self.mant, self.shift) == (o.mant, o.shift)


_P = C.c_void_p
_SZ = C.c_size_t


def _declare(L: C.CDLL) -> None:
    sig = {
        "kt_lcg_next": (C.c_uint64, [C.POINTER(C.c_uint64)]),
        "kt_sha256": (None, [_P, _SZ, _P]),
        "kt_dot_portable": (C.c_int64, [_P, _P, _SZ]),
        "kt_cpu_variant_available": (C.c_int, [C.c_int]),
        "kt_cpu_auto_variant": (C.c_int, []),
        "kt_set_max_threads": (None, [_SZ]),
        "kt_max_threads": (_SZ, []),
        "kt_resolve_threads": (_SZ, [_SZ]),
        "kt_plan_threads": (_SZ, [_SZ, _SZ]),
        "kt_linear_cpu": (None, [_P, _P, _SZ, _SZ, _SZ, C.c_int, _P]),
        "kt_linear_cpu_threads": (None, [_P, _P, _SZ, _SZ, _SZ, C.c_int, _SZ, _P]),
        "kt_linear_planted_partition": (None, [_P, _P, _SZ, _SZ, _SZ, C.c_int, _SZ, _P]),
        "kt_linear_planted_dot": (None, [_P, _P, _SZ, _SZ, _SZ, C.c_int, _P]),
        "kt_gen_demo": (None, [_SZ, _SZ, _SZ, C.c_uint64, _P, _P]),
        "kt_gen_wlevels": (None, [C.POINTER(C.c_uint64), _SZ, _P]),
        "kt_gen_w12": (None, [C.c_uint64, _SZ, _P]),
        "kt_gen_act_gauss": (None, [C.c_uint64, C.c_int64, _SZ, _P]),
        "kt_gen_act_uniform": (None, [C.c_uint64, _SZ, _P]),
        "kt_split81": (C.c_int, [C.c_int32, _P]),
        "kt_join81": (C.c_int64, [_P]),
        "kt_split256": (C.c_int, [C.c_int64, C.c_int, C.c_int, _P]),
        "kt_join256": (C.c_int64, [_P, C.c_int]),
        "kt_planes_for": (C.c_int, [_P, _SZ]),
        "kt_pack_planes": (None, [_P, _SZ, _SZ, C.c_int, C.c_int, _P]),
        "kt_flush_k": (C.c_int64, [C.c_int, C.c_int]),
        "kt_emu_linear": (None, [_P, _P, _SZ, _SZ, _SZ, C.c_int, C.c_int, C.c_int64, C.c_int, C.c_int, _P]),
        "kt_frexp": (C.c_double, [C.c_double, C.POINTER(C.c_int32)]),
        "kt_frexp_scale": (None, [C.c_double, C.c_uint32, C.POINTER(C.c_int64), C.POINTER(C.c_int32)]),
        "kt_requant": (C.c_int64, [C.c_int64, C.c_int64, C.c_int32]),
        "kt_requant_sat": (C.c_int64, [C.c_int64, C.c_int64, C.c_int32]),
        "kt_scale_from_ratio": (Scale, [C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64]),
        "kt_scale_from_f64": (Scale, [C.c_double]),
        "kt_scale_ge": (C.c_int, [Scale, Scale]),
        "kt_scale_mul": (Scale, [Scale, Scale]),
        "kt_scale_apply": (C.c_int64, [Scale, C.c_int64]),
        "kt_scale_recip": (Scale, [Scale]),
        "kt_scale_add": (Scale, [Scale, Scale]),
        "kt_scale_rsqrt": (Scale, [Scale]),
        "kt_scale_to_i32": (Scale, [Scale]),
        "kt_isqrt_u128": (C.c_uint64, [C.c_uint64, C.c_uint64]),
        "kt_quant_to": (None, [_P, _SZ, C.c_int64, _P]),
        "kt_requant_dyn": (C.c_int32, [C.c_int64, C.c_int64, C.c_int64]),
        "kt_quant_linear_forward": (None, [_P, _SZ, _SZ, Scale, _P, _SZ, Scale, _P, Scale, _SZ, _P, C.POINTER(Scale),
                                           C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
        "kt_w12_pack": (None, [_P, _SZ, _SZ, _P, _P]),
        "kt_w12_get": (C.c_int32, [_P, _P, _SZ, _SZ, _SZ]),
        "kt_w12_linear": (None, [_P, _P, _P, _SZ, _SZ, _SZ, _P]),
        "kt_requant_channels": (None, [_P, _SZ, _SZ, _P, _P, C.c_int64, C.c_int64, _P]),
        "kt_channel_scales": (None, [_P, _SZ, _SZ, C.c_int64, _P, _P]),
        "kt_gen_w12_i16": (None, [C.c_uint64, _SZ, _P]),
        "kt_gen_gauss_i32": (None, [C.c_uint64, C.c_int64, _SZ, _P]),
        "kt_channel_scales_i16": (None, [_P, _SZ, _SZ, C.c_int64, _P, _P]),
        "kt_gemm_i8w16": (C.c_int, [_P, _P, _SZ, _SZ, _SZ, _P, _P, _P, _P, _SZ]),
        "kt_moe_route": (None, [_P, _SZ, _SZ, _SZ, _P, _P, _P]),
        "kt_moe_bucket": (None, [_P, _SZ, _SZ, _SZ, _P, _P, _P]),
        "kt_moe_experts": (C.c_int, [_P, _SZ, _SZ, _SZ, _SZ, _P, _P, _P, _P, _P, _P, _P, _P, _P, C.c_int, _P, _P,
                                     _SZ]),
        "kt_moe_combine": (None, [_P, _P, _P, _P, _P, _SZ, _SZ, _SZ, _SZ, C.c_int, _P]),
        "kt_sam_entry": (None, [_P, _SZ, _SZ, _P, _P]),
        "kt_gen_uniform_i32": (None, [C.c_uint64, C.c_int64, C.c_int64, _SZ, _P]),
        "kt_gen_quant_rows": (None, [C.c_uint64, _SZ, _SZ, _P]),
        "kt_channel_scales_target_i16": (None, [_P, _SZ, _SZ, C.c_int64, C.c_int64, _P, _P]),
        "kt_argmax_i32": (C.c_int64, [_P, _SZ]),
        "kt_dec_generate": (C.c_int, [_P, _P, _SZ, _SZ, C.c_int, _P, _P, _SZ]),
        "kt_dec_rmsnorm_rows": (None, [_P, _SZ, _SZ, _P]),
        "kt_dec_rope_row": (None, [_P, _SZ, _SZ, _SZ, _P, _P]),
        "kt_dec_attend": (None, [_P, _P, _P, _SZ, _SZ, _SZ, _SZ, _P, _P, _P]),
        "kt_conv2d_i8w16": (None, [_P, _SZ, _SZ, _SZ, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _P, _P, _P, _P, _P, _SZ]),
        "kt_mlp_gelu": (C.c_int, [_P, _SZ, _SZ, _SZ, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ]),
        "kt_rd_synthetic": (_P, [C.c_uint64, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, C.c_double, C.c_double, _SZ]),
        "kt_rd_free": (None, [_P]),
        "kt_rd_generate": (C.c_int, [_P, _P, _SZ, _SZ, _P, _P, _P]),
        "kt_rd_cache_new": (_P, [_P]),
        "kt_rd_cache_free": (None, [_P]),
        "kt_rd_decode_step": (None, [_P, _P, C.c_int64, _SZ, _P, C.POINTER(Scale)]),
        "kt_rd_rmsnorm": (None, [_P, _SZ, _SZ, Scale, _P, Scale, Scale, _P, C.POINTER(Scale)]),
        "kt_rd_add": (None, [_P, Scale, _P, Scale, _SZ, _P, C.POINTER(Scale)]),
        "kt_rd_swiglu_act": (None, [_P, _P, Scale, _P, Scale, _SZ, _P, C.POINTER(Scale)]),
        "kt_rd_attention_core": (None, [_P, _P, _P, Scale, _P, Scale, _P, Scale, _SZ, _P, C.POINTER(Scale)]),
        "kt_rd_attention_append": (None, [_P, _P, _P, Scale, _P, Scale, _SZ]),
        "kt_rd_attention_prefill": (None, [_P, _SZ, _P, Scale, _P, Scale, _P, Scale, _P, C.POINTER(Scale)]),
        "kt_rd_forward": (C.c_int, [_P, _P, _SZ, _P, C.POINTER(Scale)]),
        "kt_rd_new": (_P, [_SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, C.c_double, C.c_double, _SZ]),
        "kt_rd_set_ql": (None, [_P, _SZ, C.c_int, _P, _SZ, _SZ, Scale]),
        "kt_rd_set_norm": (None, [_P, _SZ, C.c_int, _P, Scale]),
        "kt_rd_set_emb": (None, [_P, _P, Scale]),
        "kt_rd_get_ql": (Scale, [_P, _SZ, C.c_int, _P, C.POINTER(_SZ), C.POINTER(_SZ)]),
        "kt_rd_get_norm": (Scale, [_P, _SZ, C.c_int, _P, C.POINTER(Scale)]),
        "kt_rd_get_emb": (Scale, [_P, _P]),
        "kt_rd_get_lut": (None, [_P, C.c_int, _P, C.POINTER(Scale), C.POINTER(C.c_int64), C.POINTER(Scale)]),
        "kt_rd_get_rope": (Scale, [_P, _P, _P, _P, _P, _P, _P]),
        "kt_rm_synthetic": (_P, [C.c_uint64, _SZ, _SZ, _SZ, _SZ, C.c_int, C.c_int, C.c_uint64, _SZ]),
        "kt_rm_free": (None, [_P]),
        "kt_rm_route": (C.c_int64, [_P, _P, Scale, _P, _P, _P, C.POINTER(Scale)]),
        "kt_rm_combine": (None, [_P, _P, _SZ, _SZ, _P, C.c_int64, _P, C.POINTER(Scale)]),
        "kt_rm_merge_rows": (None, [_P, _P, _SZ, _SZ, _P, C.POINTER(Scale)]),
        "kt_rm_forward": (None, [_P, _P, _SZ, Scale, _P, C.POINTER(Scale)]),
        "kt_rm_expert": (None, [_P, _SZ, _P, _SZ, Scale, _P, C.POINTER(Scale)]),
        "kt_rm_get_ql": (Scale, [_P, _SZ, C.c_int, _P, C.POINTER(_SZ), C.POINTER(_SZ)]),
        "kt_rm_get_lut": (None, [_P, C.c_int, _P, C.POINTER(Scale), C.POINTER(C.c_int64), C.POINTER(Scale)]),
        "kt_rm_get_bias": (None, [_P, _P]),
        "kt_rm_probe": (Scale, [C.POINTER(C.c_uint64), _SZ, _P]),
        "kt_rm_set_bias": (None, [_P, _SZ, C.c_float]),
        "kt_rm_empty": (_P, [_SZ, _SZ, _SZ, _SZ, C.c_int, C.c_int, _SZ]),
        "kt_rm_set_ql": (None, [_P, _SZ, C.c_int, _P, Scale]),
        "kt_rm_set_bias_code": (None, [_P, _SZ, C.c_int64]),
        "kt_rm_sigmoid_codes": (None, [_P, _P, _SZ, Scale, _P]),
        "kt_rc_from_reals": (Scale, [_P, _SZ, C.c_int64, _P]),
        "kt_rc_quant_weights": (Scale, [_P, _SZ, _P]),
        "kt_rc_quant_bias": (C.c_int, [_P, _SZ, _P, C.POINTER(Scale)]),
        "kt_rc_conv2d": (None, [_P, Scale, _SZ, _SZ, _SZ, _P, Scale, _SZ, _SZ, _SZ, _SZ, _SZ, _P, Scale, _P,
                                C.POINTER(Scale)]),
        "kt_rc_gelu_table": (None, [_P, C.POINTER(Scale), C.POINTER(C.c_int64), C.POINTER(Scale)]),
        "kt_rc_apply_gelu": (None, [_P, _SZ, Scale, _P, C.POINTER(Scale)]),
        "kt_rc_feedforward": (None, [_P, _SZ, _SZ, Scale, _P, Scale, _P, Scale, _SZ, _P, Scale, _P, Scale, _P,
                                     C.POINTER(Scale)]),
        "kt_moe_forward_token": (None, [_P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _P, _P, _P, _P, _P, _P, _P, _P, C.c_int,
                                        C.c_int, _P]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


# ---------------------------------------------------------------------------------------------------------------
# hashing


def sha256_hex(a: np.ndarray) -> str:
    """SHA-256 over the array's little-endian words (apps/kt-demo/src/main.rs:57-63; kt-core/src/verify.rs:35-41)."""
    a = np.ascontiguousarray(a)
    out = (C.c_uint8 * 32)()
    lib().kt_sha256(_ptr(a), a.nbytes, out)
    return bytes(out).hex()


def sha256_py(a: np.ndarray) -> str:
    """hashlib's SHA-256 of the same bytes (an independent implementation, used to pin kt_sha256)."""
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# ---------------------------------------------------------------------------------------------------------------
# the linear accumulate


def linear_cpu(x, w, rows: int, out: int, k: int, variant: int | None = None) -> np.ndarray:
    """linear_cpu on a dot variant (crates/01-engine/kt-core/src/backend.rs:133-140; kt-runtime/src/cpu.rs).

    variant: 0 portable, 1 avx2, 2 avx512; None = the auto rank (kt-runtime/src/lib.rs:93-96)."""
    x, w = _i32(x), _i32(w)
    assert x.size == rows * k and w.size == out * k
    v = lib().kt_cpu_auto_variant() if variant is None else variant
    y = np.empty(rows * out, dtype=np.int64)
    lib().kt_linear_cpu(_ptr(x), _ptr(w), rows, out, k, v, _ptr(y))
    return y


def portable(x, w, rows: int, out: int, k: int) -> np.ndarray:
    """Portable.linear (backend.rs:143-152)."""
    return linear_cpu(x, w, rows, out, k, variant=0)


def linear_threads(x, w, rows, out, k, threads, variant=0) -> np.ndarray:
    x, w = _i32(x), _i32(w)
    y = np.full(rows * out, -1, dtype=np.int64)
    lib().kt_linear_cpu_threads(_ptr(x), _ptr(w), rows, out, k, variant, threads, _ptr(y))
    return y


def planted_partition(x, w, rows, out, k, bad: int, threads: int = 0) -> np.ndarray:
    """kt-runtime/src/planted.rs:28-59. bad: 1 FloorOffsets, 2 DropLastRun, 3 SwappedIndex."""
    x, w = _i32(x), _i32(w)
    y = np.zeros(rows * out, dtype=np.int64)
    lib().kt_linear_planted_partition(_ptr(x), _ptr(w), rows, out, k, bad, threads, _ptr(y))
    return y


def planted_dot(x, w, rows, out, k, which: int) -> np.ndarray:
    """kt-runtime/src/tests.rs:9-17. which: 10 wrapping i32 accumulator, 11 f32 accumulator."""
    x, w = _i32(x), _i32(w)
    y = np.zeros(rows * out, dtype=np.int64)
    lib().kt_linear_planted_dot(_ptr(x), _ptr(w), rows, out, k, which, _ptr(y))
    return y


def set_max_threads(n: int) -> None:
    lib().kt_set_max_threads(n)


def plan_threads(elems: int, work: int) -> int:
    return lib().kt_plan_threads(elems, min(work, 2**64 - 1))


def resolve_threads(nblocks: int) -> int:
    return lib().kt_resolve_threads(nblocks)


# ---------------------------------------------------------------------------------------------------------------
# generators


def gen_demo(m: int, n: int, k: int, seed: int = 42):
    """apps/kt-demo/src/main.rs:23-28."""
    qx = np.empty(m * k, dtype=np.int32)
    qw = np.empty(n * k, dtype=np.int32)
    lib().kt_gen_demo(m, n, k, seed, _ptr(qx), _ptr(qw))
    return qx, qw


class Stream:
    """One LCG stream (main.rs:19-22) drawing codes uniform in +-WLEVELS (gate.rs:29-36)."""

    def __init__(self, seed: int):
        self.s = C.c_uint64(seed)

    def wlevels(self, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.int32)
        lib().kt_gen_wlevels(C.byref(self.s), n, _ptr(out))
        return out


def codes(n: int, seed: int) -> np.ndarray:
    """kt-cuda/src/tests.rs:9-15: codes uniform in +-WLEVELS from a seeded LCG."""
    return Stream(seed).wlevels(n)


class Case:
    def __init__(self, label, rows, out, k, x, w):
        self.label, self.rows, self.out, self.k, self.x, self.w = label, rows, out, k, x, w


def corpus() -> list[Case]:
    """The fixed gate corpus, crates/02-runtime/kt-runtime/src/gate.rs:26-56."""
    lv = WLEVELS
    st = Stream(0x5032_0B00)
    cases = []
    for label, rows, out, k in [
        ("k=1", 1, 1, 1),
        ("odd tail", 3, 5, 7),
        ("k=33", 2, 17, 33),
        ("k=1023", 4, 64, 1023),
        ("k=4099 (long)", 1, 9, 4099),
        ("threaded 8×512×2048", 8, 512, 2048),
    ]:
        x = st.wlevels(rows * k)
        w = st.wlevels(out * k)
        cases.append(Case(label, rows, out, k, x, w))
    k = 1027
    x = np.array([-lv if i % 3 == 0 else lv for i in range(2 * k)], dtype=np.int32)
    w = np.array([lv if i % 2 == 0 else -lv for i in range(3 * k)], dtype=np.int32)
    cases.append(Case("extremes ±WLEVELS", 2, 3, k, x, w))
    x = np.full(4 * 2048, lv, dtype=np.int32)
    cases.append(Case("all +WLEVELS", 4, 4, 2048, x, x.copy()))
    return cases


def flush_case() -> Case:
    """gate.rs:61-66: the smallest k beyond one int32 flush of the reference's digit backend."""
    k = (KT_FLUSH + 1) * 16
    lv = WLEVELS
    w = np.concatenate([np.full(k, lv, dtype=np.int32), np.full(k, -lv, dtype=np.int32)])
    return Case("k beyond one int32 flush", 1, 2, k, np.full(k, lv, dtype=np.int32), w)


def gen_w12(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    lib().kt_gen_w12(seed, n, _ptr(out))
    return out


def gen_act_gauss(seed: int, sigma: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    lib().kt_gen_act_gauss(seed, sigma, n, _ptr(out))
    return out


def gen_act_uniform(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    lib().kt_gen_act_uniform(seed, n, _ptr(out))
    return out


# ---------------------------------------------------------------------------------------------------------------
# digits and the plane emulator


def split81(v: int):
    d = (C.c_int8 * 3)()
    ok = lib().kt_split81(v, d)
    return list(d) if ok else None


def join81(d) -> int:
    a = (C.c_int8 * 3)(*d)
    return lib().kt_join81(a)


def split256(v: int, p: int, wrong_carry: bool = False):
    d = (C.c_int8 * 5)()
    ok = lib().kt_split256(v, p, int(wrong_carry), d)
    return list(d)[:p] if ok else None


def planes_for(v) -> int:
    v = _i32(v)
    return lib().kt_planes_for(_ptr(v), v.size)


def pack_planes(codes_, rows, k, p, wrong_carry=False) -> np.ndarray:
    codes_ = _i32(codes_)
    kp = (k + 63) // 64 * 64
    out = np.empty(p * rows * kp, dtype=np.int8)
    lib().kt_pack_planes(_ptr(codes_), rows, k, p, int(wrong_carry), _ptr(out))
    return out.reshape(p, rows, kp)


def flush_k(px: int, pw: int) -> int:
    return lib().kt_flush_k(px, pw)


def emu_linear(x, w, rows, out, k, px=None, pw=None, flush=None, drop_top=False, wrong_carry=False) -> np.ndarray:
    """The plane product step for step on the CPU (analogue of kt-cuda/src/host.rs:53-84)."""
    x, w = _i32(x), _i32(w)
    px = planes_for(x) if px is None else px
    pw = planes_for(w) if pw is None else pw
    fk = flush_k(px, pw) if flush is None else flush
    y = np.zeros(rows * out, dtype=np.int64)
    lib().kt_emu_linear(_ptr(x), _ptr(w), rows, out, k, px, pw, fk, int(drop_top), int(wrong_carry), _ptr(y))
    return y


# ---------------------------------------------------------------------------------------------------------------
# kt-int


def requant(accum: int, mant: int, shift: int) -> int:
    return lib().kt_requant(accum, mant, shift)


def requant_sat(accum: int, mant: int, shift: int) -> int:
    return lib().kt_requant_sat(accum, mant, shift)


def frexp(x: float):
    e = C.c_int32()
    m = lib().kt_frexp(x, C.byref(e))
    return m, e.value


def frexp_scale(x: float, mant_bits: int):
    m, s = C.c_int64(), C.c_int32()
    lib().kt_frexp_scale(x, mant_bits, C.byref(m), C.byref(s))
    return m.value, s.value


def from_ratio(num: int, den: int) -> Scale:
    return lib().kt_scale_from_ratio(num >> 64, num & (2**64 - 1), den >> 64, den & (2**64 - 1))


def from_f64(x: float) -> Scale:
    return lib().kt_scale_from_f64(x)


def scale_mul(a: Scale, b: Scale) -> Scale:
    return lib().kt_scale_mul(a, b)


def scale_apply(a: Scale, v: int) -> int:
    return lib().kt_scale_apply(a, v)


def scale_recip(a: Scale) -> Scale:
    return lib().kt_scale_recip(a)


def scale_add(a: Scale, b: Scale) -> Scale:
    return lib().kt_scale_add(a, b)


def scale_rsqrt(a: Scale) -> Scale:
    return lib().kt_scale_rsqrt(a)


def scale_ge(a: Scale, b: Scale) -> bool:
    return bool(lib().kt_scale_ge(a, b))


def scale_to_i32(a: Scale) -> Scale:
    return lib().kt_scale_to_i32(a)


def isqrt_u128(n: int) -> int:
    return lib().kt_isqrt_u128(n >> 64, n & (2**64 - 1))


def quant_to(data, xmax: int) -> np.ndarray:
    data = _i32(data)
    out = np.empty_like(data)
    lib().kt_quant_to(_ptr(data), data.size, xmax, _ptr(out))
    return out


def requant_dyn(v: int, num_level: int, den: int) -> int:
    return lib().kt_requant_dyn(v, num_level, den)


def quant_linear_forward(x, rows: int, in_f: int, xs, w, out_f: int, ws, bias=None, bs=(0, 0), threads: int = 0):
    """QuantLinear::forward_int (layers.rs:275-328): (y codes rows x out_f, (mant, shift), xmax, ymax)."""
    x, w = _i32(x), _i32(w)
    assert x.size == rows * in_f and w.size == out_f * in_f
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.int64)
    y = np.empty(rows * out_f, dtype=np.int32)
    os_, xmax, ymax = Scale(), C.c_int64(), C.c_int64()
    lib().kt_quant_linear_forward(_ptr(x), rows, in_f, Scale(*xs), _ptr(w), out_f, Scale(*ws),
                                  0 if b is None else _ptr(b), Scale(*bs), threads, _ptr(y), C.byref(os_),
                                  C.byref(xmax), C.byref(ymax))
    return y.reshape(rows, out_f), (os_.mant, os_.shift), xmax.value, ymax.value


# ---------------------------------------------------------------------------------------------------------------
# the 12-bit weight path


def w12_sizes(n: int, k: int):
    """Bytes of the W12 lo and nib planes: rows rounded up to 32, k to 64."""
    lo = (n + 31) // 32 * 32 * ((k + 63) // 64 * 64)
    return lo, lo // 2


def w12_pack(codes_, n: int, k: int):
    codes_ = _i32(codes_)
    nlo, nnib = w12_sizes(n, k)
    lo = np.empty(nlo, dtype=np.int8)
    nib = np.empty(nnib, dtype=np.uint8)
    lib().kt_w12_pack(_ptr(codes_), n, k, _ptr(lo), _ptr(nib))
    return lo, nib


def w12_get(lo, nib, k, r, c) -> int:
    return lib().kt_w12_get(_ptr(lo), _ptr(nib), k, r, c)


def w12_linear(x, lo, nib, m, n, k) -> np.ndarray:
    x = _i32(x)
    y = np.empty(m * n, dtype=np.int64)
    lib().kt_w12_linear(_ptr(x), _ptr(lo), _ptr(nib), m, n, k, _ptr(y))
    return y


def requant_channels(acc, m, n, mant, shift, lo=-127, hi=127) -> np.ndarray:
    acc = np.ascontiguousarray(acc, dtype=np.int64)
    mant, shift = _i32(mant), _i32(shift)
    out = np.empty(m * n, dtype=np.int32)
    lib().kt_requant_channels(_ptr(acc), m, n, _ptr(mant), _ptr(shift), lo, hi, _ptr(out))
    return out


def channel_scales(w, n, k, sigma=40):
    w = _i32(w)
    mant = np.empty(n, dtype=np.int32)
    shift = np.empty(n, dtype=np.int32)
    lib().kt_channel_scales(_ptr(w), n, k, sigma, _ptr(mant), _ptr(shift))
    return mant, shift


# ---------------------------------------------------------------------------------------------------------------
# the layers of configs 3-5 (kt_oracle_layers.c)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def gen_w12_i16(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int16)
    lib().kt_gen_w12_i16(seed & (2**64 - 1), n, _ptr(out))
    return out


def gen_gauss_i32(seed: int, sigma: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    lib().kt_gen_gauss_i32(seed & (2**64 - 1), sigma, n, _ptr(out))
    return out


def channel_scales_i16(w, n: int, k: int, sigma: int):
    w = _c(w, np.int16)
    mant = np.empty(n, dtype=np.int32)
    shift = np.empty(n, dtype=np.int32)
    lib().kt_channel_scales_i16(_ptr(w), n, k, sigma, _ptr(mant), _ptr(shift))
    return mant, shift


def gemm_i8w16(x, w, m: int, n: int, k: int, mant=None, shift=None, threads: int = 0):
    """(acc i64 m x n, y8 int8 m x n or None): x int8 m x k against int16 codes n x k, the int8 epilogue when
    scales are given."""
    x, w = _c(x, np.int8), _c(w, np.int16)
    acc = np.empty(m * n, dtype=np.int64)
    y8 = np.empty(m * n, dtype=np.int8) if mant is not None else None
    mant_ = _c(mant, np.int32) if mant is not None else None
    shift_ = _c(shift, np.int32) if shift is not None else None
    r = lib().kt_gemm_i8w16(_ptr(x), _ptr(w), m, n, k, _ptr(mant_) if mant_ is not None else None,
                            _ptr(shift_) if shift_ is not None else None, _ptr(acc),
                            _ptr(y8) if y8 is not None else None, threads)
    if r != 0:
        raise ValueError("gemm_i8w16: k beyond the int32-exact bound")
    return acc, y8


def moe_route(logits, T: int, E: int, top_k: int, sig):
    logits, sig = _c(logits, np.int32), _c(sig, np.int16)
    sel = np.empty(T * top_k, dtype=np.int32)
    cw = np.empty(T * top_k, dtype=np.int32)
    lib().kt_moe_route(_ptr(logits), T, E, top_k, _ptr(sig), _ptr(sel), _ptr(cw))
    return sel, cw


def moe_bucket(sel, T: int, E: int, top_k: int):
    sel = _c(sel, np.int32)
    lst = np.full((E + 1) * T, -1, dtype=np.int32)
    pos = np.empty(T * top_k, dtype=np.int32)
    count = np.empty(E + 1, dtype=np.int32)
    lib().kt_moe_bucket(_ptr(sel), T, E, top_k, _ptr(lst), _ptr(pos), _ptr(count))
    return lst, pos, count


def moe_experts(x, T, H, F, G, lst, count, wgu, wd, gm, gs, dm, ds, silu, h_shift, threads: int = 0):
    """h (P x F) and d (P x H) int8 in bucket order, P = sum(count)."""
    x = _c(x, np.int8)
    lst, count = _c(lst, np.int32), _c(count, np.int32)
    wgu, wd, silu = _c(wgu, np.int16), _c(wd, np.int16), _c(silu, np.int16)
    gm, gs, dm, ds = (_c(a, np.int32) for a in (gm, gs, dm, ds))
    P = int(count.astype(np.int64).sum())
    h = np.empty(P * F, dtype=np.int8)
    d = np.empty(P * H, dtype=np.int8)
    r = lib().kt_moe_experts(_ptr(x), T, H, F, G, _ptr(lst), _ptr(count), _ptr(wgu), _ptr(wd), _ptr(gm), _ptr(gs),
                             _ptr(dm), _ptr(ds), _ptr(silu), h_shift, _ptr(h), _ptr(d), threads)
    if r != 0:
        raise ValueError("moe_experts: a dimension beyond the int32-exact bound")
    return h, d


def moe_combine(d, sel, cw, pos, count, T: int, H: int, E: int, top_k: int, out_shift: int) -> np.ndarray:
    d = _c(d, np.int8)
    sel, cw, pos, count = (_c(a, np.int32) for a in (sel, cw, pos, count))
    out = np.empty(T * H, dtype=np.int8)
    lib().kt_moe_combine(_ptr(d), _ptr(sel), _ptr(cw), _ptr(pos), _ptr(count), T, H, E, top_k, out_shift, _ptr(out))
    return out


def moe_forward_token(x, logits, T, H, F, E, top_k, wgu, wd, gm, gs, dm, ds, silu, sig, h_shift, out_shift):
    """The reference's loop order: token by token, each chosen expert on one row (slow; small shapes only)."""
    x, logits = _c(x, np.int8), _c(logits, np.int32)
    wgu, wd, silu, sig = _c(wgu, np.int16), _c(wd, np.int16), _c(silu, np.int16), _c(sig, np.int16)
    gm, gs, dm, ds = (_c(a, np.int32) for a in (gm, gs, dm, ds))
    out = np.empty(T * H, dtype=np.int8)
    lib().kt_moe_forward_token(_ptr(x), _ptr(logits), T, H, F, E, top_k, _ptr(wgu), _ptr(wd), _ptr(gm), _ptr(gs),
                               _ptr(dm), _ptr(ds), _ptr(silu), _ptr(sig), h_shift, out_shift, _ptr(out))
    return out


def moe_layer(x, logits, T, H, F, E, top_k, wgu, wd, gm, gs, dm, ds, silu, sig, h_shift, out_shift, threads=0):
    """The expert-major evaluation the GPU performs: route, bucket, experts, combine. Returns a dict of every
    intermediate (sel, cw, list, pos, count, h, d) and out."""
    sel, cw = moe_route(logits, T, E, top_k, sig)
    lst, pos, count = moe_bucket(sel, T, E, top_k)
    h, d = moe_experts(x, T, H, F, E + 1, lst, count, wgu, wd, gm, gs, dm, ds, silu, h_shift, threads)
    out = moe_combine(d, sel, cw, pos, count, T, H, E, top_k, out_shift)
    return dict(sel=sel, cw=cw, list=lst, pos=pos, count=count, h=h, d=d, out=out)


def sam_entry(img, C: int, HW: int, lut) -> np.ndarray:
    img, lut = _c(img, np.uint8), _c(lut, np.int8)
    q = np.empty(C * HW, dtype=np.int8)
    lib().kt_sam_entry(_ptr(img), C, HW, _ptr(lut), _ptr(q))
    return q


def conv2d(q, ci, h, w, wt, co, kh, kw, stride, pad, bias, mant, shift, threads: int = 0, want_acc=False):
    """Conv2d::forward_int's direct loop (conv.rs:68-130) on int8 codes: (out int8 [co][oh][ow], acc i64 or None)."""
    q, wt = _c(q, np.int8), _c(wt, np.int16)
    bias = _c(bias, np.int32) if bias is not None else None
    mant, shift = _c(mant, np.int32), _c(shift, np.int32)
    oh, ow = (h + 2 * pad - kh) // stride + 1, (w + 2 * pad - kw) // stride + 1
    out = np.empty(co * oh * ow, dtype=np.int8)
    acc = np.empty(co * oh * ow, dtype=np.int64) if want_acc else None
    lib().kt_conv2d_i8w16(_ptr(q), ci, h, w, _ptr(wt), co, kh, kw, stride, pad,
                          _ptr(bias) if bias is not None else None, _ptr(mant), _ptr(shift), _ptr(out),
                          _ptr(acc) if acc is not None else None, threads)
    return out, acc


def mlp_gelu(x, m, d, dh, wi, im, is_, gelu, wo, om, os_, threads: int = 0):
    x, wi, wo, gelu = _c(x, np.int8), _c(wi, np.int16), _c(wo, np.int16), _c(gelu, np.int8)
    im, is_, om, os_ = (_c(a, np.int32) for a in (im, is_, om, os_))
    h = np.empty(m * dh, dtype=np.int8)
    y = np.empty(m * d, dtype=np.int8)
    r = lib().kt_mlp_gelu(_ptr(x), m, d, dh, _ptr(wi), _ptr(im), _ptr(is_), _ptr(gelu), _ptr(wo), _ptr(om), _ptr(os_),
                          _ptr(h), _ptr(y), threads)
    if r:
        raise ValueError("mlp_gelu: a dimension beyond the int32-exact bound")
    return h, y


def gen_uniform(seed: int, lo: int, hi: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    lib().kt_gen_uniform_i32(seed & (2**64 - 1), lo, hi, n, _ptr(out))
    return out


def gen_quant_rows(seed: int, rows: int, cols: int) -> np.ndarray:
    out = np.empty(rows * cols, dtype=np.int16)
    lib().kt_gen_quant_rows(seed & (2**64 - 1), rows, cols, _ptr(out))
    return out


def channel_scales_target(w, n: int, k: int, sigma: int, target: int):
    w = _c(w, np.int16)
    mant = np.empty(n, dtype=np.int32)
    shift = np.empty(n, dtype=np.int32)
    lib().kt_channel_scales_target_i16(_ptr(w), n, k, sigma, target, _ptr(mant), _ptr(shift))
    return mant, shift


class DecModel(C.Structure):
    """kt_dec_model of kt_oracle_layers.c."""

    _fields_ = [(n, C.c_int64) for n in ("d", "ffn", "nh", "nkv", "hd", "layers", "vocab", "max_pos", "h_shift")] + [
        (n, C.c_void_p) for n in ("emb", "lm_mant", "lm_shift", "wqkv", "qkv_mant", "qkv_shift", "wo", "o_mant",
                                  "o_shift", "wgu", "gu_mant", "gu_shift", "wd", "d_mant", "d_shift", "rope_cos",
                                  "rope_sin", "exp_tab", "silu")]


def dec_model(shape: dict, arrays: dict):
    """A DecModel over numpy arrays (kept alive in the returned pair)."""
    keep = {}
    m = DecModel()
    for k in ("d", "ffn", "nh", "nkv", "hd", "layers", "vocab", "max_pos", "h_shift"):
        setattr(m, k, int(shape[k]))
    types = {"emb": np.int16, "wqkv": np.int16, "wo": np.int16, "wgu": np.int16, "wd": np.int16,
             "rope_cos": np.int16, "rope_sin": np.int16, "silu": np.int16}
    for k, _ in DecModel._fields_[9:]:
        a = _c(arrays[k], types.get(k, np.int32))
        keep[k] = a
        setattr(m, k, a.ctypes.data)
    return m, keep


def dec_rmsnorm(r, rows: int, d: int) -> np.ndarray:
    """The W12 decoder's RMSNorm to int8 codes (kt_dec_rmsnorm_rows)."""
    r = _c(r, np.int32)
    q = np.zeros(rows * d, dtype=np.int8)
    lib().kt_dec_rmsnorm_rows(_ptr(r), rows, d, _ptr(q))
    return q


def dec_rope(x, heads: int, hd: int, p: int, cos_t, sin_t) -> np.ndarray:
    """The W12 decoder's rotate-half RoPE of heads x hd int8 values at position p (kt_dec_rope_row)."""
    x = _c(x, np.int8).copy()
    cos_t, sin_t = _c(cos_t, np.int16), _c(sin_t, np.int16)
    lib().kt_dec_rope_row(_ptr(x), heads, hd, p, _ptr(cos_t), _ptr(sin_t))
    return x


def dec_attend(q, kl, vl, p: int, nkv: int, g: int, hd: int, exp_tab) -> np.ndarray:
    """One head of the W12 decoder's attention over positions 0..p of kv head g (kt_dec_attend)."""
    q, kl, vl, exp_tab = _c(q, np.int8), _c(kl, np.int8), _c(vl, np.int8), _c(exp_tab, np.int32)
    sc = np.zeros(p + 1, dtype=np.int64)
    o = np.zeros(hd, dtype=np.int8)
    lib().kt_dec_attend(_ptr(q), _ptr(kl), _ptr(vl), p, nkv, g, hd, _ptr(exp_tab), _ptr(sc), _ptr(o))
    return o


def dec_generate(shape: dict, arrays: dict, prompt, max_new: int, batched: bool = True, threads: int = 0):
    """generate_greedy_by on the oracle decoder: (tokens max_new int32, logits max_new x vocab int32)."""
    m, keep = dec_model(shape, arrays)
    prompt = _c(prompt, np.int32)
    toks = np.empty(max_new, dtype=np.int32)
    logits = np.empty(max_new * int(shape["vocab"]), dtype=np.int32)
    r = lib().kt_dec_generate(C.byref(m), _ptr(prompt), prompt.size, max_new, int(batched), _ptr(toks), _ptr(logits),
                              threads)
    if r:
        raise ValueError("dec_generate: shape beyond the oracle's bounds")
    return toks, logits


# ---------------------------------------------------------------------------------------------------------------
# The reference decoder at its own semantics (kt_oracle_refdec.c): DecoderModel, RmsNorm, Attention::decode_step,
# SwiGluMlp, add, generate_greedy_by and repro::run's hashes (crates/01-engine/kt-core/src/{model,layers,attention,
# generate}.rs, crates/04-ingest/kt-convert/src/repro.rs)


# repro::synthetic_model (repro.rs:260-300) and verify_repro --synthetic's input (verify_repro.rs:71-78)
SYNTH_CFG = dict(dim=32, layers=2, nh=4, nkv=2, hd=8, hidden=64, vocab=64, eps=1e-6, theta=10000.0, max_seq=256)
SYNTH_PROMPT = [3, 14, 15, 9, 26, 5, 35, 8, 9, 7, 9, 3]
SYNTH_HASH = "8109ebad0a2883838a9d133351ce421f676e8d66dbcaffc5cde000272b748d03"  # REPRODUCE.md:17


class RefModel:
    """A DecoderModel built by the oracle from the seeded float weights of repro::synthetic_model's generator."""

    def __init__(self, seed: int, cfg: dict = SYNTH_CFG):
        self.cfg = dict(cfg)
        c = self.cfg
        self.ptr = lib().kt_rd_synthetic(seed, c["dim"], c["layers"], c["nh"], c["nkv"], c["hd"], c["hidden"],
                                         c["vocab"], c["eps"], c["theta"], c["max_seq"])

    @classmethod
    def from_weights(cls, cfg: dict, emb, final_norm, lm_head, layers):
        """The oracle's model of given codes and Scales, in RefDecoder's argument order."""
        m = cls.__new__(cls)
        m.cfg = dict(cfg)
        c = m.cfg
        m.ptr = lib().kt_rd_new(c["dim"], c["layers"], c["nh"], c["nkv"], c["hd"], c["hidden"], c["vocab"], c["eps"],
                                c["theta"], c["max_seq"])
        idx = {"wq": 0, "wk": 1, "wv": 2, "wo": 3, "gate": 4, "up": 5, "down": 6}
        for l, lw in enumerate(layers):
            for n, i in idx.items():
                w = _c(lw[n][0], np.int32)
                o, k = np.asarray(lw[n][0]).shape
                lib().kt_rd_set_ql(m.ptr, l, i, _ptr(w), o, k, _sc(lw[n][1]))
            for i, n in enumerate(("in_norm", "post_norm")):
                lib().kt_rd_set_norm(m.ptr, l, i, _ptr(_c(lw[n][0], np.int32)), _sc(lw[n][1]))
        lib().kt_rd_set_norm(m.ptr, 0, 2, _ptr(_c(final_norm[0], np.int32)), _sc(final_norm[1]))
        lib().kt_rd_set_emb(m.ptr, _ptr(_c(emb[0], np.int32)), _sc(emb[1]))
        w = _c(lm_head[0], np.int32)
        lib().kt_rd_set_ql(m.ptr, 0, 7, _ptr(w), c["vocab"], c["dim"], _sc(lm_head[1]))
        return m

    def __del__(self):
        if getattr(self, "ptr", None):
            lib().kt_rd_free(self.ptr)
            self.ptr = None

    def generate(self, prompt, max_new: int):
        """(tokens, run logits_hash hex, per-position logits_hash hex list) of repro::run with no stop ids."""
        p = _c(prompt, np.int32)
        toks = np.zeros(max(max_new, 1), dtype=np.int32)
        run = (C.c_uint8 * 32)()
        npos = p.size + max(max_new - 1, 0)
        ph = np.zeros(npos * 32, dtype=np.uint8)
        if lib().kt_rd_generate(self.ptr, _ptr(p), p.size, max_new, _ptr(toks), run, _ptr(ph)):
            raise ValueError("generate: empty prompt or past the position tables")
        return toks[:max_new].tolist(), bytes(run).hex(), [bytes(ph[32 * i:32 * i + 32]).hex() for i in range(npos)]

    def forward(self, tokens):
        """CausalLM::forward_int (model.rs:361-367): the T tokens as one sequence, every op over the whole T-row
        tensor: (logits T x vocab, (mant, shift))."""
        t = _c(tokens, np.int32)
        logits, ls = np.zeros(t.size * self.cfg["vocab"], dtype=np.int32), Scale()
        if lib().kt_rd_forward(self.ptr, _ptr(t), t.size, _ptr(logits), C.byref(ls)):
            raise ValueError("forward: empty, past max_seq or a token outside the vocabulary")
        return logits.reshape(t.size, self.cfg["vocab"]), (ls.mant, ls.shift)

    def attention_prefill(self, T: int, q, qs, k, ks, v, vs):
        """Attention::forward_int between its projections over T rows (attention.rs:486-598): (o codes, scale)."""
        q, k, v = _c(q, np.int32), _c(k, np.int32), _c(v, np.int32)
        o, os_ = np.zeros(T * self.cfg["nh"] * self.cfg["hd"], dtype=np.int32), Scale()
        lib().kt_rd_attention_prefill(self.ptr, T, _ptr(q), _sc(qs), _ptr(k), _sc(ks), _ptr(v), _sc(vs), _ptr(o),
                                      C.byref(os_))
        return o, (os_.mant, os_.shift)

    def ql(self, layer: int, which: str):
        """The (codes out x in, (mant, shift)) of a projection: wq wk wv wo gate up down, or lm_head."""
        idx = {"wq": 0, "wk": 1, "wv": 2, "wo": 3, "gate": 4, "up": 5, "down": 6, "lm_head": 7}[which]
        o, i = _SZ(), _SZ()
        lib().kt_rd_get_ql(self.ptr, layer, idx, None, C.byref(o), C.byref(i))
        codes = np.zeros(o.value * i.value, dtype=np.int32)
        s = lib().kt_rd_get_ql(self.ptr, layer, idx, _ptr(codes), C.byref(o), C.byref(i))
        return codes.reshape(o.value, i.value), (s.mant, s.shift)

    def norm(self, layer: int, which: str):
        """(gamma codes, (mant, shift), eps (mant, shift)) of in_norm / post_norm / final_norm."""
        idx = {"in_norm": 0, "post_norm": 1, "final_norm": 2}[which]
        codes = np.zeros(self.cfg["dim"], dtype=np.int32)
        eps = Scale()
        s = lib().kt_rd_get_norm(self.ptr, layer, idx, _ptr(codes), C.byref(eps))
        return codes, (s.mant, s.shift), (eps.mant, eps.shift)

    def emb(self):
        codes = np.zeros(self.cfg["vocab"] * self.cfg["dim"], dtype=np.int32)
        s = lib().kt_rd_get_emb(self.ptr, _ptr(codes))
        return codes.reshape(self.cfg["vocab"], self.cfg["dim"]), (s.mant, s.shift)

    def lut(self, which: str):
        """(codes, inv_step (mant, shift), lo_index, code_scale (mant, shift)) of the exp or silu CodeLut."""
        codes = np.zeros(1 << 16, dtype=np.int64)
        inv, cs, lo = Scale(), Scale(), C.c_int64()
        lib().kt_rd_get_lut(self.ptr, 0 if which == "exp" else 1, _ptr(codes), C.byref(inv), C.byref(lo),
                            C.byref(cs))
        return codes, (inv.mant, inv.shift), lo.value, (cs.mant, cs.shift)

    def rope(self):
        """(cos mant, cos shift, cos sign, sin mant, sin shift, sin sign), each max_seq x hd/2, and 1/sqrt(hd)."""
        n = self.cfg["max_seq"] * (self.cfg["hd"] // 2)
        a = [np.zeros(n, dtype=t) for t in (np.int64, np.int32, np.int8, np.int64, np.int32, np.int8)]
        isq = lib().kt_rd_get_rope(self.ptr, *[_ptr(x) for x in a])
        return a, (isq.mant, isq.shift)

    def weights(self):
        """The model as RefDecoder's constructor takes it: (emb, final_norm, lm_head, layers)."""
        layers = []
        for l in range(self.cfg["layers"]):
            d = {n: self.norm(l, n)[:2] for n in ("in_norm", "post_norm")}
            for n in ("wq", "wk", "wv", "wo", "gate", "up", "down"):
                d[n] = self.ql(l, n)
            layers.append(d)
        return self.emb(), self.norm(0, "final_norm")[:2], self.ql(0, "lm_head"), layers


class RefCache:
    """One layer's LayerKv (attention.rs:251-265) in the oracle."""

    def __init__(self, model: RefModel):
        self.model = model
        self.ptr = lib().kt_rd_cache_new(model.ptr)

    def __del__(self):
        if getattr(self, "ptr", None):
            lib().kt_rd_cache_free(self.ptr)
            self.ptr = None


def _sc(s) -> Scale:
    return Scale(int(s[0]), int(s[1]))


def rd_rmsnorm(x, rows: int, dim: int, xs, g, gs, eps):
    """RmsNorm::forward_int (layers.rs:392-434): (codes, (mant, shift))."""
    x, g = _c(x, np.int32), _c(g, np.int32)
    y, ys = np.zeros(rows * dim, dtype=np.int32), Scale()
    lib().kt_rd_rmsnorm(_ptr(x), rows, dim, _sc(xs), _ptr(g), _sc(gs), _sc(eps), _ptr(y), C.byref(ys))
    return y, (ys.mant, ys.shift)


def rd_add(a, as_, b, bs):
    """add (layers.rs:121-136): (codes, (mant, shift))."""
    a, b = _c(a, np.int32), _c(b, np.int32)
    y, ys = np.zeros(a.size, dtype=np.int32), Scale()
    lib().kt_rd_add(_ptr(a), _sc(as_), _ptr(b), _sc(bs), a.size, _ptr(y), C.byref(ys))
    return y, (ys.mant, ys.shift)


def rd_swiglu_act(model: RefModel, g, gs, u, us):
    """SwiGluMlp::forward_int's activation with the model's SiLU CodeLut (layers.rs:615-637)."""
    g, u = _c(g, np.int32), _c(u, np.int32)
    h, hs = np.zeros(g.size, dtype=np.int32), Scale()
    lib().kt_rd_swiglu_act(model.ptr, _ptr(g), _sc(gs), _ptr(u), _sc(us), g.size, _ptr(h), C.byref(hs))
    return h, (hs.mant, hs.shift)


def rd_attention_core(cache: RefCache, q, qs, k, ks, v, vs, pos: int):
    """Attention::decode_step between its projections (attention.rs:358-458), appending to `cache`."""
    q, k, v = _c(q, np.int32), _c(k, np.int32), _c(v, np.int32)
    c = cache.model.cfg
    o, os_ = np.zeros(c["nh"] * c["hd"], dtype=np.int32), Scale()
    lib().kt_rd_attention_core(cache.model.ptr, cache.ptr, _ptr(q), _sc(qs), _ptr(k), _sc(ks), _ptr(v), _sc(vs), pos,
                               _ptr(o), C.byref(os_))
    return o, (os_.mant, os_.shift)


def rd_attention_append(cache: RefCache, k, ks, v, vs, pos: int) -> None:
    """Only the cache append of Attention::decode_step (attention.rs:366-384): k rotated at pos, k, v, their scales."""
    k, v = _c(k, np.int32), _c(v, np.int32)
    lib().kt_rd_attention_append(cache.model.ptr, cache.ptr, _ptr(k), _sc(ks), _ptr(v), _sc(vs), pos)


# ---------------------------------------------------------------------------------------------------------------
# MoeMlp at the reference's semantics (kt_oracle_refdec.c: route / route_sigmoid, combine, merge_rows, the shared
# expert; crates/01-engine/kt-core/src/layers.rs:652-1020, router.rs:29-79)


class RefMoe:
    """The reference tests' MoE (tests.rs:113-150, tests_glm.rs:31-43, 224-228) built by the oracle from the seeded
    float weights: the stream from `seed` draws the router then each expert's gate / up / down. sigmoid: 0 softmax
    router, 1 sigmoid router with bias vecf(bias_seed, E) * 0.05, 2 sigmoid router with a zero bias."""

    def __init__(self, seed: int, dim: int, E: int, top_k: int, hidden: int, norm_topk: bool = False,
                 sigmoid: int = 0, bias_seed: int = 0, shared_hidden: int = 0):
        self.dim, self.E, self.top_k, self.hidden, self.shared_hidden = dim, E, top_k, hidden, shared_hidden
        self.norm_topk, self.sigmoid = bool(norm_topk), sigmoid
        self.ptr = lib().kt_rm_synthetic(seed, dim, E, top_k, hidden, int(norm_topk), int(sigmoid == 1), bias_seed,
                                         shared_hidden)
        if sigmoid == 2:  # a sigmoid router with zero bias: the coded bias is already 0 when sigmoid == 0
            self.ptr2 = None
            lib().kt_rm_free(self.ptr)
            self.ptr = lib().kt_rm_synthetic(seed, dim, E, top_k, hidden, int(norm_topk), 1, bias_seed, shared_hidden)
            for e in range(E):
                lib().kt_rm_set_bias(self.ptr, e, 0.0)

    @classmethod
    def from_weights(cls, dim: int, router, experts, top_k: int, norm_topk: bool, bias_codes=None, shared=None):
        """The same MoeMlp over given QuantLinears (kt_rm_empty / kt_rm_set_ql): router (codes E x dim, (mant,
        shift)); experts one dict per expert of gate, up, down; bias_codes None for the softmax router, else the
        sigmoid router's E coded biases; shared None or a dict like an expert's."""
        m = cls.__new__(cls)
        E = len(experts)
        hidden = int(np.asarray(experts[0]["gate"][0]).shape[0])
        sh = int(np.asarray(shared["gate"][0]).shape[0]) if shared is not None else 0
        m.dim, m.E, m.top_k, m.hidden, m.shared_hidden = dim, E, top_k, hidden, sh
        m.norm_topk, m.sigmoid = bool(norm_topk), (0 if bias_codes is None else 1)
        m.ptr = lib().kt_rm_empty(dim, E, top_k, hidden, int(norm_topk), m.sigmoid, sh)
        idx = {"gate": 1, "up": 2, "down": 3}

        def put(e, which, q):
            codes = _c(np.asarray(q[0]).reshape(-1), np.int32)
            lib().kt_rm_set_ql(m.ptr, e, which, _ptr(codes), _sc(q[1]))

        put(0, 0, router)
        for e, ex in enumerate(experts):
            for n, w in idx.items():
                put(e, w, ex[n])
        if shared is not None:
            for n, w in idx.items():
                put(E, w, shared[n])
        if bias_codes is not None:
            for e, c in enumerate(np.asarray(bias_codes, np.int64)):
                lib().kt_rm_set_bias_code(m.ptr, e, int(c))
        return m

    def __del__(self):
        if getattr(self, "ptr", None):
            lib().kt_rm_free(self.ptr)
            self.ptr = None

    def set_bias(self, e: int, b: float) -> None:
        lib().kt_rm_set_bias(self.ptr, e, float(b))

    def route(self, x_row, xs):
        """(experts, ec, sumc, logits codes, logits scale) of MoeMlp::route for one token row."""
        x = _c(x_row, np.int32)
        sel, ec = np.zeros(self.top_k, np.int32), np.zeros(self.top_k, np.int64)
        lg, ls = np.zeros(self.E, np.int32), Scale()
        sumc = lib().kt_rm_route(self.ptr, _ptr(x), _sc(xs), _ptr(sel), _ptr(ec), _ptr(lg), C.byref(ls))
        return sel.tolist(), ec, int(sumc), lg, (ls.mant, ls.shift)

    def sigmoid_codes(self, logits, ls):
        lg = _c(logits, np.int32)
        out = np.zeros(lg.size, np.int64)
        lib().kt_rm_sigmoid_codes(self.ptr, _ptr(lg), lg.size, _sc(ls), _ptr(out))
        return out

    def forward(self, x, T: int, xs):
        """MoeMlp::forward_int of T rows: (codes T x dim, (mant, shift))."""
        x = _c(x, np.int32)
        out, os_ = np.zeros(T * self.dim, np.int32), Scale()
        lib().kt_rm_forward(self.ptr, _ptr(x), T, _sc(xs), _ptr(out), C.byref(os_))
        return out, (os_.mant, os_.shift)

    def expert(self, e: int, x, rows: int, xs):
        """SwiGluMlp::forward_int of expert e (e == E: the shared expert)."""
        x = _c(x, np.int32)
        y, ys = np.zeros(rows * self.dim, np.int32), Scale()
        lib().kt_rm_expert(self.ptr, e, _ptr(x), rows, _sc(xs), _ptr(y), C.byref(ys))
        return y, (ys.mant, ys.shift)

    def ql(self, e: int, which: str):
        """(codes out x in, (mant, shift)) of the router (which 'router') or expert e's gate / up / down."""
        idx = {"router": 0, "gate": 1, "up": 2, "down": 3}[which]
        o, i = _SZ(), _SZ()
        lib().kt_rm_get_ql(self.ptr, e, idx, None, C.byref(o), C.byref(i))
        codes = np.zeros(o.value * i.value, np.int32)
        s = lib().kt_rm_get_ql(self.ptr, e, idx, _ptr(codes), C.byref(o), C.byref(i))
        return codes.reshape(o.value, i.value), (s.mant, s.shift)

    def lut(self, which: str):
        codes = np.zeros(1 << 16, np.int64)
        inv, cs, lo = Scale(), Scale(), C.c_int64()
        lib().kt_rm_get_lut(self.ptr, {"exp": 0, "sigmoid": 1, "silu": 2}[which], _ptr(codes), C.byref(inv),
                            C.byref(lo), C.byref(cs))
        return codes, (inv.mant, inv.shift), lo.value, (cs.mant, cs.shift)

    def bias(self) -> np.ndarray:
        b = np.zeros(self.E, np.int64)
        lib().kt_rm_get_bias(self.ptr, _ptr(b))
        return b


def rm_probe(s: int, n: int):
    """IntTensor::from_reals of the reference tests' probe (tests.rs:29-32): (codes, scale, the advanced stream)."""
    st = C.c_uint64(s)
    out = np.zeros(n, np.int32)
    sc = lib().kt_rm_probe(C.byref(st), n, _ptr(out))
    return out, (sc.mant, sc.shift), st.value


def rm_combine(ys, ys_s, out_dim: int, ec, sumc: int):
    k = len(ys_s)
    y = _c(ys, np.int32)
    sarr = (Scale * k)(*[Scale(int(a), int(b)) for a, b in ys_s])
    ec = _c(ec, np.int64)
    out, os_ = np.zeros(out_dim, np.int32), Scale()
    lib().kt_rm_combine(_ptr(y), sarr, k, out_dim, _ptr(ec), sumc, _ptr(out), C.byref(os_))
    return out, (os_.mant, os_.shift)


def rm_merge_rows(rows, rs, T: int, dim: int):
    r = _c(rows, np.int32)
    sarr = (Scale * T)(*[Scale(int(a), int(b)) for a, b in rs])
    out, os_ = np.zeros(T * dim, np.int32), Scale()
    lib().kt_rm_merge_rows(_ptr(r), sarr, T, dim, _ptr(out), C.byref(os_))
    return out, (os_.mant, os_.shift)


# ---------------------------------------------------------------------------------------------------------------
# the SAM image path at the reference's semantics: Conv2d, the pixel entry, GELU, FeedForward


def vecf(seed: int, n: int):
    """The reference tests' float stream (conv.rs:471-477): ((lcg >> 40) / 2^24 * 2 - 1) as f32; (values, state)."""
    s, out = seed, np.empty(n, np.float32)
    for i in range(n):
        s = (s * 6364136223846793005 + 1442695040888963407) % 2**64
        out[i] = np.float32((s >> 40) / float(1 << 24) * 2.0 - 1.0)
    return out, s


def from_reals(real, levels: int = 1 << 28):
    """IntTensor::from_reals (tensor.rs:106-117): (codes i32, (mant, shift))."""
    r = np.ascontiguousarray(real, dtype=np.float64).reshape(-1)
    out = np.empty(r.size, np.int32)
    sc = lib().kt_rc_from_reals(_ptr(r), r.size, levels, _ptr(out))
    return out, (sc.mant, sc.shift)


def quant_weights(w):
    """Conv2d::from_weights / QuantLinear::from_weights: (12-trit codes i32, (mant, shift))."""
    f = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    out = np.empty(f.size, np.int32)
    sc = lib().kt_rc_quant_weights(_ptr(f), f.size, _ptr(out))
    return out, (sc.mant, sc.shift)


def quant_bias(b):
    """with_bias (conv.rs:49-60): (codes i64, (mant, shift)), or None for an all-zero bias."""
    f = np.ascontiguousarray(b, dtype=np.float32).reshape(-1)
    out, sc = np.empty(f.size, np.int64), Scale()
    if not lib().kt_rc_quant_bias(_ptr(f), f.size, _ptr(out), C.byref(sc)):
        return None
    return out, (sc.mant, sc.shift)


def ref_conv2d(x, xs, ci: int, h: int, w: int, wc, ws, co: int, kh: int, kw: int, stride: int, pad: int,
               bias=None):
    """Conv2d::forward_int (conv.rs:68-130): (codes co x oh x ow i32, (mant, shift)). bias: None or (codes, scale)."""
    x, wc = _i32(x), _i32(wc)
    assert x.size == ci * h * w and wc.size == co * ci * kh * kw
    oh, ow = (h + 2 * pad - kh) // stride + 1, (w + 2 * pad - kw) // stride + 1
    b = None if bias is None else np.ascontiguousarray(bias[0], dtype=np.int64)
    bs = Scale(0, 0) if bias is None else Scale(*bias[1])
    out, os_ = np.empty(co * oh * ow, np.int32), Scale()
    lib().kt_rc_conv2d(_ptr(x), Scale(*xs), ci, h, w, _ptr(wc), Scale(*ws), co, kh, kw, stride, pad,
                       0 if b is None else _ptr(b), bs, _ptr(out), C.byref(os_))
    return out.reshape(co, oh, ow), (os_.mant, os_.shift)


def gelu_table():
    """build_gelu_lut (nonlin.rs:24-26): (codes i64[65536], inv_step scale, lo_index, code scale)."""
    codes, inv, lo, cs = np.empty(1 << 16, np.int64), Scale(), C.c_int64(), Scale()
    lib().kt_rc_gelu_table(_ptr(codes), C.byref(inv), C.byref(lo), C.byref(cs))
    return codes, (inv.mant, inv.shift), lo.value, (cs.mant, cs.shift)


def apply_gelu(x, xs):
    """apply_gelu (nonlin.rs:30-45): (codes i32, the table's code scale)."""
    x = _i32(x)
    y, ys = np.empty(x.size, np.int32), Scale()
    lib().kt_rc_apply_gelu(_ptr(x), x.size, Scale(*xs), _ptr(y), C.byref(ys))
    return y, (ys.mant, ys.shift)


def feedforward(x, rows: int, dim: int, xs, wi, wis, hidden: int, wo, wos, bi=None, bo=None):
    """FeedForward::forward_int (hiera.rs:336-340): proj_in (+bias) -> apply_gelu -> proj_out (+bias).
    wi hidden x dim, wo dim x hidden codes; bi / bo None or (codes, scale)."""
    x, wi, wo = _i32(x), _i32(wi), _i32(wo)
    bip = None if bi is None else np.ascontiguousarray(bi[0], dtype=np.int64)
    bop = None if bo is None else np.ascontiguousarray(bo[0], dtype=np.int64)
    y, ys = np.empty(rows * dim, np.int32), Scale()
    lib().kt_rc_feedforward(_ptr(x), rows, dim, Scale(*xs), _ptr(wi), Scale(*wis),
                            0 if bip is None else _ptr(bip), Scale(*(bi[1] if bi else (0, 0))), hidden, _ptr(wo),
                            Scale(*wos), 0 if bop is None else _ptr(bop), Scale(*(bo[1] if bo else (0, 0))),
                            _ptr(y), C.byref(ys))
    return y.reshape(rows, dim), (ys.mant, ys.shift)
