"""The C ABI library loads and exports every function include/kt_hip.h declares; host-only helpers agree with the
oracle. No GPU call is made here."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "kt_hip.h")


def declared() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kt_hip_\w+)\s*\(", text)))


@pytest.mark.parametrize("name", ["libkt_hip.so", "libkt_hip_planted.so"])
def test_library_exports_every_declared_function(name):
    path = os.path.join(ROOT, "tritify_amd", name)
    assert os.path.exists(path), "run __graft_entry__.build() first"
    lib = C.CDLL(path)
    names = declared()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_host_helpers_agree_with_the_oracle():
    from tritify_amd import backend as B

    L = B.lib()
    for px, pw in [(1, 1), (1, 3), (3, 3), (3, 5), (5, 5)]:
        assert B.flush_k(px, pw) == O.flush_k(px, pw)
    for k in [0, 1, 63, 64, 65, 4096, 4099]:
        assert L.kt_hip_kp(k) == B.kp(k) == (k + 63) // 64 * 64
    rng = np.random.default_rng(0)
    for lo, hi in [(-128, 127), (-129, 127), (-32896, 32639), (-O.WLEVELS, O.WLEVELS), (-(2**31), 2**31 - 1)]:
        c = rng.integers(lo, hi + 1, size=100).astype(np.int64)
        c[:2] = [lo, hi]
        c = c.astype(np.int32)
        p = O.planes_for(c)
        assert B.planes_for(c) == (1 if p == 1 else 3 if p <= 3 else 5)
    assert B.fallbacks() == 0


def test_which_decode_rows_stop_at_their_sums():
    """kt_hip_quant_linear_sums_ok: the one-launch product takes rows of up to 1024 values (8192 with 3 weight
    planes) and up to 16384 outputs; the Qwen2.5-0.5B decode projections all fit."""
    from tritify_amd import backend as B

    for inp, out in [(896, 1152), (896, 896), (896, 9728), (4864, 896)]:
        assert B.quant_linear_sums_ok(inp, out, 3)
    assert B.quant_linear_sums_ok(1024, 64, 5) and not B.quant_linear_sums_ok(1025, 64, 5)
    assert not B.quant_linear_sums_ok(4864, 896, 5) and not B.quant_linear_sums_ok(8193, 64, 3)
    assert B.quant_linear_sums_ok(896, 16384, 3) and not B.quant_linear_sums_ok(896, 16385, 3)
    assert not B.quant_linear_sums_ok(896, 896, 2) and not B.quant_linear_sums_ok(0, 896, 3)


def test_the_product_build_refuses_plants():
    """Planted defects exist only in the test build (kt-runtime/Cargo.toml `plants` feature)."""
    from tritify_amd import backend as B

    h = C.c_void_p()
    e = B.lib().kt_hip_open_planted(0, B.PLANT_DROP_TOP, C.byref(h))
    assert e != 0 and not h.value


def test_the_product_never_imports_the_oracle():
    """The product package reads nothing under oracle/: it fails loudly without its own library instead."""
    pkg = os.path.join(ROOT, "tritify_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                for needle in ("import oracle", "from oracle", "libkt_oracle", "kt_oracle"):
                    assert needle not in text, (f, needle)


def test_w12_linear_rejects_bad_arguments_before_any_device_call():
    """Argument checks of kt_hip_w12_linear that need no GPU: an unknown output kind, a requant output without its
    scales, and k past the limit of the GEMM's (m > 128) or the skinny kernel's int32 accumulators."""
    from tritify_amd import backend as B

    L = B.lib()
    inval = 1  # hipErrorInvalidValue
    assert L.kt_hip_w12_linear(0, None, None, None, 4, 32, 64, None, None, 7, None, None) == inval
    assert L.kt_hip_w12_linear(0, None, None, None, 4, 32, 64, None, None, B.OUT_I8, None, None) == inval
    assert L.kt_hip_w12_linear(0, None, None, None, 129, 32, 131009, None, None, B.OUT_I64, None, None) == inval
    assert L.kt_hip_w12_linear(0, None, None, None, 128, 32, 262145, None, None, B.OUT_I64, None, None) == inval
    assert L.kt_hip_w12_linear(0, None, None, None, -1, 32, 64, None, None, B.OUT_I64, None, None) == inval
