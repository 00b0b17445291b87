"""tritify_amd: an MI355X-native (gfx950) backend for tritify's exact-integer linear accumulate.

The compute is hand-written CDNA4 HIP (tritify_amd/csrc) behind the C ABI of include/kt_hip.h; this package is the
thin Python binding of that ABI. Importing it does not load the library: the first call does, and raises ImportError
when the library has not been built.
"""
from .backend import (  # noqa: F401
    OUT_I8,
    OUT_I32,
    OUT_I64,
    PLANT_CACHE_BY_SHAPE,
    PLANT_DROP_TOP,
    PLANT_NO_FLUSH,
    PLANT_WRONG_CARRY,
    HipBackend,
    HipError,
    Weights,
    device_count,
    device_info,
    digit_gemm,
    fallbacks,
    flush_k,
    kp,
    lib,
    pack_planes,
    planes_for,
    probe_mfma,
    w12_bytes,
    w12_linear,
    w12_pack,
    w12_upload,
    weight_id_fresh,
)
