"""The cross-backend gates as a library call: kt-runtime's corpus, equality_gate and residency_gate
(crates/02-runtime/kt-runtime/src/gate.rs:1-140) over this build's backends, through the C ABI (kt_hip_gate_*,
tritify_amd/csrc/kt_gate.cpp). The command-line face is tritify_amd/kt_runtime_probe (runtime_probe.rs).

    from tritify_amd import gate, HipBackend
    ok, reports = gate.equality_gate([gate.portable(), gate.of(HipBackend(0))])
    for r in reports: print(r.backend, r.hash, r.diverged)

A backend is the engine's Portable (the reference of both gates), a HipBackend (product or planted build), or any
Python callable `fn(x, weight_id, w, rows, out, k) -> i64 array` wrapped by `from_callable`.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import backend as B

NAME_LEN = 96
DIVERGED = -1

_LINEAR_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.POINTER(C.c_int32), C.c_uint64, C.POINTER(C.c_int32), C.c_size_t,
                         C.c_size_t, C.c_size_t, C.POINTER(C.c_int64))


class _Case(C.Structure):
    _fields_ = [("label", C.c_char_p), ("id", C.c_uint64), ("rows", C.c_size_t), ("out", C.c_size_t),
                ("k", C.c_size_t), ("x", C.POINTER(C.c_int32)), ("w", C.POINTER(C.c_int32))]


class _Backend(C.Structure):
    _fields_ = [("name", C.c_char * NAME_LEN), ("linear_weights", _LINEAR_FN), ("ctx", C.c_void_p)]


class _Report(C.Structure):
    _fields_ = [("backend", C.c_char * NAME_LEN), ("hash", C.c_char * 65), ("diverged", C.c_uint64),
                ("error", C.c_int)]


def _declare(L) -> None:
    if getattr(L, "_gate_declared", False):
        return
    L.kt_hip_gate_corpus.restype = C.c_size_t
    L.kt_hip_gate_corpus.argtypes = [C.POINTER(C.POINTER(_Case))]
    L.kt_hip_gate_bound_cases.restype = C.c_size_t
    L.kt_hip_gate_bound_cases.argtypes = [C.POINTER(C.POINTER(_Case))]
    L.kt_hip_gate_portable.restype = C.c_int
    L.kt_hip_gate_portable.argtypes = [C.POINTER(_Backend)]
    L.kt_hip_gate_backend.restype = C.c_int
    L.kt_hip_gate_backend.argtypes = [C.c_void_p, C.POINTER(_Backend)]
    L.kt_hip_equality_gate.restype = C.c_int
    L.kt_hip_equality_gate.argtypes = [C.POINTER(_Backend), C.c_size_t, C.POINTER(_Case), C.c_size_t,
                                       C.POINTER(_Report)]
    L.kt_hip_residency_gate.restype = C.c_int
    L.kt_hip_residency_gate.argtypes = [C.POINTER(_Backend), C.POINTER(_Case), C.c_size_t, C.c_char_p, C.c_size_t]
    L.kt_hip_portable_linear.restype = C.c_int
    L.kt_hip_portable_linear.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_size_t, C.c_void_p]
    L._gate_declared = True


def _lib(planted: bool = False):
    L = B.lib(planted)
    _declare(L)
    return L


@dataclass
class Case:
    """One corpus or bound case (gate.rs:13-22): x rows x k, w out x k, the weights' id."""
    label: str
    id: int
    rows: int
    out: int
    k: int
    x: np.ndarray
    w: np.ndarray


@dataclass
class Report:
    """GateReport (gate.rs:71-79)."""
    backend: str
    hash: str
    diverged: list
    error: int


class GateBackend:
    """A backend as the gates call it; keeps whatever it wraps alive."""

    def __init__(self, raw: _Backend, keep=None):
        self.raw, self._keep = raw, keep

    @property
    def name(self) -> str:
        return self.raw.name.decode()


def _cases(fn) -> list:
    arr = C.POINTER(_Case)()
    n = fn(C.byref(arr))
    out = []
    for i in range(n):
        c = arr[i]
        x = np.ctypeslib.as_array(c.x, shape=(c.rows * c.k,)).copy()
        w = np.ctypeslib.as_array(c.w, shape=(c.out * c.k,)).copy()
        out.append(Case(c.label.decode(), int(c.id), int(c.rows), int(c.out), int(c.k), x, w))
    return out


def corpus() -> list:
    """corpus() (gate.rs:26-58): the fixed corpus, the same bytes on every machine."""
    return _cases(_lib().kt_hip_gate_corpus)


def bound_cases() -> list:
    """flush_case() (gate.rs:60-69) and this backend's own bound cases; each answer is +-k * code^2."""
    return _cases(_lib().kt_hip_gate_bound_cases)


def portable() -> GateBackend:
    """The engine's Portable (backend.rs:143-160), the gates' reference."""
    raw = _Backend()
    B.check(_lib().kt_hip_gate_portable(C.byref(raw)), "gate portable")
    return GateBackend(raw)


def of(b: "B.HipBackend") -> GateBackend:
    """A HipBackend (the product's or the planted build's) as a gate backend."""
    L = b._lib
    _declare(L)
    raw = _Backend()
    B.check(L.kt_hip_gate_backend(b._h, C.byref(raw)), "gate backend")
    return GateBackend(raw, keep=b)


def from_callable(name: str, fn) -> GateBackend:
    """Any backend: fn(x, weight_id, w, rows, out, k) -> rows * out i64 values."""
    def call(_ctx, x, wid, w, rows, out, k, y):
        try:
            xa = np.ctypeslib.as_array(x, shape=(rows * k,)) if rows * k else np.zeros(0, np.int32)
            wa = np.ctypeslib.as_array(w, shape=(out * k,)) if out * k else np.zeros(0, np.int32)
            got = np.asarray(fn(xa, int(wid), wa, int(rows), int(out), int(k)), dtype=np.int64).reshape(-1)
            if got.size != rows * out:
                return 1
            if got.size:
                np.ctypeslib.as_array(y, shape=(rows * out,))[:] = got
            return 0
        except Exception:
            return 1

    cb = _LINEAR_FN(call)
    raw = _Backend()
    raw.name = name.encode()[:NAME_LEN - 1]
    raw.linear_weights = cb
    return GateBackend(raw, keep=cb)


def _case_array(cases):
    arr = (_Case * len(cases))()
    keep = []
    for i, c in enumerate(cases):
        x = np.ascontiguousarray(c.x, dtype=np.int32)
        w = np.ascontiguousarray(c.w, dtype=np.int32)
        lab = c.label.encode()
        keep += [x, w, lab]
        arr[i] = _Case(lab, c.id, c.rows, c.out, c.k, x.ctypes.data_as(C.POINTER(C.c_int32)),
                       w.ctypes.data_as(C.POINTER(C.c_int32)))
    return arr, keep


def equality_gate(backends, cases=None):
    """equality_gate (gate.rs:81-106): (all byte-identical, one Report per backend); the first backend is the
    reference."""
    cases = corpus() if cases is None else cases
    arr, _keep = _case_array(cases)
    bs = (_Backend * len(backends))(*[b.raw for b in backends])
    reps = (_Report * len(backends))()
    rc = _lib().kt_hip_equality_gate(bs, len(backends), arr, len(cases), reps)
    if rc not in (0, DIVERGED):
        B.check(rc, "equality gate")
    out = [Report(r.backend.decode(), r.hash.decode(), [c.label for i, c in enumerate(cases) if r.diverged >> i & 1],
                  int(r.error)) for r in reps]
    return rc == 0, out


def residency_gate(b: GateBackend, cases=None):
    """residency_gate (gate.rs:108-140): None if it holds, else the message naming the first differing case."""
    cases = corpus() if cases is None else cases
    arr, _keep = _case_array(cases)
    msg = C.create_string_buffer(512)
    rc = _lib().kt_hip_residency_gate(C.byref(b.raw), arr, len(cases), msg, 512)
    if rc == 0:
        return None
    if rc != DIVERGED:
        B.check(rc, "residency gate")
    return msg.value.decode()


def bound_holds(b: GateBackend, case: Case) -> bool:
    """The backend's answer on one bound case equals Portable's."""
    x = np.ascontiguousarray(case.x, np.int32)
    w = np.ascontiguousarray(case.w, np.int32)
    y = np.zeros(case.rows * case.out, np.int64)
    rc = b.raw.linear_weights(b.raw.ctx, x.ctypes.data_as(C.POINTER(C.c_int32)), case.id,
                              w.ctypes.data_as(C.POINTER(C.c_int32)), case.rows, case.out, case.k,
                              y.ctypes.data_as(C.POINTER(C.c_int64)))
    want = np.zeros_like(y)
    _lib().kt_hip_portable_linear(x.ctypes.data, w.ctypes.data, case.rows, case.out, case.k, want.ctypes.data)
    return rc == 0 and np.array_equal(y, want)
