"""The gates as a product feature, on the CPU (kt-runtime/src/gate.rs:1-140, tests_cuda.rs:17-72): the library's
corpus is the reference's byte for byte (against the oracle's restatement), the engine's Portable through the
equality gate gives the reference's corpus hash 781285bb..., the bound cases have their closed-form answers, and the
gates catch planted defects in caller-supplied backends -- a dropped top term by the equality gate, a shape-keyed
cache by the residency gate only. The command line (kt_runtime_probe) runs on a host without a GPU. No GPU call."""
import os
import subprocess

import numpy as np

from oracle import oracle as O

CORPUS_HASH = "781285bb99bcd9cb5233f708466676db41e717b6971ce70508b57ed291478352"  # kt-runtime/src/tests_cuda.rs:9
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_the_corpus_is_the_references():
    from tritify_amd import gate

    got, want = gate.corpus(), O.corpus()
    assert [c.label for c in got] == [c.label for c in want]
    for g, w in zip(got, want):
        assert (g.rows, g.out, g.k) == (w.rows, w.out, w.k)
        assert np.array_equal(g.x, w.x) and np.array_equal(g.w, w.w), g.label
    assert len({c.id for c in got}) == len(got)


def test_portable_through_the_gate_gives_the_corpus_hash():
    from tritify_amd import gate

    ok, reps = gate.equality_gate([gate.portable(), gate.portable()])
    assert ok and [r.hash for r in reps] == [CORPUS_HASH] * 2 and not reps[0].diverged


def test_bound_cases_closed_forms():
    from tritify_amd import gate

    cases = gate.bound_cases()
    assert cases[0].k == (O.KT_FLUSH + 1) * 16 and cases[0].label == O.flush_case().label
    p = gate.portable()
    for c in cases:
        code = int(c.x[0])
        assert (c.x == code).all() and c.rows == 1 and c.out == 2
        y = np.zeros(2, np.int64)
        gate._lib().kt_hip_portable_linear(c.x.ctypes.data, c.w.ctypes.data, 1, 2, c.k, y.ctypes.data)
        assert y.tolist() == [c.k * code * code, -c.k * code * code], c.label
        assert gate.bound_holds(p, c)


def test_the_gates_catch_planted_defects_in_any_backend():
    from tritify_amd import gate

    def exact(x, wid, w, rows, out, k):
        return O.portable(x, w, rows, out, k)

    def drop_top(x, wid, w, rows, out, k):  # loses the top base-256 digit product of every term (DropPlane22-like)
        xh, wh = (x.astype(np.int64) + 2**15) >> 16, (w.astype(np.int64) + 2**15) >> 16
        y = O.portable(x, w, rows, out, k).reshape(rows, out)
        return (y - (xh.reshape(rows, k) << 16) @ (wh.reshape(out, k) << 16).T).reshape(-1)

    cache = {}

    def by_shape(x, wid, w, rows, out, k):  # resident weights keyed by shape only (CacheByShape)
        key = (out, k)
        if key not in cache:
            cache[key] = w.copy()
        return O.portable(x, cache[key], rows, out, k)

    ok, reps = gate.equality_gate([gate.portable(), gate.from_callable("exact", exact),
                                   gate.from_callable("drop-top", drop_top)])
    assert not ok
    assert reps[1].hash == CORPUS_HASH and not reps[1].diverged
    assert reps[2].diverged and reps[2].hash != CORPUS_HASH
    shaped = gate.from_callable("by-shape", by_shape)
    ok, _ = gate.equality_gate([gate.portable(), shaped])
    assert ok, "every corpus case has its own shape"
    msg = gate.residency_gate(shaped)
    assert msg is not None and "twin 0 of one shape differs in round 0" in msg  # the corpus k=1023 filled it
    assert gate.residency_gate(gate.from_callable("exact", exact)) is None


def test_the_probe_runs_on_a_host_without_a_gpu():
    exe = os.path.join(ROOT, "tritify_amd", "kt_runtime_probe")
    r = subprocess.run([exe, "--no-speed"], capture_output=True, text=True, timeout=120,
                       env=dict(os.environ, HIP_VISIBLE_DEVICES=""))
    assert r.returncode == 0, r.stdout + r.stderr
    assert f"gate        : portable   {CORPUS_HASH}  identical" in r.stdout
    assert "verdict     : every backend byte-identical" in r.stdout
