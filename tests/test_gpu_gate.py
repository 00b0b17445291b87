"""The gates as a product feature on the MI355X (kt-runtime/src/tests_cuda.rs:17-72 through the library's gates, not
the test's own): the device backend at the default budget and at a 1-byte budget gives the reference's corpus hash,
holds residency and every bound case; each planted defect of libkt_hip_planted.so is caught by the gate that the
reference's test names for it; and kt_runtime_probe --budget-1 --plants says the same and exits 0."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

CORPUS_HASH = "781285bb99bcd9cb5233f708466676db41e717b6971ce70508b57ed291478352"  # kt-runtime/src/tests_cuda.rs:9
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def test_the_device_backends_pass_every_gate(torch_dev):
    import tritify_amd as T
    from tritify_amd import gate

    say("case: gates on hip (default budget, budget 1)")
    hbs = [T.HipBackend(0), T.HipBackend(0, budget=1)]
    bs = [gate.of(b) for b in hbs]
    ok, reps = gate.equality_gate([gate.portable()] + bs)
    assert ok, [(r.backend, r.diverged, r.error) for r in reps]
    assert [r.hash for r in reps] == [CORPUS_HASH] * 3
    for b in bs:
        assert gate.residency_gate(b) is None, b.name
        for c in gate.bound_cases():
            say(f"case: {b.name} bound {c.label} k={c.k}")
            assert gate.bound_holds(b, c), (b.name, c.label)
    assert T.fallbacks() == 0
    for b in hbs:
        b.close()


def test_every_plant_is_caught_by_its_gate(torch_dev):
    import tritify_amd as T
    from tritify_amd import gate

    for plant in (T.PLANT_DROP_TOP, T.PLANT_WRONG_CARRY):
        hb = T.HipBackend(0, plant=plant)
        say(f"case: plant {plant} equality gate")
        ok, reps = gate.equality_gate([gate.portable(), gate.of(hb)])
        assert not ok and reps[1].diverged, hb.name()
        hb.close()
    hb = T.HipBackend(0, plant=T.PLANT_NO_FLUSH)
    b = gate.of(hb)
    say("case: plant NoFlush")
    assert gate.equality_gate([gate.portable(), b])[0], "the corpus never reaches the bound"
    own = gate.bound_cases()[1:]
    assert own and not any(gate.bound_holds(b, c) for c in own)
    hb.close()
    hb = T.HipBackend(0, plant=T.PLANT_CACHE_BY_SHAPE)
    say("case: plant CacheByShape")
    msg = gate.residency_gate(gate.of(hb))
    assert msg is not None and "differs" in msg
    hb.close()


def test_the_probe_command_line(torch_dev):
    say("case: kt_runtime_probe --budget-1 --plants")
    exe = os.path.join(ROOT, "tritify_amd", "kt_runtime_probe")
    r = subprocess.run([exe, "--budget-1", "--plants"], capture_output=True, text=True, timeout=300)
    say(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.count(CORPUS_HASH) == 3
    assert r.stdout.count(" caught  ") == 4 and "NOT CAUGHT" not in r.stdout
    assert r.stdout.count("residency   :") == 2 and r.stdout.count(" holds") == 2
    assert "DIVERGED" not in r.stdout and "verdict     : every backend byte-identical" in r.stdout
