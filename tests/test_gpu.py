"""Parity of the MI355X backend with the CPU oracle, through the C ABI. Run on a GPU box with -m gpu.

Mirrors the reference's backend tests: crates/02-runtime/kt-runtime/src/tests_cuda.rs (the corpus hash, residency,
the bound case, every planted defect caught), crates/02-runtime/kt-cuda/src/tests.rs (tails, extremes, bounds), and
the benchmark workloads (config 1 through the LinearBackend path; config 2 through the 12-bit-weight path) checked
byte for byte: against the oracle at sizes it computes in seconds, and against the committed fixture hashes at full
size.
"""
import json
import os
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "goldens.json")))
CORPUS_HASH = "781285bb99bcd9cb5233f708466676db41e717b6971ce70508b57ed291478352"  # kt-runtime/src/tests_cuda.rs:9
KT_DEMO_HASH = "de67ba758bd0d1fb574fa64d7ff326e9d17f536d7725659228bebddcc6478bfa"  # README.md:74


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def tb():
    import tritify_amd

    return tritify_amd


# ----------------------------------------------------------------------------------------------------------------
# the MFMA lane layout the kernels assume


def test_mfma_lane_layout(torch_dev):
    """One 32x32x32 and one 16x16x64 int8 MFMA on known operands: the C registers sit where the kernels read them
    (32x32: lane l, register r -> row 8(r/4) + 4(l/32) + r%4, column l%32; 16x16: row 4(l/16) + r, column l%16),
    given operand bytes placed as lane l = row (l mod R), k = 16 (l div R) .. +16."""
    torch = torch_dev
    say("case: mfma layout probe")
    rng = np.random.default_rng(0)
    a = rng.integers(-128, 128, size=(64, 16), dtype=np.int8)
    b = rng.integers(-128, 128, size=(64, 16), dtype=np.int8)
    ad = torch.from_numpy(a.copy()).cuda()
    bd = torch.from_numpy(b.copy()).cuda()
    c32 = torch.zeros(64 * 16, dtype=torch.int32, device="cuda")
    c16 = torch.zeros(64 * 4, dtype=torch.int32, device="cuda")
    tb().probe_mfma(ad, bd, c32, c16)
    torch.cuda.synchronize()
    c32, c16 = c32.cpu().numpy().reshape(64, 16), c16.cpu().numpy().reshape(64, 4)
    # 32x32x32: A[i][k] is lane (i + 32*(k//16)) byte k%16; B likewise with the column
    A = np.zeros((32, 32), np.int64)
    B = np.zeros((32, 32), np.int64)
    for l in range(64):
        A[l % 32, 16 * (l // 32):16 * (l // 32) + 16] = a[l]
        B[l % 32, 16 * (l // 32):16 * (l // 32) + 16] = b[l]
    C = A @ B.T
    for l in range(64):
        for r in range(16):
            assert c32[l, r] == C[8 * (r // 4) + 4 * (l // 32) + r % 4, l % 32], (l, r)
    A = np.zeros((16, 64), np.int64)
    B = np.zeros((16, 64), np.int64)
    for l in range(64):
        A[l % 16, 16 * (l // 16):16 * (l // 16) + 16] = a[l]
        B[l % 16, 16 * (l // 16):16 * (l // 16) + 16] = b[l]
    C = A @ B.T
    for l in range(64):
        for r in range(4):
            assert c16[l, r] == C[4 * (l // 16) + r, l % 16], (l, r)


# ----------------------------------------------------------------------------------------------------------------
# the LinearBackend path (digit planes)


def gate(b, cases):
    """equality_gate for one backend against the oracle (kt-runtime/src/gate.rs:79-104): (hash, diverged labels)."""
    ys, diverged = [], []
    for c in cases:
        say(f"case: {b.name()} corpus {c.label} ({c.rows}x{c.out}x{c.k})")
        y = b.linear_weights(c.x, c.weights, c.rows, c.out, c.k)
        ys.append(y)
        if not np.array_equal(y, O.portable(c.x, c.w, c.rows, c.out, c.k)):
            diverged.append(c.label)
    return O.sha256_hex(np.concatenate(ys)), diverged


def corpus_with_ids():
    cs = O.corpus()
    for c in cs:
        c.weights = tb().Weights(tb().weight_id_fresh(), c.w)
    return cs


def residency_gate(b, cases):
    """gate.rs:109-140: the corpus twice, then two weight matrices of one shape interleaved four times."""
    for p in (1, 2):
        for c in cases:
            if not np.array_equal(b.linear_weights(c.x, c.weights, c.rows, c.out, c.k),
                                  O.portable(c.x, c.w, c.rows, c.out, c.k)):
                return f"{b.name()}: pass {p}, case '{c.label}' differs"
    x = next(c.x for c in cases if c.label == "k=1023")
    pair = [(tb().weight_id_fresh(), O.codes(64 * 1023, s)) for s in (11, 12)]
    for rnd in range(4):
        for i, (wid, w) in enumerate(pair):
            if not np.array_equal(b.linear_weights(x, tb().Weights(wid, w), 4, 64, 1023), O.portable(x, w, 4, 64, 1023)):
                return f"{b.name()}: twin {i} of one shape differs in round {rnd}"
    return None


def test_the_backend_gives_the_corpus_hash_and_holds_residency_and_the_bound():
    """kt-runtime/src/tests_cuda.rs:17-45 on the MI355X, with the default budget and with a budget of 1 byte."""
    HB = tb().HipBackend
    cases = corpus_with_ids()
    bound = O.flush_case()
    for b, resident in [(HB(0), True), (HB(0, budget=1), False)]:
        h, diverged = gate(b, cases)
        assert not diverged, (b.name(), diverged)
        assert h == CORPUS_HASH == GOLD["corpus_sha256"], b.name()
        assert residency_gate(b, cases) is None
        assert (b.resident_bytes() > 0) == resident, b.name()
        say(f"case: {b.name()} flush case k={bound.k}")
        y = b.linear(bound.x, bound.w, 1, 2, bound.k)
        assert list(y) == [bound.k * O.WLEVELS**2, -bound.k * O.WLEVELS**2]
        assert b.name().startswith("hip:")
        b.close()
    assert tb().fallbacks() == 0


@pytest.mark.parametrize("px,code", [(1, -128), (3, -8_421_504)])
def test_this_builds_own_bound_case(px, code):
    """At the backend's int32 flush bound plus one chunk, with every digit at -128, the accumulators would wrap
    without the flush; the backend is exact there (the NoFlush firing control is in the planted test below)."""
    b = tb().HipBackend(0)
    k = tb().flush_k(px, px) + 256
    x = np.full(k, code, dtype=np.int32)
    w = np.concatenate([x, -x])
    say(f"case: bound px={px} k={k}")
    y = b.linear(x, w, 1, 2, k)
    assert list(y) == [k * code * code, -k * code * code]
    b.close()


def test_every_planted_defect_is_caught():
    """kt-runtime/src/tests_cuda.rs:47-72 with this backend's plants (libkt_hip_planted.so)."""
    T = tb()
    cases = corpus_with_ids()
    for plant in (T.PLANT_DROP_TOP, T.PLANT_WRONG_CARRY):
        b = T.HipBackend(0, plant=plant)
        _, diverged = gate(b, cases)
        assert diverged, b.name()
        say(f"equality gate: {b.name()} diverges on {diverged}")
        b.close()
    b = T.HipBackend(0, plant=T.PLANT_NO_FLUSH)
    _, diverged = gate(b, cases)
    assert not diverged, "the corpus never reaches the bound"
    for px, code in [(1, -128), (3, -8_421_504)]:
        k = T.flush_k(px, px) + 256
        x = np.full(k, code, dtype=np.int32)
        say(f"case: planted NoFlush bound px={px}")
        assert b.linear(x, x, 1, 1, k)[0] != k * code * code
    b.close()
    b = T.HipBackend(0, plant=T.PLANT_CACHE_BY_SHAPE)
    assert residency_gate(b, cases) is not None
    b.close()


def test_kt_demo_and_config1_hashes(hip_backend):
    """apps/kt-demo (README.md:74) and benchmark config 1 through the LinearBackend ABI."""
    qx, qw = O.gen_demo(64, 768, 768, 42)
    assert O.sha256_hex(hip_backend.linear(qx, qw, 64, 768, 768)) == KT_DEMO_HASH
    g = GOLD["config1"]
    qx, qw = O.gen_demo(64, 1024, 1024, 42)
    y = hip_backend.linear(qx, qw, 64, 1024, 1024)
    assert O.sha256_hex(y) == g["y_i64_sha256"] and O.sha256_hex(y.astype(np.int32)) == g["y_i32_sha256"]


def test_tails_mixed_planes_and_any_i32(hip_backend):
    """kt-cuda/src/tests.rs:54-65 shapes, every plane pairing, and full-range i32 codes (wrapping i64)."""
    rng = np.random.default_rng(7)
    ranges = {1: (-128, 127), 3: (-O.WLEVELS, O.WLEVELS), 5: (-(2**31), 2**31 - 1)}
    shapes = [(1, 1, 1), (3, 5, 7), (2, 17, 33), (16, 16, 16), (17, 33, 50), (1, 9, 4099), (20, 40, 300),
              (65, 129, 64), (130, 70, 129), (257, 3, 200)]
    for px in (1, 3, 5):
        for pw in (1, 3, 5):
            for rows, out, k in shapes:
                x = rng.integers(*ranges[px], size=rows * k, endpoint=True).astype(np.int32)
                w = rng.integers(*ranges[pw], size=out * k, endpoint=True).astype(np.int32)
                say(f"case: planes {px}x{pw} {rows}x{out}x{k}")
                assert np.array_equal(hip_backend.linear(x, w, rows, out, k), O.portable(x, w, rows, out, k)), \
                    (px, pw, rows, out, k)


def test_empty_shapes(hip_backend):
    for rows, out, k in [(0, 5, 3), (4, 0, 3), (0, 0, 0)]:
        y = hip_backend.linear(np.zeros(rows * k, np.int32), np.zeros(out * k, np.int32), rows, out, k)
        assert y.size == 0
    y = hip_backend.linear(np.zeros(0, np.int32), np.zeros(0, np.int32), 3, 4, 0)
    assert np.array_equal(y, np.zeros(12, np.int64))


def test_device_level_digit_gemm(torch_dev):
    """kt_hip_pack_planes + kt_hip_digit_gemm on device buffers (the kt_cuda_digit_gemm level)."""
    torch = torch_dev
    T = tb()
    rows, out, k = 37, 91, 333
    x, w = O.codes(rows * k, 1), O.codes(out * k, 2)
    kp = T.kp(k)
    xd, wd = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    xa = torch.empty(3 * rows * kp, dtype=torch.int8, device="cuda")
    wb = torch.empty(3 * out * kp, dtype=torch.int8, device="cuda")
    y = torch.empty(rows * out, dtype=torch.int64, device="cuda")
    T.pack_planes(xd, rows, k, 3, xa)
    T.pack_planes(wd, out, k, 3, wb)
    torch.cuda.synchronize()
    assert np.array_equal(xa.cpu().numpy().reshape(3, rows, kp), O.pack_planes(x, rows, k, 3))
    T.digit_gemm(xa, 3, wb, 3, y, rows, out, k)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), O.portable(x, w, rows, out, k))


# ----------------------------------------------------------------------------------------------------------------
# the 12-bit-weight path


def _w12_device(torch, w, n, k):
    T = tb()
    nlo, nnib = T.w12_bytes(n, k)
    lo = torch.empty(nlo, dtype=torch.int8, device="cuda")
    nib = torch.empty(nnib, dtype=torch.uint8, device="cuda")
    T.w12_upload(w, n, k, lo, nib)
    return lo, nib


def _x_device(torch, x, m, k):
    kp = tb().kp(k)
    xp = np.zeros((m, kp), np.int8)
    xp[:, :k] = x.reshape(m, k)
    return torch.from_numpy(xp).cuda()


def test_w12_pack_matches_the_oracle_layout(torch_dev):
    torch = torch_dev
    rng = np.random.default_rng(3)
    for n, k in [(1, 1), (3, 33), (64, 64), (17, 200), (5, 4096)]:
        w = rng.integers(-2048, 2048, size=n * k).astype(np.int32)
        lo, nib = _w12_device(torch, w, n, k)
        olo, onib = O.w12_pack(w, n, k)
        assert np.array_equal(lo.cpu().numpy(), olo) and np.array_equal(nib.cpu().numpy(), onib), (n, k)
    with pytest.raises(tb().HipError):
        _w12_device(torch, np.array([2048], np.int32), 1, 1)


def test_stream_read_touches_every_byte(torch_dev):
    """kt_hip_stream_read (the read-floor probe): the XOR of its per-chunk words is the XOR of every 32-bit word of
    the buffer, for empty, one-load, ragged-chunk and config-2-sized buffers; a length that is not a multiple of 16
    is refused."""
    torch = torch_dev
    T = tb()
    rng = np.random.default_rng(3)
    out = torch.empty(T.backend.STREAM_READ_CTAS, dtype=torch.int32, device="cuda")
    for nbytes in (0, 16, 16 * 1001, 4096 * 4096 * 3 // 2):
        buf = rng.integers(-(2**31), 2**31, size=max(nbytes // 4, 1), dtype=np.int64).astype(np.int32)[: nbytes // 4]
        src = torch.from_numpy(buf.copy() if nbytes else np.zeros(4, np.int32)).cuda()
        say(f"case: stream read {nbytes} bytes")
        out.fill_(0x5A5A5A5A)
        T.backend.stream_read(src, nbytes, out)
        torch.cuda.synchronize()
        want = np.bitwise_xor.reduce(buf.view(np.uint32)) if nbytes else np.uint32(0)
        assert np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32)) == want, nbytes
    with pytest.raises(T.HipError):
        T.backend.stream_read(src, 24, out)


@pytest.mark.parametrize("out_kind", [0, 1, 2])
def test_w12_linear_against_the_oracle(torch_dev, out_kind):
    """GEMV (m <= 8) and MFMA GEMM (m > 8) for tails in m, n and k, every output kind."""
    torch = torch_dev
    T = tb()
    rng = np.random.default_rng(10 + out_kind)
    for m, n, k in [(1, 1, 1), (1, 5, 7), (2, 33, 100), (3, 64, 64), (4, 130, 1000), (5, 17, 4096), (8, 256, 2048),
                    (9, 70, 129), (16, 4096, 512), (17, 65, 64), (33, 200, 300), (64, 64, 4096), (65, 129, 640),
                    (100, 96, 2000), (96, 1000, 4096), (128, 512, 1024), (129, 100, 256), (130, 300, 96), (300, 257, 448)]:
        x = rng.integers(-128, 128, size=m * k).astype(np.int32)
        w = rng.integers(-2048, 2048, size=n * k).astype(np.int32)
        mant, shift = O.channel_scales(w, n, k, 40)
        lo, nib = _w12_device(torch, w, n, k)
        xd = _x_device(torch, x, m, k)
        md, sd = torch.from_numpy(mant).cuda(), torch.from_numpy(shift).cuda()
        dt = {0: torch.int64, 1: torch.int32, 2: torch.int8}[out_kind]
        y = torch.empty(m * n, dtype=dt, device="cuda")
        say(f"case: w12 out_kind={out_kind} {m}x{n}x{k}")
        T.w12_linear(xd, lo, nib, m, n, k, y, out_kind, md, sd)
        torch.cuda.synchronize()
        acc = O.portable(x, w, m, n, k)
        if out_kind == 0:
            want = acc
        elif out_kind == 1:
            want = O.requant_channels(acc, m, n, mant, shift, -(2**31), 2**31 - 1)
        else:
            want = O.requant_channels(acc, m, n, mant, shift, -127, 127).astype(np.int8)
        assert np.array_equal(y.cpu().numpy(), want), (m, n, k)


def test_w12_extremes(torch_dev):
    """Every product at its largest magnitude on the skinny kernel and on the GEMM, at k = 4096 and at k = 20000
    (where the row-sum term -1920 * sum(x) no longer fits int32)."""
    torch = torch_dev
    T = tb()
    n = 64
    for m, k in [(1, 4096), (64, 4096), (128, 4096), (129, 4096), (3, 20000), (100, 20000), (129, 20000)]:
        for xv, wv in [(-128, -2048), (127, 2047), (-128, 2047), (127, -2048)]:
            x = np.full(m * k, xv, np.int32)
            w = np.full(n * k, wv, np.int32)
            lo, nib = _w12_device(torch, w, n, k)
            y = torch.empty(m * n, dtype=torch.int64, device="cuda")
            say(f"case: w12 extremes m={m} x={xv} w={wv}")
            T.w12_linear(_x_device(torch, x, m, k), lo, nib, m, n, k, y)
            torch.cuda.synchronize()
            assert (y.cpu().numpy() == k * xv * wv).all()


def test_w12_int32_bound_at_k_8192(torch_dev):
    """x = -128 against w = -2048 over k = 8192 sums to exactly 2^31, one past int32: the skinny kernel (m <= 128) and
    the GEMM (m > 128) must both carry it into i64 and requantize it exactly."""
    torch = torch_dev
    T = tb()
    k, n = 8192, 40
    w = np.full(n * k, -2048, np.int32)
    lo, nib = _w12_device(torch, w, n, k)
    mant = np.full(n, 1, np.int32)
    shift = np.full(n, 24, np.int32)  # 2^31 / 2^24 = 128 -> clamps to 127 for int8, 128 for int32
    md, sd = torch.from_numpy(mant).cuda(), torch.from_numpy(shift).cuda()
    for m in (1, 33, 65, 130, 200):
        x = np.full(m * k, -128, np.int32)
        xd = _x_device(torch, x, m, k)
        say(f"case: w12 2^31 bound m={m}")
        y = torch.empty(m * n, dtype=torch.int64, device="cuda")
        q32 = torch.empty(m * n, dtype=torch.int32, device="cuda")
        T.w12_linear(xd, lo, nib, m, n, k, y)
        T.w12_linear(xd, lo, nib, m, n, k, q32, T.OUT_I32, md, sd)
        torch.cuda.synchronize()
        assert (y.cpu().numpy() == 2**31).all() and (q32.cpu().numpy() == 128).all(), m


def test_w12_few_columns_and_long_k(torch_dev):
    """Few 16-column blocks against long k (past the int32 range of one dot, up to 70000) on the skinny kernel,
    every output kind, against the oracle; every launch twice, so nothing depends on state a launch leaves."""
    torch = torch_dev
    T = tb()
    rng = np.random.default_rng(21)
    cases = [(1, 32, 8192), (2, 64, 20000), (8, 40, 12345), (32, 100, 9000), (33, 96, 16384), (64, 33, 70000),
             (17, 1000, 4096), (5, 4096, 896)]
    data = []
    for m, n, k in cases:
        x = rng.integers(-128, 128, size=m * k).astype(np.int32)
        w = rng.integers(-2048, 2048, size=n * k).astype(np.int32)
        mant, shift = O.channel_scales(w, n, k, 40)
        acc = O.portable(x, w, m, n, k)
        data.append((m, n, k, x, w, mant, shift, acc))
    for rep in range(2):
        for m, n, k, x, w, mant, shift, acc in data:
            lo, nib = _w12_device(torch, w, n, k)
            xd = _x_device(torch, x, m, k)
            md, sd = torch.from_numpy(mant).cuda(), torch.from_numpy(shift).cuda()
            say(f"case: w12 long k {m}x{n}x{k} rep {rep}")
            y = torch.empty(m * n, dtype=torch.int64, device="cuda")
            q32 = torch.empty(m * n, dtype=torch.int32, device="cuda")
            q8 = torch.empty(m * n, dtype=torch.int8, device="cuda")
            T.w12_linear(xd, lo, nib, m, n, k, y)
            T.w12_linear(xd, lo, nib, m, n, k, q32, T.OUT_I32, md, sd)
            T.w12_linear(xd, lo, nib, m, n, k, q8, T.OUT_I8, md, sd)
            torch.cuda.synchronize()
            assert np.array_equal(y.cpu().numpy(), acc), (m, n, k)
            assert np.array_equal(q32.cpu().numpy(), O.requant_channels(acc, m, n, mant, shift, -(2**31),
                                                                         2**31 - 1)), (m, n, k)
            assert np.array_equal(q8.cpu().numpy(), O.requant_channels(acc, m, n, mant, shift, -127, 127)), (m, n, k)


def test_w12_requant_edges(torch_dev):
    """Every pairing of edge multipliers and shifts (one output channel each; shifts from -2^31 to 2^31 - 1) on the
    skinny kernel, the int32-fast GEMM (k <= 8128) and the i64 GEMM (longer k), against the oracle's exact clamp."""
    from test_oracle import EDGE_MANT, EDGE_SHIFT

    torch = torch_dev
    T = tb()
    pairs = [(mm, ss) for mm in EDGE_MANT for ss in EDGE_SHIFT]
    n = len(pairs)
    mant = np.array([p[0] for p in pairs], np.int32)
    shift = np.array([p[1] for p in pairs], np.int32)
    md, sd = torch.from_numpy(mant).cuda(), torch.from_numpy(shift).cuda()
    rng = np.random.default_rng(22)
    for m, k in [(3, 4096), (70, 9000), (130, 4096), (140, 9000)]:
        x = rng.integers(-128, 128, size=m * k).astype(np.int32)
        w = rng.integers(-2048, 2048, size=n * k).astype(np.int32)
        w[: 2 * k] = -2048  # two channels at the largest magnitude
        x[:k] = -128
        lo, nib = _w12_device(torch, w, n, k)
        xd = _x_device(torch, x, m, k)
        acc = O.portable(x, w, m, n, k)
        say(f"case: w12 requant edges {m}x{n}x{k}")
        q32 = torch.empty(m * n, dtype=torch.int32, device="cuda")
        q8 = torch.empty(m * n, dtype=torch.int8, device="cuda")
        T.w12_linear(xd, lo, nib, m, n, k, q32, T.OUT_I32, md, sd)
        T.w12_linear(xd, lo, nib, m, n, k, q8, T.OUT_I8, md, sd)
        torch.cuda.synchronize()
        assert np.array_equal(q32.cpu().numpy(), O.requant_channels(acc, m, n, mant, shift, -(2**31), 2**31 - 1))
        assert np.array_equal(q8.cpu().numpy(), O.requant_channels(acc, m, n, mant, shift, -127, 127))


def test_w12_two_streams(torch_dev):
    """Launches interleaved on two streams give the oracle's result on each."""
    torch = torch_dev
    T = tb()
    rng = np.random.default_rng(23)
    m, n, k = 4, 256, 8192
    ws = [rng.integers(-2048, 2048, size=n * k).astype(np.int32) for _ in range(2)]
    x = rng.integers(-128, 128, size=m * k).astype(np.int32)
    xd = _x_device(torch, x, m, k)
    devs = [_w12_device(torch, w, n, k) for w in ws]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    ys = [torch.empty(m * n, dtype=torch.int64, device="cuda") for _ in range(2)]
    torch.cuda.synchronize()
    say("case: w12 two streams")
    for rep in range(4):
        for i in range(2):
            T.w12_linear(xd, devs[i][0], devs[i][1], m, n, k, ys[i], stream=streams[i])
    torch.cuda.synchronize()
    for i in range(2):
        assert np.array_equal(ys[i].cpu().numpy(), O.portable(x, ws[i], m, n, k)), i


@pytest.mark.parametrize("m,n,k", [(2048, 4096, 64), (2100, 3900, 100), (2305, 4000, 704), (4096, 2080, 1000)])
def test_w12_dma_tile_kernel(torch_dev, m, n, k):
    """Shapes whose 256 x 128 tiles cover every CU take the DMA-fed GEMM: ragged rows (a one-row last tile) and
    columns (a last tile of one or a partial column block), k of one and two 64-deep k-tiles (fewer than the ring
    keeps in flight) and longer; every output kind, the residual add included, against the oracle."""
    torch = torch_dev
    T = tb()
    rng = np.random.default_rng(m + n + k)
    x = rng.integers(-128, 128, size=m * k).astype(np.int32)
    w = rng.integers(-2048, 2048, size=n * k).astype(np.int32)
    mant, shift = O.channel_scales(w, n, k, 40)
    lo, nib = _w12_device(torch, w, n, k)
    xd = _x_device(torch, x, m, k)
    md, sd = torch.from_numpy(mant).cuda(), torch.from_numpy(shift).cuda()
    acc = O.linear_threads(x, w, m, n, k, 16, O.lib().kt_cpu_auto_variant())
    q32 = O.requant_channels(acc, m, n, mant, shift, -(2**31), 2**31 - 1)
    res = rng.integers(-(2**31), 2**31, size=m * n, dtype=np.int64).astype(np.int32)
    res[:4] = [2**31 - 1, -(2**31), 5, -5]  # saturating adds at both ends
    wants = {T.OUT_I64: acc, T.OUT_I32: q32,
             T.OUT_I8: O.requant_channels(acc, m, n, mant, shift, -127, 127).astype(np.int8),
             T.OUT_I32_ADD: np.clip(res.astype(np.int64) + q32, -(2**31), 2**31 - 1).astype(np.int32)}
    for kind, want in wants.items():
        say(f"case: w12 dma tile {m}x{n}x{k} out_kind={kind}")
        y = torch.from_numpy(res.copy()).cuda() if kind == T.OUT_I32_ADD else \
            torch.empty(m * n, dtype={T.OUT_I64: torch.int64, T.OUT_I32: torch.int32, T.OUT_I8: torch.int8}[kind],
                        device="cuda")
        T.w12_linear(xd, lo, nib, m, n, k, y, kind, md, sd)
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        assert np.array_equal(got, want), (kind, np.argwhere(got != want)[:5].tolist())


def test_w12_dma_tile_kernel_past_int32(torch_dev):
    """The DMA-fed GEMM at k = 8200 (past the int32 recombination: the i64 epilogue) with every product at its
    largest magnitude: each output is k * x * w exactly."""
    torch = torch_dev
    T = tb()
    m, n, k = 2048, 4096, 8200
    for xv, wv in [(-128, -2048), (127, -2048)]:
        lo, nib = _w12_device(torch, np.full(n * k, wv, np.int32), n, k)
        xd = torch.full((m, T.kp(k)), xv, dtype=torch.int8, device="cuda")
        xd[:, k:] = 0
        y = torch.empty(m * n, dtype=torch.int64, device="cuda")
        say(f"case: w12 dma tile past int32 x={xv} w={wv}")
        T.w12_linear(xd, lo, nib, m, n, k, y)
        torch.cuda.synchronize()
        assert bool((y == k * xv * wv).all().item())


def test_config2_full_size_against_fixtures(torch_dev):
    """benchmark config 2 at its full shape (N = K = 4096, M in {1, 16, 128, 2048}): the i64 accumulators and the
    requantized int8 outputs hash to the fixtures the CPU oracle produced (tests/golden/goldens.json)."""
    torch = torch_dev
    T = tb()
    g = GOLD["config2"]
    N, K = g["N"], g["K"]
    w = O.gen_w12(g["w_seed"], N * K)
    x = O.gen_act_gauss(g["x_seed"], g["sigma"], max(g["Ms"]) * K)
    mant, shift = O.channel_scales(w, N, K, g["sigma"])
    assert O.sha256_hex(w) == g["w_sha256"] and O.sha256_hex(x) == g["x_sha256"]
    lo, nib = _w12_device(torch, w, N, K)
    md, sd = torch.from_numpy(mant).cuda(), torch.from_numpy(shift).cuda()
    xd_all = torch.from_numpy(x.astype(np.int8)).cuda()
    for m in g["Ms"]:
        want = g["outputs"][str(m)]
        acc = torch.empty(m * N, dtype=torch.int64, device="cuda")
        q = torch.empty(m * N, dtype=torch.int8, device="cuda")
        say(f"case: config2 M={m}")
        T.w12_linear(xd_all[: m * K], lo, nib, m, N, K, acc, T.OUT_I64)
        T.w12_linear(xd_all[: m * K], lo, nib, m, N, K, q, T.OUT_I8, md, sd)
        torch.cuda.synchronize()
        assert O.sha256_hex(acc.cpu().numpy()) == want["acc_i64_sha256"], m
        assert O.sha256_hex(q.cpu().numpy()) == want["out_i8_sha256"], m


@pytest.mark.parametrize("m,n,k", [(512, 2048, 512), (161, 250, 448), (520, 4010, 200)])
def test_w12_small_tile_variants_every_output(torch_dev, m, n, k):
    """The dense W12 products on the smaller CTA tiles chosen when 128 x 128 tiles leave CUs idle: 512 x 2048 x 512
    lands on the 64 x 64 variant (tiles_h = 128, tiles_q = 256), the ragged 161 x 250 x 448 on 32 x 64, the ragged
    520 x 4010 x 200 on 64 x 128 (tiles_h = 288); each for i64, i32, int8, the saturating residual add (from residuals
    at both int32 limits) and the int8 code table."""
    torch = torch_dev
    T = tb()
    rng = np.random.default_rng(m + n + k)
    x = rng.integers(-128, 128, size=m * k).astype(np.int32)
    w = rng.integers(-2048, 2048, size=n * k).astype(np.int32)
    mant, shift = O.channel_scales(w, n, k, 40)
    mant[::7] = 2**31 - 1  # some channels far past int8 / int32 after the requant
    lo, nib = _w12_device(torch, w, n, k)
    xd = _x_device(torch, x, m, k)
    md, sd = torch.from_numpy(mant).cuda(), torch.from_numpy(shift).cuda()
    acc = O.portable(x, w, m, n, k)
    for out_kind in (0, 1, 2, 3):
        say(f"case: w12 small-tile {m}x{n}x{k} out_kind={out_kind}")
        dt = {0: torch.int64, 1: torch.int32, 2: torch.int8, 3: torch.int32}[out_kind]
        prev = rng.integers(-(2**31), 2**31, size=m * n, dtype=np.int64).astype(np.int32)
        prev[::5] = 2**31 - 1
        prev[1::5] = -(2**31)
        y = torch.from_numpy(prev.copy()).cuda() if out_kind == 3 else torch.empty(m * n, dtype=dt, device="cuda")
        T.w12_linear(xd, lo, nib, m, n, k, y, out_kind, md, sd)
        torch.cuda.synchronize()
        if out_kind == 0:
            want = acc
        elif out_kind == 1:
            want = O.requant_channels(acc, m, n, mant, shift, -(2**31), 2**31 - 1)
        elif out_kind == 2:
            want = O.requant_channels(acc, m, n, mant, shift, -127, 127).astype(np.int8)
        else:
            q = O.requant_channels(acc, m, n, mant, shift, -(2**31), 2**31 - 1).astype(np.int64)
            want = np.clip(prev.astype(np.int64) + q, -(2**31), 2**31 - 1).astype(np.int32)
        assert np.array_equal(y.cpu().numpy(), want), out_kind
    say(f"case: w12 small-tile {m}x{n}x{k} lut")
    lut = rng.integers(-128, 128, size=255).astype(np.int8)
    y = torch.empty(m * n, dtype=torch.int8, device="cuda")
    T.w12_linear_lut(xd, lo, nib, m, n, k, y, md, sd, torch.from_numpy(lut).cuda())
    torch.cuda.synchronize()
    q8 = O.requant_channels(acc, m, n, mant, shift, -127, 127).astype(np.int64)
    assert np.array_equal(y.cpu().numpy(), lut[q8 + 127])
