// The cross-backend gates of kt-runtime (crates/02-runtime/kt-runtime/src/gate.rs:1-140) as library calls: the
// fixed corpus, the bound cases, the equality gate (every backend byte-identical to the first, one SHA-256 per
// backend over every accumulator) and the residency gate (the corpus twice, then two weight matrices of one shape
// interleaved). A backend is a name plus a linear_weights function, so the gates take this library's HIP backend,
// a planted build's, the engine's Portable, or any caller's.
//
// Portable here is the engine's own CPU kernel (kt-core/src/backend.rs:66-160: i64 dot products, wrapping as the
// reference's release build, rows x out split over threads). It is the gates' reference and nothing else: the HIP
// backend never hands a call to it.
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "kt_hip.h"

namespace {

constexpr int32_t WLEVELS = 265720;  // layers.rs:16

// ---- SHA-256 (FIPS 180-4) ----------------------------------------------------------------------------------------
struct Sha256 {
    uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a, 0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    uint8_t buf[64];
    size_t fill = 0;
    uint64_t bytes = 0;

    static uint32_t rotr(uint32_t v, int n) { return (v >> n) | (v << (32 - n)); }
    void block(const uint8_t* p) {
        static const uint32_t K[64] = {
            0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
            0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
            0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
            0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
            0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
            0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
            0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
            0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};
        uint32_t w[64];
        for (int i = 0; i < 16; i++)
            w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 | (uint32_t)p[4 * i + 2] << 8 | p[4 * i + 3];
        for (int i = 16; i < 64; i++) {
            const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
        for (int i = 0; i < 64; i++) {
            const uint32_t t1 = hh + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + K[i] + w[i];
            const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
            hh = g, g = f, f = e, e = d + t1, d = c, c = b, b = a, a = t1 + t2;
        }
        h[0] += a, h[1] += b, h[2] += c, h[3] += d, h[4] += e, h[5] += f, h[6] += g, h[7] += hh;
    }
    void update(const void* data, size_t n) {
        const uint8_t* p = (const uint8_t*)data;
        bytes += n;
        while (n > 0) {
            const size_t take = std::min(n, 64 - fill);
            memcpy(buf + fill, p, take);
            fill += take, p += take, n -= take;
            if (fill == 64) block(buf), fill = 0;
        }
    }
    std::string hex() {
        const uint64_t bits = bytes * 8;
        const uint8_t one = 0x80, zero = 0;
        update(&one, 1);
        while (fill != 56) update(&zero, 1);
        uint8_t len[8];
        for (int i = 0; i < 8; i++) len[i] = (uint8_t)(bits >> (56 - 8 * i));
        update(len, 8);
        char out[65];
        for (int i = 0; i < 8; i++) snprintf(out + 8 * i, 9, "%08x", h[i]);
        return std::string(out, 64);
    }
};

// One LCG stream of codes uniform in +-WLEVELS (gate.rs:29-36).
struct Lcg {
    uint64_t s;
    int32_t next() {
        s = s * 6364136223846793005ULL + 1442695040888963407ULL;
        return (int32_t)((s >> 33) % (2 * (uint64_t)WLEVELS + 1)) - WLEVELS;
    }
    std::vector<int32_t> codes(size_t n) {
        std::vector<int32_t> v(n);
        for (auto& c : v) c = next();
        return v;
    }
};

struct OwnedCase {
    std::string label;
    uint64_t id;
    size_t rows, out, k;
    std::vector<int32_t> x, w;
};

std::mutex g_mu;
std::vector<OwnedCase> g_corpus, g_bounds;
std::vector<kt_gate_case> g_corpus_view, g_bounds_view;

kt_gate_case view_of(const OwnedCase& c) {
    kt_gate_case v{};
    v.label = c.label.c_str();
    v.id = c.id;
    v.rows = c.rows, v.out = c.out, v.k = c.k;
    v.x = c.x.data(), v.w = c.w.data();
    return v;
}

// gate.rs:26-58: six seeded cases (tails no SIMD width divides, a long dot, a threaded fill), then the extremes.
void build_corpus() {
    if (!g_corpus.empty()) return;
    Lcg st{0x50320b00ULL};
    const struct {
        const char* label;
        size_t rows, out, k;
    } shapes[] = {{"k=1", 1, 1, 1},       {"odd tail", 3, 5, 7},           {"k=33", 2, 17, 33},
                  {"k=1023", 4, 64, 1023}, {"k=4099 (long)", 1, 9, 4099}, {"threaded 8\xc3\x97" "512\xc3\x97" "2048", 8, 512, 2048}};
    for (const auto& s : shapes) {
        OwnedCase c{s.label, kt_hip_weight_id_fresh(), s.rows, s.out, s.k, {}, {}};
        c.x = st.codes(s.rows * s.k);
        c.w = st.codes(s.out * s.k);
        g_corpus.push_back(std::move(c));
    }
    {  // every product is +-WLEVELS^2
        const size_t k = 1027;
        OwnedCase c{"extremes \xc2\xb1WLEVELS", kt_hip_weight_id_fresh(), 2, 3, k, {}, {}};
        for (size_t i = 0; i < 2 * k; i++) c.x.push_back(i % 3 == 0 ? -WLEVELS : WLEVELS);
        for (size_t i = 0; i < 3 * k; i++) c.w.push_back(i % 2 == 0 ? WLEVELS : -WLEVELS);
        g_corpus.push_back(std::move(c));
    }
    {
        OwnedCase c{"all +WLEVELS", kt_hip_weight_id_fresh(), 4, 4, 2048, std::vector<int32_t>(4 * 2048, WLEVELS), {}};
        c.w = c.x;
        g_corpus.push_back(std::move(c));
    }
    for (const auto& c : g_corpus) g_corpus_view.push_back(view_of(c));
}

// The bound cases: the reference's flush_case (gate.rs:60-69: the smallest k beyond one int32 flush of its digit
// backend, every code +WLEVELS against a +WLEVELS and a -WLEVELS row), then this backend's own: one 256-deep chunk
// past its int32 flush bound with every digit of every plane at -128, the largest magnitude a digit product adds,
// for 1-plane and 3-plane codes (an unflushed accumulator wraps on each).
void build_bounds() {
    if (!g_bounds.empty()) return;
    const size_t kt_flush = (size_t)(2147483647LL / (16 * 40 * 40)), ref_k = (kt_flush + 1) * 16;
    {
        OwnedCase c{"k beyond one int32 flush", kt_hip_weight_id_fresh(), 1, 2, ref_k,
                    std::vector<int32_t>(ref_k, WLEVELS), {}};
        c.w.assign(ref_k, WLEVELS);
        c.w.insert(c.w.end(), ref_k, -WLEVELS);
        g_bounds.push_back(std::move(c));
    }
    const struct {
        int planes;
        int32_t code;
        const char* label;
    } own[] = {{1, -128, "k past the 1-plane flush, digits -128"}, {3, -8421504, "k past the 3-plane flush, digits -128"}};
    for (const auto& o : own) {
        const size_t k = (size_t)kt_hip_flush_k(o.planes, o.planes) + 256;
        OwnedCase c{o.label, kt_hip_weight_id_fresh(), 1, 2, k, std::vector<int32_t>(k, o.code), {}};
        c.w.assign(k, o.code);
        c.w.insert(c.w.end(), k, -o.code);
        g_bounds.push_back(std::move(c));
    }
    for (const auto& c : g_bounds) g_bounds_view.push_back(view_of(c));
}

// Portable::linear (backend.rs:133-160): y[r, o] = sum_i x[r, i] w[o, i] in wrapping i64.
void portable(const int32_t* x, const int32_t* w, size_t rows, size_t out, size_t k, int64_t* y) {
    const size_t n = rows * out;
    if (n == 0) return;
    const double work = (double)n * (double)k;
    size_t t = std::min<size_t>(std::max<unsigned>(1, std::thread::hardware_concurrency()), 16);
    t = std::max<size_t>(1, std::min<size_t>({t, n, (size_t)(work / (1 << 20)) + 1}));
    auto run = [&](size_t lo, size_t hi) {
        for (size_t e = lo; e < hi; e++) {
            const int32_t* a = x + (e / out) * k;
            const int32_t* b = w + (e % out) * k;
            uint64_t s = 0;
            for (size_t i = 0; i < k; i++) s += (uint64_t)((int64_t)a[i] * (int64_t)b[i]);
            y[e] = (int64_t)s;
        }
    };
    if (t == 1) return run(0, n);
    std::vector<std::thread> pool;
    const size_t chunk = (n + t - 1) / t;
    for (size_t lo = 0; lo < n; lo += chunk) pool.emplace_back(run, lo, std::min(n, lo + chunk));
    for (auto& th : pool) th.join();
}

int portable_fn(void*, const int32_t* x, uint64_t, const int32_t* w, size_t rows, size_t out, size_t k, int64_t* y) {
    portable(x, w, rows, out, k, y);
    return 0;
}

int hip_fn(void* ctx, const int32_t* x, uint64_t id, const int32_t* w, size_t rows, size_t out, size_t k,
           int64_t* y) {
    return kt_hip_linear_weights((kt_hip_backend*)ctx, x, id, w, rows, out, k, y);
}

void set_name(char* dst, const char* src) {
    strncpy(dst, src, KT_GATE_NAME_LEN - 1);
    dst[KT_GATE_NAME_LEN - 1] = 0;
}

int call(const kt_gate_backend* b, const kt_gate_case& c, std::vector<int64_t>& y) {
    y.assign(c.rows * c.out, 0);
    return b->linear_weights(b->ctx, c.x, c.id, c.w, c.rows, c.out, c.k, y.data());
}

}  // namespace

extern "C" {

size_t kt_hip_gate_corpus(const kt_gate_case** cases) {
    std::lock_guard<std::mutex> g(g_mu);
    build_corpus();
    if (cases) *cases = g_corpus_view.data();
    return g_corpus_view.size();
}

size_t kt_hip_gate_bound_cases(const kt_gate_case** cases) {
    std::lock_guard<std::mutex> g(g_mu);
    build_bounds();
    if (cases) *cases = g_bounds_view.data();
    return g_bounds_view.size();
}

int kt_hip_gate_portable(kt_gate_backend* out) {
    if (!out) return KT_GATE_EINVAL;
    memset(out, 0, sizeof(*out));
    set_name(out->name, "portable");
    out->linear_weights = portable_fn;
    return 0;
}

int kt_hip_gate_backend(kt_hip_backend* b, kt_gate_backend* out) {
    if (!b || !out) return KT_GATE_EINVAL;
    memset(out, 0, sizeof(*out));
    const int e = kt_hip_name(b, out->name, KT_GATE_NAME_LEN);
    if (e) return e;
    out->linear_weights = hip_fn;
    out->ctx = b;
    return 0;
}

int kt_hip_portable_linear(const int32_t* x, const int32_t* w, size_t rows, size_t out, size_t k, int64_t* y) {
    if ((rows * out > 0 && (!y || (k > 0 && (!x || !w))))) return KT_GATE_EINVAL;
    portable(x, w, rows, out, k, y);
    return 0;
}

int kt_hip_equality_gate(const kt_gate_backend* backends, size_t n, const kt_gate_case* cases, size_t ncases,
                         kt_gate_report* reports) {
    if (!backends || n == 0 || !cases || ncases == 0 || ncases > 64 || !reports) return KT_GATE_EINVAL;
    std::vector<std::vector<int64_t>> ref(ncases);
    bool all_same = true;
    for (size_t b = 0; b < n; b++) {
        kt_gate_report& r = reports[b];
        memset(&r, 0, sizeof(r));
        set_name(r.backend, backends[b].name);
        Sha256 h;
        std::vector<int64_t> y;
        for (size_t c = 0; c < ncases; c++) {
            const int e = call(&backends[b], cases[c], y);
            if (e && !r.error) r.error = e;
            if (e) y.assign(cases[c].rows * cases[c].out, 0);
            h.update(y.data(), y.size() * sizeof(int64_t));  // little-endian i64, as the reference hashes them
            if (b == 0) ref[c] = e ? std::vector<int64_t>() : y;
            if (e || y != ref[c]) r.diverged |= 1ULL << c;
        }
        memcpy(r.hash, h.hex().c_str(), 65);
        all_same &= r.diverged == 0;
    }
    return all_same ? 0 : KT_GATE_DIVERGED;
}

int kt_hip_residency_gate(const kt_gate_backend* b, const kt_gate_case* cases, size_t ncases, char* msg,
                          size_t len) {
    if (!b || !cases || (msg && len == 0)) return KT_GATE_EINVAL;
    auto fail = [&](const std::string& m) {
        if (msg) snprintf(msg, len, "%s", m.c_str());
        return KT_GATE_DIVERGED;
    };
    std::vector<int64_t> got, want;
    for (int pass = 1; pass <= 2; pass++)
        for (size_t c = 0; c < ncases; c++) {
            const kt_gate_case& cs = cases[c];
            const int e = call(b, cs, got);
            want.assign(cs.rows * cs.out, 0);
            portable(cs.x, cs.w, cs.rows, cs.out, cs.k, want.data());
            if (e || got != want)
                return fail(std::string(b->name) + ": pass " + std::to_string(pass) + ", case '" + cs.label +
                            "' differs" + (e ? " (error " + std::to_string(e) + ")" : ""));
        }
    // two weight matrices of one shape (4 x 1023 against 64 x 1023), interleaved four times
    std::vector<int32_t> x;
    for (size_t c = 0; c < ncases; c++)
        if (!strcmp(cases[c].label, "k=1023") && cases[c].rows == 4 && cases[c].k == 1023)
            x.assign(cases[c].x, cases[c].x + 4 * 1023);
    if (x.empty()) x = Lcg{7}.codes(4 * 1023);
    const uint64_t ids[2] = {kt_hip_weight_id_fresh(), kt_hip_weight_id_fresh()};
    const std::vector<int32_t> twins[2] = {Lcg{11}.codes(64 * 1023), Lcg{12}.codes(64 * 1023)};
    for (int round = 0; round < 4; round++)
        for (int i = 0; i < 2; i++) {
            kt_gate_case cs{"twin", ids[i], 4, 64, 1023, x.data(), twins[i].data()};
            const int e = call(b, cs, got);
            want.assign(4 * 64, 0);
            portable(x.data(), twins[i].data(), 4, 64, 1023, want.data());
            if (e || got != want)
                return fail(std::string(b->name) + ": twin " + std::to_string(i) + " of one shape differs in round " +
                            std::to_string(round));
        }
    if (msg) msg[0] = 0;
    return 0;
}

}  // extern "C"
