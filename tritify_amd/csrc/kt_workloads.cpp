// Host-side generators of the benchmark workloads' synthetic inputs (integer-only, identical on every machine), for
// the shapes where numpy is too slow: config 3's decoder weights, config 4's 129 experts and config 5's image. The
// stream is the reference's LCG, s <- s * 6364136223846793005 + 1442695040888963407 mod 2^64, drawn as s >> 33
// (apps/kt-demo/src/main.rs:19-22). tritify_amd/workloads.py holds the same definitions in numpy; the tests check
// that both agree with each other and with the committed fixture hashes. No GPU is used here.

#include <stddef.h>
#include <stdint.h>

#include <thread>
#include <vector>

#include "kt_hip.h"

namespace {

constexpr uint64_t LCG_A = 6364136223846793005ULL, LCG_C = 1442695040888963407ULL;

inline uint64_t lcg(uint64_t& s) {
    s = s * LCG_A + LCG_C;
    return s;
}

// The state after n steps from s: the affine map (A, C)^n applied by squaring.
uint64_t lcg_jump(uint64_t s, uint64_t n) {
    uint64_t a = LCG_A, c = LCG_C, ja = 1, jc = 0;
    while (n) {
        if (n & 1) ja = ja * a, jc = jc * a + c;
        c = c * a + c, a = a * a;
        n >>= 1;
    }
    return s * ja + jc;
}

// Split [0, n) over the host cores; f(begin, end) per part.
template <class F>
void parallel_for(size_t n, size_t grain, F f) {
    size_t hw = std::thread::hardware_concurrency();
    size_t parts = n / grain;
    if (parts > hw) parts = hw;
    if (parts <= 1) {
        f((size_t)0, n);
        return;
    }
    std::vector<std::thread> th;
    const size_t chunk = (n + parts - 1) / parts;
    for (size_t p = 1; p < parts; p++) {
        const size_t b = p * chunk, e = b + chunk < n ? b + chunk : n;
        if (b < e) th.emplace_back(f, b, e);
    }
    f((size_t)0, chunk < n ? chunk : n);
    for (auto& t : th) t.join();
}

uint64_t isqrt64(uint64_t n) {
    if (n < 2) return n;
    uint64_t x = (uint64_t)1 << ((64 - __builtin_clzll(n) + 1) / 2);
    for (;;) {
        const uint64_t y = (x + n / x) >> 1;
        if (y >= x) return x;
        x = y;
    }
}

int bits128(unsigned __int128 v) {
    int b = 0;
    while (v) b++, v >>= 1;
    return b;
}

}  // namespace

extern "C" {

void kt_hip_gen_w12(uint64_t seed, size_t n, int32_t* out) {
    const uint64_t s0 = seed ^ 0x9E3779B97F4A7C15ULL;
    parallel_for(n, 1 << 20, [&](size_t b, size_t e) {
        uint64_t s = lcg_jump(s0, b);
        for (size_t i = b; i < e; i++) out[i] = (int32_t)((lcg(s) >> 33) % 4096) - 2048;
    });
}

void kt_hip_gen_gauss(uint64_t seed, int64_t sigma, int64_t clip, size_t n, int32_t* out) {
    const uint64_t s0 = seed ^ 0xD1B54A32D192ED03ULL;
    parallel_for(n, 1 << 18, [&](size_t b, size_t e) {
        uint64_t s = lcg_jump(s0, 12 * (uint64_t)b);
        for (size_t i = b; i < e; i++) {
            int64_t sum = 0;
            for (int j = 0; j < 12; j++) sum += (int64_t)((lcg(s) >> 33) & 0xFFFF);
            const int64_t t = 2 * sum - 12 * 65535;
            const int64_t mag = ((t < 0 ? -t : t) * sigma + 65536) >> 17;
            int64_t v = t < 0 ? -mag : mag;
            if (clip > 0) v = v > clip ? clip : (v < -clip ? -clip : v);
            out[i] = (int32_t)v;
        }
    });
}

void kt_hip_gen_uniform(uint64_t seed, int64_t lo, int64_t hi, size_t n, int32_t* out) {
    const uint64_t s0 = seed ^ 0x9E3779B97F4A7C15ULL, range = (uint64_t)(hi - lo + 1);
    parallel_for(n, 1 << 20, [&](size_t b, size_t e) {
        uint64_t s = lcg_jump(s0, b);
        for (size_t i = b; i < e; i++) out[i] = (int32_t)((int64_t)((lcg(s) >> 33) % range) + lo);
    });
}

void kt_hip_channel_scales(const int32_t* w, size_t n, size_t k, int64_t sigma, int64_t target, int32_t* mant,
                           int32_t* shift) {
    parallel_for(n, 64, [&](size_t b, size_t e) {
        for (size_t o = b; o < e; o++) {
            uint64_t ss = 0;
            for (size_t c = 0; c < k; c++) ss += (uint64_t)((int64_t)w[o * k + c] * w[o * k + c]);
            const uint64_t root = isqrt64(ss);
            if (root == 0) {
                mant[o] = 0, shift[o] = 0;
                continue;
            }
            // Scale::from_ratio(target, 4 * sigma * root) (kt-int/src/lib.rs:191-212), then an int32 mantissa
            unsigned __int128 num = (unsigned __int128)target, den = (unsigned __int128)(4 * (uint64_t)sigma) * root;
            while (bits128(num) > 64 || bits128(den) > 64) num >>= 1, den >>= 1;
            if (den == 0) den = 1;
            int s = 31 - (bits128(num) - bits128(den));
            unsigned __int128 m;
            if (s >= 0) {
                m = ((num << s) + den / 2) / den;
            } else {
                const unsigned __int128 dd = den << (-s);
                m = (num + dd / 2) / dd;
            }
            while (m >= ((unsigned __int128)1 << 31)) m = (m + 1) >> 1, s -= 1;
            mant[o] = (int32_t)m, shift[o] = s;
        }
    });
}

void kt_hip_gen_quant_rows(uint64_t seed, size_t rows, size_t cols, int32_t* out) {
    const uint64_t s0 = seed ^ 0xD1B54A32D192ED03ULL;
    parallel_for(rows, 16, [&](size_t b, size_t e) {
        uint64_t s = lcg_jump(s0, 12 * (uint64_t)b * cols);
        for (size_t r = b; r < e; r++) {
            int32_t* v = out + r * cols;
            int64_t mx = 0;
            for (size_t c = 0; c < cols; c++) {
                int64_t sum = 0;
                for (int j = 0; j < 12; j++) sum += (int64_t)((lcg(s) >> 33) & 0xFFFF);
                const int64_t t = 2 * sum - 12 * 65535;
                const int64_t mag = ((t < 0 ? -t : t) * (1 << 20) + 65536) >> 17;
                v[c] = (int32_t)(t < 0 ? -mag : mag);
                mx = mag > mx ? mag : mx;
            }
            for (size_t c = 0; c < cols; c++) {
                if (mx == 0) {
                    v[c] = 0;
                    continue;
                }
                const int64_t a = 2047 * (int64_t)v[c], q = (2 * (a < 0 ? -a : a) + mx) / (2 * mx);
                v[c] = (int32_t)(a < 0 ? -q : q);
            }
        }
    });
}

}  // extern "C"
