/*
 * kt_oracle.c -- TEST INFRASTRUCTURE ONLY. A CPU restatement, in plain C, of tritify's exact-integer linear
 * accumulate and the integer arithmetic around it. It is the checker the GPU path is compared with and the timed
 * CPU baseline; it is never part of the product. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.
 *
 * Every function names the reference file:line it restates (paths relative to the tritify repository root).
 * Integer arithmetic only, except the two offline calibration helpers kt_frexp / kt_frexp_scale /
 * kt_scale_from_f64, which restate the reference's offline float code.
 *
 * Pinning (how each part is checked, tests/test_oracle.py):
 *   - lcg, gen_demo, linear_cpu, sha256: kt-demo golden de67ba75... (README.md:74) and the config-1 hashes.
 *   - corpus + linear_cpu + sha256: CORPUS_HASH 781285bb... (kt-runtime/src/tests_cuda.rs:9).
 *   - flush case: closed form k*WLEVELS^2 (kt-runtime/src/gate.rs:61-66).
 *   - split81 / join81: exhaustive over +-WLEVELS, split(+-WLEVELS) = [+-40]*3 (kt-cuda/src/tests.rs:21-34).
 *   - split256 (this build's digit scheme): exhaustive round trip over every code of each plane count's range.
 *   - plane emulator: equals linear_cpu on the corpus; wraps exactly at the flush bound (brute-force i32 model).
 *   - requant / Scale: the reference's doc-test known answers (kt-int/src/lib.rs:35-39, 561-650), closed forms,
 *     and an f64 cross-check within 1 ulp as the reference's own tests do.
 *   - quant_to / requant_dyn: brute force with Python integers on random and edge inputs.
 *   - w12 pack / w12 accumulate: the recombination equals the direct i64 sum (exhaustive over the 4096 codes).
 */
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

typedef __int128 i128;
typedef unsigned __int128 u128;

/* crates/01-engine/kt-core/src/layers.rs:16,18 */
#define WLEVELS 265720LL
#define ACT_LEVELS (1LL << 28)

/* ------------------------------------------------------------------------------------------------------------ */
/* LCG: apps/kt-demo/src/main.rs:19-22 (also gate.rs:32, kt-cuda/src/tests.rs:9-14)                              */
/* ------------------------------------------------------------------------------------------------------------ */
static inline uint64_t lcg(uint64_t* s) {
    *s = *s * 6364136223846793005ULL + 1442695040888963407ULL;
    return *s;
}

uint64_t kt_lcg_next(uint64_t* s) { return lcg(s); }

/* ------------------------------------------------------------------------------------------------------------ */
/* SHA-256 (FIPS 180-4). The reference hashes with sha2 0.10.9 (Cargo.lock); outputs are pinned by the goldens.  */
/* ------------------------------------------------------------------------------------------------------------ */
typedef struct {
    uint32_t h[8];
    uint64_t len;
    uint8_t buf[64];
    size_t nbuf;
} kt_sha256_ctx;

static const uint32_t SHA_K[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};

static inline uint32_t ror(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

static void sha_block(kt_sha256_ctx* c, const uint8_t* p) {
    uint32_t w[64];
    for (int i = 0; i < 16; i++)
        w[i] = ((uint32_t)p[4 * i] << 24) | ((uint32_t)p[4 * i + 1] << 16) | ((uint32_t)p[4 * i + 2] << 8) | p[4 * i + 3];
    for (int i = 16; i < 64; i++) {
        uint32_t s0 = ror(w[i - 15], 7) ^ ror(w[i - 15], 18) ^ (w[i - 15] >> 3);
        uint32_t s1 = ror(w[i - 2], 17) ^ ror(w[i - 2], 19) ^ (w[i - 2] >> 10);
        w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = c->h[0], b = c->h[1], cc = c->h[2], d = c->h[3], e = c->h[4], f = c->h[5], g = c->h[6], h = c->h[7];
    for (int i = 0; i < 64; i++) {
        uint32_t t1 = h + (ror(e, 6) ^ ror(e, 11) ^ ror(e, 25)) + ((e & f) ^ (~e & g)) + SHA_K[i] + w[i];
        uint32_t t2 = (ror(a, 2) ^ ror(a, 13) ^ ror(a, 22)) + ((a & b) ^ (a & cc) ^ (b & cc));
        h = g; g = f; f = e; e = d + t1; d = cc; cc = b; b = a; a = t1 + t2;
    }
    c->h[0] += a; c->h[1] += b; c->h[2] += cc; c->h[3] += d; c->h[4] += e; c->h[5] += f; c->h[6] += g; c->h[7] += h;
}

void kt_sha256_init(kt_sha256_ctx* c) {
    static const uint32_t H0[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                                   0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    memcpy(c->h, H0, sizeof H0);
    c->len = 0;
    c->nbuf = 0;
}

void kt_sha256_update(kt_sha256_ctx* c, const void* data, size_t n) {
    const uint8_t* p = (const uint8_t*)data;
    c->len += n;
    if (c->nbuf) {
        size_t take = 64 - c->nbuf < n ? 64 - c->nbuf : n;
        memcpy(c->buf + c->nbuf, p, take);
        c->nbuf += take; p += take; n -= take;
        if (c->nbuf == 64) { sha_block(c, c->buf); c->nbuf = 0; }
    }
    while (n >= 64) { sha_block(c, p); p += 64; n -= 64; }
    if (n) { memcpy(c->buf, p, n); c->nbuf = n; }
}

void kt_sha256_final(kt_sha256_ctx* c, uint8_t out[32]) {
    uint64_t bits = c->len * 8;
    uint8_t pad = 0x80;
    kt_sha256_update(c, &pad, 1);
    uint8_t z = 0;
    while (c->nbuf != 56) kt_sha256_update(c, &z, 1);
    uint8_t lb[8];
    for (int i = 0; i < 8; i++) lb[i] = (uint8_t)(bits >> (56 - 8 * i));
    kt_sha256_update(c, lb, 8);
    for (int i = 0; i < 8; i++) {
        out[4 * i] = (uint8_t)(c->h[i] >> 24); out[4 * i + 1] = (uint8_t)(c->h[i] >> 16);
        out[4 * i + 2] = (uint8_t)(c->h[i] >> 8); out[4 * i + 3] = (uint8_t)c->h[i];
    }
}

size_t kt_sha256_ctx_size(void) { return sizeof(kt_sha256_ctx); }

/* One-shot hash of a byte buffer. The test hashes of i64/i32 arrays are over their little-endian words, which on
 * x86-64 are the in-memory bytes (apps/kt-demo/src/main.rs:57-63, kt-core/src/verify.rs:35-41). */
void kt_sha256(const void* data, size_t n, uint8_t out[32]) {
    kt_sha256_ctx c;
    kt_sha256_init(&c);
    kt_sha256_update(&c, data, n);
    kt_sha256_final(&c, out);
}

/* ------------------------------------------------------------------------------------------------------------ */
/* The CPU dot variants: crates/01-engine/kt-core/src/backend.rs:66-69 (dot_portable) and                       */
/* crates/02-runtime/kt-runtime/src/cpu.rs:150-177 (the same loop compiled with avx2 / avx512f enabled).         */
/* Release-mode Rust sums wrap on i64 overflow; the sum here is carried in uint64_t to wrap the same way.       */
/* ------------------------------------------------------------------------------------------------------------ */
static inline __attribute__((always_inline)) int64_t dot_loop(const int32_t* a, const int32_t* b, size_t k) {
    uint64_t acc = 0;
    for (size_t i = 0; i < k; i++) acc += (uint64_t)((int64_t)a[i] * (int64_t)b[i]);
    return (int64_t)acc;
}

int64_t kt_dot_portable(const int32_t* a, const int32_t* b, size_t k) { return dot_loop(a, b, k); }

__attribute__((target("avx2"))) int64_t kt_dot_avx2(const int32_t* a, const int32_t* b, size_t k) {
    return dot_loop(a, b, k);
}

__attribute__((target("avx512f"))) int64_t kt_dot_avx512(const int32_t* a, const int32_t* b, size_t k) {
    return dot_loop(a, b, k);
}

typedef int64_t (*dot_fn)(const int32_t*, const int32_t*, size_t);

/* Variant ids: 0 portable, 1 avx2, 2 avx512 (kt-runtime/src/cpu.rs:10-19). Returns 1 if this host can run it. */
int kt_cpu_variant_available(int v) {
    __builtin_cpu_init();
    switch (v) {
        case 0: return 1;
        case 1: return __builtin_cpu_supports("avx2") ? 1 : 0;
        case 2: return __builtin_cpu_supports("avx512f") ? 1 : 0;
        default: return 0;
    }
}

/* The auto rank on x86-64: avx512 > avx2 > portable (kt-runtime/src/lib.rs:93-96). */
int kt_cpu_auto_variant(void) {
    if (kt_cpu_variant_available(2)) return 2;
    if (kt_cpu_variant_available(1)) return 1;
    return 0;
}

static dot_fn variant_fn(int v) {
    switch (v) {
        case 1: return kt_dot_avx2;
        case 2: return kt_dot_avx512;
        default: return kt_dot_portable;
    }
}

/* ------------------------------------------------------------------------------------------------------------ */
/* Thread plan and partition: backend.rs:74-139, layers.rs:41-77 (max_threads / resolve_threads).              */
/* ------------------------------------------------------------------------------------------------------------ */
#define WORK_PER_SPAWN ((size_t)1 << 17) /* backend.rs:74 */
#define SERIAL_BELOW ((size_t)1 << 20)   /* backend.rs:79 */

static size_t g_max_threads = 0; /* layers.rs:48 -- 0 = every core (TRITIFY_THREADS semantics) */

void kt_set_max_threads(size_t n) { g_max_threads = n; }
size_t kt_max_threads(void) { return g_max_threads; }

static size_t host_cores(void) {
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (size_t)n : 1;
}

/* layers.rs:72-77 */
size_t kt_resolve_threads(size_t nblocks) {
    size_t cap = g_max_threads;
    size_t want = cap == 0 ? host_cores() : cap;
    if (want < 1) want = 1;
    size_t nb = nblocks < 1 ? 1 : nblocks;
    return want < nb ? want : nb;
}

/* Integer floor square root of a usize (Rust's usize::isqrt). */
static size_t isqrt_usize(size_t n) {
    if (n < 2) return n;
    size_t x = (size_t)1 << ((64 - __builtin_clzll((unsigned long long)n) + 1) / 2);
    for (;;) {
        size_t y = (x + n / x) >> 1;
        if (y >= x) return x;
        x = y;
    }
}

static size_t sat_mul(size_t a, size_t b) {
    size_t r;
    return __builtin_mul_overflow(a, b, &r) ? SIZE_MAX : r;
}

/* backend.rs:89-94 */
size_t kt_plan_threads(size_t elems, size_t work) {
    if (work < SERIAL_BELOW) return 1;
    size_t t = kt_resolve_threads(elems);
    size_t s = isqrt_usize(work / WORK_PER_SPAWN);
    if (s < t) t = s;
    return t < 1 ? 1 : t;
}

typedef struct {
    const int32_t* x;
    const int32_t* w;
    size_t out, k;
    dot_fn dot;
    int64_t* y;
    size_t start, len;
    int bad; /* a planted partition defect (kt-runtime/src/planted.rs:8-16); 0 = none */
    size_t rows;
} run_arg;

/* Element i of the flat rows x out buffer is dot(x[i / out], w[i % out]) (backend.rs:129-138). */
static void* run_worker(void* p) {
    run_arg* a = (run_arg*)p;
    for (size_t e = 0; e < a->len; e++) {
        size_t i = a->start + e;
        const int32_t *xr, *wr;
        if (a->bad == 3) { /* SwappedIndex: (i % rows, i / rows) */
            xr = a->x + (i % a->rows) * a->k;
            wr = a->w + (i / a->rows) * a->k;
        } else {
            xr = a->x + (i / a->out) * a->k;
            wr = a->w + (i % a->out) * a->k;
        }
        a->y[e] = a->dot(xr, wr, a->k);
    }
    return NULL;
}

/* fill_partitioned (backend.rs:101-127) specialised to the linear accumulate, with the planted partitions of
 * kt-runtime/src/planted.rs:28-59 (bad = 1 FloorOffsets, 2 DropLastRun, 3 SwappedIndex; threads forced when > 0). */
static void fill_linear(const int32_t* x, const int32_t* w, size_t rows, size_t out, size_t k, dot_fn dot,
                        int64_t* y, size_t threads, int bad) {
    size_t len = rows * out;
    if (len == 0) return;
    size_t t = threads < 1 ? 1 : (threads > len ? len : threads);
    size_t chunk = (len + t - 1) / t;
    size_t runs = (len + chunk - 1) / chunk;
    if (runs == 1 && bad == 0) {
        run_arg a = {x, w, out, k, dot, y, 0, len, 0, rows};
        run_worker(&a);
        return;
    }
    run_arg* args = (run_arg*)calloc(runs, sizeof(run_arg));
    pthread_t* th = (pthread_t*)calloc(runs, sizeof(pthread_t));
    for (size_t ci = 0; ci < runs; ci++) {
        size_t at = ci * chunk; /* a run's first index is the length before it */
        size_t n = len - at < chunk ? len - at : chunk;
        size_t start = bad == 1 ? ci * (len / t) : at;
        args[ci] = (run_arg){x, w, out, k, dot, y + at, start, n, bad, rows};
    }
    /* the calling thread takes the first run; the others are spawned (backend.rs:114-126) */
    for (size_t ci = 1; ci < runs; ci++) {
        if (bad == 2 && ci == runs - 1) continue; /* DropLastRun */
        pthread_create(&th[ci], NULL, run_worker, &args[ci]);
    }
    if (!(bad == 2 && runs == 1)) run_worker(&args[0]);
    for (size_t ci = 1; ci < runs; ci++) {
        if (bad == 2 && ci == runs - 1) continue;
        pthread_join(th[ci], NULL);
    }
    free(args);
    free(th);
}

/* linear_cpu (backend.rs:133-140): the threaded CPU driver on one dot variant. y is rows*out, caller-owned. */
void kt_linear_cpu(const int32_t* x, const int32_t* w, size_t rows, size_t out, size_t k, int variant, int64_t* y) {
    size_t threads = kt_plan_threads(rows * out, sat_mul(sat_mul(rows, out), k));
    fill_linear(x, w, rows, out, k, variant_fn(variant), y, threads, 0);
}

/* The same with an explicit worker count (tests_partition.rs:31-38 drives fill_partitioned this way). */
void kt_linear_cpu_threads(const int32_t* x, const int32_t* w, size_t rows, size_t out, size_t k, int variant,
                           size_t threads, int64_t* y) {
    fill_linear(x, w, rows, out, k, variant_fn(variant), y, threads, 0);
}

/* kt-runtime/src/planted.rs:28-59: a planted partition. threads == 0 uses the engine's own plan. */
void kt_linear_planted_partition(const int32_t* x, const int32_t* w, size_t rows, size_t out, size_t k, int bad,
                                 size_t threads, int64_t* y) {
    size_t planned = kt_plan_threads(rows * out, sat_mul(sat_mul(rows, out), k));
    size_t t = threads ? threads : planned;
    fill_linear(x, w, rows, out, k, kt_dot_portable, y, t, bad);
}

/* kt-runtime/src/tests.rs:9-17: the two planted dot kernels the gate must catch. variant 10 = wrapping i32
 * accumulator, 11 = f32 accumulator. Serial (they are firing controls, not timed). */
void kt_linear_planted_dot(const int32_t* x, const int32_t* w, size_t rows, size_t out, size_t k, int which,
                           int64_t* y) {
    for (size_t r = 0; r < rows; r++)
        for (size_t o = 0; o < out; o++) {
            const int32_t* a = x + r * k;
            const int32_t* b = w + o * k;
            if (which == 10) {
                uint32_t s = 0;
                for (size_t i = 0; i < k; i++) s += (uint32_t)a[i] * (uint32_t)b[i];
                y[r * out + o] = (int64_t)(int32_t)s;
            } else {
                float s = 0.0f;
                for (size_t i = 0; i < k; i++) s += (float)a[i] * (float)b[i];
                y[r * out + o] = (int64_t)s;
            }
        }
}

/* ------------------------------------------------------------------------------------------------------------ */
/* Generators                                                                                                     */
/* ------------------------------------------------------------------------------------------------------------ */

/* apps/kt-demo/src/main.rs:23-28: one stream seeded seed ^ 0x9E3779B97F4A7C15; qx (m*k, in [-127,127]) first,
 * then qw (n*k, in {-1,0,1}). */
void kt_gen_demo(size_t m, size_t n, size_t k, uint64_t seed, int32_t* qx, int32_t* qw) {
    uint64_t s = seed ^ 0x9E3779B97F4A7C15ULL;
    for (size_t i = 0; i < m * k; i++) qx[i] = (int32_t)((lcg(&s) >> 33) % 255) - 127;
    for (size_t i = 0; i < n * k; i++) qw[i] = (int32_t)((lcg(&s) >> 33) % 3) - 1;
}

/* Codes uniform in +-WLEVELS from a stream (gate.rs:29-36; kt-cuda/src/tests.rs:9-15 with its own seed). */
void kt_gen_wlevels(uint64_t* state, size_t n, int32_t* out) {
    for (size_t i = 0; i < n; i++) out[i] = (int32_t)((lcg(state) >> 33) % (2 * (uint64_t)WLEVELS + 1)) - (int32_t)WLEVELS;
}

/* The benchmark config-2 generators (this build's own definitions; integer only, no libm):
 *  - weights: uniform signed 12-bit codes in [-2048, 2047]: ((s >> 33) % 4096) - 2048 on a stream seeded
 *    seed ^ 0x9E3779B97F4A7C15 (the kt-demo convention, main.rs:24);
 *  - activations: round(N(0, sigma)) clipped to +-127, where N(0,1) is the Irwin-Hall sum of 12 uniforms
 *    u_i = (s >> 33) & 0xFFFF (variance 12 * (2^32 - 1)/12 ~ 2^32, so std 2^16) on a stream seeded
 *    seed ^ 0xD1B54A32D192ED03; x = round_half_away((sum - 6*65535.5) * sigma / 65536), done in integers as
 *    t = 2*sum - 12*65535 (= 2*(sum - 6*65535.5)), x = sign(t) * ((|t|*sigma + 65536) >> 17). */
void kt_gen_w12(uint64_t seed, size_t n, int32_t* out) {
    uint64_t s = seed ^ 0x9E3779B97F4A7C15ULL;
    for (size_t i = 0; i < n; i++) out[i] = (int32_t)((lcg(&s) >> 33) % 4096) - 2048;
}

void kt_gen_act_gauss(uint64_t seed, int64_t sigma, size_t n, int32_t* out) {
    uint64_t s = seed ^ 0xD1B54A32D192ED03ULL;
    for (size_t i = 0; i < n; i++) {
        int64_t sum = 0;
        for (int j = 0; j < 12; j++) sum += (int64_t)((lcg(&s) >> 33) & 0xFFFF);
        int64_t t = 2 * sum - 12 * 65535;
        int64_t mag = ((t < 0 ? -t : t) * sigma + 65536) >> 17;
        int64_t v = t < 0 ? -mag : mag;
        if (v > 127) v = 127;
        if (v < -127) v = -127;
        out[i] = (int32_t)v;
    }
}

/* int8 activations uniform in [-127, 127] (configs 4 and 5 inputs), stream seed ^ 0x9E3779B97F4A7C15. */
void kt_gen_act_uniform(uint64_t seed, size_t n, int32_t* out) {
    uint64_t s = seed ^ 0x9E3779B97F4A7C15ULL;
    for (size_t i = 0; i < n; i++) out[i] = (int32_t)((lcg(&s) >> 33) % 255) - 127;
}

/* ------------------------------------------------------------------------------------------------------------ */
/* Digits                                                                                                         */
/* ------------------------------------------------------------------------------------------------------------ */

/* kt-cuda/src/digits.rs:40-53: three balanced base-81 digits, low first. Returns 0 outside +-WLEVELS. */
int kt_split81(int32_t v, int8_t d[3]) {
    if ((v < 0 ? -(int64_t)v : (int64_t)v) > WLEVELS) return 0;
    int32_t r = v;
    for (int i = 0; i < 3; i++) {
        int32_t lo = (((r + 40) % 81) + 81) % 81 - 40; /* rem_euclid */
        d[i] = (int8_t)lo;
        r = (r - lo) / 81;
    }
    return r == 0;
}

/* kt-cuda/src/digits.rs:69-71 */
int64_t kt_join81(const int8_t d[3]) { return (int64_t)d[0] + 81 * ((int64_t)d[1] + 81 * (int64_t)d[2]); }

/* This build's digit scheme: P balanced base-256 digits d_i in [-128, 127], v = sum 256^i d_i, low first.
 * d = ((r + 128) mod 256) - 128, r = (r - d) / 256. Returns 0 if P digits do not reach v. `wrong_carry`
 * truncates r / 256 instead (the analogue of the reference's WrongCarry plant, digits.rs:54-66). */
int kt_split256(int64_t v, int p, int wrong_carry, int8_t* d) {
    int64_t r = v;
    for (int i = 0; i < p; i++) {
        int64_t lo = (((r + 128) % 256) + 256) % 256 - 128;
        d[i] = (int8_t)lo;
        r = wrong_carry ? r / 256 : (r - lo) / 256;
    }
    return wrong_carry ? 1 : r == 0;
}

int64_t kt_join256(const int8_t* d, int p) {
    int64_t v = 0;
    for (int i = p - 1; i >= 0; i--) v = v * 256 + d[i];
    return v;
}

/* The fewest balanced base-256 digits (1, 2, 3, 4 or 5) that hold every code of a slice. */
int kt_planes_for(const int32_t* v, size_t n) {
    int64_t lo = 0, hi = 0;
    for (size_t i = 0; i < n; i++) {
        if (v[i] < lo) lo = v[i];
        if (v[i] > hi) hi = v[i];
    }
    int64_t mn = -128, mx = 127;
    for (int p = 1; p <= 5; p++) {
        if (lo >= mn && hi <= mx) return p;
        mn = mn * 256 - 128; /* one more digit: 256*range + [-128, 127] */
        mx = mx * 256 + 127;
    }
    return 5;
}

/* Plane layout of the device operands: [plane][row][kp] int8, kp = k rounded up to 64, zero padding. */
void kt_pack_planes(const int32_t* codes, size_t rows, size_t k, int p, int wrong_carry, int8_t* out) {
    size_t kp = (k + 63) / 64 * 64;
    memset(out, 0, (size_t)p * rows * kp);
    int8_t d[5];
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < k; c++) {
            kt_split256(codes[r * k + c], p, wrong_carry, d);
            for (int i = 0; i < p; i++) out[((size_t)i * rows + r) * kp + c] = d[i];
        }
}

/* The i32-accumulator flush interval of a (px, pw) plane product: the most pairs one group sums is min(px,pw),
 * each term at most 128*128 = 16384 in magnitude, so an int32 group sum is safe for
 * floor((2^31 - 1) / (min(px,pw) * 16384)) k-values; rounded down to the 256-value chunk granularity. */
int64_t kt_flush_k(int px, int pw) {
    int64_t n = px < pw ? px : pw;
    int64_t f = 2147483647LL / (n * 16384);
    return f / 256 * 256;
}

/* The plane product on the CPU, step for step (the analogue of kt-cuda/src/host.rs:53-84): per group g = i + j an
 * int32 sum that wraps like the device accumulator, added into i64 as 256^g * C_g (wrapping) every flush_k
 * k-values. Planted knobs: flush_k <= 0 never flushes (NoFlush); drop_top skips the top group (the (px-1,pw-1)
 * pair, the analogue of DropPlane22); wrong_carry splits x with the truncating carry (WrongCarry). */
void kt_emu_linear(const int32_t* x, const int32_t* w, size_t rows, size_t out, size_t k, int px, int pw,
                   int64_t flush_k, int drop_top, int wrong_carry, int64_t* y) {
    int ng = px + pw - 1;
    int8_t* xd = (int8_t*)malloc((size_t)px * (k ? k : 1));
    int8_t* wd = (int8_t*)malloc((size_t)pw * (k ? k : 1));
    int8_t d[5];
    for (size_t r = 0; r < rows; r++) {
        for (size_t c = 0; c < k; c++) {
            kt_split256(x[r * k + c], px, wrong_carry, d);
            for (int i = 0; i < px; i++) xd[(size_t)i * k + c] = d[i];
        }
        for (size_t o = 0; o < out; o++) {
            for (size_t c = 0; c < k; c++) {
                kt_split256(w[o * k + c], pw, 0, d);
                for (int j = 0; j < pw; j++) wd[(size_t)j * k + c] = d[j];
            }
            uint64_t acc = 0;
            size_t c0 = 0;
            while (c0 < k) {
                size_t c1 = (flush_k <= 0 || (size_t)flush_k >= k - c0) ? k : c0 + (size_t)flush_k;
                uint32_t s[9] = {0};
                for (size_t c = c0; c < c1; c++)
                    for (int i = 0; i < px; i++)
                        for (int j = 0; j < pw; j++)
                            s[i + j] += (uint32_t)((int32_t)xd[(size_t)i * k + c] * (int32_t)wd[(size_t)j * k + c]);
                for (int g = 0; g < ng; g++) {
                    if (drop_top && g == ng - 1) continue;
                    if (8 * g >= 64) continue; /* 256^g = 0 mod 2^64 */
                    acc += (uint64_t)((int64_t)(int32_t)s[g]) << (8 * g);
                }
                c0 = c1;
            }
            y[r * out + o] = (int64_t)acc;
        }
    }
    free(xd);
    free(wd);
}

/* ------------------------------------------------------------------------------------------------------------ */
/* kt-int: crates/00-kernels/kt-int/src/lib.rs                                                                    */
/* ------------------------------------------------------------------------------------------------------------ */

/* lib.rs:46-60 */
double kt_frexp(double x, int32_t* e_out) {
    if (x == 0.0 || !(x - x == 0.0)) { *e_out = 0; return x; }
    uint64_t bits;
    memcpy(&bits, &x, 8);
    int32_t ef = (int32_t)((bits >> 52) & 0x7ff);
    if (ef == 0) {
        int32_t e;
        double m = kt_frexp(x * 9007199254740992.0, &e);
        *e_out = e - 53;
        return m;
    }
    *e_out = ef - 1022;
    uint64_t mb = (bits & ~(0x7ffULL << 52)) | (1022ULL << 52);
    double m;
    memcpy(&m, &mb, 8);
    return m;
}

/* Rust's f64::round: half away from zero (no libm: the value is at most 2^53 here, so adding 0.5 and truncating
 * in the integer domain is exact for the magnitudes that arise; ties go away from zero). */
static int64_t round_away(double v) {
    double a = v < 0 ? -v : v;
    int64_t t = (int64_t)a;                   /* trunc */
    if (a - (double)t >= 0.5) t += 1;         /* exact: a - t is exact for a < 2^52 */
    return v < 0 ? -t : t;
}

/* lib.rs:65-73 */
void kt_frexp_scale(double scale, uint32_t mant_bits, int64_t* mant, int32_t* shift) {
    if (!(scale > 0.0 && scale - scale == 0.0)) { *mant = 0; *shift = 0; return; }
    int32_t e;
    double m = kt_frexp(scale, &e);
    *mant = round_away(m * (double)(1ULL << mant_bits));
    *shift = (int32_t)mant_bits - e;
}

/* lib.rs:78-86: round(accum * mant / 2^shift), i128 product, round half away from zero. */
int64_t kt_requant(int64_t accum, int64_t mant, int32_t shift) {
    i128 prod = (i128)accum * (i128)mant;
    if (shift <= 0) return (int64_t)(prod << (-shift));
    i128 half = (i128)1 << (shift - 1);
    i128 r = prod >= 0 ? (prod + half) >> shift : -(((-prod) + half) >> shift);
    return (int64_t)r;
}

typedef struct {
    int64_t mant;
    int32_t shift;
} kt_scale;

static int bits_u128(u128 x) {
    if (x == 0) return 0;
    uint64_t hi = (uint64_t)(x >> 64);
    if (hi) return 128 - __builtin_clzll(hi);
    return 64 - __builtin_clzll((uint64_t)x);
}

/* lib.rs:191-212 (num, den as (hi, lo) u64 pairs so the C ABI carries u128 values). */
kt_scale kt_scale_from_ratio(uint64_t num_hi, uint64_t num_lo, uint64_t den_hi, uint64_t den_lo) {
    u128 num = ((u128)num_hi << 64) | num_lo, den = ((u128)den_hi << 64) | den_lo;
    kt_scale z = {0, 0};
    if (num == 0) return z;
    if (den == 0) abort(); /* the reference asserts den > 0 */
    while (bits_u128(num) > 64 || bits_u128(den) > 64) { num >>= 1; den >>= 1; }
    if (den == 0) den = 1;
    int s = 31 - (bits_u128(num) - bits_u128(den));
    u128 mant;
    if (s >= 0) {
        u128 numer = num << s;
        mant = (numer + den / 2) / den;
    } else {
        u128 dd = den << (-s);
        mant = (num + dd / 2) / dd;
    }
    kt_scale r = {(int64_t)mant, s};
    return r;
}

/* lib.rs:215-222 */
kt_scale kt_scale_from_f64(double x) {
    kt_scale z = {0, 0};
    if (!(x > 0.0 && x - x == 0.0)) return z;
    int32_t e;
    double m = kt_frexp(x, &e);
    kt_scale r = {round_away(m * (double)(1ULL << 31)), 31 - e};
    return r;
}

/* lib.rs:227-248 */
int kt_scale_ge(kt_scale a, kt_scale o) {
    if (a.mant == 0) return o.mant == 0;
    if (o.mant == 0) return 1;
    u128 ma = (u128)a.mant, mb = (u128)o.mant;
    int d = o.shift - a.shift;
    if (d >= 0) {
        if ((uint32_t)d + (uint32_t)bits_u128(ma) > 127) return 1;
        return (ma << d) >= mb;
    }
    uint32_t e = (uint32_t)(-d);
    if (e + (uint32_t)bits_u128(mb) > 127) return 0;
    return ma >= (mb << e);
}

/* lib.rs:252-258 */
kt_scale kt_scale_mul(kt_scale a, kt_scale o) {
    kt_scale z = {0, 0};
    if (a.mant == 0 || o.mant == 0) return z;
    u128 p = (u128)a.mant * (u128)o.mant;
    kt_scale q = kt_scale_from_ratio((uint64_t)(p >> 64), (uint64_t)p, 0, 1);
    q.shift += a.shift + o.shift;
    return q;
}

/* lib.rs:261-272 */
int64_t kt_scale_apply(kt_scale a, int64_t value) {
    if (a.mant == 0) return 0;
    return kt_requant(value, a.mant, a.shift);
}

/* lib.rs:275-280 */
kt_scale kt_scale_recip(kt_scale a) {
    if (a.mant == 0) abort();
    kt_scale r = kt_scale_from_ratio(0, 1ULL << 40, 0, (uint64_t)a.mant);
    kt_scale out = {r.mant, r.shift - a.shift + 40};
    return out;
}

/* lib.rs:285-303 */
kt_scale kt_scale_add(kt_scale a, kt_scale o) {
    if (a.mant == 0) return o;
    if (o.mant == 0) return a;
    int s = a.shift > o.shift ? a.shift : o.shift;
    uint32_t da = (uint32_t)(s - a.shift), db = (uint32_t)(s - o.shift);
    if (da >= 96) return a;
    if (db >= 96) return o;
    u128 sum = ((u128)a.mant << da) + ((u128)o.mant << db);
    kt_scale fr = kt_scale_from_ratio((uint64_t)(sum >> 64), (uint64_t)sum, 0, 1);
    kt_scale r = {fr.mant, fr.shift + s};
    return r;
}

/* lib.rs:327-340 */
static u128 isqrt_u128(u128 n) {
    if (n == 0) return 0;
    int bits = bits_u128(n);
    u128 x = (u128)1 << ((bits + 1) / 2);
    for (;;) {
        u128 y = (x + n / x) >> 1;
        if (y >= x) return x;
        x = y;
    }
}

/* isqrt_u128 over (hi, lo); returns the low 64 bits of the root (roots of u128 values fit u64). */
uint64_t kt_isqrt_u128(uint64_t hi, uint64_t lo) { return (uint64_t)isqrt_u128(((u128)hi << 64) | lo); }

/* lib.rs:307-318 */
kt_scale kt_scale_rsqrt(kt_scale a) {
    if (a.mant <= 0) abort();
    u128 m = (u128)a.mant;
    int32_t s = a.shift;
    if (s & 1) { m <<= 1; s += 1; }
    u128 r = isqrt_u128(m << 62);
    kt_scale t = {(int64_t)r, 31 + s / 2};
    return kt_scale_recip(t);
}

/* An int32 multiplier for the per-channel requant epilogue (this build's rule): from_ratio gives a mantissa in
 * [2^30, 2^32]; halve it with rounding (and lower the shift) until it is below 2^31. */
kt_scale kt_scale_to_i32(kt_scale a) {
    while (a.mant >= (1LL << 31)) {
        a.mant = (a.mant + 1) >> 1;
        a.shift -= 1;
    }
    return a;
}

/* ------------------------------------------------------------------------------------------------------------ */
/* layers.rs:23-39: quant_to and requant_dyn                                                                      */
/* ------------------------------------------------------------------------------------------------------------ */
void kt_quant_to(const int32_t* data, size_t n, int64_t xmax, int32_t* out) {
    int64_t half = xmax / 2;
    for (size_t i = 0; i < n; i++) {
        int64_t num = (int64_t)data[i] * WLEVELS;
        out[i] = (int32_t)(num >= 0 ? (num + half) / xmax : -((-num + half) / xmax));
    }
}

int32_t kt_requant_dyn(int64_t v, int64_t num_level, int64_t den) {
    i128 prod = (i128)v * (i128)num_level;
    i128 half = (i128)den / 2;
    i128 r = prod >= 0 ? (prod + half) / den : -(((-prod) + half) / den);
    return (int32_t)r;
}

/* |v| with the two's-complement wrap of i64::abs in a release build (i64::MIN stays negative). */
static int64_t abs_wrap(int64_t v) { return v < 0 ? (int64_t)(0 - (uint64_t)v) : v; }

/*
 * QuantLinear::forward_int (layers.rs:275-328) for rows x in i32 codes at scale xs against out x in weight codes at
 * scale ws, with optional i64 bias codes at scale bs (NULL: no bias). Writes the rows x out i32 output codes and
 * returns their scale in *os; *xmax_out and *ymax_out receive the two per-call maxima (0 when not reached).
 *   1. xmax = max |x|; xmax == 0 -> the bias codes (as i32) at bs, or zeros at Scale::ZERO     (279-295)
 *   2. qx = quant_to(x, xmax); c = from_ratio(xmax, WLEVELS) * xs * ws; c == 0 -> zeros        (297-302)
 *   3. bias_in_c[o] = (bs * c^-1).apply(bias[o])                                                (304-307)
 *   4. acc = linear(qx, w) + bias_in_c  (wrapping i64)                                          (312-320)
 *   5. ymax = max |acc|; 0 -> zeros; y = requant_dyn(acc, ACT_LEVELS, ymax),
 *      os = from_ratio(ymax, ACT_LEVELS) * c                                                    (321-327)
 */
void kt_quant_linear_forward(const int32_t* x, size_t rows, size_t in, kt_scale xs, const int32_t* w, size_t out,
                             kt_scale ws, const int64_t* bias, kt_scale bs, size_t threads, int32_t* y, kt_scale* os,
                             int64_t* xmax_out, int64_t* ymax_out) {
    const size_t n = rows * out;
    const kt_scale zero = {0, 0};
    int64_t xmax = 0;
    for (size_t i = 0; i < rows * in; i++) {
        const int64_t a = abs_wrap((int64_t)x[i]);
        if (a > xmax) xmax = a;
    }
    *xmax_out = xmax, *ymax_out = 0, *os = zero;
    if (xmax == 0) {
        for (size_t i = 0; i < n; i++) y[i] = bias ? (int32_t)bias[i % out] : 0;
        if (bias) *os = bs;
        return;
    }
    int32_t* qx = (int32_t*)malloc(rows * in * sizeof(int32_t) + 1);
    int64_t* acc = (int64_t*)malloc(n * sizeof(int64_t) + 1);
    if (!qx || !acc) abort();
    kt_quant_to(x, rows * in, xmax, qx);
    const kt_scale c = kt_scale_mul(kt_scale_mul(kt_scale_from_ratio(0, (uint64_t)xmax, 0, WLEVELS), xs), ws);
    if (c.mant == 0) {
        memset(y, 0, n * sizeof(int32_t));
        free(qx), free(acc);
        return;
    }
    fill_linear(qx, w, rows, out, in, variant_fn(kt_cpu_auto_variant()), acc,
                threads ? threads : kt_plan_threads(n, sat_mul(n, in)), 0);
    if (bias) {
        const kt_scale f = kt_scale_mul(bs, kt_scale_recip(c));
        for (size_t i = 0; i < n; i++) acc[i] = (int64_t)((uint64_t)acc[i] + (uint64_t)kt_scale_apply(f, bias[i % out]));
    }
    int64_t ymax = 0;
    for (size_t i = 0; i < n; i++) {
        const int64_t a = abs_wrap(acc[i]);
        if (a > ymax) ymax = a;
    }
    *ymax_out = ymax;
    if (ymax == 0) {
        memset(y, 0, n * sizeof(int32_t));
    } else {
        for (size_t i = 0; i < n; i++) y[i] = kt_requant_dyn(acc[i], ACT_LEVELS, ymax);
        *os = kt_scale_mul(kt_scale_from_ratio(0, (uint64_t)ymax, 0, ACT_LEVELS), c);
    }
    free(qx), free(acc);
}

/* ------------------------------------------------------------------------------------------------------------ */
/* The 12-bit weight path (benchmark configs 2-5; this build's own format, restated here as the checker)          */
/* ------------------------------------------------------------------------------------------------------------ */

/* W12 layout (this build's 12-bit weight format) for an n x k matrix of codes v in [-2048, 2047]. Digits:
 *   lo = (v & 255) - 128 in [-128, 127] (an int8 plane), hi = (v + 2048) >> 8 in [0, 15], so v = lo + 256 hi - 1920
 *   and sum_k x v = S_lo + 256 S_hi - 1920 sum_k x.
 * Fragment tiling: np = n rounded up to 32, kp = k rounded up to 64. The matrix is cut into blocks of 32 rows x 32 k;
 * block (nb, kb) (kb fastest, kp/32 per row block) holds 64 "lanes" of 16 lo bytes and 8 nib bytes each. Lane
 * l = (n % 32) + 32 h, h = (k % 32) / 16, covers t = k % 16 = 0..15 of its row:
 *   lo byte  ((nb * KB + kb) * 64 + l) * 16 + t;
 *   nib byte ((nb * KB + kb) * 64 + l) * 8 + 4 (t / 8) + (t % 4), low nibble for t % 8 < 4, high nibble otherwise,
 * so a lane's 8 nib bytes as dwords D0, D1 unpack to hi in t order as D0 & 0x0F0F0F0F, (D0 >> 4) & 0x0F0F0F0F,
 * D1 & 0x0F0F0F0F, (D1 >> 4) & 0x0F0F0F0F. Padding rows and k are lo = 0, hi = 0. */
static size_t w12_lo_index(size_t kp, size_t r, size_t c) {
    size_t KB = kp / 32, nb = r / 32, kb = c / 32, lane = (r % 32) + 32 * ((c % 32) / 16);
    return ((nb * KB + kb) * 64 + lane) * 16 + (c % 16);
}

static size_t w12_nib_index(size_t kp, size_t r, size_t c, int* high) {
    size_t KB = kp / 32, nb = r / 32, kb = c / 32, lane = (r % 32) + 32 * ((c % 32) / 16), t = c % 16;
    *high = (t % 8) >= 4;
    return ((nb * KB + kb) * 64 + lane) * 8 + 4 * (t / 8) + (t % 4);
}

size_t kt_w12_lo_bytes(size_t n, size_t k) { return (n + 31) / 32 * 32 * ((k + 63) / 64 * 64); }

void kt_w12_pack(const int32_t* codes, size_t n, size_t k, int8_t* lo, uint8_t* nib) {
    size_t kp = (k + 63) / 64 * 64, np = (n + 31) / 32 * 32;
    memset(lo, 0, np * kp);
    memset(nib, 0, np * kp / 2);
    for (size_t r = 0; r < n; r++)
        for (size_t c = 0; c < k; c++) {
            int32_t v = codes[r * k + c];
            lo[w12_lo_index(kp, r, c)] = (int8_t)((v & 255) - 128);
            int high;
            size_t b = w12_nib_index(kp, r, c, &high);
            uint32_t hi = (uint32_t)(v + 2048) >> 8;
            nib[b] |= (uint8_t)(high ? hi << 4 : hi);
        }
}

/* Decode one code back from the W12 layout (for the exhaustive round-trip test). */
int32_t kt_w12_get(const int8_t* lo, const uint8_t* nib, size_t k, size_t r, size_t c) {
    size_t kp = (k + 63) / 64 * 64;
    int high;
    uint8_t b = nib[w12_nib_index(kp, r, c, &high)];
    int32_t hi = high ? (b >> 4) : (b & 15);
    return (int32_t)lo[w12_lo_index(kp, r, c)] + 256 * hi - 1920;
}

/* The exact accumulators of int8 activations x (m x k, values in [-128,127] as i32) against 12-bit weights in the
 * W12 layout, computed the way the device does -- two int32 plane sums and the row-sum correction, recombined in
 * i64 -- so a layout or recombination mistake shows up against kt_linear_cpu. */
void kt_w12_linear(const int32_t* x, const int8_t* lo, const uint8_t* nib, size_t m, size_t n, size_t k,
                   int64_t* y) {
    size_t kp = (k + 63) / 64 * 64;
    for (size_t r = 0; r < m; r++) {
        int64_t rs = 0;
        for (size_t c = 0; c < k; c++) rs += x[r * k + c];
        for (size_t o = 0; o < n; o++) {
            int32_t s_lo = 0, s_hi = 0;
            for (size_t c = 0; c < k; c++) {
                int high;
                uint8_t b = nib[w12_nib_index(kp, o, c, &high)];
                int32_t h = high ? (b >> 4) : (b & 15);
                s_lo += x[r * k + c] * (int32_t)lo[w12_lo_index(kp, o, c)];
                s_hi += x[r * k + c] * h;
            }
            y[r * n + o] = (int64_t)s_lo + 256 * (int64_t)s_hi - 1920 * rs;
        }
    }
}

/* requant's value without the wrap: round(accum * mant / 2^shift) half away from zero, saturated to i64, for any
 * int32 shift. Equals kt_requant (lib.rs:78-86) wherever that value fits i64; kt_requant casts a larger one to i64
 * with wrap-around (and shifts of 128 or more are outside its i128 arithmetic). */
int64_t kt_requant_sat(int64_t accum, int64_t mant, int32_t shift) {
    i128 prod = (i128)accum * (i128)mant; /* |prod| <= 2^126 */
    if (prod == 0) return 0;
    int neg = prod < 0;
    u128 mag = neg ? (u128)(-prod) : (u128)prod, limit = (u128)1 << 63, q;
    if (shift <= 0) {
        int64_t up = -(int64_t)shift;
        if (up >= 64) q = limit;
        else q = (mag >= ((u128)1 << (63 - up))) ? limit : mag << up;
    } else if (shift >= 127) {
        q = 0;
    } else {
        q = (mag + ((u128)1 << (shift - 1))) >> shift;
    }
    if (q >= limit) return neg ? INT64_MIN : INT64_MAX;
    return neg ? -(int64_t)q : (int64_t)q;
}

/* The per-channel epilogue: out = clamp(requant(acc, mant[n], shift[n]), lo, hi) (kt-int/src/lib.rs:78-86 per
 * output channel, without the i64 wrap; the clamp is this build's int8 / int32 output). */
void kt_requant_channels(const int64_t* acc, size_t m, size_t n, const int32_t* mant, const int32_t* shift,
                         int64_t lo, int64_t hi, int32_t* out) {
    for (size_t r = 0; r < m; r++)
        for (size_t o = 0; o < n; o++) {
            int64_t v = kt_requant_sat(acc[r * n + o], mant[o], shift[o]);
            if (v < lo) v = lo;
            if (v > hi) v = hi;
            out[r * n + o] = (int32_t)v;
        }
}

/* The config-2 per-channel scale (this build's rule, integers only): with ss_n = sum_k w[n,k]^2 and the activation
 * sigma, map 4 standard deviations of the accumulator, 4 * sigma * isqrt(ss_n), to 127:
 * scale_n = to_i32(from_ratio(127, 4 * sigma * isqrt(ss_n))). A zero row gets mant 0. */
void kt_channel_scales(const int32_t* w, size_t n, size_t k, int64_t sigma, int32_t* mant, int32_t* shift) {
    for (size_t o = 0; o < n; o++) {
        uint64_t ss = 0;
        for (size_t c = 0; c < k; c++) ss += (uint64_t)((int64_t)w[o * k + c] * w[o * k + c]);
        uint64_t root = (uint64_t)isqrt_u128(ss);
        if (root == 0) { mant[o] = 0; shift[o] = 0; continue; }
        kt_scale s = kt_scale_from_ratio(0, 127, 0, 4 * (uint64_t)sigma * root);
        s = kt_scale_to_i32(s);
        mant[o] = (int32_t)s.mant;
        shift[o] = s.shift;
    }
}
