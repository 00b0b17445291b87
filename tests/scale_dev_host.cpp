// The device Scale arithmetic (tritify_amd/csrc/kt_scale_dev.h) built for the host with g++, behind plain C entry
// points, so that tests/test_scale_dev.py can check every arithmetic path of the same source on the CPU.
#include "kt_scale_dev.h"

using kt::i128;
using kt::Sc;
using kt::u128;

static u128 join(uint64_t hi, uint64_t lo) { return ((u128)hi << 64) | lo; }
static void split(u128 v, uint64_t* hi, uint64_t* lo) { *hi = (uint64_t)(v >> 64), *lo = (uint64_t)v; }
static void put(Sc s, int64_t* m, int32_t* sh) { *m = s.mant, *sh = s.shift; }

extern "C" {

void sd_udiv128(uint64_t nh, uint64_t nl, uint64_t dh, uint64_t dl, uint64_t* qh, uint64_t* ql) {
    split(kt::udiv128(join(nh, nl), join(dh, dl)), qh, ql);
}
uint64_t sd_isqrt(uint64_t nh, uint64_t nl) { return (uint64_t)kt::isqrt_u128(join(nh, nl)); }
void sd_from_ratio(uint64_t nh, uint64_t nl, uint64_t dh, uint64_t dl, int64_t* m, int32_t* s) {
    put(kt::from_ratio(join(nh, nl), join(dh, dl)), m, s);
}
void sd_mul(int64_t am, int32_t as, int64_t bm, int32_t bs, int64_t* m, int32_t* s) {
    put(kt::sc_mul(Sc{am, as}, Sc{bm, bs}), m, s);
}
void sd_add(int64_t am, int32_t as, int64_t bm, int32_t bs, int64_t* m, int32_t* s) {
    put(kt::sc_add(Sc{am, as}, Sc{bm, bs}), m, s);
}
void sd_recip(int64_t am, int32_t as, int64_t* m, int32_t* s) { put(kt::sc_recip(Sc{am, as}), m, s); }
void sd_rsqrt(int64_t am, int32_t as, int64_t* m, int32_t* s) { put(kt::sc_rsqrt(Sc{am, as}), m, s); }
int sd_ge(int64_t am, int32_t as, int64_t bm, int32_t bs) { return kt::sc_ge(Sc{am, as}, Sc{bm, bs}); }
int64_t sd_apply(int64_t am, int32_t as, int64_t v) { return kt::sc_apply(Sc{am, as}, v); }
int64_t sd_apply32(int64_t am, int32_t as, int32_t v) { return kt::sc_apply32(Sc{am, as}, v); }
int32_t sd_requant_dyn(int64_t v, int64_t den) { return kt::requant_dyn_dev(v, den); }
uint64_t sd_udiv_small_q(uint64_t nh, uint64_t nl, int64_t d) { return kt::udiv_small_q(join(nh, nl), d); }
}

extern "C" int32_t sd_rq_apply(int64_t den, int64_t v) { return kt::rq_apply(kt::rq_den(den), v); }
extern "C" uint64_t sd_udiv64_small(uint64_t n, uint64_t d) { return kt::udiv64_small(n, d); }
