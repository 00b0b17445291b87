// kt-int's integer Scale (crates/00-kernels/kt-int/src/lib.rs:175-340) on the device, for the reference-semantics
// layers: a non-negative scale mant * 2^-shift with a ~31-bit mantissa, composed with 128-bit integer arithmetic.
// Every function gives the integers of its kt-int counterpart; these run in one thread per tensor (or per cached
// step), never per element, except sc_apply and requant_dyn_dev.
//
// The same source compiles as host C++ (g++, no HIP headers) so that the exactness of every arithmetic path can be
// checked on the CPU against the restatement of kt-int and against Python's integers.
#pragma once

#include <stdint.h>

#ifdef __HIPCC__
#include <hip/hip_runtime.h>
#define KT_SC_FN __host__ __device__ inline
#define KT_SC_COLD __host__ __device__ inline __attribute__((noinline))
#else
#include <math.h>
#define KT_SC_FN inline
#define KT_SC_COLD inline __attribute__((noinline))
#endif

namespace kt {

typedef unsigned __int128 u128;
typedef __int128 i128;

struct Sc {
    int64_t mant;
    int32_t shift;
};

KT_SC_FN int bits_u128(u128 v) {
    const uint64_t hi = (uint64_t)(v >> 64), lo = (uint64_t)v;
    return hi ? 128 - __builtin_clzll(hi) : (lo ? 64 - __builtin_clzll(lo) : 0);
}

// floor(n / d) for d > 0, exact for every input:
//  - d a power of two below 2^64: a shift;
//  - d below 2^64 and the quotient below 2^49 (bits(n) - bits(d) < 49; every quotient of from_ratio, whose mantissa
//    is below 2^33, and of isqrt's Newton steps): a double-precision estimate, whose relative error is at most
//    5 * 2^-53 (the conversions of n's two halves and of d, their sum, the quotient), so at most 5/16 absolute,
//    corrected against the exact i128 remainder (n < 2^113 here, so the remainder fits). On the GPU this is a
//    few dozen instructions, where a 64-bit integer division is a long software sequence;
//  - both below 2^64: the 64-bit division;
//  - otherwise restoring long division.
// The last two are rare in the layers' Scale chains and long in code: they stay out of line (udiv128_rest), so the
// inlined copies at every call site are short (one-token kernels fetch their straight-line code cold each launch).
KT_SC_COLD u128 udiv128_rest(u128 n, u128 d) {
    if ((n >> 64) == 0 && (d >> 64) == 0) return (u128)((uint64_t)n / (uint64_t)d);
    u128 q = 0, r = 0;
    for (int i = bits_u128(n) - 1; i >= 0; i--) {
        r = (r << 1) | ((n >> i) & 1);
        if (r >= d) r -= d, q |= (u128)1 << i;
    }
    return q;
}
KT_SC_FN u128 udiv128(u128 n, u128 d) {
    // from_ratio's normalizations divide by powers of two (Scale::mul by 1, a negative shift by 2^-s): a shift
    if ((d >> 64) == 0 && (uint64_t)d != 0 && ((uint64_t)d & ((uint64_t)d - 1)) == 0)
        return n >> __builtin_ctzll((uint64_t)d);
    if ((d >> 64) == 0 && bits_u128(n) - bits_u128(d) < 49) {
        const uint64_t d64 = (uint64_t)d;
        const double dn = (double)(uint64_t)(n >> 64) * 18446744073709551616.0 + (double)(uint64_t)n;
        uint64_t q = (uint64_t)(dn / (double)d64);
        i128 rem = (i128)n - (i128)q * (i128)d64;
        while (rem < 0) q--, rem += (i128)d64;
        while (rem >= (i128)d64) q++, rem -= (i128)d64;
        return (u128)q;
    }
    return udiv128_rest(n, d);
}

// floor(n / d) for d < 2^32 and a quotient below 2^40: the double quotient is within 2^-12 of the exact one (the
// conversion of n and the division each add a relative error of at most 2^-53), so the floor is at most one away,
// and the remainder, in (-2^33, 2^33), is exact in 64-bit wrapping arithmetic.
KT_SC_FN uint64_t udiv64_small(uint64_t n, uint64_t d) {
    uint64_t q = (uint64_t)((double)n / (double)d);
    const int64_t rem = (int64_t)(n - q * d);
    if (rem < 0) q--;
    else if (rem >= (int64_t)d) q++;
    return q;
}

// Scale::from_ratio (lib.rs:191-212): a 31-bit-normalized mantissa of num / den, rounded.
KT_SC_FN Sc from_ratio(u128 num, u128 den) {
    if (num == 0) return Sc{0, 0};
    // the same integers in 64-bit arithmetic where the operands allow (no halving applies below 2^64):
    if (den == 1 && (num >> 64) == 0) {  // Scale::mul and Scale::add: a division by a power of two
        const uint64_t n = (uint64_t)num;
        const int s = 32 - (64 - __builtin_clzll(n));  // 31 - (bits(n) - bits(1))
        if (s >= 0) return Sc{(int64_t)(n << s), s};
        const int k = -s;  // floor((n + 2^(k-1)) / 2^k), without the sum's overflow
        return Sc{(int64_t)((n >> k) + ((n >> (k - 1)) & 1)), s};
    }
    if ((num >> 62) == 0 && den != 0 && (den >> 32) == 0) {  // num < 2^62, den < 2^32: quotients below 2^33
        const uint64_t n = (uint64_t)num, d = (uint64_t)den;
        const int s = 31 - ((64 - __builtin_clzll(n)) - (64 - __builtin_clzll(d)));
        if (s >= 0) return Sc{(int64_t)udiv64_small((n << s) + d / 2, d), s};  // n << s has 31 + bits(d) bits
        const uint64_t dd = d << (-s);                                          // bits(n) - 31 bits
        return Sc{(int64_t)udiv64_small(n + dd / 2, dd), s};
    }
    {  // the reference halves both until each fits 64 bits: that many halvings as one shift
        const int bn = bits_u128(num), bd = bits_u128(den), k = (bn > bd ? bn : bd) - 64;
        if (k > 0) num >>= k, den >>= k;
    }
    if (den == 0) den = 1;
    const int s = 31 - (bits_u128(num) - bits_u128(den));
    u128 m;
    if (s >= 0) {
        m = udiv128((num << s) + den / 2, den);
    } else {
        const u128 dd = den << (-s);
        m = udiv128(num + dd / 2, dd);
    }
    return Sc{(int64_t)m, s};
}

// Scale::mul (lib.rs:252-258)
KT_SC_FN Sc sc_mul(Sc a, Sc b) {
    if (a.mant == 0 || b.mant == 0) return Sc{0, 0};
    const uint64_t am = (uint64_t)a.mant, bm = (uint64_t)b.mant;
    Sc q = from_ratio((am >> 32) == 0 && (bm >> 32) == 0 ? (u128)(am * bm) : (u128)am * (u128)bm, 1);
    q.shift += a.shift + b.shift;
    return q;
}

// Scale::recip (lib.rs:275-280); a.mant > 0.
KT_SC_FN Sc sc_recip(Sc a) {
    const Sc r = from_ratio((u128)1 << 40, (u128)(uint64_t)a.mant);
    return Sc{r.mant, r.shift - a.shift + 40};
}

// Scale::ge (lib.rs:227-248): a >= o by value.
KT_SC_FN bool sc_ge(Sc a, Sc o) {
    if (a.mant == 0) return o.mant == 0;
    if (o.mant == 0) return true;
    const int d = o.shift - a.shift;
    {  // mantissas below 2^33 and shifts within 30 of each other: the same comparison in 64 bits
        const uint64_t ua = (uint64_t)a.mant, ub = (uint64_t)o.mant;
        if ((ua >> 33) == 0 && (ub >> 33) == 0 && d <= 30 && d >= -30)
            return d >= 0 ? (ua << d) >= ub : ua >= (ub << -d);
    }
    const u128 ma = (u128)(uint64_t)a.mant, mb = (u128)(uint64_t)o.mant;
    if (d >= 0) {
        if (d + bits_u128(ma) > 127) return true;
        return (ma << d) >= mb;
    }
    const int e = -d;
    if (e + bits_u128(mb) > 127) return false;
    return ma >= (mb << e);
}

// Scale::add (lib.rs:285-303)
KT_SC_FN Sc sc_add(Sc a, Sc o) {
    if (a.mant == 0) return o;
    if (o.mant == 0) return a;
    const int s = a.shift > o.shift ? a.shift : o.shift;
    const int da = s - a.shift, db = s - o.shift;
    if (da >= 96) return a;
    if (db >= 96) return o;
    const u128 sum = ((u128)(uint64_t)a.mant << da) + ((u128)(uint64_t)o.mant << db);
    const Sc fr = from_ratio(sum, 1);
    return Sc{fr.mant, fr.shift + s};
}

// isqrt_u128 (lib.rs:327-340): floor(sqrt(n)), which the reference's Newton iteration from above (start
// 2^ceil(bits/2) >= sqrt(n), stop when a step no longer decreases) arrives at. Below 2^104 the same integer comes
// from the double-precision root corrected to the exact floor: the estimate is within 2 of sqrt(n) there (the
// conversion and the root each add a relative error of at most 2^-53 to a value below 2^52), and the two loops move
// it to the r with r^2 <= n < (r + 1)^2, which is unique. Larger n take the Newton iteration itself.
KT_SC_COLD u128 isqrt_newton(u128 n) {  // n >= 2^104: the reference's iteration itself
    u128 x = (u128)1 << ((bits_u128(n) + 1) / 2);
    for (;;) {
        const u128 y = (x + udiv128(n, x)) >> 1;
        if (y >= x) return x;
        x = y;
    }
}
KT_SC_FN u128 isqrt_u128(u128 n) {
    if (n == 0) return 0;
    if (bits_u128(n) <= 104) {
        const double dn = (double)(uint64_t)(n >> 64) * 18446744073709551616.0 + (double)(uint64_t)n;
        uint64_t r = (uint64_t)sqrt(dn);
        while ((u128)r * r > n) r--;
        while ((u128)(r + 1) * (r + 1) <= n) r++;
        return (u128)r;
    }
    return isqrt_newton(n);
}

// Scale::rsqrt (lib.rs:307-318); a.mant > 0.
KT_SC_FN Sc sc_rsqrt(Sc a) {
    u128 m = (u128)(uint64_t)a.mant;
    int s = a.shift;
    if (s & 1) m <<= 1, s += 1;
    const u128 r = isqrt_u128(m << 62);
    return sc_recip(Sc{(int64_t)r, 31 + s / 2});
}

// Scale::apply (lib.rs:261-272): round(value * a) half away from zero, i128 product, wrapped to i64.
KT_SC_FN int64_t sc_apply(Sc a, int64_t value) {
    if (a.mant == 0) return 0;
    const i128 prod = (i128)value * (i128)a.mant;
    if (a.shift <= 0) return (int64_t)(prod << (-a.shift));
    const i128 half = (i128)1 << (a.shift - 1);
    return (int64_t)(prod >= 0 ? (prod + half) >> a.shift : -(((-prod) + half) >> a.shift));
}

// Scale::apply of an int32 code with 64-bit arithmetic where that is exact: |mant| < 2^32 and 0 <= shift <= 63 keep
// |v * mant| below 2^63 and its sum with the rounding addend 2^(shift - 1) below 2^64 (unsigned); other Scales go
// through the i128 sc_apply. The same rounding, half away from zero.
KT_SC_COLD int64_t sc_apply_wide(Sc a, int64_t v) { return sc_apply(a, v); }
KT_SC_FN int64_t sc_apply32(Sc a, int32_t v) {
    if (a.mant > -((int64_t)1 << 32) && a.mant < ((int64_t)1 << 32) && a.shift >= 0 && a.shift <= 63) {
        const uint64_t m = (uint64_t)(uint32_t)(a.mant < 0 ? -a.mant : a.mant);
        const uint64_t x = (uint64_t)(uint32_t)(v < 0 ? 0u - (uint32_t)v : (uint32_t)v);
        const uint64_t p = x * m;
        const uint64_t q = a.shift == 0 ? p : (p + ((uint64_t)1 << (a.shift - 1))) >> a.shift;
        return (v < 0) != (a.mant < 0) ? (int64_t)(0 - q) : (int64_t)q;
    }
    return sc_apply_wide(a, v);  // a Scale outside the 64-bit range: rare, out of line
}

// floor(n / d) for 0 < d < 2^63 when the quotient is below 2^40: the double estimate's absolute error is then below
// 2^40 * 2^-50 (three roundings of relative size 2^-53 each), so one correction step each way suffices; two are
// allowed.
KT_SC_FN uint64_t udiv_small_q(u128 n, int64_t d) {
    const double dn = (double)(uint64_t)(n >> 64) * 18446744073709551616.0 + (double)(uint64_t)n;
    const double qd = dn / (double)d;
    uint64_t q = qd <= 0.0 ? 0 : (uint64_t)qd;
    i128 rem = (i128)n - (i128)q * (i128)d;
#pragma unroll
    for (int i = 0; i < 2; i++)
        if (rem < 0) q--, rem += d;
#pragma unroll
    for (int i = 0; i < 2; i++)
        if (rem >= d) q++, rem -= d;
    return q;
}

// requant_dyn(v, 2^28, den) (crates/01-engine/kt-core/src/layers.rs:33-39) for |v| <= den: the quotient is at most
// 2^28, within udiv_small_q's range.
KT_SC_FN int32_t requant_dyn_dev(int64_t v, int64_t den) {
    const uint64_t a = v < 0 ? 0 - (uint64_t)v : (uint64_t)v;
    const uint64_t q = udiv_small_q(((u128)a << 28) + (u128)(uint64_t)(den / 2), den);
    return (int32_t)(v < 0 ? 0 - q : q);
}

// requant_dyn(v, 2^28, den) for many v over one den, without a division per value: q = floor((|v| 2^28 + den / 2)
// / den) estimated as |v| * (2^28 / den) + 1/2 in double precision (relative error below 2^-51 on a value at most
// 2^28, so within one of q) and corrected by the exact remainder. For den < 2^62 and |v| <= den that remainder lies
// in (-2^62, 2^63), so its 64-bit wrapping value is exact. Every other input (|v| > den, den <= 0, den >= 2^62)
// takes requant_dyn_cold, the reference's own i128 arithmetic.
struct RqDen {
    int64_t den;
    uint64_t half;
    double rinv;
};
KT_SC_FN RqDen rq_den(int64_t den) {
    return RqDen{den, (uint64_t)(den / 2), den > 0 ? 268435456.0 / (double)den : 0.0};
}
// requant_dyn(v, 2^28, den) for any v and den != 0 exactly as layers.rs:33-39 computes it: the i128 product, half =
// den / 2 truncated, the truncating i128 quotient (signs from the numerator and den), the result wrapped to i32. The
// reference's division by a zero den panics; 0 is returned for it.
KT_SC_COLD int32_t requant_dyn_cold(int64_t v, int64_t den) {
    if (den == 0) return 0;
    const i128 prod = (i128)v * ((i128)1 << 28), half = (i128)(den / 2);
    const i128 num = prod >= 0 ? prod + half : -prod + half;  // |num| < 2^92
    const u128 un = num < 0 ? (u128)(-num) : (u128)num;
    const u128 ud = den < 0 ? (u128)(0 - (uint64_t)den) : (u128)(uint64_t)den;
    const u128 uq = udiv128(un, ud);
    const i128 q = ((num < 0) != (den < 0)) ? -(i128)uq : (i128)uq;  // num / den, truncated
    const i128 r = prod >= 0 ? q : -q;
    return (int32_t)(uint32_t)(uint64_t)(u128)r;
}
KT_SC_FN int32_t rq_apply(const RqDen& r, int64_t v) {
    const uint64_t a = v < 0 ? 0 - (uint64_t)v : (uint64_t)v;
    if (r.den <= 0 || r.den >= ((int64_t)1 << 62) || a > (uint64_t)r.den) return requant_dyn_cold(v, r.den);
    uint64_t q = (uint64_t)((double)a * r.rinv + 0.5);
    const int64_t rem = (int64_t)((a << 28) + r.half - q * (uint64_t)r.den);
    if (rem < 0) q--;
    else if (rem >= r.den) q++;
    return (int32_t)(v < 0 ? 0 - q : q);
}

}  // namespace kt
