/*
 * kt_oracle.h -- TEST INFRASTRUCTURE ONLY. Prototypes shared by the two halves of the CPU oracle:
 * kt_oracle.c (the reference's integer path) and kt_oracle_layers.c (the layers of benchmark configs 3-5 around the
 * 12-bit GEMM). Never part of the product.
 */
#ifndef KT_ORACLE_H
#define KT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

typedef struct {
    int64_t mant;
    int32_t shift;
} kt_scale;

uint64_t kt_lcg_next(uint64_t* s);
int64_t kt_requant_sat(int64_t accum, int64_t mant, int32_t shift);
kt_scale kt_scale_from_ratio(uint64_t num_hi, uint64_t num_lo, uint64_t den_hi, uint64_t den_lo);
kt_scale kt_scale_to_i32(kt_scale a);
uint64_t kt_isqrt_u128(uint64_t hi, uint64_t lo);
size_t kt_resolve_threads(size_t nblocks);

#endif /* KT_ORACLE_H */
