// Wave reductions without LDS on gfx950 (wave64): DPP moves between the lanes of one 16-lane row (the xor-1 and xor-2
// partners within quads, then the 8- and 16-lane mirrors) pair every lane with lanes holding disjoint, equal-sized
// groups, so four steps leave each row's reduction (maximum, wrapping sum, a lexicographic order) in all of its
// lanes; the four rows' results (lanes 0, 16, 32, 48) are then read into scalars and combined there. Every lane of
// the wave must be active.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kt {

namespace {

template <int CTRL>
__device__ inline uint64_t dpp64(uint64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)v, CTRL, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(v >> 32), CTRL, 0xF, 0xF, false);
    return ((uint64_t)hi << 32) | lo;
}
__device__ inline uint64_t lane64(uint64_t v, int l) {
    return ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l) << 32) |
           (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
}
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;
__device__ inline int64_t max64(int64_t a, int64_t b) { return b > a ? b : a; }
__device__ inline int64_t row_max_i64(int64_t v) {
    v = max64(v, (int64_t)dpp64<DPP_XOR1>((uint64_t)v));
    v = max64(v, (int64_t)dpp64<DPP_XOR2>((uint64_t)v));
    v = max64(v, (int64_t)dpp64<DPP_HALF_MIRROR>((uint64_t)v));
    return max64(v, (int64_t)dpp64<DPP_MIRROR>((uint64_t)v));
}
__device__ inline uint64_t row_sum_u64(uint64_t v) {  // wrapping
    v += dpp64<DPP_XOR1>(v);
    v += dpp64<DPP_XOR2>(v);
    v += dpp64<DPP_HALF_MIRROR>(v);
    return v + dpp64<DPP_MIRROR>(v);
}
// a u128 (hi, lo) summed over each row
template <int CTRL>
__device__ inline void add128_dpp(uint64_t& hi, uint64_t& lo) {
    const uint64_t ohi = dpp64<CTRL>(hi), olo = dpp64<CTRL>(lo), t = lo + olo;
    hi += ohi + (t < lo), lo = t;
}
__device__ inline void add128_row(uint64_t& hi, uint64_t& lo) {
    add128_dpp<DPP_XOR1>(hi, lo);
    add128_dpp<DPP_XOR2>(hi, lo);
    add128_dpp<DPP_HALF_MIRROR>(hi, lo);
    add128_dpp<DPP_MIRROR>(hi, lo);
}
__device__ inline int64_t wave_max_i64(int64_t v) {
    v = row_max_i64(v);
    return max64(max64((int64_t)lane64(v, 0), (int64_t)lane64(v, 16)),
                 max64((int64_t)lane64(v, 32), (int64_t)lane64(v, 48)));
}
__device__ inline uint64_t wave_sum_u64(uint64_t v) {
    v = row_sum_u64(v);
    return lane64(v, 0) + lane64(v, 16) + lane64(v, 32) + lane64(v, 48);
}
template <int CTRL>
__device__ inline uint32_t dpp32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
}
__device__ inline int32_t wave_sum_i32(int32_t v) {  // wrapping
    v += (int32_t)dpp32<DPP_XOR1>((uint32_t)v);
    v += (int32_t)dpp32<DPP_XOR2>((uint32_t)v);
    v += (int32_t)dpp32<DPP_HALF_MIRROR>((uint32_t)v);
    v += (int32_t)dpp32<DPP_MIRROR>((uint32_t)v);
    return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) + __builtin_amdgcn_readlane(v, 32) +
           __builtin_amdgcn_readlane(v, 48);
}
__device__ inline uint32_t wave_max_u32(uint32_t v) {
    auto mx = [](uint32_t a, uint32_t b) { return b > a ? b : a; };
    v = mx(v, dpp32<DPP_XOR1>(v));
    v = mx(v, dpp32<DPP_XOR2>(v));
    v = mx(v, dpp32<DPP_HALF_MIRROR>(v));
    v = mx(v, dpp32<DPP_MIRROR>(v));
    return mx(mx((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 16)),
              mx((uint32_t)__builtin_amdgcn_readlane((int)v, 32), (uint32_t)__builtin_amdgcn_readlane((int)v, 48)));
}

__device__ inline int32_t wave_max_i32(int32_t v) {
    auto mx = [](int32_t a, int32_t b) { return b > a ? b : a; };
    v = mx(v, (int32_t)dpp32<DPP_XOR1>((uint32_t)v));
    v = mx(v, (int32_t)dpp32<DPP_XOR2>((uint32_t)v));
    v = mx(v, (int32_t)dpp32<DPP_HALF_MIRROR>((uint32_t)v));
    v = mx(v, (int32_t)dpp32<DPP_MIRROR>((uint32_t)v));
    return mx(mx(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
              mx(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
// x plus its value in lane l ^ 1, l ^ 2 (DPP), l ^ 16 and l ^ 32 (the lane-swap instructions: swapping the odd
// 16-lane rows of one copy of x with the even rows of another, or the upper 32 lanes with the lower 32, leaves
// every lane's partner in one of the two copies), wrapping: no LDS.
__device__ inline int32_t add_xor1(int32_t x) { return x + (int32_t)dpp32<DPP_XOR1>((uint32_t)x); }
__device__ inline int32_t add_xor2(int32_t x) { return x + (int32_t)dpp32<DPP_XOR2>((uint32_t)x); }
__device__ inline int32_t add_xor16(int32_t x) {
    const auto p = __builtin_amdgcn_permlane16_swap((unsigned)x, (unsigned)x, false, false);
    return (int32_t)(p[0] + p[1]);
}
__device__ inline int32_t add_xor32(int32_t x) {
    const auto p = __builtin_amdgcn_permlane32_swap((unsigned)x, (unsigned)x, false, false);
    return (int32_t)(p[0] + p[1]);
}

}  // namespace

}  // namespace kt
