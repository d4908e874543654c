// fns_lanes.hpp - cross-lane exchange on the 64-lane gfx950 wave without the LDS crossbar.
//
// xor_lane<O>(v) returns v of lane (lane ^ O), O in {1, 2, 4, 8, 16, 32}, built from VALU data movement only:
//   O = 1, 2 : DPP quad_perm;   O = 4 : DPP row_half_mirror then quad reversal;   O = 8 : DPP row_ror:8;
//   O = 16   : v_permlane16_swap (gfx950; swaps the odd and even 16-lane rows);
//   O = 32   : v_permlane32_swap (swaps the two 32-lane halves).
// ds_bpermute-based shuffles cost ~50 ns each when chained (measured); these cost a few cycles. Because xor_lane
// is an exact xor permutation, butterflies built on it perform the same additions in the same order as the xor
// shuffles they replace (the Q8_1 sums must match the reference bit for bit). All lanes must be active.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace fns::dev {

template <int O> __device__ __forceinline__ int xor_lane_i(int v) {
    if constexpr (O == 1) {
        return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    } else if constexpr (O == 2) {
        return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    } else if constexpr (O == 4) {
        const int m = __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);  // row_half_mirror: i -> 7 - i
        return __builtin_amdgcn_update_dpp(0, m, 0x1B, 0xF, 0xF, false);          // quad_perm [3,2,1,0]
    } else if constexpr (O == 8) {
        return __builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, false);  // row_ror:8
    } else if constexpr (O == 16) {
        const auto p = __builtin_amdgcn_permlane16_swap((unsigned) v, (unsigned) v, false, false);
        return (int) ((threadIdx.x & 16) ? p[0] : p[1]);
    } else {
        static_assert(O == 32, "xor_lane: offset must be 1, 2, 4, 8, 16 or 32");
        const auto p = __builtin_amdgcn_permlane32_swap((unsigned) v, (unsigned) v, false, false);
        return (int) ((threadIdx.x & 32) ? p[0] : p[1]);
    }
}

template <int O> __device__ __forceinline__ float xor_lane(float v) {
    return __builtin_bit_cast(float, xor_lane_i<O>(__builtin_bit_cast(int, v)));
}

// Sum over aligned groups of W lanes (power of two <= 64), xor butterfly from W/2 down to 1: every lane of the group
// receives the sum, computed in the same order as `for (o = W/2; o; o >>= 1) v += shfl_xor(v, o)`.
template <int W> __device__ __forceinline__ float lanes_sum(float v) {
    if constexpr (W >= 64) v += xor_lane<32>(v);
    if constexpr (W >= 32) v += xor_lane<16>(v);
    if constexpr (W >= 16) v += xor_lane<8>(v);
    if constexpr (W >= 8) v += xor_lane<4>(v);
    if constexpr (W >= 4) v += xor_lane<2>(v);
    if constexpr (W >= 2) v += xor_lane<1>(v);
    return v;
}

template <int W> __device__ __forceinline__ int lanes_sum_i(int v) {
    if constexpr (W >= 64) v += xor_lane_i<32>(v);
    if constexpr (W >= 32) v += xor_lane_i<16>(v);
    if constexpr (W >= 16) v += xor_lane_i<8>(v);
    if constexpr (W >= 8) v += xor_lane_i<4>(v);
    if constexpr (W >= 4) v += xor_lane_i<2>(v);
    if constexpr (W >= 2) v += xor_lane_i<1>(v);
    return v;
}

template <int W> __device__ __forceinline__ float lanes_max(float v) {
    if constexpr (W >= 64) v = fmaxf(v, xor_lane<32>(v));
    if constexpr (W >= 32) v = fmaxf(v, xor_lane<16>(v));
    if constexpr (W >= 16) v = fmaxf(v, xor_lane<8>(v));
    if constexpr (W >= 8) v = fmaxf(v, xor_lane<4>(v));
    if constexpr (W >= 4) v = fmaxf(v, xor_lane<2>(v));
    if constexpr (W >= 2) v = fmaxf(v, xor_lane<1>(v));
    return v;
}

// Max of a 64-bit unsigned value over the whole wave (every lane receives it).
template <int O> __device__ __forceinline__ uint64_t max_xor_u64(uint64_t v) {
    const uint32_t lo = (uint32_t) xor_lane_i<O>((int) (uint32_t) v), hi = (uint32_t) xor_lane_i<O>((int) (uint32_t) (v >> 32));
    const uint64_t o = ((uint64_t) hi << 32) | lo;
    return o > v ? o : v;
}
__device__ __forceinline__ uint64_t lanes_max_u64(uint64_t v) {
    v = max_xor_u64<32>(v);
    v = max_xor_u64<16>(v);
    v = max_xor_u64<8>(v);
    v = max_xor_u64<4>(v);
    v = max_xor_u64<2>(v);
    return max_xor_u64<1>(v);
}

// Q8_1 of one value per lane, 32-lane blocks (lanes 0-31, 32-63): the reference's op order (d = amax / 127,
// q = roundf(x / d), ds = (d, sum) with xor butterflies 16 .. 1). Returns q; d, sum and the 16-lane integer sum of q
// (for the K-quant min term) and the block's max |v| are valid in every lane of the block.
struct Q8Lane {
    int q;
    float d, sum, amax;
    int qsum16, qsum32;
};
__device__ __forceinline__ Q8Lane q8_1_lane(float v) {
    float amax = fabsf(v), sum = v;
    amax = fmaxf(amax, xor_lane<16>(amax));
    sum += xor_lane<16>(sum);
    amax = fmaxf(amax, xor_lane<8>(amax));
    sum += xor_lane<8>(sum);
    amax = fmaxf(amax, xor_lane<4>(amax));
    sum += xor_lane<4>(sum);
    amax = fmaxf(amax, xor_lane<2>(amax));
    sum += xor_lane<2>(sum);
    amax = fmaxf(amax, xor_lane<1>(amax));
    sum += xor_lane<1>(sum);
    Q8Lane r;
    r.amax = amax;
    r.d = amax / 127.0f;
    r.q = amax == 0.0f ? 0 : (int) (int8_t) roundf(v / r.d);
    r.sum = sum;
    r.qsum16 = lanes_sum_i<16>(r.q);
    r.qsum32 = r.qsum16 + xor_lane_i<16>(r.qsum16);
    return r;
}

}  // namespace fns::dev
