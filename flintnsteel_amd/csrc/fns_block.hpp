// fns_block.hpp - LDS staging of packed weights and activation rows (LDS-DMA helpers), and the Q8_1 activation row
// image the GEMV code reads from LDS. Block layouts: see fns_common.hpp.
#pragma once

#include "fns_common.hpp"

namespace fns::dev {

// ---- LDS staging of packed weights ------------------------------------------------------------------------------
// LDS-DMA (global_load_lds_dwordx4): each wave instruction moves 1 KiB of consecutive global bytes (fully coalesced
// 128-bit loads) to 1 KiB of consecutive LDS at the wave-uniform base given in M0, lane i filling bytes 16 i ..
// 16 i + 15; the data never passes through VGPRs. It is visible after dma_wait() (all of this wave's vector loads
// complete) and a workgroup barrier.
// One wave's LDS DMA of the bytes [begin, end) of src (rounded outward to 16-byte boundaries) to the same offsets of
// dst; src and dst 16-byte aligned. Pieces that two waves both cover receive the same bytes from each.
__device__ __forceinline__ void dma_wave(uint8_t *dst, const uint8_t *src, int begin, int end) {
    const int lane = threadIdx.x % kWave;
    const int b = begin & ~15, e = (end + 15) & ~15;
    for (int p = b; p < e; p += 1024) {
        if (p + lane * 16 < e)
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *) (src + p + lane * 16),
                                             (__attribute__((address_space(3))) void *) (dst + p), 16, 0, 0);
    }
}
// LDS DMA of `bytes` (a multiple of 16) by waves first_wave .. NW-1 of the workgroup (1 KiB per wave instruction).
template <int NW>
__device__ __forceinline__ void dma_waves_from(uint8_t *dst, const uint8_t *src, int bytes, int first_wave) {
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    if (wave < first_wave) return;
    for (int p = (wave - first_wave) * 1024; p < bytes; p += (NW - first_wave) * 1024) {
        if (p + lane * 16 < bytes)
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *) (src + p + lane * 16),
                                             (__attribute__((address_space(3))) void *) (dst + p), 16, 0, 0);
    }
}
// s_waitcnt vmcnt(0) (gfx9 encoding: expcnt and lgkmcnt left at their maxima).
__device__ __forceinline__ void dma_wait() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// 16 bytes at a 2-byte-aligned address (LDS, or global through a generic pointer): one unaligned 16-byte load
// (gfx950 runs with unaligned LDS and global access enabled, and the compiler emits ds_read_b128 / flat_load_dwordx4
// for it); nothing outside the 16 bytes is touched.
__device__ __forceinline__ uint4 lds16u(const uint8_t *p) {
    uint4 v;
    __builtin_memcpy(&v, __builtin_assume_aligned(p, 2), 16);
    return v;
}

__device__ __forceinline__ float sbyte_f(uint32_t w, int k) { return (float) (int) (int8_t) ((w >> (8 * k)) & 0xffu); }
__device__ __forceinline__ float fmaf_(float a, float b, float c) { return __builtin_fmaf(a, b, c); }

// Activation row image (npad columns, a multiple of 512), kept in LDS and copied there verbatim from global memory:
//   int8 q, 256 columns then 16 bytes of padding per 256 | f32 d[npad/32] | f32 s16[npad/16] | f32 s32[npad/32]
// with s16 / s32 = d * (sum of the quantised values of the 16 / 32 columns). The padding puts the 256-column blocks of
// a row on different LDS banks (lanes taking consecutive blocks read 16-byte pieces that would otherwise all map to
// the same banks), and img_bytes rounds the image to 64 mod 256 bytes so consecutive images are skewed as well.
constexpr int kImgQRow = 272;
__host__ __device__ constexpr int img_q_bytes(int npad) { return npad / 256 * kImgQRow; }
__host__ __device__ constexpr int img_bytes(int npad) {
    const int b = img_q_bytes(npad) + (npad / 32 + npad / 16 + npad / 32) * 4;
    return b + ((64 - b % 256) + 256) % 256;
}
__host__ __device__ constexpr int img_q_index(int i) { return i + (i >> 8) * (kImgQRow - 256); }
struct ActImg {
    const int8_t *q;
    const float *d, *s16, *s32;
};
__device__ __forceinline__ ActImg act_img(const uint8_t *base, int npad) {
    const float *d = (const float *) (base + img_q_bytes(npad));
    return ActImg{(const int8_t *) base, d, d + npad / 32, d + npad / 32 + npad / 16};
}

constexpr uint32_t kLo4 = 0x0F0F0F0Fu;

// 16-value group term of Q6_K / Q3_K: d8 * (u . a) - bias * s16, with u the unsigned codes.
__device__ __forceinline__ float group_term(int dotu, float d8, float s16, float bias) {
    return fmaf_(d8, (float) dotu, -bias * s16);
}

}  // namespace fns::dev
