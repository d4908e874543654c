// fns_block.hpp - one whole 256-value K-quant block per lane: the block's packed bytes are loaded into registers
// (9 / 11 / 13 / 7 sixteen-byte fragments for Q4_K / Q5_K / Q6_K / Q3_K), its header (d, dmin, 6-bit scales) is
// decoded once, and its dot product with a Q8_1 activation row (LDS image) is formed sub-block by sub-block:
//   Q4_K / Q5_K: d * sum_s sc_s * d8_s * (q_s . a_s) - dmin * sum_s m_s * (d8_s * sum a_s)       (s: 32 values)
//   Q6_K       : d * sum_g sc_g * (d8_g * (u_g . a_g) - 32 * d8_g * sum a_g)                      (g: 16 values)
//   Q3_K       : d * sum_g sc_g * (d8_g * (u_g . a_g) -  4 * d8_g * sum a_g)                      (g: 16 values)
// with exact integer dot products (v_dot4 on int8 lanes) and the weights' zero points (32, 4) folded into the
// activation sums, so the unsigned codes u are never re-biased per byte. Block layouts: see fns_common.hpp.
#pragma once

#include "fns_common.hpp"

namespace fns::dev {

template <int T> struct BlockRegs;
template <> struct BlockRegs<T_Q4_K> { uint4 v[9]; };
template <> struct BlockRegs<T_Q5_K> { uint4 v[11]; };
template <> struct BlockRegs<T_Q6_K> { uint4 v[13]; uint32_t d; };
template <> struct BlockRegs<T_Q3_K> { uint4 v[6]; uint4 tail; };

template <int T> __device__ __forceinline__ void block_load(const uint8_t *blk, BlockRegs<T> &b);

template <> __device__ __forceinline__ void block_load<T_Q4_K>(const uint8_t *blk, BlockRegs<T_Q4_K> &b) {
#pragma unroll
    for (int i = 0; i < 9; ++i) b.v[i] = gload<uint4>(blk + 16 * i);
}
template <> __device__ __forceinline__ void block_load<T_Q5_K>(const uint8_t *blk, BlockRegs<T_Q5_K> &b) {
#pragma unroll
    for (int i = 0; i < 11; ++i) b.v[i] = gload<uint4>(blk + 16 * i);
}
template <> __device__ __forceinline__ void block_load<T_Q6_K>(const uint8_t *blk, BlockRegs<T_Q6_K> &b) {
#pragma unroll
    for (int i = 0; i < 13; ++i) b.v[i] = gload16u(blk + 16 * i);
    b.d = gload<uint16_t>(blk + 208);
}
template <> __device__ __forceinline__ void block_load<T_Q3_K>(const uint8_t *blk, BlockRegs<T_Q3_K> &b) {
#pragma unroll
    for (int i = 0; i < 6; ++i) b.v[i] = gload16u(blk + 16 * i);
    b.tail = gload16u(blk + 94);  // bytes 94..109: scales at +2, d at +14
}

// ---- LDS staging of packed weights ------------------------------------------------------------------------------
// dma_to_lds copies `bytes` (a multiple of 16; src and dst 16-byte aligned) from global memory into LDS with the
// gfx950 LDS-DMA load (global_load_lds_dwordx4): each wave instruction moves 1 KiB of consecutive global bytes (fully
// coalesced 128-bit loads) to 1 KiB of consecutive LDS at the wave-uniform base given in M0, lane i filling bytes
// 16 i .. 16 i + 15; the data never passes through VGPRs. Pieces are dealt round-robin over the NT / 64 waves.
// The data is visible after dma_wait() (all of this wave's vector loads complete) and a workgroup barrier.
template <int NT>
__device__ __forceinline__ void dma_to_lds(uint8_t *dst, const uint8_t *src, int bytes) {
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    for (int p = wave * 1024; p < bytes; p += NT * 16) {
        if (p + lane * 16 < bytes)
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *) (src + p + lane * 16),
                                             (__attribute__((address_space(3))) void *) (dst + p), 16, 0, 0);
    }
}
// Gathering form: piece i of 16 bytes comes from src_of(16 i) (any 16-byte-aligned global address per piece) and lands
// at dst + 16 i.
template <int NT, class F>
__device__ __forceinline__ void dma_gather_to_lds(uint8_t *dst, int bytes, F src_of) {
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    for (int p = wave * 1024; p < bytes; p += NT * 16) {
        if (p + lane * 16 < bytes)
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *) src_of(p + lane * 16),
                                             (__attribute__((address_space(3))) void *) (dst + p), 16, 0, 0);
    }
}
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

// Whole block from LDS (Q4_K / Q5_K blocks sit at 16-byte-aligned offsets of a staged region; Q6_K / Q3_K at 2-byte).
template <int T> __device__ __forceinline__ void lds_block_load(const uint8_t *blk, BlockRegs<T> &b);
template <> __device__ __forceinline__ void lds_block_load<T_Q4_K>(const uint8_t *blk, BlockRegs<T_Q4_K> &b) {
#pragma unroll
    for (int i = 0; i < 9; ++i) b.v[i] = *(const uint4 *) (blk + 16 * i);
}
template <> __device__ __forceinline__ void lds_block_load<T_Q5_K>(const uint8_t *blk, BlockRegs<T_Q5_K> &b) {
#pragma unroll
    for (int i = 0; i < 11; ++i) b.v[i] = *(const uint4 *) (blk + 16 * i);
}
template <> __device__ __forceinline__ void lds_block_load<T_Q6_K>(const uint8_t *blk, BlockRegs<T_Q6_K> &b) {
#pragma unroll
    for (int i = 0; i < 13; ++i) b.v[i] = lds16u(blk + 16 * i);
    const uintptr_t a = (uintptr_t) (blk + 208);
    b.d = (*(const uint32_t *) (a & ~(uintptr_t) 3) >> ((a & 3u) * 8u)) & 0xffffu;
}
template <> __device__ __forceinline__ void lds_block_load<T_Q3_K>(const uint8_t *blk, BlockRegs<T_Q3_K> &b) {
#pragma unroll
    for (int i = 0; i < 6; ++i) b.v[i] = lds16u(blk + 16 * i);
    b.tail = lds16u(blk + 94);
}

__device__ __forceinline__ uint32_t comp(const uint4 &v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }
__device__ __forceinline__ float ubyte_f(uint32_t w, int k) { return (float) ((w >> (8 * k)) & 0xffu); }
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

template <int T> __device__ __forceinline__ float block_dot(const BlockRegs<T> &b, const ActImg &x, int col0);

constexpr uint32_t kLo4 = 0x0F0F0F0Fu;

template <> __device__ __forceinline__ float block_dot<T_Q4_K>(const BlockRegs<T_Q4_K> &b, const ActImg &x, int col0) {
    const int8_t *qb = x.q + (col0 >> 8) * kImgQRow;
    const uint4 h = b.v[0];
    const uint32_t sc_lo = h.y & 0x3F3F3F3Fu, m_lo = h.z & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (h.w & kLo4) | ((h.y >> 2) & 0x30303030u);
    const uint32_t m_hi = ((h.w >> 4) & kLo4) | ((h.z >> 2) & 0x30303030u);
    float sumd = 0.0f, summ = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const uint4 q0 = b.v[1 + 2 * g], q1 = b.v[2 + 2 * g];  // qs[32g .. 32g+31]
        const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const int c = col0 + 64 * g;
        const int4 a0 = *(const int4 *) (qb + (c - col0)), a1 = *(const int4 *) (qb + (c - col0) + 16);
        const int4 e0 = *(const int4 *) (qb + (c - col0) + 32), e1 = *(const int4 *) (qb + (c - col0) + 48);
        const int a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        const int e[8] = {e0.x, e0.y, e0.z, e0.w, e1.x, e1.y, e1.z, e1.w};
        int dl = 0, dh = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            dl = dot4((int) (q[i] & kLo4), a[i], dl);
            dh = dot4((int) ((q[i] >> 4) & kLo4), e[i], dh);
        }
        const uint32_t scw = g < 2 ? sc_lo : sc_hi, mw = g < 2 ? m_lo : m_hi;
        const int k0 = 2 * (g & 1);
        const int blk = c >> 5;
        sumd = fmaf_(ubyte_f(scw, k0) * x.d[blk], (float) dl, sumd);
        sumd = fmaf_(ubyte_f(scw, k0 + 1) * x.d[blk + 1], (float) dh, sumd);
        summ = fmaf_(ubyte_f(mw, k0), x.s32[blk], summ);
        summ = fmaf_(ubyte_f(mw, k0 + 1), x.s32[blk + 1], summ);
    }
    return half_to_float(h.x & 0xffffu) * sumd - half_to_float(h.x >> 16) * summ;
}

template <> __device__ __forceinline__ float block_dot<T_Q5_K>(const BlockRegs<T_Q5_K> &b, const ActImg &x, int col0) {
    const int8_t *qb = x.q + (col0 >> 8) * kImgQRow;
    const uint4 h = b.v[0];
    const uint32_t sc_lo = h.y & 0x3F3F3F3Fu, m_lo = h.z & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (h.w & kLo4) | ((h.y >> 2) & 0x30303030u);
    const uint32_t m_hi = ((h.w >> 4) & kLo4) | ((h.z >> 2) & 0x30303030u);
    const uint32_t qh[8] = {b.v[1].x, b.v[1].y, b.v[1].z, b.v[1].w, b.v[2].x, b.v[2].y, b.v[2].z, b.v[2].w};
    float sumd = 0.0f, summ = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const uint4 q0 = b.v[3 + 2 * g], q1 = b.v[4 + 2 * g];
        const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const int c = col0 + 64 * g;
        const int4 a0 = *(const int4 *) (qb + (c - col0)), a1 = *(const int4 *) (qb + (c - col0) + 16);
        const int4 e0 = *(const int4 *) (qb + (c - col0) + 32), e1 = *(const int4 *) (qb + (c - col0) + 48);
        const int a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        const int e[8] = {e0.x, e0.y, e0.z, e0.w, e1.x, e1.y, e1.z, e1.w};
        int dl = 0, dh = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            // fifth bit: qh bit 2g (low values) and 2g+1 (high values), moved to bit 4 of each byte
            const uint32_t bl = (2 * g <= 4 ? (qh[i] << (4 - 2 * g)) : (qh[i] >> (2 * g - 4))) & 0x10101010u;
            const uint32_t bh = (2 * g + 1 <= 4 ? (qh[i] << (3 - 2 * g)) : (qh[i] >> (2 * g - 3))) & 0x10101010u;
            dl = dot4((int) ((q[i] & kLo4) | bl), a[i], dl);
            dh = dot4((int) (((q[i] >> 4) & kLo4) | bh), e[i], dh);
        }
        const uint32_t scw = g < 2 ? sc_lo : sc_hi, mw = g < 2 ? m_lo : m_hi;
        const int k0 = 2 * (g & 1);
        const int blk = c >> 5;
        sumd = fmaf_(ubyte_f(scw, k0) * x.d[blk], (float) dl, sumd);
        sumd = fmaf_(ubyte_f(scw, k0 + 1) * x.d[blk + 1], (float) dh, sumd);
        summ = fmaf_(ubyte_f(mw, k0), x.s32[blk], summ);
        summ = fmaf_(ubyte_f(mw, k0 + 1), x.s32[blk + 1], summ);
    }
    return half_to_float(h.x & 0xffffu) * sumd - half_to_float(h.x >> 16) * summ;
}

// 16-value group term of Q6_K / Q3_K: d8 * (u . a) - bias * s16, with u the unsigned codes.
__device__ __forceinline__ float group_term(int dotu, float d8, float s16, float bias) {
    return fmaf_(d8, (float) dotu, -bias * s16);
}

template <> __device__ __forceinline__ float block_dot<T_Q6_K>(const BlockRegs<T_Q6_K> &b, const ActImg &x, int col0) {
    const int8_t *qb = x.q + (col0 >> 8) * kImgQRow;
    const uint4 sc = b.v[12];  // int8 scales[16]
    float sum = 0.0f;
#pragma unroll
    for (int n = 0; n < 2; ++n) {
        const uint4 A0 = b.v[4 * n], A1 = b.v[4 * n + 1];      // ql[64n .. 64n+31]
        const uint4 B0 = b.v[4 * n + 2], B1 = b.v[4 * n + 3];  // ql[64n+32 .. 64n+63]
        const uint4 Q0 = b.v[8 + 2 * n], Q1 = b.v[9 + 2 * n];  // qh[32n .. 32n+31]
        const uint32_t A[8] = {A0.x, A0.y, A0.z, A0.w, A1.x, A1.y, A1.z, A1.w};
        const uint32_t B[8] = {B0.x, B0.y, B0.z, B0.w, B1.x, B1.y, B1.z, B1.w};
        const uint32_t Q[8] = {Q0.x, Q0.y, Q0.z, Q0.w, Q1.x, Q1.y, Q1.z, Q1.w};
#pragma unroll
        for (int kind = 0; kind < 4; ++kind) {  // values 128n + 32 kind + l
#pragma unroll
            for (int half = 0; half < 2; ++half) {  // l in [16 half, 16 half + 16)
                const int c = col0 + 128 * n + 32 * kind + 16 * half;
                const int4 a = *(const int4 *) (qb + (c - col0));
                const int av[4] = {a.x, a.y, a.z, a.w};
                int du = 0;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const int i = 4 * half + w;
                    uint32_t u;
                    if (kind == 0) u = (A[i] & kLo4) | ((Q[i] << 4) & 0x30303030u);
                    else if (kind == 1) u = (B[i] & kLo4) | ((Q[i] << 2) & 0x30303030u);
                    else if (kind == 2) u = ((A[i] >> 4) & kLo4) | (Q[i] & 0x30303030u);
                    else u = ((B[i] >> 4) & kLo4) | ((Q[i] >> 2) & 0x30303030u);
                    du = dot4((int) u, av[w], du);
                }
                const int gi = 8 * n + 2 * kind + half;
                const float s = sbyte_f(comp(sc, gi >> 2), gi & 3);
                sum = fmaf_(s, group_term(du, x.d[c >> 5], x.s16[c >> 4], 32.0f), sum);
            }
        }
    }
    return half_to_float(b.d) * sum;
}

template <> __device__ __forceinline__ float block_dot<T_Q3_K>(const BlockRegs<T_Q3_K> &b, const ActImg &x, int col0) {
    const int8_t *qb = x.q + (col0 >> 8) * kImgQRow;
    const uint4 t = b.tail;
    // scale bytes 0..11 start at byte 2 of the tail: realign to words S0 (scales 0-3), S1 (4-7), S2 (8-11)
    const uint32_t S0 = __builtin_amdgcn_alignbit(t.y, t.x, 16), S1 = __builtin_amdgcn_alignbit(t.z, t.y, 16);
    const uint32_t S2 = __builtin_amdgcn_alignbit(t.w, t.z, 16);
    // 6-bit scale of group g (stored + 32): low nibble from S0/S1 (g < 8) or their high nibbles (g >= 8), top two
    // bits from S2 byte g%4 at shift 2*(g/4)
    const uint32_t SC[4] = {(S0 & kLo4) | ((S2 << 4) & 0x30303030u), (S1 & kLo4) | ((S2 << 2) & 0x30303030u),
                            ((S0 >> 4) & kLo4) | (S2 & 0x30303030u), ((S1 >> 4) & kLo4) | ((S2 >> 2) & 0x30303030u)};
    const uint32_t HM[8] = {b.v[0].x, b.v[0].y, b.v[0].z, b.v[0].w, b.v[1].x, b.v[1].y, b.v[1].z, b.v[1].w};
    float sum = 0.0f;
#pragma unroll
    for (int n = 0; n < 2; ++n) {
        const uint4 q0 = b.v[2 + 2 * n], q1 = b.v[3 + 2 * n];  // qs[32n .. 32n+31]
        const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {  // values 128n + 32j + l
            const int hs = 4 * n + j;  // hmask bit of this (n, j)
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const int c = col0 + 128 * n + 32 * j + 16 * half;
                const int4 a = *(const int4 *) (qb + (c - col0));
                const int av[4] = {a.x, a.y, a.z, a.w};
                int du = 0;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const int i = 4 * half + w;
                    const uint32_t hb = (hs <= 2 ? (HM[i] << (2 - hs)) : (HM[i] >> (hs - 2))) & 0x04040404u;
                    const uint32_t u = ((q[i] >> (2 * j)) & 0x03030303u) | hb;
                    du = dot4((int) u, av[w], du);
                }
                const int g = 8 * n + 2 * j + half;
                const float s = ubyte_f(SC[g >> 2], g & 3) - 32.0f;
                sum = fmaf_(s, group_term(du, x.d[c >> 5], x.s16[c >> 4], 4.0f), sum);
            }
        }
    }
    return half_to_float(t.w >> 16) * sum;
}

}  // namespace fns::dev
