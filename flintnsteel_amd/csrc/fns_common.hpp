// fns_common.hpp - shared device helpers of the MI355X (gfx950, wave64) MoE FFN kernels.
//
// GGUF block layouts (byte offsets; the layouts are those of the GGUF file format, ggml-common.h of llama.cpp
// 19ab5a5e, which the reference compiles from an external checkout):
//   Q8_1  36 B / 32 values : half d | half s (sum of the unquantised values) | int8 qs[32]
//   Q3_K 110 B / 256 values: hmask[32] @0 | qs[64] @32 | scales[12] @96 | half d @108
//   Q4_K 144 B / 256 values: half d @0 | half dmin @2 | scales[12] @4 | qs[128] @16
//   Q5_K 176 B / 256 values: half d @0 | half dmin @2 | scales[12] @4 | qh[32] @16 | qs[128] @48
//   Q6_K 210 B / 256 values: ql[128] @0 | qh[64] @128 | int8 scales[16] @192 | half d @208
//   Q8_0  34 B / 32 values : half d | int8 qs[32]  (the kernels handle 8 consecutive blocks, 272 B, as one unit)
// Q3_K and Q6_K blocks are only 2-byte aligned inside a row; gfx950 global loads accept unaligned addresses, so the
// 16-byte fragments below are read with memcpy-style loads at their true addresses.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "fns_lanes.hpp"

// Phase-timing hooks. The library build defines them as no-ops; a tuning build passes -DFNS_PROBE_HEADER=<file> to
// record wall-clock marks at these points instead.
#ifdef FNS_PROBE_HEADER
#include FNS_PROBE_HEADER
#else
#define FNS_MARK(k, wg, i) ((void) (wg))
#define MMQ_MARK(i) ((void) 0)
#define MMQ_NOTE(v) ((void) 0)
#define PF_MARK(k, i) ((void) 0)
#endif

namespace fns::dev {

constexpr int kWave = 64;

enum : int {
    T_Q8_0 = 8, T_Q8_1 = 9, T_Q3_K = 11, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14,
    T_IQ3_XXS = 18, T_IQ3_S = 21, T_IQ2_S = 22, T_IQ4_XS = 23, T_BF16 = 30
};

template <int T> struct Traits;
template <> struct Traits<T_Q3_K> { static constexpr int bytes = 110, slots = 4; };
template <> struct Traits<T_Q4_K> { static constexpr int bytes = 144, slots = 8; };
template <> struct Traits<T_Q5_K> { static constexpr int bytes = 176, slots = 8; };
template <> struct Traits<T_Q6_K> { static constexpr int bytes = 210, slots = 8; };
// Q8_0 (34 B per 32 values: half d | int8 qs[32]): the kernels' 256-value unit is 8 consecutive blocks (272 B).
template <> struct Traits<T_Q8_0> { static constexpr int bytes = 272, slots = 4; };
// IQ formats (256 values per block; decoded by the quarter kernels only):
//   IQ4_XS 136 B: half d | u16 scales_h | scales_l[4] | qs[128] (4-bit indices into the IQ4_NL values)
//   IQ3_XXS 98 B: half d | grid indices[64] | 8 x u32 (4 x 7 sign bits + 4-bit scale per 32 values)
//   IQ3_S  110 B: half d | grid indices[64] | qh[8] (9th index bits) | signs[32] | scales[4] (4 bits per 32 values)
//   IQ2_S   82 B: half d | grid indices[32] | signs[32] | qh[8] (2 high index bits per 8 values) | scales[8]
template <> struct Traits<T_IQ4_XS> { static constexpr int bytes = 136, slots = 4; };
template <> struct Traits<T_IQ3_XXS> { static constexpr int bytes = 98, slots = 4; };
template <> struct Traits<T_IQ3_S> { static constexpr int bytes = 110, slots = 4; };
template <> struct Traits<T_IQ2_S> { static constexpr int bytes = 82, slots = 4; };

__host__ __device__ constexpr int block_bytes(int t) {
    return t == T_Q3_K ? 110 : t == T_Q4_K ? 144 : t == T_Q5_K ? 176 : t == T_Q6_K ? 210 : t == T_Q8_0 ? 272
         : t == T_IQ4_XS ? 136 : t == T_IQ3_XXS ? 98 : t == T_IQ3_S ? 110 : t == T_IQ2_S ? 82 : 0;
}

__device__ __forceinline__ float half_to_float(uint32_t bits16) {
    return (float) __builtin_bit_cast(_Float16, (uint16_t) bits16);
}
__device__ __forceinline__ uint32_t float_to_half(float f) {  // round to nearest even
    return (uint32_t) __builtin_bit_cast(uint16_t, (_Float16) f);
}

// 16 bytes at an address that may be only 2-byte aligned.
__device__ __forceinline__ uint4 load16(const uint8_t *p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}

__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// exp(x): Cody-Waite reduction with ln2 split in a 17-bit head and a tail, degree-7 Taylor polynomial on
// |r| <= ln2/2, scaling by 2^n in two exact steps. Explicit fmaf everywhere: the CPU oracle evaluates the same
// sequence and gets the same bits.
__device__ __forceinline__ float fns_expf(float x) {
    if (x < -104.0f) return 0.0f;
    if (x > 88.72f) return __builtin_inff();
    const float n = __builtin_rintf(x * 1.44269504088896341f);
    float r = __builtin_fmaf(n, -0.693145751953125f, x);
    r = __builtin_fmaf(n, -1.42860682030941723e-6f, r);
    float p = 1.0f / 5040.0f;
    p = __builtin_fmaf(p, r, 1.0f / 720.0f);
    p = __builtin_fmaf(p, r, 1.0f / 120.0f);
    p = __builtin_fmaf(p, r, 1.0f / 24.0f);
    p = __builtin_fmaf(p, r, 1.0f / 6.0f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    int ni = (int) n;
    const int h = ni < -100 ? -64 : (ni > 127 ? 1 : 0);
    ni -= h;
    const float s1 = __builtin_bit_cast(float, (uint32_t) (ni + 127) << 23);
    const float s2 = __builtin_bit_cast(float, (uint32_t) (h + 127) << 23);
    return (p * s1) * s2;
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + fns_expf(-g)); }

// Butterfly sum over aligned groups of W lanes (W a power of two <= 64); every lane of the group gets the sum.
template <int W> __device__ __forceinline__ float group_sum(float v) { return lanes_sum<W>(v); }

// Per-byte subtraction of a constant c in [1, 127] for bytes u in [0, 127 - c] ... [0, 127]: (u + 128 - c) ^ 0x80
// never carries across bytes and yields the two's-complement byte u - c.
template <int C> __device__ __forceinline__ int bytes_sub(int w) {
    constexpr uint32_t add = 0x01010101u * (uint32_t) (128 - C);
    return (int) (((uint32_t) w + add) ^ 0x80808080u);
}

// Activation row in LDS: int8 q[npad] (16-byte aligned), float d[npad/32] (Q8_1 scale), float s16[npad/16] and
// float s32[npad/32] (d * sum of the quantised values of each 16 / 32 columns, for the K-quant min / zero terms).
struct ActView {
    const int8_t *q;
    const float *d;
    const float *s16;
};

__host__ __device__ constexpr int act_lds_bytes(int npad) { return npad + npad / 32 * 4 + npad / 16 * 4 + npad / 32 * 4; }

// Copies one Q8_1 row (nblk blocks of 36 bytes) from global memory into the LDS image.
__device__ __forceinline__ void stage_q8_1_row(const uint8_t *__restrict__ src, int nblk, int8_t *q, float *d,
                                               float *s16, int tid, int nthreads) {
    float *s32 = s16 + 2 * nblk;
    for (int b = tid; b < nblk; b += nthreads) {
        const uint32_t *w = (const uint32_t *) (src + (size_t) b * 36);
        uint32_t v[9];
#pragma unroll
        for (int i = 0; i < 9; ++i) v[i] = w[i];
        const float db = half_to_float(v[0] & 0xffffu);
        int sa = 0, sb = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) sa = dot4((int) v[1 + i], 0x01010101, sa);
#pragma unroll
        for (int i = 0; i < 4; ++i) sb = dot4((int) v[5 + i], 0x01010101, sb);
        uint4 *dq = (uint4 *) (q + 32 * b);
        dq[0] = make_uint4(v[1], v[2], v[3], v[4]);
        dq[1] = make_uint4(v[5], v[6], v[7], v[8]);
        d[b] = db;
        s16[2 * b] = db * (float) sa;
        s16[2 * b + 1] = db * (float) sb;
        s32[b] = db * (float) (sa + sb);
    }
}

// ---- per-type slot products -------------------------------------------------------------------------------
// A "slot" is one 16-byte fragment of packed quants and the values it encodes: 32 values for Q4_K/Q5_K/Q6_K
// (8 slots per block), 64 values for Q3_K (4 slots per block). A lane keeps the same slot position j (and so the
// same activation columns) for every row it processes: the activation side (ActFrag) is read from LDS once and
// reused; frag_dot returns the slot's contribution to W_row . x in fp32 (exact integer sub-block dots, fp32 scales).

// Loads through the global address space (the expert pointers come from a table in memory, which would otherwise
// make the compiler emit generic flat loads).
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
template <class V> __device__ __forceinline__ V gload(const uint8_t *p) {
    if constexpr (sizeof(V) == 16) {
        const u32x4_t v = *(const __attribute__((address_space(1))) u32x4_t *) p;
        return __builtin_bit_cast(V, v);
    } else {
        return *(const __attribute__((address_space(1))) V *) p;
    }
}
// 16 bytes at a global address that may be only 2-byte aligned.
__device__ __forceinline__ uint4 gload16u(const uint8_t *p) {
    uint4 v;
    __builtin_memcpy(&v, (const __attribute__((address_space(1))) uint8_t *) p, 16);
    return v;
}

struct Frag {
    uint4 a, b, c;  // raw fragments (meaning depends on the type)
    uint32_t e;     // Q6_K: the f16 d
};

template <int T> __device__ __forceinline__ void slot_load(const uint8_t *blk, int j, Frag &f);

template <> __device__ __forceinline__ void slot_load<T_Q4_K>(const uint8_t *blk, int j, Frag &f) {
    f.a = gload<uint4>(blk);                // d, dmin, scales
    f.b = gload<uint4>(blk + 16 + 16 * j);  // qs[16j .. 16j+15]
}
template <> __device__ __forceinline__ void slot_load<T_Q5_K>(const uint8_t *blk, int j, Frag &f) {
    f.a = gload<uint4>(blk);
    f.c = gload<uint4>(blk + 16 + 16 * (j & 1));  // qh[16h .. 16h+15]
    f.b = gload<uint4>(blk + 48 + 16 * j);
}
template <> __device__ __forceinline__ void slot_load<T_Q6_K>(const uint8_t *blk, int j, Frag &f) {
    const int n = j >> 2, jj = j & 3;
    f.b = gload16u(blk + 64 * n + 16 * jj);              // ql
    f.c = gload16u(blk + 128 + 32 * n + 16 * (jj & 1));  // qh
    f.a = gload16u(blk + 192);                           // scales[0..15]
    f.e = gload<uint16_t>(blk + 208);
}
template <> __device__ __forceinline__ void slot_load<T_Q3_K>(const uint8_t *blk, int j, Frag &f) {
    f.b = gload16u(blk + 32 + 16 * j);   // qs[16j .. 16j+15]
    f.c = gload16u(blk + 16 * (j & 1));  // hmask[16h .. 16h+15]
    f.a = gload16u(blk + 94);            // bytes 94..109: scales[0..11] at +2, d at +14
}

__device__ __forceinline__ uint32_t word(const uint4 &v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}
__device__ __forceinline__ uint32_t byte_of(const uint4 &v, int i) { return (word(v, i >> 2) >> (8 * (i & 3))) & 0xffu; }

// Activation registers of one slot.
template <int T> struct ActFrag {
    int4 q0, q1;
    float d0, d1, s0, s1;
};
template <> struct ActFrag<T_Q3_K> {
    int4 q[4];
    float d[4];
};

template <int T> __device__ __forceinline__ ActFrag<T> act_frag(const ActView &x, int j, int col0);

// Q4_K / Q5_K slot j: g = j/2, h = j%2; low nibbles = values 64g+16h+t (sub-block 2g), high = values +32 (2g+1).
template <> __device__ __forceinline__ ActFrag<T_Q4_K> act_frag<T_Q4_K>(const ActView &x, int j, int col0) {
    const int clo = col0 + 64 * (j >> 1) + 16 * (j & 1), chi = clo + 32;
    ActFrag<T_Q4_K> r;
    r.q0 = *(const int4 *) (x.q + clo);
    r.q1 = *(const int4 *) (x.q + chi);
    r.d0 = x.d[clo >> 5];
    r.d1 = x.d[chi >> 5];
    r.s0 = x.s16[clo >> 4];
    r.s1 = x.s16[chi >> 4];
    return r;
}
template <> __device__ __forceinline__ ActFrag<T_Q5_K> act_frag<T_Q5_K>(const ActView &x, int j, int col0) {
    const ActFrag<T_Q4_K> a = act_frag<T_Q4_K>(x, j, col0);
    return ActFrag<T_Q5_K>{a.q0, a.q1, a.d0, a.d1, a.s0, a.s1};
}
// Q6_K slot j: n = j/4, jj = j%4; low values 128n+16jj+t, high values +64.
template <> __device__ __forceinline__ ActFrag<T_Q6_K> act_frag<T_Q6_K>(const ActView &x, int j, int col0) {
    const int clo = col0 + 128 * (j >> 2) + 16 * (j & 3), chi = clo + 64;
    ActFrag<T_Q6_K> r;
    r.q0 = *(const int4 *) (x.q + clo);
    r.q1 = *(const int4 *) (x.q + chi);
    r.d0 = x.d[clo >> 5];
    r.d1 = x.d[chi >> 5];
    r.s0 = r.s1 = 0.0f;
    return r;
}
// Q3_K slot j (0..3): n = j/2, h = j%2; group jj holds values 128n+32jj+16h+t.
template <> __device__ __forceinline__ ActFrag<T_Q3_K> act_frag<T_Q3_K>(const ActView &x, int j, int col0) {
    ActFrag<T_Q3_K> r;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
        const int c = col0 + 128 * (j >> 1) + 32 * jj + 16 * (j & 1);
        r.q[jj] = *(const int4 *) (x.q + c);
        r.d[jj] = x.d[c >> 5];
    }
    return r;
}

// 6-bit scales/mins of sub-blocks 2g and 2g+1 of a Q4_K/Q5_K block (scale bytes in h.y, h.z, h.w), extracted with
// word-wide masks: bytes 0-3 of sc(0..3) = w1 & 63, m(0..3) = w2 & 63; sc(4..7) = low nibbles of w3 | top bits of w1,
// m(4..7) = high nibbles of w3 | top bits of w2 (ggml get_scale_min_k4, four values at a time).
__device__ __forceinline__ void scales_k4(const uint4 &h, int g, int &sc0, int &sc1, int &m0, int &m1) {
    const uint32_t w1 = h.y, w2 = h.z, w3 = h.w;
    const uint32_t sc_lo = w1 & 0x3F3F3F3Fu, m_lo = w2 & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (w3 & 0x0F0F0F0Fu) | ((w1 >> 2) & 0x30303030u);
    const uint32_t m_hi = ((w3 >> 4) & 0x0F0F0F0Fu) | ((w2 >> 2) & 0x30303030u);
    const uint32_t scw = g < 2 ? sc_lo : sc_hi, mw = g < 2 ? m_lo : m_hi;
    const int sh = 16 * (g & 1);
    sc0 = (int) ((scw >> sh) & 0xFFu);
    sc1 = (int) ((scw >> (sh + 8)) & 0xFFu);
    m0 = (int) ((mw >> sh) & 0xFFu);
    m1 = (int) ((mw >> (sh + 8)) & 0xFFu);
}

template <int T> __device__ __forceinline__ float frag_dot(const Frag &f, int j, const ActFrag<T> &x);

template <> __device__ __forceinline__ float frag_dot<T_Q4_K>(const Frag &f, int j, const ActFrag<T_Q4_K> &x) {
    int dlo = 0, dhi = 0;
    dlo = dot4((int) (f.b.x & 0x0F0F0F0Fu), x.q0.x, dlo);
    dlo = dot4((int) (f.b.y & 0x0F0F0F0Fu), x.q0.y, dlo);
    dlo = dot4((int) (f.b.z & 0x0F0F0F0Fu), x.q0.z, dlo);
    dlo = dot4((int) (f.b.w & 0x0F0F0F0Fu), x.q0.w, dlo);
    dhi = dot4((int) ((f.b.x >> 4) & 0x0F0F0F0Fu), x.q1.x, dhi);
    dhi = dot4((int) ((f.b.y >> 4) & 0x0F0F0F0Fu), x.q1.y, dhi);
    dhi = dot4((int) ((f.b.z >> 4) & 0x0F0F0F0Fu), x.q1.z, dhi);
    dhi = dot4((int) ((f.b.w >> 4) & 0x0F0F0F0Fu), x.q1.w, dhi);
    int sc0, sc1, m0, m1;
    scales_k4(f.a, j >> 1, sc0, sc1, m0, m1);
    const float d = half_to_float(f.a.x & 0xffffu), dmin = half_to_float(f.a.x >> 16);
    const float sd = (float) (sc0 * dlo) * x.d0 + (float) (sc1 * dhi) * x.d1;
    const float sm = (float) m0 * x.s0 + (float) m1 * x.s1;
    return d * sd - dmin * sm;
}

// Q5_K: as Q4_K with a fifth bit from qh[16h+t]: bit 2g (low values) and bit 2g+1 (high values).
template <> __device__ __forceinline__ float frag_dot<T_Q5_K>(const Frag &f, int j, const ActFrag<T_Q5_K> &x) {
    const int g = j >> 1;
    const int sl = 2 * g, sh = 2 * g + 1;
    auto lo = [&](uint32_t q, uint32_t qh) { return (int) ((q & 0x0F0F0F0Fu) | (((qh >> sl) & 0x01010101u) << 4)); };
    auto hi = [&](uint32_t q, uint32_t qh) {
        return (int) (((q >> 4) & 0x0F0F0F0Fu) | (((qh >> sh) & 0x01010101u) << 4));
    };
    int dlo = 0, dhi = 0;
    dlo = dot4(lo(f.b.x, f.c.x), x.q0.x, dlo);
    dlo = dot4(lo(f.b.y, f.c.y), x.q0.y, dlo);
    dlo = dot4(lo(f.b.z, f.c.z), x.q0.z, dlo);
    dlo = dot4(lo(f.b.w, f.c.w), x.q0.w, dlo);
    dhi = dot4(hi(f.b.x, f.c.x), x.q1.x, dhi);
    dhi = dot4(hi(f.b.y, f.c.y), x.q1.y, dhi);
    dhi = dot4(hi(f.b.z, f.c.z), x.q1.z, dhi);
    dhi = dot4(hi(f.b.w, f.c.w), x.q1.w, dhi);
    int sc0, sc1, m0, m1;
    scales_k4(f.a, g, sc0, sc1, m0, m1);
    const float d = half_to_float(f.a.x & 0xffffu), dmin = half_to_float(f.a.x >> 16);
    const float sd = (float) (sc0 * dlo) * x.d0 + (float) (sc1 * dhi) * x.d1;
    const float sm = (float) m0 * x.s0 + (float) m1 * x.s1;
    return d * sd - dmin * sm;
}

// Q6_K slot j: n = j/4, jj = j%4; ql low nibble = value 128n+16jj+t, high nibble = value +64; two qh bits from
// qh[32n+16(jj%2)+t] at shift 2*(jj/2) (low) and 2*(jj/2)+4 (high); 6-bit value - 32. Scales (int8, 16 values each):
// group 8n+jj (low) and 8n+jj+4 (high).
template <> __device__ __forceinline__ float frag_dot<T_Q6_K>(const Frag &f, int j, const ActFrag<T_Q6_K> &x) {
    const int n = j >> 2, jj = j & 3;
    const int shl = 2 * (jj >> 1), shh = shl + 4;
    auto lo = [&](uint32_t q, uint32_t qh) {
        return bytes_sub<32>((int) ((q & 0x0F0F0F0Fu) | (((qh >> shl) & 0x03030303u) << 4)));
    };
    auto hi = [&](uint32_t q, uint32_t qh) {
        return bytes_sub<32>((int) (((q >> 4) & 0x0F0F0F0Fu) | (((qh >> shh) & 0x03030303u) << 4)));
    };
    int dlo = 0, dhi = 0;
    dlo = dot4(lo(f.b.x, f.c.x), x.q0.x, dlo);
    dlo = dot4(lo(f.b.y, f.c.y), x.q0.y, dlo);
    dlo = dot4(lo(f.b.z, f.c.z), x.q0.z, dlo);
    dlo = dot4(lo(f.b.w, f.c.w), x.q0.w, dlo);
    dhi = dot4(hi(f.b.x, f.c.x), x.q1.x, dhi);
    dhi = dot4(hi(f.b.y, f.c.y), x.q1.y, dhi);
    dhi = dot4(hi(f.b.z, f.c.z), x.q1.z, dhi);
    dhi = dot4(hi(f.b.w, f.c.w), x.q1.w, dhi);
    const int glo = 8 * n + jj;  // 0..11; the high group is glo + 4 (same word position + 1 word)
    const uint32_t wlo = word(f.a, glo >> 2);
    const uint32_t whi = word(f.a, (glo >> 2) + 1);
    const int sclo = (int) (int8_t) ((wlo >> (8 * (glo & 3))) & 0xffu);
    const int schi = (int) (int8_t) ((whi >> (8 * (glo & 3))) & 0xffu);
    const float d = half_to_float(f.e);
    return d * ((float) (sclo * dlo) * x.d0 + (float) (schi * dhi) * x.d1);
}

// Q3_K slot j (0..3): qs[16j+t] (n = j/2, h = j%2) holds 2-bit values for jj = 0..3 at value 128n+32jj+16h+t; the
// high bit is hmask[16h+t] bit 4n+jj (set: +0, clear: -4). Scale group 8n+2jj+h, 6-bit value - 32, packed in
// 12 bytes (low nibbles in bytes 0..7, high 2-bit pairs in bytes 8..11). f.a holds block bytes 94..109.
template <> __device__ __forceinline__ float frag_dot<T_Q3_K>(const Frag &f, int j, const ActFrag<T_Q3_K> &x) {
    const int n = j >> 1, h = j & 1;
    float acc = 0.0f;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
        const int hs = 4 * n + jj;
        auto val = [&](uint32_t q, uint32_t hm) {
            return bytes_sub<4>((int) (((q >> (2 * jj)) & 0x03030303u) | (((hm >> hs) & 0x01010101u) << 2)));
        };
        int dd = 0;
        dd = dot4(val(f.b.x, f.c.x), x.q[jj].x, dd);
        dd = dot4(val(f.b.y, f.c.y), x.q[jj].y, dd);
        dd = dot4(val(f.b.z, f.c.z), x.q[jj].z, dd);
        dd = dot4(val(f.b.w, f.c.w), x.q[jj].w, dd);
        const int g = 8 * n + 2 * jj + h;
        // scales field byte i is f.a byte i + 2
        const uint32_t lo4 = g < 8 ? (byte_of(f.a, 2 + g) & 0xFu) : (byte_of(f.a, 2 + g - 8) >> 4);
        const uint32_t hi2 = (byte_of(f.a, 2 + 8 + (g & 3)) >> (2 * (g >> 2))) & 3u;
        const int sc = (int) (lo4 | (hi2 << 4)) - 32;
        acc += (float) (sc * dd) * x.d[jj];
    }
    return half_to_float(f.a.w >> 16) * acc;
}

template <int T> __device__ __forceinline__ float slot_dot(const Frag &f, int j, int col0, const ActView &x) {
    return frag_dot<T>(f, j, act_frag<T>(x, j, col0));
}

}  // namespace fns::dev
