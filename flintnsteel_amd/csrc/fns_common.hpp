// fns_common.hpp - shared device helpers of the MI355X (gfx950, wave64) MoE FFN kernels.
//
// GGUF block layouts (byte offsets; the layouts are those of the GGUF file format, ggml-common.h of llama.cpp
// 19ab5a5e, which the reference compiles from an external checkout):
//   Q8_1  36 B / 32 values : half d | half s (sum of the unquantised values) | int8 qs[32]
//   Q3_K 110 B / 256 values: hmask[32] @0 | qs[64] @32 | scales[12] @96 | half d @108
//   Q4_K 144 B / 256 values: half d @0 | half dmin @2 | scales[12] @4 | qs[128] @16
//   Q5_K 176 B / 256 values: half d @0 | half dmin @2 | scales[12] @4 | qh[32] @16 | qs[128] @48
//   Q6_K 210 B / 256 values: ql[128] @0 | qh[64] @128 | int8 scales[16] @192 | half d @208
// Q3_K and Q6_K blocks are only 2-byte aligned inside a row; gfx950 global loads accept unaligned addresses, so the
// 16-byte fragments below are read with memcpy-style loads at their true addresses.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace fns::dev {

constexpr int kWave = 64;

enum : int { T_Q8_0 = 8, T_Q8_1 = 9, T_Q3_K = 11, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_BF16 = 30 };

template <int T> struct Traits;
template <> struct Traits<T_Q3_K> { static constexpr int bytes = 110, slots = 4; };
template <> struct Traits<T_Q4_K> { static constexpr int bytes = 144, slots = 8; };
template <> struct Traits<T_Q5_K> { static constexpr int bytes = 176, slots = 8; };
template <> struct Traits<T_Q6_K> { static constexpr int bytes = 210, slots = 8; };

__host__ __device__ constexpr int block_bytes(int t) {
    return t == T_Q3_K ? 110 : t == T_Q4_K ? 144 : t == T_Q5_K ? 176 : t == T_Q6_K ? 210 : t == T_Q8_0 ? 34 : 0;
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
template <int W> __device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// Per-byte subtraction of a constant c in [1, 127] for bytes u in [0, 127 - c] ... [0, 127]: (u + 128 - c) ^ 0x80
// never carries across bytes and yields the two's-complement byte u - c.
template <int C> __device__ __forceinline__ int bytes_sub(int w) {
    constexpr uint32_t add = 0x01010101u * (uint32_t) (128 - C);
    return (int) (((uint32_t) w + add) ^ 0x80808080u);
}

// Activation row in LDS: int8 q[npad] (16-byte aligned), float d[npad/32] (Q8_1 scale), float s16[npad/16]
// (d * sum of the 16 quantised values of each half block, for the K-quant min term).
struct ActView {
    const int8_t *q;
    const float *d;
    const float *s16;
};

__host__ __device__ constexpr int act_lds_bytes(int npad) { return npad + npad / 32 * 4 + npad / 16 * 4; }

// Copies one Q8_1 row (nblk blocks of 36 bytes) from global memory into the LDS view.
__device__ __forceinline__ void stage_q8_1_row(const uint8_t *__restrict__ src, int nblk, int8_t *q, float *d,
                                               float *s16, int tid, int nthreads) {
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
    }
}

// ---- per-type slot products -------------------------------------------------------------------------------
// A "slot" is one 16-byte fragment of packed quants and the values it encodes: 32 values for Q4_K/Q5_K/Q6_K
// (8 slots per block), 64 values for Q3_K (4 slots per block). slot_dot returns that fragment's contribution to
// W_row . x in fp32; integer dot products are exact, scales are applied per 16- or 32-value group.

struct Frag {
    uint4 a, b, c;  // raw fragments (meaning depends on the type)
    uint32_t e;     // Q6_K: the f16 d
};

template <int T> __device__ __forceinline__ void slot_load(const uint8_t *blk, int j, Frag &f);

template <> __device__ __forceinline__ void slot_load<T_Q4_K>(const uint8_t *blk, int j, Frag &f) {
    f.a = *(const uint4 *) blk;               // d, dmin, scales
    f.b = *(const uint4 *) (blk + 16 + 16 * j);  // qs[16j .. 16j+15]
}
template <> __device__ __forceinline__ void slot_load<T_Q5_K>(const uint8_t *blk, int j, Frag &f) {
    f.a = *(const uint4 *) blk;
    f.c = *(const uint4 *) (blk + 16 + 16 * (j & 1));  // qh[16h .. 16h+15]
    f.b = *(const uint4 *) (blk + 48 + 16 * j);
}
template <> __device__ __forceinline__ void slot_load<T_Q6_K>(const uint8_t *blk, int j, Frag &f) {
    const int n = j >> 2, jj = j & 3;
    f.b = load16(blk + 64 * n + 16 * jj);                    // ql
    f.c = load16(blk + 128 + 32 * n + 16 * (jj & 1));        // qh
    f.a = load16(blk + 192);                                 // scales[0..15]
    uint16_t dh;
    __builtin_memcpy(&dh, blk + 208, 2);
    f.e = dh;
}
template <> __device__ __forceinline__ void slot_load<T_Q3_K>(const uint8_t *blk, int j, Frag &f) {
    f.b = load16(blk + 32 + 16 * j);           // qs[16j .. 16j+15]
    f.c = load16(blk + 16 * (j & 1));          // hmask[16h .. 16h+15]
    f.a = load16(blk + 94);                    // bytes 94..109: scales[0..11] at +2, d at +14
}

__device__ __forceinline__ uint32_t word(const uint4 &v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}
__device__ __forceinline__ uint32_t byte_of(const uint4 &v, int i) { return (word(v, i >> 2) >> (8 * (i & 3))) & 0xffu; }

// 6-bit scale and min of sub-block s (0..7) from the 12-byte K-quant scale field held in words 1..3 of `h`
// (h = first 16 bytes of a Q4_K/Q5_K block).
__device__ __forceinline__ void scale_min_k4(const uint4 &h, int s, int &sc, int &m) {
    const int o = 4;  // scales start at byte 4 of the block
    if (s < 4) {
        sc = (int) (byte_of(h, o + s) & 63u);
        m = (int) (byte_of(h, o + s + 4) & 63u);
    } else {
        sc = (int) ((byte_of(h, o + s + 4) & 0xFu) | ((byte_of(h, o + s - 4) >> 6) << 4));
        m = (int) ((byte_of(h, o + s + 4) >> 4) | ((byte_of(h, o + s) >> 6) << 4));
    }
}

template <int T> __device__ __forceinline__ float slot_dot(const Frag &f, int j, int col0, const ActView &x);

// Q4_K slot j: qs[16j..16j+15]; g = j/2, h = j%2. Low nibbles = values 64g+16h+t (sub-block 2g), high nibbles =
// values 64g+32+16h+t (sub-block 2g+1). Block value = d*sc*q - dmin*m.
template <> __device__ __forceinline__ float slot_dot<T_Q4_K>(const Frag &f, int j, int col0, const ActView &x) {
    const int g = j >> 1, h = j & 1;
    const int clo = col0 + 64 * g + 16 * h, chi = clo + 32;
    const int4 alo = *(const int4 *) (x.q + clo);
    const int4 ahi = *(const int4 *) (x.q + chi);
    int dlo = 0, dhi = 0;
    dlo = dot4((int) (f.b.x & 0x0F0F0F0Fu), alo.x, dlo);
    dlo = dot4((int) (f.b.y & 0x0F0F0F0Fu), alo.y, dlo);
    dlo = dot4((int) (f.b.z & 0x0F0F0F0Fu), alo.z, dlo);
    dlo = dot4((int) (f.b.w & 0x0F0F0F0Fu), alo.w, dlo);
    dhi = dot4((int) ((f.b.x >> 4) & 0x0F0F0F0Fu), ahi.x, dhi);
    dhi = dot4((int) ((f.b.y >> 4) & 0x0F0F0F0Fu), ahi.y, dhi);
    dhi = dot4((int) ((f.b.z >> 4) & 0x0F0F0F0Fu), ahi.z, dhi);
    dhi = dot4((int) ((f.b.w >> 4) & 0x0F0F0F0Fu), ahi.w, dhi);
    int sc0, m0, sc1, m1;
    scale_min_k4(f.a, 2 * g, sc0, m0);
    scale_min_k4(f.a, 2 * g + 1, sc1, m1);
    const float d = half_to_float(f.a.x & 0xffffu), dmin = half_to_float(f.a.x >> 16);
    const float sd = (float) (sc0 * dlo) * x.d[clo >> 5] + (float) (sc1 * dhi) * x.d[chi >> 5];
    const float sm = (float) m0 * x.s16[clo >> 4] + (float) m1 * x.s16[chi >> 4];
    return d * sd - dmin * sm;
}

// Q5_K: as Q4_K with a fifth bit from qh[16h+t]: bit 2g (low values) and bit 2g+1 (high values).
template <> __device__ __forceinline__ float slot_dot<T_Q5_K>(const Frag &f, int j, int col0, const ActView &x) {
    const int g = j >> 1, h = j & 1;
    const int clo = col0 + 64 * g + 16 * h, chi = clo + 32;
    const int4 alo = *(const int4 *) (x.q + clo);
    const int4 ahi = *(const int4 *) (x.q + chi);
    const int sl = 2 * g, sh = 2 * g + 1;
    auto lo = [&](uint32_t q, uint32_t qh) { return (int) ((q & 0x0F0F0F0Fu) | (((qh >> sl) & 0x01010101u) << 4)); };
    auto hi = [&](uint32_t q, uint32_t qh) {
        return (int) (((q >> 4) & 0x0F0F0F0Fu) | (((qh >> sh) & 0x01010101u) << 4));
    };
    int dlo = 0, dhi = 0;
    dlo = dot4(lo(f.b.x, f.c.x), alo.x, dlo);
    dlo = dot4(lo(f.b.y, f.c.y), alo.y, dlo);
    dlo = dot4(lo(f.b.z, f.c.z), alo.z, dlo);
    dlo = dot4(lo(f.b.w, f.c.w), alo.w, dlo);
    dhi = dot4(hi(f.b.x, f.c.x), ahi.x, dhi);
    dhi = dot4(hi(f.b.y, f.c.y), ahi.y, dhi);
    dhi = dot4(hi(f.b.z, f.c.z), ahi.z, dhi);
    dhi = dot4(hi(f.b.w, f.c.w), ahi.w, dhi);
    int sc0, m0, sc1, m1;
    scale_min_k4(f.a, 2 * g, sc0, m0);
    scale_min_k4(f.a, 2 * g + 1, sc1, m1);
    const float d = half_to_float(f.a.x & 0xffffu), dmin = half_to_float(f.a.x >> 16);
    const float sd = (float) (sc0 * dlo) * x.d[clo >> 5] + (float) (sc1 * dhi) * x.d[chi >> 5];
    const float sm = (float) m0 * x.s16[clo >> 4] + (float) m1 * x.s16[chi >> 4];
    return d * sd - dmin * sm;
}

// Q6_K slot j: n = j/4, jj = j%4; ql[64n+16jj+t] low nibble = value 128n+16jj+t, high nibble = value +64; two qh
// bits from qh[32n+16(jj%2)+t] at shift 2*(jj/2) (low) and 2*(jj/2)+4 (high); 6-bit value - 32. Scales (int8,
// 16 values each): group 8n+jj (low) and 8n+jj+4 (high). f.a holds scales[0..15], f.e the f16 d.
template <> __device__ __forceinline__ float slot_dot<T_Q6_K>(const Frag &f, int j, int col0, const ActView &x) {
    const int n = j >> 2, jj = j & 3;
    const int clo = col0 + 128 * n + 16 * jj, chi = clo + 64;
    const int4 alo = *(const int4 *) (x.q + clo);
    const int4 ahi = *(const int4 *) (x.q + chi);
    const int shl = 2 * (jj >> 1), shh = shl + 4;
    auto lo = [&](uint32_t q, uint32_t qh) {
        return bytes_sub<32>((int) ((q & 0x0F0F0F0Fu) | (((qh >> shl) & 0x03030303u) << 4)));
    };
    auto hi = [&](uint32_t q, uint32_t qh) {
        return bytes_sub<32>((int) (((q >> 4) & 0x0F0F0F0Fu) | (((qh >> shh) & 0x03030303u) << 4)));
    };
    int dlo = 0, dhi = 0;
    dlo = dot4(lo(f.b.x, f.c.x), alo.x, dlo);
    dlo = dot4(lo(f.b.y, f.c.y), alo.y, dlo);
    dlo = dot4(lo(f.b.z, f.c.z), alo.z, dlo);
    dlo = dot4(lo(f.b.w, f.c.w), alo.w, dlo);
    dhi = dot4(hi(f.b.x, f.c.x), ahi.x, dhi);
    dhi = dot4(hi(f.b.y, f.c.y), ahi.y, dhi);
    dhi = dot4(hi(f.b.z, f.c.z), ahi.z, dhi);
    dhi = dot4(hi(f.b.w, f.c.w), ahi.w, dhi);
    const int glo = 8 * n + jj, ghi = glo + 4;
    const int sclo = (int) (int8_t) byte_of(f.a, glo);
    const int schi = (int) (int8_t) byte_of(f.a, ghi);
    const float d = half_to_float(f.e);
    return d * ((float) (sclo * dlo) * x.d[clo >> 5] + (float) (schi * dhi) * x.d[chi >> 5]);
}

// Q3_K slot j (0..3): qs[16j+t] (n = j/2, h = j%2) holds 2-bit values for jj = 0..3 at value 128n+32jj+16h+t; the
// high bit is hmask[16h+t] bit 4n+jj (set: +0, clear: -4). Scale group 8n+2jj+h, 6-bit value - 32, packed in
// 12 bytes (low nibbles in bytes 0..7, high 2-bit pairs in bytes 8..11). f.a holds block bytes 94..109.
template <> __device__ __forceinline__ float slot_dot<T_Q3_K>(const Frag &f, int j, int col0, const ActView &x) {
    const int n = j >> 1, h = j & 1;
    float acc = 0.0f;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
        const int c = col0 + 128 * n + 32 * jj + 16 * h;
        const int4 a = *(const int4 *) (x.q + c);
        const int hs = 4 * n + jj;
        auto val = [&](uint32_t q, uint32_t hm) {
            return bytes_sub<4>((int) (((q >> (2 * jj)) & 0x03030303u) | (((hm >> hs) & 0x01010101u) << 2)));
        };
        int dd = 0;
        dd = dot4(val(f.b.x, f.c.x), a.x, dd);
        dd = dot4(val(f.b.y, f.c.y), a.y, dd);
        dd = dot4(val(f.b.z, f.c.z), a.z, dd);
        dd = dot4(val(f.b.w, f.c.w), a.w, dd);
        const int g = 8 * n + 2 * jj + h;
        // scales field byte i is f.a byte i + 2
        const uint32_t lo4 = g < 8 ? (byte_of(f.a, 2 + g) & 0xFu) : (byte_of(f.a, 2 + g - 8) >> 4);
        const uint32_t hi2 = (byte_of(f.a, 2 + 8 + (g & 3)) >> (2 * (g >> 2))) & 3u;
        const int sc = (int) (lo4 | (hi2 << 4)) - 32;
        acc += (float) (sc * dd) * x.d[c >> 5];
    }
    return half_to_float(f.a.w >> 16) * acc;
}

}  // namespace fns::dev
