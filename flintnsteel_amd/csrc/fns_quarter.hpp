// fns_quarter.hpp - dot product of one quarter of a 256-value K-quant block (64 consecutive values) with a Q8_1
// activation row image (fns_block.hpp layout). Quarters let 32 lanes share one row of a 2048-wide matrix (8 blocks x 4
// quarters), so each lane runs a short dependency chain and many waves share a SIMD; a lane reads only the bytes its
// quarter needs (header + 32 of the 128 qs bytes for Q4_K, for example).
//   Q4_K / Q5_K quarter g: sub-blocks 2g (low nibbles of qs[32g..32g+31]) and 2g+1 (high nibbles), each
//                          d * sc * d8 * (q . a) - dmin * m * (d8 * sum a)
//   Q6_K quarter 2n+h    : values 128n + 64h .. +63: ql[64n..64n+63] nibble h, qh[32n..32n+31] bit pairs 2h, 2h+1;
//                          d * sum_g sc_g * (d8 * (u . a) - 32 * d8 * sum a) over its four 16-value groups
//   Q3_K quarter 2n+h    : values 128n + 64h .. +63: qs[32n..32n+31] bit pairs 2j (j = 2h, 2h+1), hmask bit 4n+j;
//                          d * sum_g (sc_g - 32) * (d8 * (u . a) - 4 * d8 * sum a)
//   Q8_0 quarter q       : blocks 2q and 2q+1 of 8 consecutive 34-byte blocks; sum_b (d_b * d8) * (q_b . a)
// The integer products are exact (v_dot4 on int8 lanes); the zero points (32 for Q6_K, 4 for Q3_K) are folded into
// the activation sums (group_term), so the unsigned codes are never re-biased per byte.
#pragma once

#include "fns_block.hpp"

#include <type_traits>

namespace fns::dev {

// Loader policies. Aligned16 (16-byte-aligned) and Any2 (2-byte-aligned) read weights in global memory through
// global-address-space pointers: global loads count on the vector-memory counter only, so the compiler can keep
// several quarters' loads in flight while LDS reads of the activations complete (a generic pointer becomes a flat
// load, which counts on both counters and made it wait after every quarter). Padded reads blocks staged in LDS.
typedef uint32_t gv4u __attribute__((ext_vector_type(4)));
typedef gv4u gv4u_a2 __attribute__((aligned(2)));
typedef uint32_t gu32_a2 __attribute__((aligned(2)));
typedef __attribute__((address_space(1))) const gv4u GV4;
typedef __attribute__((address_space(1))) const gv4u_a2 GV4a2;
typedef __attribute__((address_space(1))) const gu32_a2 GU32a2;
struct Aligned16 {
    static __device__ __forceinline__ uint4 ld(const uint8_t *p) {
        const gv4u v = *(GV4 *) p;
        return make_uint4(v.x, v.y, v.z, v.w);
    }
    static __device__ __forceinline__ uint32_t ld32(const uint8_t *p) { return *(GU32a2 *) p; }
};
struct Any2 {
    static __device__ __forceinline__ uint4 ld(const uint8_t *p) {
        const gv4u v = *(GV4a2 *) p;
        return make_uint4(v.x, v.y, v.z, v.w);
    }
    static __device__ __forceinline__ uint32_t ld32(const uint8_t *p) { return *(GU32a2 *) p; }
};
// Padded: blocks staged in LDS at a 16-byte-aligned stride (kStageBytes), each block's last 16-byte piece holding the
// block's last 16 bytes (so no piece reads past the block); for Q4_K / Q5_K / Q8_0 / IQ types the same as Aligned16
// (their staged layout is the verbatim one).
struct Padded {
    static __device__ __forceinline__ uint4 ld(const uint8_t *p) { return *(const uint4 *) p; }
    static __device__ __forceinline__ uint32_t ld32(const uint8_t *p) { return *(const uint32_t *) p; }
};
template <int T> constexpr int kStageBytes = T == T_Q6_K ? 224 : T == T_Q3_K ? 112 : Traits<T>::bytes;
// 4 bytes at a 2-byte-aligned address.
__device__ __forceinline__ uint32_t ld32u(const uint8_t *p) {
    uint32_t v;
    __builtin_memcpy(&v, __builtin_assume_aligned(p, 2), 4);
    return v;
}

// The activation side of one quarter (64 consecutive columns of block bb, quarter qt) in registers: the 64 int8 values
// as 16 dwords, the Q8_1 scales of its two 32-column blocks, d * (sum of the quantised values) of its four 16-column
// groups and of its two 32-column blocks. Loaded once, it serves every weight row that has the same quarter.
struct ActQ {
    int a[16];
    float d[2], s16[4], s32[2];
};
__device__ __forceinline__ ActQ act_q(const ActImg &x, int bb, int qt) {
    ActQ r;
    const int8_t *p = x.q + bb * kImgQRow + 64 * qt;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int4 v = *(const int4 *) (p + 16 * i);
        r.a[4 * i] = v.x;
        r.a[4 * i + 1] = v.y;
        r.a[4 * i + 2] = v.z;
        r.a[4 * i + 3] = v.w;
    }
    const int b32 = bb * 8 + 2 * qt;
    r.d[0] = x.d[b32];
    r.d[1] = x.d[b32 + 1];
#pragma unroll
    for (int g = 0; g < 4; ++g) r.s16[g] = x.s16[2 * b32 + g];
    r.s32[0] = x.s32[b32];
    r.s32[1] = x.s32[b32 + 1];
    return r;
}

// Quarter dot against an activation quarter in registers (qt: the quarter's index in its block).
template <int T, class L> __device__ __forceinline__ float quarter_dot_r(const uint8_t *blk, const ActQ &x, int qt);

// Q4_K / Q5_K share the header decoding: 6-bit scale and min of sub-blocks 2qt, 2qt+1 (bytes k0, k0+1 of the words).
__device__ __forceinline__ void k4_scales(const uint4 &h, int qt, uint32_t &scw, uint32_t &mw) {
    const uint32_t sc_lo = h.y & 0x3F3F3F3Fu, m_lo = h.z & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (h.w & kLo4) | ((h.y >> 2) & 0x30303030u);
    const uint32_t m_hi = ((h.w >> 4) & kLo4) | ((h.z >> 2) & 0x30303030u);
    scw = qt < 2 ? sc_lo : sc_hi;
    mw = qt < 2 ? m_lo : m_hi;
}
__device__ __forceinline__ float ubyte_dyn(uint32_t w, int k) { return (float) ((w >> (8 * k)) & 0xffu); }

__device__ __forceinline__ float k4_finish(const uint4 &h, const ActQ &x, int qt, int dl, int dh) {
    uint32_t scw, mw;
    k4_scales(h, qt, scw, mw);
    const int k0 = 2 * (qt & 1);
    float sumd = ubyte_dyn(scw, k0) * x.d[0] * (float) dl;
    sumd = fmaf_(ubyte_dyn(scw, k0 + 1) * x.d[1], (float) dh, sumd);
    float summ = ubyte_dyn(mw, k0) * x.s32[0];
    summ = fmaf_(ubyte_dyn(mw, k0 + 1), x.s32[1], summ);
    return half_to_float(h.x & 0xffffu) * sumd - half_to_float(h.x >> 16) * summ;
}

template <class L> __device__ __forceinline__ float q4k_quarter(const uint8_t *blk, const ActQ &x, int qt) {
    const uint4 h = L::ld(blk);
    const uint4 q0 = L::ld(blk + 16 + 32 * qt), q1 = L::ld(blk + 32 + 32 * qt);
    const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    int dl = 0, dh = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        dl = dot4((int) (q[i] & kLo4), x.a[i], dl);
        dh = dot4((int) ((q[i] >> 4) & kLo4), x.a[8 + i], dh);
    }
    return k4_finish(h, x, qt, dl, dh);
}
template <> __device__ __forceinline__ float quarter_dot_r<T_Q4_K, Aligned16>(const uint8_t *blk, const ActQ &x, int qt) {
    return q4k_quarter<Aligned16>(blk, x, qt);
}
template <> __device__ __forceinline__ float quarter_dot_r<T_Q4_K, Any2>(const uint8_t *blk, const ActQ &x, int qt) {
    return q4k_quarter<Any2>(blk, x, qt);
}
template <> __device__ __forceinline__ float quarter_dot_r<T_Q4_K, Padded>(const uint8_t *blk, const ActQ &x, int qt) {
    return q4k_quarter<Padded>(blk, x, qt);
}

template <class L> __device__ __forceinline__ float q5k_quarter(const uint8_t *blk, const ActQ &x, int qt) {
    const uint4 h = L::ld(blk);
    const uint4 h0 = L::ld(blk + 16), h1 = L::ld(blk + 32);
    const uint4 q0 = L::ld(blk + 48 + 32 * qt), q1 = L::ld(blk + 64 + 32 * qt);
    const uint32_t qh[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
    const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    int dl = 0, dh = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        // fifth bit: qh bit 2qt (low values) and 2qt+1 (high values), moved to bit 4 of each byte
        const uint32_t bl = ((qh[i] >> (2 * qt)) & 0x01010101u) << 4;
        const uint32_t bh = ((qh[i] >> (2 * qt + 1)) & 0x01010101u) << 4;
        dl = dot4((int) ((q[i] & kLo4) | bl), x.a[i], dl);
        dh = dot4((int) (((q[i] >> 4) & kLo4) | bh), x.a[8 + i], dh);
    }
    return k4_finish(h, x, qt, dl, dh);
}
template <> __device__ __forceinline__ float quarter_dot_r<T_Q5_K, Aligned16>(const uint8_t *blk, const ActQ &x, int qt) {
    return q5k_quarter<Aligned16>(blk, x, qt);
}
template <> __device__ __forceinline__ float quarter_dot_r<T_Q5_K, Any2>(const uint8_t *blk, const ActQ &x, int qt) {
    return q5k_quarter<Any2>(blk, x, qt);
}
template <> __device__ __forceinline__ float quarter_dot_r<T_Q5_K, Padded>(const uint8_t *blk, const ActQ &x, int qt) {
    return q5k_quarter<Padded>(blk, x, qt);
}

// Q6_K and Q3_K blocks are only 2-byte aligned: both policies read through Any2.
// L = Padded: the block is staged in LDS at a 16-byte-aligned address with its last piece (bytes 194 .. 209) at
// offset 208; otherwise a 2-byte-aligned block in global memory.
template <class L> __device__ __forceinline__ float q6k_quarter(const uint8_t *blk, const ActQ &x, int qt) {
    constexpr bool PAD = std::is_same<L, Padded>::value;
    const int n = qt >> 1, hh = qt & 1;
    auto ld = [&](int o) { return PAD ? L::ld(blk + o) : Any2::ld(blk + o); };
    const uint4 A0 = ld(64 * n), A1 = ld(64 * n + 16);       // ql[64n .. 64n+31]
    const uint4 B0 = ld(64 * n + 32), B1 = ld(64 * n + 48);  // ql[64n+32 .. 64n+63]
    const uint4 Q0 = ld(128 + 32 * n), Q1 = ld(144 + 32 * n);  // qh[32n .. 32n+31]
    const uint32_t scw = PAD ? L::ld32(blk + 192 + 4 * qt) : Any2::ld32(blk + 192 + 4 * qt);  // int8 scales of groups 4qt .. 4qt+3
    const uint32_t dbits = PAD ? L::ld32(blk + 220) >> 16 : Any2::ld32(blk + 208) & 0xffffu;
    const uint32_t A[8] = {A0.x, A0.y, A0.z, A0.w, A1.x, A1.y, A1.z, A1.w};
    const uint32_t B[8] = {B0.x, B0.y, B0.z, B0.w, B1.x, B1.y, B1.z, B1.w};
    const uint32_t Q[8] = {Q0.x, Q0.y, Q0.z, Q0.w, Q1.x, Q1.y, Q1.z, Q1.w};
    const int sh = 4 * hh;
    int du[4] = {0, 0, 0, 0};  // groups: A half 0, A half 1, B half 0, B half 1
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t qh = Q[i] >> sh;
        const uint32_t ua = ((A[i] >> sh) & kLo4) | ((qh << 4) & 0x30303030u);
        const uint32_t ub = ((B[i] >> sh) & kLo4) | ((qh << 2) & 0x30303030u);
        du[i >> 2] = dot4((int) ua, x.a[i], du[i >> 2]);
        du[2 + (i >> 2)] = dot4((int) ub, x.a[8 + i], du[2 + (i >> 2)]);
    }
    float sum = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; ++g) sum = fmaf_(sbyte_f(scw, g), group_term(du[g], x.d[g >> 1], x.s16[g], 32.0f), sum);
    return half_to_float(dbits) * sum;
}
template <> __device__ __forceinline__ float quarter_dot_r<T_Q6_K, Aligned16>(const uint8_t *blk, const ActQ &x, int qt) {
    return q6k_quarter<Any2>(blk, x, qt);
}
template <> __device__ __forceinline__ float quarter_dot_r<T_Q6_K, Any2>(const uint8_t *blk, const ActQ &x, int qt) {
    return q6k_quarter<Any2>(blk, x, qt);
}
template <> __device__ __forceinline__ float quarter_dot_r<T_Q6_K, Padded>(const uint8_t *blk, const ActQ &x, int qt) {
    return q6k_quarter<Padded>(blk, x, qt);
}

// L = Padded: the block is staged in LDS at a 16-byte-aligned address with its last piece (bytes 94 .. 109) at
// offset 96; otherwise a 2-byte-aligned block in global memory.
template <class L> __device__ __forceinline__ float q3k_quarter(const uint8_t *blk, const ActQ &x, int qt) {
    constexpr bool PAD = std::is_same<L, Padded>::value;
    const int n = qt >> 1, hh = qt & 1;
    auto ld = [&](int o) { return PAD ? L::ld(blk + o) : Any2::ld(blk + o); };
    const uint4 H0 = ld(0), H1 = ld(16);                          // hmask[0 .. 31]
    const uint4 q0 = ld(32 + 32 * n), q1 = ld(48 + 32 * n);  // qs[32n .. 32n+31]
    const uint4 t = ld(PAD ? 96 : 94);                            // scales at +2, d at +14
    const uint32_t HM[8] = {H0.x, H0.y, H0.z, H0.w, H1.x, H1.y, H1.z, H1.w};
    const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    const uint32_t S0 = __builtin_amdgcn_alignbit(t.y, t.x, 16), S1 = __builtin_amdgcn_alignbit(t.z, t.y, 16);
    const uint32_t S2 = __builtin_amdgcn_alignbit(t.w, t.z, 16);
    // scales of groups 4qt .. 4qt+3: low nibbles from S0 (qt even) or S1 (qt odd), shifted by 4 for qt >= 2; top two
    // bits from S2 at bit pair qt of each byte
    const uint32_t lo = ((hh ? S1 : S0) >> (4 * n)) & kLo4;
    const uint32_t hi = (uint32_t) ((((uint64_t) S2) << 4) >> (2 * qt)) & 0x30303030u;
    const uint32_t scw = lo | hi;
    int du[4] = {0, 0, 0, 0};  // groups: j0 half 0, j0 half 1, j1 half 0, j1 half 1 (j0 = 2hh, j1 = 2hh + 1)
    const int j0 = 2 * hh;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t hm = HM[i] >> (4 * n + j0);
        const uint32_t u0 = ((q[i] >> (2 * j0)) & 0x03030303u) | ((hm << 2) & 0x04040404u);
        const uint32_t u1 = ((q[i] >> (2 * j0 + 2)) & 0x03030303u) | ((hm << 1) & 0x04040404u);
        du[i >> 2] = dot4((int) u0, x.a[i], du[i >> 2]);
        du[2 + (i >> 2)] = dot4((int) u1, x.a[8 + i], du[2 + (i >> 2)]);
    }
    float sum = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; ++g)
        sum = fmaf_(ubyte_dyn(scw, g) - 32.0f, group_term(du[g], x.d[g >> 1], x.s16[g], 4.0f), sum);
    return half_to_float(t.w >> 16) * sum;
}
template <> __device__ __forceinline__ float quarter_dot_r<T_Q3_K, Aligned16>(const uint8_t *blk, const ActQ &x, int qt) {
    return q3k_quarter<Any2>(blk, x, qt);
}
template <> __device__ __forceinline__ float quarter_dot_r<T_Q3_K, Any2>(const uint8_t *blk, const ActQ &x, int qt) {
    return q3k_quarter<Any2>(blk, x, qt);
}
template <> __device__ __forceinline__ float quarter_dot_r<T_Q3_K, Padded>(const uint8_t *blk, const ActQ &x, int qt) {
    return q3k_quarter<Padded>(blk, x, qt);
}

// Q8_0 quarter qt = blocks 2qt and 2qt+1 of the 8-block unit (68 bytes at offset 68 qt, 2-byte aligned at least):
// sum over the two blocks of (d_w * d8) * (q_w . a), the block product of ggml vec_dot_q8_0_q8_1.
template <class L> __device__ __forceinline__ float q80_quarter(const uint8_t *blk, const ActQ &x, int qt) {
    const uint8_t *p = blk + 68 * qt;
    // (Padded: LDS data, 2-byte aligned within the staged unit; otherwise global memory)
    auto ld = [&](int o) { return std::is_same<L, Padded>::value ? lds16u(p + o) : Any2::ld(p + o); };
    const uint4 A0 = ld(0), A1 = ld(16), A2 = ld(32), A3 = ld(48);
    const uint32_t W[17] = {A0.x, A0.y, A0.z, A0.w, A1.x, A1.y, A1.z, A1.w, A2.x, A2.y, A2.z, A2.w, A3.x, A3.y, A3.z, A3.w,
                            std::is_same<L, Padded>::value ? ld32u(p + 64) : Any2::ld32(p + 64)};
    int s0 = 0, s1 = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        s0 = dot4((int) __builtin_amdgcn_alignbit(W[i + 1], W[i], 16), x.a[i], s0);  // block 0 codes: bytes 2 .. 33
        s1 = dot4((int) W[9 + i], x.a[8 + i], s1);                                    // block 1 codes: bytes 36 .. 67
    }
    const float d0 = half_to_float(W[0] & 0xffffu) * x.d[0], d1 = half_to_float(W[8] >> 16) * x.d[1];
    return fmaf_(d1, (float) s1, d0 * (float) s0);
}
template <> __device__ __forceinline__ float quarter_dot_r<T_Q8_0, Aligned16>(const uint8_t *blk, const ActQ &x, int qt) {
    return q80_quarter<Any2>(blk, x, qt);
}
template <> __device__ __forceinline__ float quarter_dot_r<T_Q8_0, Any2>(const uint8_t *blk, const ActQ &x, int qt) {
    return q80_quarter<Any2>(blk, x, qt);
}
template <> __device__ __forceinline__ float quarter_dot_r<T_Q8_0, Padded>(const uint8_t *blk, const ActQ &x, int qt) {
    return q80_quarter<Padded>(blk, x, qt);
}

// ---- IQ formats: quarter qt = sub-blocks 2qt and 2qt+1 (32 values each). Per sub-block the integer arithmetic of
// the reference's GPU products (src/ggml/ggml_mmvq.cu:101-157 for IQ3_XXS / IQ3_S; ggml vecdotq.cuh
// vec_dot_iq4_xs_q8_1 / vec_dot_iq2_s_q8_1 for IQ4_XS / IQ2_S): an exact v_dot4 sum, the sub-block scale applied in
// integers (C division truncating toward zero), then (d_w * d8) * sum in fp32; the quarter returns the two sub-block
// terms added in order.

// The IQ3_XXS / IQ3_S / IQ2_S codebooks (ggml's iq3xxs_grid, iq3s_grid, iq2s_grid). The library does not carry them:
// the engine registers its copies once per device (fns_hip_set_iq_grids), which fills this array of every translation
// unit that decodes IQ blocks. Codebook values are positive bytes (never 0), which the sign step below relies on.
struct IqGrids {
    uint32_t iq3xxs[256];
    uint32_t iq3s[512];
    uint64_t iq2s[1024];
};
static __device__ IqGrids g_iq_grids;
// LDS copies of the two small codebooks (1 and 2 KiB) for the GEMV kernels: an LDS read per lookup instead of a
// gathered global load. Every kernel that decodes IQ3_XXS or IQ3_S blocks fills them first (iq_grids_to_lds) and
// reaches a workgroup barrier before its first lookup. (The 8 KiB IQ2_S codebook stays in global memory.)
static __shared__ uint32_t s_iq3xxs_grid[256];
static __shared__ uint32_t s_iq3s_grid[512];
template <int T> __device__ __forceinline__ void iq_grids_to_lds(int tid, int nthreads) {
    if constexpr (T == T_IQ3_XXS) {
        for (int i = tid; i < 256; i += nthreads) s_iq3xxs_grid[i] = g_iq_grids.iq3xxs[i];
    } else if constexpr (T == T_IQ3_S) {
        for (int i = tid; i < 512; i += nthreads) s_iq3s_grid[i] = g_iq_grids.iq3s[i];
    }
}
template <int T> constexpr bool kIqLdsGrid = T == T_IQ3_XXS || T == T_IQ3_S;

// The IQ4_NL values {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113} as four byte tables.
constexpr uint32_t kIq4T0 = 0xBFAD9881u, kIq4T1 = 0xF6EADDCFu, kIq4T2 = 0x26190D01u, kIq4T3 = 0x71594535u;
// Four 4-bit indices (one per byte) -> their four int8 values: v_perm picks from entries 0-7 and 8-15, bit 3 chooses.
__device__ __forceinline__ uint32_t iq4nl_values(uint32_t nib) {
    const uint32_t sel = nib & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(kIq4T1, kIq4T0, sel), hi = __builtin_amdgcn_perm(kIq4T3, kIq4T2, sel);
    const uint32_t e = (nib >> 3) & 0x01010101u;
    const uint32_t m = (e << 8) - e;  // 0xff in the bytes whose index is >= 8
    return (hi & m) | (lo & ~m);
}
// Four sign bits -> one bit per byte (bit j -> byte j, bit 0).
__device__ __forceinline__ uint32_t spread4(uint32_t s4) { return (s4 * 0x00204081u) & 0x01010101u; }
// Four positive codebook bytes with the signs of spread4 applied: per byte (g ^ 0xff) + 1 = -g, which cannot carry
// into the next byte because g >= 1.
__device__ __forceinline__ int signed_grid(uint32_t g, uint32_t e) { return (int) ((g ^ ((e << 8) - e)) + e); }
// The 7 stored sign bits of an IQ3_XXS group plus the eighth that makes the count of negative signs even.
__device__ __forceinline__ uint32_t ksigns(uint32_t v7) { return v7 | ((uint32_t) (__builtin_popcount(v7) & 1) << 7); }
__device__ __forceinline__ uint32_t ld8u(const uint8_t *p) { return (uint32_t) *p; }

__device__ __forceinline__ float iq4xs_quarter(const uint8_t *blk, const ActQ &x, int qt) {
    const uint32_t h0 = ld32u(blk), sl = ld32u(blk + 4);
    const float d = half_to_float(h0 & 0xffffu);
    const uint32_t sh = h0 >> 16;
    float acc = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int ib = 2 * qt + h;
        const uint4 q = lds16u(blk + 8 + 16 * ib);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
        int s = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s = dot4((int) iq4nl_values(w[i] & kLo4), x.a[8 * h + i], s);
            s = dot4((int) iq4nl_values((w[i] >> 4) & kLo4), x.a[8 * h + 4 + i], s);
        }
        const int ls = (int) (((sl >> (8 * (ib >> 1) + 4 * (ib & 1))) & 0xfu) | (((sh >> (2 * ib)) & 3u) << 4));
        s *= ls - 32;
        acc += (d * x.d[h]) * (float) s;
    }
    return acc;
}

__device__ __forceinline__ float iq3xxs_quarter(const uint8_t *blk, const ActQ &x, int qt) {
    const float d = half_to_float(ld32u(blk) & 0xffffu);
    float acc = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int ib = 2 * qt + h;
        const uint32_t i0 = ld32u(blk + 2 + 8 * ib), i1 = ld32u(blk + 6 + 8 * ib);
        const uint32_t aux = ld32u(blk + 66 + 4 * ib);
        int s = 0;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t idx = l < 2 ? i0 : i1, sh = 16 * (l & 1);
            const uint32_t sg = ksigns((aux >> (7 * l)) & 127u);
            const uint32_t g0 = s_iq3xxs_grid[(idx >> sh) & 0xffu], g1 = s_iq3xxs_grid[(idx >> (sh + 8)) & 0xffu];
            s = dot4(signed_grid(g0, spread4(sg & 0xfu)), x.a[8 * h + 2 * l], s);
            s = dot4(signed_grid(g1, spread4(sg >> 4)), x.a[8 * h + 2 * l + 1], s);
        }
        const int ls = (int) (aux >> 28);
        s = (ls * s + s / 2) / 2;
        acc += (d * x.d[h]) * (float) s;
    }
    return acc;
}

__device__ __forceinline__ float iq3s_quarter(const uint8_t *blk, const ActQ &x, int qt) {
    const float d = half_to_float(ld32u(blk) & 0xffffu);
    const uint32_t scw = ld32u(blk + 106);
    float acc = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int ib = 2 * qt + h;
        const uint32_t i0 = ld32u(blk + 2 + 8 * ib), i1 = ld32u(blk + 6 + 8 * ib);
        const uint32_t qh = ld8u(blk + 66 + ib), sg = ld32u(blk + 74 + 4 * ib);
        int s = 0;
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            const uint32_t gi = (((l < 4 ? i0 : i1) >> (8 * (l & 3))) & 0xffu) | (((qh >> l) & 1u) << 8);
            const uint32_t sb = (sg >> (4 * l)) & 0xfu;  // byte l/2, nibble l%2
            s = dot4(signed_grid(s_iq3s_grid[gi], spread4(sb)), x.a[8 * h + l], s);
        }
        s *= 1 + 2 * (int) ((scw >> (8 * (ib >> 1) + 4 * (ib & 1))) & 0xfu);
        acc += (d * x.d[h]) * (float) s;
    }
    return acc;
}

__device__ __forceinline__ float iq2s_quarter(const uint8_t *blk, const ActQ &x, int qt) {
    const float d = half_to_float(ld32u(blk) & 0xffffu);
    float acc = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int ib = 2 * qt + h;
        const uint32_t idx = ld32u(blk + 2 + 4 * ib), sg = ld32u(blk + 34 + 4 * ib);
        const uint32_t qh = ld8u(blk + 66 + ib), sc = ld8u(blk + 74 + ib);
        int s2[2] = {0, 0};
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t gi = ((idx >> (8 * l)) & 0xffu) | (((qh >> (2 * l)) & 3u) << 8);
            const uint64_t g = g_iq_grids.iq2s[gi];
            const uint32_t sb = (sg >> (8 * l)) & 0xffu;
            s2[l >> 1] = dot4(signed_grid((uint32_t) g, spread4(sb & 0xfu)), x.a[8 * h + 2 * l], s2[l >> 1]);
            s2[l >> 1] = dot4(signed_grid((uint32_t) (g >> 32), spread4(sb >> 4)), x.a[8 * h + 2 * l + 1], s2[l >> 1]);
        }
        const int ls0 = (int) (sc & 0xfu), ls1 = (int) (sc >> 4);
        const int s = (s2[0] * ls0 + s2[1] * ls1 + (s2[0] + s2[1]) / 2) / 4;
        acc += (d * x.d[h]) * (float) s;
    }
    return acc;
}

#define FNS_IQ_QUARTER(T, F)                                                                                        \
    template <> __device__ __forceinline__ float quarter_dot_r<T, Aligned16>(const uint8_t *blk, const ActQ &x, int qt) { \
        return F(blk, x, qt);                                                                                        \
    }                                                                                                                \
    template <> __device__ __forceinline__ float quarter_dot_r<T, Any2>(const uint8_t *blk, const ActQ &x, int qt) {     \
        return F(blk, x, qt);                                                                                        \
    }                                                                                                                \
    template <> __device__ __forceinline__ float quarter_dot_r<T, Padded>(const uint8_t *blk, const ActQ &x, int qt) {   \
        return F(blk, x, qt);                                                                                        \
    }
FNS_IQ_QUARTER(T_IQ4_XS, iq4xs_quarter)
FNS_IQ_QUARTER(T_IQ3_XXS, iq3xxs_quarter)
FNS_IQ_QUARTER(T_IQ3_S, iq3s_quarter)
FNS_IQ_QUARTER(T_IQ2_S, iq2s_quarter)
#undef FNS_IQ_QUARTER

// Copies the codebooks into this translation unit's g_iq_grids on the current device.
static inline hipError_t upload_iq_grids(const IqGrids *host) {
    return hipMemcpyToSymbol(HIP_SYMBOL(g_iq_grids), host, sizeof(IqGrids), 0, hipMemcpyHostToDevice);
}

// The quarter dot against an activation row image (the activation quarter read from LDS for this one product).
template <int T, class L> __device__ __forceinline__ float quarter_dot(const uint8_t *blk, const ActImg &x, int bb, int qt) {
    return quarter_dot_r<T, L>(blk, act_q(x, bb, qt), qt);
}

// A Q4_K quarter's weight bytes (header, the 32 code bytes of the quarter), loaded apart from the arithmetic so a caller
// can have several quarters' loads in flight before the first dot product.
struct Q4Frag {
    uint4 h, q0, q1;
};
template <class L> __device__ __forceinline__ Q4Frag q4k_frag(const uint8_t *blk, int qt) {
    return Q4Frag{L::ld(blk), L::ld(blk + 16 + 32 * qt), L::ld(blk + 32 + 32 * qt)};
}
// quarter_dot_nc's Q4_K arithmetic on a loaded fragment.
template <int NC>
__device__ __forceinline__ void q4k_nc(const Q4Frag &f, const ActImg (&x)[NC], int ncol, int bb, int qt, float (&acc)[NC]) {
    const uint32_t q[8] = {f.q0.x, f.q0.y, f.q0.z, f.q0.w, f.q1.x, f.q1.y, f.q1.z, f.q1.w};
    int lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        lo[i] = (int) (q[i] & kLo4);
        hi[i] = (int) ((q[i] >> 4) & kLo4);
    }
#pragma unroll
    for (int n = 0; n < NC; ++n) {
        if (NC == 1 || n < ncol) {
            const ActQ a = act_q(x[n], bb, qt);
            int dl = 0, dh = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                dl = dot4(lo[i], a.a[i], dl);
                dh = dot4(hi[i], a.a[8 + i], dh);
            }
            acc[n] += k4_finish(f.h, a, qt, dl, dh);
        }
    }
}

// The same dot for NC activation columns (n < ncol live; NC == 1 ignores ncol): acc[n] += quarter_dot(blk, x[n]).
// Q4_K reads and unpacks the weight quarter once for all columns; each column's arithmetic is exactly that of
// quarter_dot (a verify column equals the batch-1 result bit for bit). Other types call quarter_dot per column.
template <int T, class L, int NC>
__device__ __forceinline__ void quarter_dot_nc(const uint8_t *blk, const ActImg (&x)[NC], int ncol, int bb, int qt,
                                               float (&acc)[NC]) {
    if constexpr (T == T_Q4_K) {
        q4k_nc<NC>(q4k_frag<L>(blk, qt), x, ncol, bb, qt, acc);
    } else {
#pragma unroll
        for (int n = 0; n < NC; ++n)
            if (NC == 1 || n < ncol) acc[n] += quarter_dot<T, L>(blk, x[n], bb, qt);
    }
}

}  // namespace fns::dev
