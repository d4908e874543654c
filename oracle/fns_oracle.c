/* fns_oracle.c - CPU restatement of the MoE FFN hot path (TEST INFRASTRUCTURE ONLY; see fns_oracle.h).
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off: every fp32 expression below is evaluated exactly as
 * written, which is what makes the Q8_1 and routing restatements bit-comparable with the HIP kernels).
 */
#include "fns_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK_K 256
#define QK8 32

/* ---- GGUF block layouts (ggml-common.h of llama.cpp 19ab5a5e; sizes are part of the GGUF format) ---- */
typedef struct { uint16_t d; int8_t qs[32]; } blk_q8_0;
typedef struct { uint16_t d, s; int8_t qs[32]; } blk_q8_1;
typedef struct { uint8_t hmask[32]; uint8_t qs[64]; uint8_t scales[12]; uint16_t d; } blk_q3_K;
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; } blk_q4_K;
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qh[32]; uint8_t qs[128]; } blk_q5_K;
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } blk_q6_K;

_Static_assert(sizeof(blk_q8_0) == 34, "q8_0 block is 34 bytes");
_Static_assert(sizeof(blk_q8_1) == 36, "q8_1 block is 36 bytes");
_Static_assert(sizeof(blk_q3_K) == 110, "q3_K block is 110 bytes");
_Static_assert(sizeof(blk_q4_K) == 144, "q4_K block is 144 bytes");
_Static_assert(sizeof(blk_q5_K) == 176, "q5_K block is 176 bytes");
_Static_assert(sizeof(blk_q6_K) == 210, "q6_K block is 210 bytes");

/* IQ formats (ggml-common.h block_iq4_xs / block_iq3_xxs / block_iq3_s / block_iq2_s). */
typedef struct { uint16_t d; uint16_t scales_h; uint8_t scales_l[4]; uint8_t qs[128]; } blk_iq4_xs;
typedef struct { uint16_t d; uint8_t qs[96]; } blk_iq3_xxs;  /* 64 grid indices, then 8 words of signs + scale */
typedef struct { uint16_t d; uint8_t qs[64]; uint8_t qh[8]; uint8_t signs[32]; uint8_t scales[4]; } blk_iq3_s;
typedef struct { uint16_t d; uint8_t qs[64]; uint8_t qh[8]; uint8_t scales[8]; } blk_iq2_s;  /* qs: 32 idx, 32 signs */
_Static_assert(sizeof(blk_iq4_xs) == 136, "iq4_xs block is 136 bytes");
_Static_assert(sizeof(blk_iq3_xxs) == 98, "iq3_xxs block is 98 bytes");
_Static_assert(sizeof(blk_iq3_s) == 110, "iq3_s block is 110 bytes");
_Static_assert(sizeof(blk_iq2_s) == 82, "iq2_s block is 82 bytes");

/* ggml's non-linear 4-bit values of IQ4_NL / IQ4_XS (kvalues_iq4nl). */
static const int8_t kvalues_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

/* The lattice codebooks of IQ3_XXS (256 x 4 bytes), IQ3_S (512 x 4) and IQ2_S (1024 x 8) are ggml's tables
 * (iq3xxs_grid, iq3s_grid, iq2s_grid); they are not in this container, so the caller registers them here (the tests
 * register seeded tables of the right size and value sets, and the HIP library gets the same ones). */
static uint32_t g_iq3xxs_grid[256], g_iq3s_grid[512];
static uint64_t g_iq2s_grid[1024];
static int g_iq_grids_set;

void or_set_iq_grids(const uint32_t *iq3xxs, const uint32_t *iq3s, const uint64_t *iq2s) {
    memcpy(g_iq3xxs_grid, iq3xxs, sizeof g_iq3xxs_grid);
    memcpy(g_iq3s_grid, iq3s, sizeof g_iq3s_grid);
    memcpy(g_iq2s_grid, iq2s, sizeof g_iq2s_grid);
    g_iq_grids_set = 1;
}

/* ksigns_iq2xs[v]: the 7 stored sign bits v plus an eighth that makes the count of negative signs even. */
static int ksign_bits(uint32_t v7) { return (int) (v7 | ((uint32_t) (__builtin_popcount(v7) & 1) << 7)); }

/* ---- half precision ---- */
uint16_t or_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t) (sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t) (sign | 0x7c00u); /* >= 65520 rounds to infinity */
    if (ax < 0x38800000u) {                                     /* below 2^-14: f16 subnormal */
        float af;
        memcpy(&af, &ax, 4);
        const uint32_t r = (uint32_t) rintf(af * 16777216.0f); /* exact scaling by 2^24, round to even */
        return (uint16_t) (sign | r);
    }
    const uint32_t e = (ax >> 23) - 127u + 15u;
    const uint32_t m = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t) (sign | h);
}

float or_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t) h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        float f = (float) m * (1.0f / 16777216.0f);
        memcpy(&bits, &f, 4);
        bits |= sign;
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* exp(x): Cody-Waite reduction x = n ln2 + r (ln2 split in a 17-bit head and a tail), Taylor polynomial of degree 7
 * on |r| <= ln2/2 (truncation error < 6e-9 relative), scaling by 2^n in two exact steps. The HIP kernels evaluate the
 * identical sequence (flintnsteel_amd/csrc/fns_common.hpp: fns_expf), so gating probabilities are bit-identical. */
float or_expf(float x) {
    if (x < -104.0f) return 0.0f;
    if (x > 88.72f) return INFINITY;
    const float n = rintf(x * 1.44269504088896341f);
    float r = fmaf(n, -0.693145751953125f, x);
    r = fmaf(n, -1.42860682030941723e-6f, r);
    float p = 1.0f / 5040.0f;
    p = fmaf(p, r, 1.0f / 720.0f);
    p = fmaf(p, r, 1.0f / 120.0f);
    p = fmaf(p, r, 1.0f / 24.0f);
    p = fmaf(p, r, 1.0f / 6.0f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    int ni = (int) n;
    /* 2^ni = 2^(ni - h) * 2^h with both factors normal floats */
    const int h = ni < -100 ? -64 : (ni > 127 ? 1 : 0);
    ni -= h;
    uint32_t b1 = (uint32_t) (ni + 127) << 23, b2 = (uint32_t) (h + 127) << 23;
    float s1, s2;
    memcpy(&s1, &b1, 4);
    memcpy(&s2, &b2, 4);
    return (p * s1) * s2;
}

/* ---- sizes ---- */
size_t or_block_bytes(int type) {
    switch (type) {
        case OR_Q8_0: return sizeof(blk_q8_0);
        case OR_Q8_1: return sizeof(blk_q8_1);
        case OR_Q3_K: return sizeof(blk_q3_K);
        case OR_Q4_K: return sizeof(blk_q4_K);
        case OR_Q5_K: return sizeof(blk_q5_K);
        case OR_Q6_K: return sizeof(blk_q6_K);
        case OR_IQ4_XS: return sizeof(blk_iq4_xs);
        case OR_IQ3_XXS: return sizeof(blk_iq3_xxs);
        case OR_IQ3_S: return sizeof(blk_iq3_s);
        case OR_IQ2_S: return sizeof(blk_iq2_s);
        default: return 0;
    }
}

int or_block_elems(int type) {
    switch (type) {
        case OR_Q8_0: case OR_Q8_1: return 32;
        case OR_Q3_K: case OR_Q4_K: case OR_Q5_K: case OR_Q6_K: return QK_K;
        case OR_IQ4_XS: case OR_IQ3_XXS: case OR_IQ3_S: case OR_IQ2_S: return QK_K;
        default: return 0;
    }
}

int or_is_iq(int type) {
    return type == OR_IQ4_XS || type == OR_IQ3_XXS || type == OR_IQ3_S || type == OR_IQ2_S;
}

size_t or_row_bytes(int type, int64_t ncols) {
    const int be = or_block_elems(type);
    if (!be || ncols % be) return 0;
    return (size_t) (ncols / be) * or_block_bytes(type);
}

/* ---- ggml reference quantisers (ggml-quants.c quantize_row_*_ref), restated ---- */
static int nearest_int(float f) { return (int) rintf(f); } /* round half to even, as ggml's 1.5*2^23 trick */

/* Scale and (negated) min of n values on the grid 0..nmax, weighted least squares over nstep candidate scales. */
static float make_qkx2_quants(int n, int nmax, const float *x, const float *w, uint8_t *L, float *the_min,
                              uint8_t *Laux, float rmin, float rdelta, int nstep) {
    float mn = x[0], mx = x[0], sum_w = w[0], sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < mn) mn = x[i];
        if (x[i] > mx) mx = x[i];
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    if (mn > 0) mn = 0;
    if (mx == mn) {
        memset(L, 0, (size_t) n);
        *the_min = -mn;
        return 0.0f;
    }
    float iscale = nmax / (mx - mn);
    float scale = 1 / iscale;
    float best_error = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * (x[i] - mn));
        l = l < 0 ? 0 : (l > nmax ? nmax : l);
        L[i] = (uint8_t) l;
        float diff = scale * L[i] + mn - x[i];
        diff = diff * diff;
        best_error += w[i] * diff;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (mx - mn);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * (x[i] - mn));
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            Laux[i] = (uint8_t) l;
            sum_l += w[i] * l;
            sum_l2 += w[i] * l * l;
            sum_xl += w[i] * l * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float cur_error = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * Laux[i] + this_min - x[i];
                diff = diff * diff;
                cur_error += w[i] * diff;
            }
            if (cur_error < best_error) {
                memcpy(L, Laux, (size_t) n);
                best_error = cur_error;
                scale = this_scale;
                mn = this_min;
            }
        }
    }
    *the_min = -mn;
    return scale;
}

#define GROUP_MAX_EPS 1e-15f

/* Signed grid -nmax..nmax-1 with rmse weighting x^2 (ggml make_qx_quants, rmse_type 1). L = l + nmax. */
static float make_qx_quants(int n, int nmax, const float *x, int8_t *L) {
    float mx = 0, amax = 0;
    for (int i = 0; i < n; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; mx = x[i]; }
    }
    if (amax < GROUP_MAX_EPS) {
        memset(L, 0, (size_t) n);
        return 0.0f;
    }
    float iscale = -nmax / mx;
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
        L[i] = (int8_t) (l + nmax);
        const float w = x[i] * x[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    float scale = suml2 ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -(nmax + 0.1f * is) / mx;
        sumlx = suml2 = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * x[i]);
            l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
            const float w = x[i] * x[i];
            sumlx += w * x[i] * l;
            suml2 += w * l * l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) {
                int l = nearest_int(iscale * x[i]);
                l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
                L[i] = (int8_t) (nmax + l);
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

/* Signed grid -nmax..nmax-1 refined by coordinate descent on the x^2-weighted error (ggml make_q3_quants, rmse). */
static float make_q3_quants(int n, int nmax, const float *x, int8_t *L) {
    float mx = 0, amax = 0;
    for (int i = 0; i < n; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; mx = x[i]; }
    }
    if (amax < GROUP_MAX_EPS) {
        memset(L, 0, (size_t) n);
        return 0.0f;
    }
    const float iscale = -nmax / mx;
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
        L[i] = (int8_t) l;
        const float w = x[i] * x[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    for (int itry = 0; itry < 5; ++itry) {
        int n_changed = 0;
        for (int i = 0; i < n; ++i) {
            const float w = x[i] * x[i];
            float slx = sumlx - w * x[i] * L[i];
            if (slx > 0) {
                float sl2 = suml2 - w * L[i] * L[i];
                int new_l = nearest_int(x[i] * sl2 / slx);
                new_l = new_l < -nmax ? -nmax : (new_l > nmax - 1 ? nmax - 1 : new_l);
                if (new_l != L[i]) {
                    slx += w * x[i] * new_l;
                    sl2 += w * new_l * new_l;
                    if (sl2 > 0 && slx * slx * suml2 > sumlx * sumlx * sl2) {
                        L[i] = (int8_t) new_l;
                        sumlx = slx;
                        suml2 = sl2;
                        ++n_changed;
                    }
                }
            }
        }
        if (!n_changed) break;
    }
    for (int i = 0; i < n; ++i) L[i] = (int8_t) (L[i] + nmax);
    return sumlx / suml2;
}

/* 6-bit scale/min pair j of the 12-byte K-quant scale field (ggml get_scale_min_k4). */
static void scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t) ((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t) ((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

static void pack_scale_min_k4(uint8_t *scales, const uint8_t *ls, const uint8_t *lm) {
    memset(scales, 0, 12);
    for (int j = 0; j < 8; ++j) {
        if (j < 4) {
            scales[j] = ls[j];
            scales[j + 4] = lm[j];
        } else {
            scales[j + 4] = (uint8_t) ((ls[j] & 0xF) | ((lm[j] & 0xF) << 4));
            scales[j - 4] |= (uint8_t) ((ls[j] >> 4) << 6);
            scales[j] |= (uint8_t) ((lm[j] >> 4) << 6);
        }
    }
}

/* Shared by Q4_K (nmax 15) and Q5_K (nmax 31): per 32-value sub-block weighted scale/min, then 6-bit super scales. */
static void quant_kx_block(const float *x, int nmax, float rmin, int nstep, uint16_t *d_out, uint16_t *dmin_out,
                           uint8_t *scales, uint8_t *L) {
    float mins[8], scl[8], weights[32];
    uint8_t Laux[32];
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; ++j) {
        float sum_x2 = 0;
        for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
        const float av_x = sqrtf(sum_x2 / 32);
        for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(x[32 * j + l]);
        scl[j] = make_qkx2_quants(32, nmax, x + 32 * j, weights, L + 32 * j, &mins[j], Laux, rmin, 0.1f, nstep);
        if (scl[j] > max_scale) max_scale = scl[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    uint8_t ls[8], lm[8];
    for (int j = 0; j < 8; ++j) {
        int a = nearest_int(inv_scale * scl[j]), b = nearest_int(inv_min * mins[j]);
        ls[j] = (uint8_t) (a > 63 ? 63 : a);
        lm[j] = (uint8_t) (b > 63 ? 63 : b);
    }
    pack_scale_min_k4(scales, ls, lm);
    *d_out = or_f32_to_f16(max_scale / 63.f);
    *dmin_out = or_f32_to_f16(max_min / 63.f);
    for (int j = 0; j < 8; ++j) {
        uint8_t sc, m;
        scale_min_k4(j, scales, &sc, &m);
        const float d = or_f16_to_f32(*d_out) * sc;
        if (!d) continue;
        const float dm = or_f16_to_f32(*dmin_out) * m;
        for (int ii = 0; ii < 32; ++ii) {
            int l = nearest_int((x[32 * j + ii] + dm) / d);
            L[32 * j + ii] = (uint8_t) (l < 0 ? 0 : (l > nmax ? nmax : l));
        }
    }
}

static void quant_q4_K(const float *x, blk_q4_K *y) {
    uint8_t L[QK_K];
    quant_kx_block(x, 15, -1.0f, 20, &y->d, &y->dmin, y->scales, L);
    uint8_t *q = y->qs;
    for (int j = 0; j < QK_K; j += 64, q += 32)
        for (int l = 0; l < 32; ++l) q[l] = (uint8_t) (L[j + l] | (L[j + l + 32] << 4));
}

static void quant_q5_K(const float *x, blk_q5_K *y) {
    uint8_t L[QK_K];
    quant_kx_block(x, 31, -0.5f, 15, &y->d, &y->dmin, y->scales, L);
    memset(y->qh, 0, sizeof y->qh);
    uint8_t *ql = y->qs, m1 = 1, m2 = 2;
    for (int n = 0; n < QK_K; n += 64, ql += 32) {
        for (int j = 0; j < 32; ++j) {
            int l1 = L[n + j], l2 = L[n + j + 32];
            if (l1 > 15) { l1 -= 16; y->qh[j] |= m1; }
            if (l2 > 15) { l2 -= 16; y->qh[j] |= m2; }
            ql[j] = (uint8_t) (l1 | (l2 << 4));
        }
        m1 = (uint8_t) (m1 << 2);
        m2 = (uint8_t) (m2 << 2);
    }
}

static void quant_q6_K(const float *x, blk_q6_K *y) {
    int8_t L[QK_K];
    float scl[16];
    float max_scale = 0, max_abs_scale = 0;
    for (int ib = 0; ib < 16; ++ib) {
        scl[ib] = make_qx_quants(16, 32, x + 16 * ib, L + 16 * ib);
        const float as = fabsf(scl[ib]);
        if (as > max_abs_scale) { max_abs_scale = as; max_scale = scl[ib]; }
    }
    if (max_abs_scale < GROUP_MAX_EPS) {
        memset(y, 0, sizeof *y);
        return;
    }
    const float iscale = -128.f / max_scale;
    y->d = or_f32_to_f16(1 / iscale);
    for (int ib = 0; ib < 16; ++ib) {
        int v = nearest_int(iscale * scl[ib]);
        y->scales[ib] = (int8_t) (v > 127 ? 127 : v);
    }
    for (int j = 0; j < 16; ++j) {
        const float d = or_f16_to_f32(y->d) * y->scales[j];
        if (!d) continue;
        for (int ii = 0; ii < 16; ++ii) {
            int l = nearest_int(x[16 * j + ii] / d);
            l = l < -32 ? -32 : (l > 31 ? 31 : l);
            L[16 * j + ii] = (int8_t) (l + 32);
        }
    }
    uint8_t *ql = y->ql, *qh = y->qh;
    for (int j = 0; j < QK_K; j += 128, ql += 64, qh += 32) {
        for (int l = 0; l < 32; ++l) {
            const uint8_t q1 = L[j + l] & 0xF, q2 = L[j + l + 32] & 0xF, q3 = L[j + l + 64] & 0xF,
                          q4 = L[j + l + 96] & 0xF;
            ql[l] = (uint8_t) (q1 | (q3 << 4));
            ql[l + 32] = (uint8_t) (q2 | (q4 << 4));
            qh[l] = (uint8_t) ((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) | ((L[j + l + 64] >> 4) << 4) |
                               ((L[j + l + 96] >> 4) << 6));
        }
    }
}

static void quant_q3_K(const float *x, blk_q3_K *y) {
    int8_t L[QK_K];
    float scl[16];
    float max_scale = 0, amax = 0;
    for (int j = 0; j < 16; ++j) {
        scl[j] = make_q3_quants(16, 4, x + 16 * j, L + 16 * j);
        const float s = fabsf(scl[j]);
        if (s > amax) { amax = s; max_scale = scl[j]; }
    }
    memset(y->scales, 0, 12);
    if (max_scale) {
        const float iscale = -32.f / max_scale;
        for (int j = 0; j < 16; ++j) {
            int l = nearest_int(iscale * scl[j]);
            l = (l < -32 ? -32 : (l > 31 ? 31 : l)) + 32;
            if (j < 8) y->scales[j] = (uint8_t) (l & 0xF);
            else y->scales[j - 8] |= (uint8_t) ((l & 0xF) << 4);
            l >>= 4;
            y->scales[j % 4 + 8] |= (uint8_t) (l << (2 * (j / 4)));
        }
        y->d = or_f32_to_f16(1 / iscale);
    } else {
        y->d = 0;
    }
    for (int j = 0; j < 16; ++j) {
        int sc = j < 8 ? y->scales[j] & 0xF : y->scales[j - 8] >> 4;
        sc = (sc | (((y->scales[8 + j % 4] >> (2 * (j / 4))) & 3) << 4)) - 32;
        const float d = or_f16_to_f32(y->d) * sc;
        if (!d) continue;
        for (int ii = 0; ii < 16; ++ii) {
            int l = nearest_int(x[16 * j + ii] / d);
            l = l < -4 ? -4 : (l > 3 ? 3 : l);
            L[16 * j + ii] = (int8_t) (l + 4);
        }
    }
    memset(y->hmask, 0, 32);
    int m = 0;
    uint8_t hm = 1;
    for (int j = 0; j < QK_K; ++j) {
        if (L[j] > 3) {
            y->hmask[m] |= hm;
            L[j] = (int8_t) (L[j] - 4);
        }
        if (++m == QK_K / 8) {
            m = 0;
            hm = (uint8_t) (hm << 1);
        }
    }
    for (int j = 0; j < QK_K; j += 128)
        for (int l = 0; l < 32; ++l)
            y->qs[j / 4 + l] = (uint8_t) (L[j + l] | (L[j + l + 32] << 2) | (L[j + l + 64] << 4) | (L[j + l + 96] << 6));
}

static void quant_q8_0(const float *x, blk_q8_0 *y) {
    float amax = 0;
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(x[i]));
    const float d = amax / 127;
    const float id = d ? 1.0f / d : 0.0f;
    y->d = or_f32_to_f16(d);
    for (int i = 0; i < 32; ++i) y->qs[i] = (int8_t) roundf(x[i] * id);
}

int or_quantize(int type, const float *x, void *out, int64_t nrows, int64_t ncols, int nthreads) {
    const int be = or_block_elems(type);
    if (!be || type == OR_Q8_1 || ncols % be) return -1;
    const int64_t nb = nrows * (ncols / be);
    const size_t bb = or_block_bytes(type);
    (void) nthreads;
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
    for (int64_t i = 0; i < nb; ++i) {
        const float *xb = x + i * be;
        void *yb = (char *) out + (size_t) i * bb;
        switch (type) {
            case OR_Q8_0: quant_q8_0(xb, (blk_q8_0 *) yb); break;
            case OR_Q3_K: quant_q3_K(xb, (blk_q3_K *) yb); break;
            case OR_Q4_K: quant_q4_K(xb, (blk_q4_K *) yb); break;
            case OR_Q5_K: quant_q5_K(xb, (blk_q5_K *) yb); break;
            case OR_Q6_K: quant_q6_K(xb, (blk_q6_K *) yb); break;
        }
    }
    return 0;
}

/* ---- dequantisation (ggml dequantize_row_*, in float64) ---- */
static void deq_q4_K(const blk_q4_K *b, double *y) {
    const double d = or_f16_to_f32(b->d), dmin = or_f16_to_f32(b->dmin);
    const uint8_t *q = b->qs;
    for (int j = 0, is = 0; j < QK_K; j += 64, q += 32, is += 2) {
        uint8_t sc, m;
        scale_min_k4(is, b->scales, &sc, &m);
        const double d1 = d * sc, m1 = dmin * m;
        scale_min_k4(is + 1, b->scales, &sc, &m);
        const double d2 = d * sc, m2 = dmin * m;
        for (int l = 0; l < 32; ++l) y[j + l] = d1 * (q[l] & 0xF) - m1;
        for (int l = 0; l < 32; ++l) y[j + 32 + l] = d2 * (q[l] >> 4) - m2;
    }
}

static void deq_q5_K(const blk_q5_K *b, double *y) {
    const double d = or_f16_to_f32(b->d), dmin = or_f16_to_f32(b->dmin);
    const uint8_t *ql = b->qs;
    uint8_t u1 = 1, u2 = 2;
    for (int j = 0, is = 0; j < QK_K; j += 64, ql += 32, is += 2) {
        uint8_t sc, m;
        scale_min_k4(is, b->scales, &sc, &m);
        const double d1 = d * sc, m1 = dmin * m;
        scale_min_k4(is + 1, b->scales, &sc, &m);
        const double d2 = d * sc, m2 = dmin * m;
        for (int l = 0; l < 32; ++l) y[j + l] = d1 * ((ql[l] & 0xF) + (b->qh[l] & u1 ? 16 : 0)) - m1;
        for (int l = 0; l < 32; ++l) y[j + 32 + l] = d2 * ((ql[l] >> 4) + (b->qh[l] & u2 ? 16 : 0)) - m2;
        u1 = (uint8_t) (u1 << 2);
        u2 = (uint8_t) (u2 << 2);
    }
}

static void deq_q6_K(const blk_q6_K *b, double *y) {
    const double d = or_f16_to_f32(b->d);
    const uint8_t *ql = b->ql, *qh = b->qh;
    const int8_t *sc = b->scales;
    for (int n = 0; n < QK_K; n += 128, ql += 64, qh += 32, sc += 8) {
        for (int l = 0; l < 32; ++l) {
            const int is = l / 16;
            const int q1 = (int) ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
            const int q2 = (int) ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = (int) ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = (int) ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            y[n + l] = d * sc[is + 0] * q1;
            y[n + l + 32] = d * sc[is + 2] * q2;
            y[n + l + 64] = d * sc[is + 4] * q3;
            y[n + l + 96] = d * sc[is + 6] * q4;
        }
    }
}

static int q3_scale(const uint8_t *s, int j) {
    const int lo = j < 8 ? s[j] & 0xF : s[j - 8] >> 4;
    const int hi = (s[8 + j % 4] >> (2 * (j / 4))) & 3;
    return (lo | (hi << 4)) - 32;
}

static void deq_q3_K(const blk_q3_K *b, double *y) {
    const double d = or_f16_to_f32(b->d);
    const uint8_t *q = b->qs;
    uint8_t m = 1;
    int is = 0;
    for (int n = 0; n < QK_K; n += 128, q += 32) {
        int shift = 0;
        for (int j = 0; j < 4; ++j, shift += 2, m = (uint8_t) (m << 1)) {
            double dl = d * q3_scale(b->scales, is++);
            for (int l = 0; l < 16; ++l)
                y[n + 32 * j + l] = dl * ((int) ((q[l] >> shift) & 3) - ((b->hmask[l] & m) ? 0 : 4));
            dl = d * q3_scale(b->scales, is++);
            for (int l = 0; l < 16; ++l)
                y[n + 32 * j + 16 + l] = dl * ((int) ((q[l + 16] >> shift) & 3) - ((b->hmask[l + 16] & m) ? 0 : 4));
        }
    }
}

static void deq_q8_0(const blk_q8_0 *b, double *y) {
    const double d = or_f16_to_f32(b->d);
    for (int i = 0; i < 32; ++i) y[i] = d * b->qs[i];
}

/* IQ dequantisation (ggml-quants.c dequantize_row_iq4_xs / iq3_xxs / iq3_s / iq2_s): per 32-value sub-block a
 * scale, then codebook values with signs. Sub-block scale formulas are the dequantiser's; the integer rounding of
 * the GPU dot products is restated in or_iq_dot below. */
static void deq_iq4_xs(const blk_iq4_xs *b, double *y) {
    const double d = or_f16_to_f32(b->d);
    for (int ib = 0; ib < 8; ++ib) {
        const int ls = ((b->scales_l[ib / 2] >> (4 * (ib % 2))) & 0xf) | (((b->scales_h >> (2 * ib)) & 3) << 4);
        const double dl = d * (ls - 32);
        for (int j = 0; j < 16; ++j) {
            y[32 * ib + j] = dl * kvalues_iq4nl[b->qs[16 * ib + j] & 0xf];
            y[32 * ib + 16 + j] = dl * kvalues_iq4nl[b->qs[16 * ib + j] >> 4];
        }
    }
}
static void deq_iq3_xxs(const blk_iq3_xxs *b, double *y) {
    const double d = or_f16_to_f32(b->d);
    for (int ib = 0; ib < 8; ++ib) {
        uint32_t aux;
        memcpy(&aux, b->qs + 64 + 4 * ib, 4);
        const double db = d * (0.5 + (aux >> 28)) * 0.5;
        for (int l = 0; l < 4; ++l) {
            const int s = ksign_bits((aux >> (7 * l)) & 127);
            for (int h = 0; h < 2; ++h) {
                const uint32_t g = g_iq3xxs_grid[b->qs[8 * ib + 2 * l + h]];
                for (int j = 0; j < 4; ++j)
                    y[32 * ib + 8 * l + 4 * h + j] = db * (double) ((g >> (8 * j)) & 0xff) * ((s >> (4 * h + j)) & 1 ? -1 : 1);
            }
        }
    }
}
static void deq_iq3_s(const blk_iq3_s *b, double *y) {
    const double d = or_f16_to_f32(b->d);
    for (int ib = 0; ib < 8; ++ib) {
        const double db = d * (1 + 2 * ((b->scales[ib / 2] >> (4 * (ib % 2))) & 0xf));
        for (int l = 0; l < 8; ++l) {
            const uint32_t g = g_iq3s_grid[b->qs[8 * ib + l] | (((b->qh[ib] >> l) & 1) << 8)];
            const int s = b->signs[4 * ib + l / 2] >> (4 * (l % 2));
            for (int j = 0; j < 4; ++j)
                y[32 * ib + 4 * l + j] = db * (double) ((g >> (8 * j)) & 0xff) * ((s >> j) & 1 ? -1 : 1);
        }
    }
}
static void deq_iq2_s(const blk_iq2_s *b, double *y) {
    const double d = or_f16_to_f32(b->d);
    for (int ib = 0; ib < 8; ++ib) {
        for (int l = 0; l < 4; ++l) {
            const double dl = d * (0.5 + ((b->scales[ib] >> (4 * (l / 2))) & 0xf)) * 0.25;
            const uint64_t g = g_iq2s_grid[b->qs[4 * ib + l] | (((b->qh[ib] >> (2 * l)) & 3) << 8)];
            const int s = b->qs[32 + 4 * ib + l];
            for (int j = 0; j < 8; ++j)
                y[32 * ib + 8 * l + j] = dl * (double) ((g >> (8 * j)) & 0xff) * ((s >> j) & 1 ? -1 : 1);
        }
    }
}

/* One 32-value sub-block dot of an IQ block with a Q8_1 block, in the integer arithmetic of the reference's GPU
 * products (src/ggml/ggml_mmvq.cu:101-157 for IQ3_XXS / IQ3_S; ggml vecdotq.cuh vec_dot_iq4_xs_q8_1 /
 * vec_dot_iq2_s_q8_1 for the others): an exact integer sum, the sub-block scale applied in integers (C division
 * truncating toward zero), then d_w * d8 in fp32 times the integer. */
static double iq_sub_dot(int type, const void *blk, int ib, const int8_t *q8, float d8) {
    long sumi = 0;
    float dw = 0.0f;
    switch (type) {
        case OR_IQ4_XS: {
            const blk_iq4_xs *b = (const blk_iq4_xs *) blk;
            for (int j = 0; j < 16; ++j)
                sumi += kvalues_iq4nl[b->qs[16 * ib + j] & 0xf] * q8[j] + kvalues_iq4nl[b->qs[16 * ib + j] >> 4] * q8[16 + j];
            const int ls = ((b->scales_l[ib / 2] >> (4 * (ib % 2))) & 0xf) | (((b->scales_h >> (2 * ib)) & 3) << 4);
            sumi *= ls - 32;
            dw = or_f16_to_f32(b->d);
            break;
        }
        case OR_IQ3_XXS: {
            const blk_iq3_xxs *b = (const blk_iq3_xxs *) blk;
            uint32_t aux;
            memcpy(&aux, b->qs + 64 + 4 * ib, 4);
            for (int l = 0; l < 4; ++l) {
                const int s = ksign_bits((aux >> (7 * l)) & 127);
                for (int h = 0; h < 2; ++h) {
                    const uint32_t g = g_iq3xxs_grid[b->qs[8 * ib + 2 * l + h]];
                    for (int j = 0; j < 4; ++j) {
                        const int v = (int) ((g >> (8 * j)) & 0xff);
                        sumi += ((s >> (4 * h + j)) & 1 ? -v : v) * q8[8 * l + 4 * h + j];
                    }
                }
            }
            const long ls = aux >> 28;
            sumi = (ls * sumi + sumi / 2) / 2;
            dw = or_f16_to_f32(b->d);
            break;
        }
        case OR_IQ3_S: {
            const blk_iq3_s *b = (const blk_iq3_s *) blk;
            for (int l = 0; l < 8; ++l) {
                const uint32_t g = g_iq3s_grid[b->qs[8 * ib + l] | (((b->qh[ib] >> l) & 1) << 8)];
                const int s = b->signs[4 * ib + l / 2] >> (4 * (l % 2));
                for (int j = 0; j < 4; ++j) {
                    const int v = (int) ((g >> (8 * j)) & 0xff);
                    sumi += ((s >> j) & 1 ? -v : v) * q8[4 * l + j];
                }
            }
            sumi *= 1 + 2 * ((b->scales[ib / 2] >> (4 * (ib % 2))) & 0xf);
            dw = or_f16_to_f32(b->d);
            break;
        }
        case OR_IQ2_S: {
            const blk_iq2_s *b = (const blk_iq2_s *) blk;
            long s2[2] = {0, 0};
            for (int l = 0; l < 4; ++l) {
                const uint64_t g = g_iq2s_grid[b->qs[4 * ib + l] | (((b->qh[ib] >> (2 * l)) & 3) << 8)];
                const int s = b->qs[32 + 4 * ib + l];
                for (int j = 0; j < 8; ++j) {
                    const int v = (int) ((g >> (8 * j)) & 0xff);
                    s2[l / 2] += ((s >> j) & 1 ? -v : v) * q8[8 * l + j];
                }
            }
            const long ls0 = b->scales[ib] & 0xf, ls1 = b->scales[ib] >> 4;
            sumi = (s2[0] * ls0 + s2[1] * ls1 + (s2[0] + s2[1]) / 2) / 4;
            dw = or_f16_to_f32(b->d);
            break;
        }
    }
    return (double) (dw * d8) * (double) sumi;
}

static void deq_block(int type, const void *blk, double *y) {
    switch (type) {
        case OR_IQ4_XS: deq_iq4_xs((const blk_iq4_xs *) blk, y); break;
        case OR_IQ3_XXS: deq_iq3_xxs((const blk_iq3_xxs *) blk, y); break;
        case OR_IQ3_S: deq_iq3_s((const blk_iq3_s *) blk, y); break;
        case OR_IQ2_S: deq_iq2_s((const blk_iq2_s *) blk, y); break;
        case OR_Q8_0: deq_q8_0((const blk_q8_0 *) blk, y); break;
        case OR_Q3_K: deq_q3_K((const blk_q3_K *) blk, y); break;
        case OR_Q4_K: deq_q4_K((const blk_q4_K *) blk, y); break;
        case OR_Q5_K: deq_q5_K((const blk_q5_K *) blk, y); break;
        case OR_Q6_K: deq_q6_K((const blk_q6_K *) blk, y); break;
    }
}

int or_dequantize(int type, const void *in, double *out, int64_t nrows, int64_t ncols) {
    const int be = or_block_elems(type);
    if (!be || type == OR_Q8_1 || ncols % be) return -1;
    const int64_t nb = nrows * (ncols / be);
    const size_t bb = or_block_bytes(type);
    for (int64_t i = 0; i < nb; ++i) deq_block(type, (const char *) in + (size_t) i * bb, out + i * be);
    return 0;
}

/* ---- Q8_1 (GPU op order of the reference) ---- */
size_t or_q8_1_row_bytes(int64_t ncols) { return (size_t) ((ncols + 511) / 512 * 512 / QK8) * sizeof(blk_q8_1); }

void or_quantize_q8_1(const float *x, void *xq, int64_t ncols, int64_t nrows) {
    const int64_t nblk = (ncols + 511) / 512 * 512 / QK8;
    for (int64_t r = 0; r < nrows; ++r) {
        blk_q8_1 *y = (blk_q8_1 *) ((char *) xq + (size_t) r * or_q8_1_row_bytes(ncols));
        for (int64_t b = 0; b < nblk; ++b) {
            float v[32], am[32], s[32];
            for (int i = 0; i < 32; ++i) {
                const int64_t c = b * 32 + i;
                v[i] = c < ncols ? x[r * ncols + c] : 0.0f;
                am[i] = fabsf(v[i]);
                s[i] = v[i];
            }
            /* 32-lane xor butterfly, offsets 16, 8, 4, 2, 1: lane i adds lane i^o (all lanes end equal) */
            for (int o = 16; o > 0; o >>= 1) {
                float na[32], ns[32];
                for (int i = 0; i < 32; ++i) {
                    na[i] = fmaxf(am[i], am[i ^ o]);
                    ns[i] = s[i] + s[i ^ o];
                }
                memcpy(am, na, sizeof am);
                memcpy(s, ns, sizeof s);
            }
            const float amax = am[0], sum = s[0];
            const float d = amax / 127.0f;
            for (int i = 0; i < 32; ++i) y[b].qs[i] = amax == 0.0f ? 0 : (int8_t) roundf(v[i] / d);
            y[b].d = or_f32_to_f16(d);
            y[b].s = or_f32_to_f16(sum);
        }
    }
}

void or_dequantize_q8_1(const void *xq, double *out, int64_t ncols, int64_t nrows) {
    for (int64_t r = 0; r < nrows; ++r) {
        const blk_q8_1 *y = (const blk_q8_1 *) ((const char *) xq + (size_t) r * or_q8_1_row_bytes(ncols));
        for (int64_t c = 0; c < ncols; ++c)
            out[r * ncols + c] = (double) or_f16_to_f32(y[c / 32].d) * y[c / 32].qs[c % 32];
    }
}

/* ---- router and gating ---- */
void or_router_f32(const float *w, const float *x, float *logits, int64_t ncols, int64_t n_expert, int64_t n_tok) {
    for (int64_t t = 0; t < n_tok; ++t)
        for (int64_t e = 0; e < n_expert; ++e) {
            double s = 0;
            for (int64_t i = 0; i < ncols; ++i) s += (double) w[e * ncols + i] * (double) x[t * ncols + i];
            logits[t * n_expert + e] = (float) s;
        }
}

/* One wave of 64 lanes holds expert lane + 64*j (j < 4). The HIP kernel (route_topk) performs exactly these fp32
 * operations; argmax is order-independent (ties -> lower index), the softmax sum is restated lane by lane. */
int or_route_topk(const float *logits, int32_t *ids, float *w, float *probs, float *margin, int n_expert, int k,
                  int n_tok, int gating, int norm) {
    if (n_expert < 1 || n_expert > 256 || k < 1 || k > 16 || k > n_expert) return -1;
    for (int t = 0; t < n_tok; ++t) {
        const float *lg = logits + (size_t) t * n_expert;
        float p[256];
        if (gating == 0) {
            float m = -INFINITY;
            for (int e = 0; e < n_expert; ++e) m = fmaxf(m, lg[e]);
            float ev[256], lane[64];
            for (int e = 0; e < n_expert; ++e) ev[e] = or_expf(lg[e] - m);
            for (int l = 0; l < 64; ++l) {
                float s = 0.0f;
                for (int j = 0; j < 4; ++j) {
                    const int e = l + 64 * j;
                    s = s + (e < n_expert ? ev[e] : 0.0f);
                }
                lane[l] = s;
            }
            for (int o = 32; o > 0; o >>= 1) {
                float nl[64];
                for (int l = 0; l < 64; ++l) nl[l] = lane[l] + lane[l ^ o];
                memcpy(lane, nl, sizeof lane);
            }
            const float inv = 1.0f / lane[0];
            for (int e = 0; e < n_expert; ++e) p[e] = ev[e] * inv;
        } else {
            for (int e = 0; e < n_expert; ++e) p[e] = 1.0f / (1.0f + or_expf(-lg[e]));
        }
        if (probs) memcpy(probs + (size_t) t * n_expert, p, sizeof(float) * (size_t) n_expert);
        float sel[16], sum = 0.0f;
        int taken[256] = {0};
        for (int r = 0; r < k; ++r) {
            int best = -1;
            for (int e = 0; e < n_expert; ++e)
                if (!taken[e] && (best < 0 || p[e] > p[best])) best = e;
            taken[best] = 1;
            ids[(size_t) t * k + r] = best;
            sel[r] = p[best];
            sum += p[best];
        }
        for (int r = 0; r < k; ++r) w[(size_t) t * k + r] = norm ? sel[r] / fmaxf(sum, 6.103515625e-5f) : sel[r];
        if (margin) {
            /* logit gap between the k-th selected expert and the best unselected one */
            float lk = lg[ids[(size_t) t * k + k - 1]], best_out = -INFINITY;
            for (int e = 0; e < n_expert; ++e)
                if (!taken[e] && lg[e] > best_out) best_out = lg[e];
            margin[t] = k < n_expert ? lk - best_out : INFINITY;
        }
    }
    return 0;
}

/* ---- expert GEMV in float64 ---- */
int or_mmvq_experts(int type, const void *const *table, int64_t ncols, int64_t nrows, const void *xq, int64_t n_xq,
                    int64_t x_div, const int32_t *ids, int64_t n_ids, double *dst) {
    const int be = or_block_elems(type);
    if (!be || type == OR_Q8_1 || ncols % be || n_xq < 1 || x_div < 1) return -1;
    const size_t rb = or_row_bytes(type, ncols);
    if (or_is_iq(type)) {  /* the reference's integer sub-block products, float64 across sub-blocks */
        for (int64_t c = 0; c < n_ids; ++c) {
            const blk_q8_1 *xb = (const blk_q8_1 *) ((const char *) xq + (size_t) ((c / x_div) % n_xq) *
                                                                             or_q8_1_row_bytes(ncols));
            const char *base = (const char *) table[ids[c]];
            for (int64_t r = 0; r < nrows; ++r) {
                double s = 0;
                for (int64_t b = 0; b < ncols / QK_K; ++b)
                    for (int ib = 0; ib < 8; ++ib)
                        s += iq_sub_dot(type, base + (size_t) r * rb + (size_t) b * or_block_bytes(type), ib,
                                        xb[b * 8 + ib].qs, or_f16_to_f32(xb[b * 8 + ib].d));
                dst[c * nrows + r] = s;
            }
        }
        return 0;
    }
    double *xd = (double *) malloc(sizeof(double) * (size_t) ncols);
    double *wr = (double *) malloc(sizeof(double) * (size_t) ncols);
    if (!xd || !wr) { free(xd); free(wr); return -1; }
    for (int64_t c = 0; c < n_ids; ++c) {
        const int64_t row = (c / x_div) % n_xq;
        or_dequantize_q8_1((const char *) xq + (size_t) row * or_q8_1_row_bytes(ncols), xd, ncols, 1);
        const char *base = (const char *) table[ids[c]];
        for (int64_t r = 0; r < nrows; ++r) {
            or_dequantize(type, base + (size_t) r * rb, wr, 1, ncols);
            double s = 0;
            for (int64_t i = 0; i < ncols; ++i) s += wr[i] * xd[i];
            dst[c * nrows + r] = s;
        }
    }
    free(xd);
    free(wr);
    return 0;
}

void or_swiglu(const double *gate, const double *up, double *act, int64_t n) {
    for (int64_t i = 0; i < n; ++i) act[i] = up[i] * (gate[i] / (1.0 + exp(-gate[i])));
}

float or_amax_guard_scale(const float *row, int64_t n) {
    float m = 0.0f;
    for (int64_t i = 0; i < n; ++i) m = fmaxf(m, fabsf(row[i]));
    float e = m * (1.0f / 1024.0f);
    e = logf(e);
    e = e * 1.4426950408889634f;
    e = ceilf(e);
    e = fminf(fmaxf(e, 0.0f), 127.0f);
    e = e * 0.6931471805599453f;
    return expf(e);
}

void or_moe_combine(const float *dexp, const float *escale, const float *w, const float *sh, const float *x, float *out,
                    int64_t n, int k, int64_t n_tok) {
    for (int64_t t = 0; t < n_tok; ++t) {
        const float *d = dexp + (size_t) t * k * n;
        const float *e = escale ? escale + (size_t) t * k : NULL;
        const float *ww = w + (size_t) t * k;
        for (int64_t i = 0; i < n; ++i) {
            float moe = (d[i] * (e ? e[0] : 1.0f)) * ww[0];
            for (int j = 1; j < k; ++j) moe = moe + (d[(size_t) j * n + i] * (e ? e[j] : 1.0f)) * ww[j];
            const float s = sh ? sh[t * n + i] : 0.0f;
            out[t * n + i] = (moe + s) + (x ? x[t * n + i] : 0.0f);
        }
    }
}

int or_compact_ids(const int32_t *ids, int64_t n_tok, int k, int n_expert, int x_rows_per_tok, int32_t *bounds,
                   int32_t *src, int32_t *dst) {
    for (int e = 0; e <= n_expert; ++e) bounds[e] = 0;
    for (int64_t i = 0; i < n_tok * k; ++i) {
        if (ids[i] < 0 || ids[i] >= n_expert) return -1;
        bounds[ids[i] + 1]++;
    }
    int distinct = 0;
    for (int e = 0; e < n_expert; ++e) {
        distinct += bounds[e + 1] > 0;
        bounds[e + 1] += bounds[e];
    }
    int32_t *fill = (int32_t *) malloc(sizeof(int32_t) * (size_t) n_expert);
    if (!fill) return -1;
    memcpy(fill, bounds, sizeof(int32_t) * (size_t) n_expert);
    for (int64_t t = 0; t < n_tok; ++t)
        for (int j = 0; j < k; ++j) {
            const int e = ids[t * k + j];
            const int p = fill[e]++;
            src[p] = (int32_t) (t * x_rows_per_tok + (x_rows_per_tok == 1 ? 0 : j));
            dst[p] = (int32_t) (t * k + j);
        }
    free(fill);
    return distinct;
}

/* ---- CPU baseline: batch-1 layer, integer dot products per sub-block (not ggml) ---- */

/* Unpack one K-quant block into int8 values v[256] and per-16-value float scale/min pairs (32-value groups for
 * Q4_K/Q5_K, 16-value groups for Q3_K/Q6_K): value = sc[g] * v - mn[g]. */
static int unpack_block(int type, const void *blk, int8_t *v, float *sc, float *mn) {
    switch (type) {
        case OR_Q4_K: case OR_Q5_K: {
            const blk_q4_K *b4 = (const blk_q4_K *) blk;
            const blk_q5_K *b5 = (const blk_q5_K *) blk;
            const float d = or_f16_to_f32(type == OR_Q4_K ? b4->d : b5->d);
            const float dmin = or_f16_to_f32(type == OR_Q4_K ? b4->dmin : b5->dmin);
            const uint8_t *scales = type == OR_Q4_K ? b4->scales : b5->scales;
            const uint8_t *qs = type == OR_Q4_K ? b4->qs : b5->qs;
            for (int j = 0; j < 4; ++j)
                for (int l = 0; l < 32; ++l) {
                    int lo = qs[32 * j + l] & 0xF, hi = qs[32 * j + l] >> 4;
                    if (type == OR_Q5_K) {
                        lo += (b5->qh[l] >> (2 * j)) & 1 ? 16 : 0;
                        hi += (b5->qh[l] >> (2 * j + 1)) & 1 ? 16 : 0;
                    }
                    v[64 * j + l] = (int8_t) lo;
                    v[64 * j + 32 + l] = (int8_t) hi;
                }
            for (int g = 0; g < 8; ++g) {
                uint8_t s, m;
                scale_min_k4(g, scales, &s, &m);
                sc[g] = d * s;
                mn[g] = dmin * m;
            }
            return 32;
        }
        case OR_Q6_K: {
            const blk_q6_K *b = (const blk_q6_K *) blk;
            const float d = or_f16_to_f32(b->d);
            for (int n = 0; n < 2; ++n)
                for (int l = 0; l < 32; ++l) {
                    const uint8_t *ql = b->ql + 64 * n, *qh = b->qh + 32 * n;
                    v[128 * n + l] = (int8_t) (((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32);
                    v[128 * n + l + 32] = (int8_t) (((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
                    v[128 * n + l + 64] = (int8_t) (((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
                    v[128 * n + l + 96] = (int8_t) (((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
                }
            for (int g = 0; g < 16; ++g) {
                sc[g] = d * b->scales[g];
                mn[g] = 0;
            }
            return 16;
        }
        case OR_Q3_K: {
            const blk_q3_K *b = (const blk_q3_K *) blk;
            const float d = or_f16_to_f32(b->d);
            for (int n = 0; n < 2; ++n)
                for (int j = 0; j < 4; ++j)
                    for (int l = 0; l < 32; ++l) {
                        const int q = (b->qs[32 * n + l] >> (2 * j)) & 3;
                        const int h = (b->hmask[l] >> (4 * n + j)) & 1;
                        v[128 * n + 32 * j + l] = (int8_t) (q - (h ? 0 : 4));
                    }
            for (int g = 0; g < 16; ++g) {
                sc[g] = d * q3_scale(b->scales, g);
                mn[g] = 0;
            }
            return 16;
        }
    }
    return 0;
}

static float cpu_dot_row(int type, const char *row, const blk_q8_1 *xq, const int *xsum, int64_t ncols) {
    const size_t bb = or_block_bytes(type);
    float acc = 0.0f;
    int8_t v[256];
    float sc[16], mn[16];
    for (int64_t b = 0; b < ncols / 256; ++b) {
        const int g = unpack_block(type, row + b * bb, v, sc, mn);
        for (int s = 0; s < 256 / g; ++s) {
            const int c0 = (int) (b * 256 + s * g);
            const blk_q8_1 *q = &xq[c0 / 32];
            const int8_t *qs = q->qs + c0 % 32;
            int isum = 0;
            for (int i = 0; i < g; ++i) isum += v[s * g + i] * qs[i];
            const float d8 = or_f16_to_f32(q->d);
            int ys = 0;
            if (g == 32) ys = xsum[c0 / 32];
            acc += d8 * (sc[s] * (float) isum - mn[s] * (float) ys);
        }
    }
    return acc;
}

int or_cpu_moe_layer(int gu_type, int down_type, const float *router_w, const void *const *table, size_t gate_off,
                     size_t up_off, size_t down_off, const float *x, float *out, int64_t hidden, int64_t inter,
                     int n_expert, int k, int nthreads) {
    if (hidden % 256 || inter % 256 || k > 16 || n_expert > 256) return -1;
    const int nt = nthreads > 0 ? nthreads : 1;
    float logits[256], w[16];
    int32_t ids[16];
#pragma omp parallel for num_threads(nt)
    for (int e = 0; e < n_expert; ++e) {
        float s = 0.0f;
        for (int64_t i = 0; i < hidden; ++i) s += router_w[e * hidden + i] * x[i];
        logits[e] = s;
    }
    or_route_topk(logits, ids, w, NULL, NULL, n_expert, k, 1, 0, 1);
    const size_t hb = or_q8_1_row_bytes(hidden), ib = or_q8_1_row_bytes(inter);
    blk_q8_1 *xq = (blk_q8_1 *) malloc(hb), *aq = (blk_q8_1 *) malloc(ib * (size_t) k);
    int *xsum = (int *) malloc(sizeof(int) * (size_t) (hb / 36)), *asum = (int *) malloc(sizeof(int) * (ib / 36) * k);
    float *act = (float *) malloc(sizeof(float) * (size_t) (inter * k));
    float *dexp = (float *) malloc(sizeof(float) * (size_t) (hidden * k));
    if (!xq || !aq || !xsum || !asum || !act || !dexp) return -1;
    or_quantize_q8_1(x, xq, hidden, 1);
    for (size_t b = 0; b < hb / 36; ++b) {
        int s = 0;
        for (int i = 0; i < 32; ++i) s += xq[b].qs[i];
        xsum[b] = s;
    }
    const size_t gu_rb = or_row_bytes(gu_type, hidden), dn_rb = or_row_bytes(down_type, inter);
#pragma omp parallel for schedule(static) num_threads(nt)
    for (int64_t i = 0; i < inter * k; ++i) {
        const int j = (int) (i / inter);
        const int64_t r = i % inter;
        const char *base = (const char *) table[ids[j]];
        const float g = cpu_dot_row(gu_type, base + gate_off + r * gu_rb, xq, xsum, hidden);
        const float u = cpu_dot_row(gu_type, base + up_off + r * gu_rb, xq, xsum, hidden);
        act[i] = u * (g / (1.0f + expf(-g)));
    }
    or_quantize_q8_1(act, aq, inter, k);
    for (int j = 0; j < k; ++j) {
        const blk_q8_1 *row = (const blk_q8_1 *) ((const char *) aq + (size_t) j * ib);
        for (size_t b = 0; b < ib / 36; ++b) {
            int s = 0;
            for (int i = 0; i < 32; ++i) s += row[b].qs[i];
            asum[j * (ib / 36) + b] = s;
        }
    }
#pragma omp parallel for schedule(static) num_threads(nt)
    for (int64_t i = 0; i < hidden * k; ++i) {
        const int j = (int) (i / hidden);
        const int64_t r = i % hidden;
        const char *base = (const char *) table[ids[j]];
        dexp[i] = cpu_dot_row(down_type, base + down_off + r * dn_rb,
                              (const blk_q8_1 *) ((const char *) aq + (size_t) j * ib), asum + j * (ib / 36), inter);
    }
    or_moe_combine(dexp, NULL, w, NULL, NULL, out, hidden, k, 1);
    free(xq); free(aq); free(xsum); free(asum); free(act); free(dexp);
    return 0;
}
