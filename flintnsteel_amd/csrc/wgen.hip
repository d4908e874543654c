// wgen.hip - synthetic, seeded weights and activations on the GPU: Philox-4x32-10 normals and GGUF K-quant weight
// quantisers (ggml's reference quantisers quantize_row_q{3,4,5,6}_K_ref, llama.cpp 19ab5a5e, restated).
//
// The configs ask for weights "made by quantising N(0, 0.02) fp32 with ggml's reference quantizer"; 48 layers of 128
// experts is ~29 G weights, far too many for a host quantiser, so the quantisers run here, one thread per 256-value
// block, with the fp32 operations in the same order as the ggml algorithm (no contraction, IEEE division and square
// root). The tests compare them byte for byte with the CPU oracle's restatement.
#include "fns_common.hpp"
#include "fns_host.hpp"
#include "fns_internal.hpp"

namespace fns {

using namespace fns::dev;

namespace {

// ---- Philox-4x32-10 (Salmon et al., SC'11) + Box-Muller ----
__device__ __forceinline__ uint4 philox(uint4 c, uint2 k) {
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = (uint64_t) 0xD2511F53u * c.x, p1 = (uint64_t) 0xCD9E8D57u * c.z;
        c = make_uint4((uint32_t) (p1 >> 32) ^ c.y ^ k.x, (uint32_t) p1, (uint32_t) (p0 >> 32) ^ c.w ^ k.y, (uint32_t) p0);
        k.x += 0x9E3779B9u;
        k.y += 0xBB67AE85u;
    }
    return c;
}

__device__ __forceinline__ float u01(uint32_t v) { return ((float) (v >> 8) + 0.5f) * (1.0f / 16777216.0f); }

__global__ void k_fill_normal(float *__restrict__ out, int64_t n, uint64_t seed, uint64_t offset, float mean,
                              float std) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;  // one counter = 4 outputs
    if (4 * i >= n) return;
    const uint64_t ctr = offset / 4 + (uint64_t) i;
    const uint4 r = philox(make_uint4((uint32_t) ctr, (uint32_t) (ctr >> 32), 0x5eed, 0), make_uint2((uint32_t) seed,
                                                                                                       (uint32_t) (seed >> 32)));
    const float a = sqrtf(-2.0f * logf(u01(r.x))), b = sqrtf(-2.0f * logf(u01(r.z)));
    const float t1 = 6.2831853071795865f * u01(r.y), t2 = 6.2831853071795865f * u01(r.w);
    float v[4] = {a * cosf(t1), a * sinf(t1), b * cosf(t2), b * sinf(t2)};
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (4 * i + j < n) out[4 * i + j] = mean + std * v[j];
}

// ---- ggml reference quantisers ----
__device__ __forceinline__ int nearest(float f) { return (int) __builtin_rintf(f); }
__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }
__device__ __forceinline__ uint16_t f16bits(float f) { return (uint16_t) float_to_half(f); }
__device__ __forceinline__ float f16val(uint16_t h) { return half_to_float(h); }

// Weighted scale/min search over the grid 0..nmax (ggml make_qkx2_quants, squared error).
__device__ float qkx2(const float *x, const float *w, uint8_t *L, float *the_min, int nmax, float rmin, float rdelta,
                      int nstep) {
    float mn = x[0], mx = x[0], sum_w = w[0], sum_x = sum_w * x[0];
    for (int i = 1; i < 32; ++i) {
        if (x[i] < mn) mn = x[i];
        if (x[i] > mx) mx = x[i];
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    if (mn > 0) mn = 0;
    if (mx == mn) {
        for (int i = 0; i < 32; ++i) L[i] = 0;
        *the_min = -mn;
        return 0.0f;
    }
    float iscale = nmax / (mx - mn);
    float scale = 1 / iscale;
    float best_error = 0;
    for (int i = 0; i < 32; ++i) {
        const int l = clampi(nearest(iscale * (x[i] - mn)), 0, nmax);
        L[i] = (uint8_t) l;
        float diff = scale * L[i] + mn - x[i];
        diff = diff * diff;
        best_error += w[i] * diff;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (mx - mn);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < 32; ++i) {
            const int l = clampi(nearest(iscale * (x[i] - mn)), 0, nmax);
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
            for (int i = 0; i < 32; ++i) {
                const int l = clampi(nearest(iscale * (x[i] - mn)), 0, nmax);
                float diff = this_scale * l + this_min - x[i];
                diff = diff * diff;
                cur_error += w[i] * diff;
            }
            if (cur_error < best_error) {
                for (int i = 0; i < 32; ++i) L[i] = (uint8_t) clampi(nearest(iscale * (x[i] - mn)), 0, nmax);
                best_error = cur_error;
                scale = this_scale;
                mn = this_min;
            }
        }
    }
    *the_min = -mn;
    return scale;
}

__device__ __forceinline__ void scale_min_k4b(int j, const uint8_t *q, int &sc, int &m) {
    if (j < 4) {
        sc = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// Q4_K (nmax 15, rmin -1, 20 steps) and Q5_K (nmax 31, rmin -0.5, 15 steps): shared scale/min part.
template <int NMAX>
__device__ void quant_kx(const float *__restrict__ x, uint8_t *scales, uint16_t &dh, uint16_t &dminh, uint8_t *L) {
    constexpr float rmin = NMAX == 15 ? -1.0f : -0.5f;
    constexpr int nstep = NMAX == 15 ? 20 : 15;
    float mins[8], scl[8], wts[32], xs[32];
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; ++j) {
        float sum_x2 = 0;
        for (int l = 0; l < 32; ++l) {
            xs[l] = x[32 * j + l];
            sum_x2 += xs[l] * xs[l];
        }
        const float av_x = sqrtf(sum_x2 / 32);
        for (int l = 0; l < 32; ++l) wts[l] = av_x + fabsf(xs[l]);
        scl[j] = qkx2(xs, wts, L + 32 * j, &mins[j], NMAX, rmin, 0.1f, nstep);
        if (scl[j] > max_scale) max_scale = scl[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    for (int j = 0; j < 12; ++j) scales[j] = 0;
    for (int j = 0; j < 8; ++j) {
        const int ls = min(63, nearest(inv_scale * scl[j]));
        const int lm = min(63, nearest(inv_min * mins[j]));
        if (j < 4) {
            scales[j] = (uint8_t) ls;
            scales[j + 4] = (uint8_t) lm;
        } else {
            scales[j + 4] = (uint8_t) ((ls & 0xF) | ((lm & 0xF) << 4));
            scales[j - 4] |= (uint8_t) ((ls >> 4) << 6);
            scales[j] |= (uint8_t) ((lm >> 4) << 6);
        }
    }
    dh = f16bits(max_scale / 63.f);
    dminh = f16bits(max_min / 63.f);
    for (int j = 0; j < 8; ++j) {
        int sc, m;
        scale_min_k4b(j, scales, sc, m);
        const float d = f16val(dh) * sc;
        if (!d) continue;
        const float dm = f16val(dminh) * m;
        for (int ii = 0; ii < 32; ++ii) L[32 * j + ii] = (uint8_t) clampi(nearest((x[32 * j + ii] + dm) / d), 0, NMAX);
    }
}

__device__ void quant_q4_K(const float *x, uint8_t *y) {
    uint8_t L[256], scales[12];
    uint16_t dh, dminh;
    quant_kx<15>(x, scales, dh, dminh, L);
    uint8_t blk[144];
    blk[0] = dh & 0xff; blk[1] = dh >> 8; blk[2] = dminh & 0xff; blk[3] = dminh >> 8;
    for (int j = 0; j < 12; ++j) blk[4 + j] = scales[j];
    for (int j = 0; j < 4; ++j)
        for (int l = 0; l < 32; ++l) blk[16 + 32 * j + l] = (uint8_t) (L[64 * j + l] | (L[64 * j + l + 32] << 4));
    for (int i = 0; i < 144; ++i) y[i] = blk[i];
}

__device__ void quant_q5_K(const float *x, uint8_t *y) {
    uint8_t L[256], scales[12];
    uint16_t dh, dminh;
    quant_kx<31>(x, scales, dh, dminh, L);
    uint8_t blk[176];
    blk[0] = dh & 0xff; blk[1] = dh >> 8; blk[2] = dminh & 0xff; blk[3] = dminh >> 8;
    for (int j = 0; j < 12; ++j) blk[4 + j] = scales[j];
    uint8_t *qh = blk + 16, *ql = blk + 48;
    for (int j = 0; j < 32; ++j) qh[j] = 0;
    uint8_t m1 = 1, m2 = 2;
    for (int n = 0; n < 256; n += 64, ql += 32) {
        for (int j = 0; j < 32; ++j) {
            int l1 = L[n + j], l2 = L[n + j + 32];
            if (l1 > 15) { l1 -= 16; qh[j] |= m1; }
            if (l2 > 15) { l2 -= 16; qh[j] |= m2; }
            ql[j] = (uint8_t) (l1 | (l2 << 4));
        }
        m1 = (uint8_t) (m1 << 2);
        m2 = (uint8_t) (m2 << 2);
    }
    for (int i = 0; i < 176; ++i) y[i] = blk[i];
}

constexpr float kGroupMaxEps = 1e-15f;

// ggml make_qx_quants with rmse_type 1 (weights x^2), 16 values, grid -nmax..nmax-1; L = l + nmax.
__device__ float qx16(const float *x, int8_t *L, int nmax) {
    float mx = 0, amax = 0;
    for (int i = 0; i < 16; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; mx = x[i]; }
    }
    if (amax < kGroupMaxEps) {
        for (int i = 0; i < 16; ++i) L[i] = 0;
        return 0.0f;
    }
    float iscale = -nmax / mx;
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < 16; ++i) {
        const int l = clampi(nearest(iscale * x[i]), -nmax, nmax - 1);
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
        for (int i = 0; i < 16; ++i) {
            const int l = clampi(nearest(iscale * x[i]), -nmax, nmax - 1);
            const float w = x[i] * x[i];
            sumlx += w * x[i] * l;
            suml2 += w * l * l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < 16; ++i) L[i] = (int8_t) (nmax + clampi(nearest(iscale * x[i]), -nmax, nmax - 1));
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

__device__ void quant_q6_K(const float *x, uint8_t *y) {
    int8_t L[256];
    float scl[16], xs[16];
    float max_scale = 0, max_abs_scale = 0;
    for (int ib = 0; ib < 16; ++ib) {
        for (int i = 0; i < 16; ++i) xs[i] = x[16 * ib + i];
        scl[ib] = qx16(xs, L + 16 * ib, 32);
        const float as = fabsf(scl[ib]);
        if (as > max_abs_scale) { max_abs_scale = as; max_scale = scl[ib]; }
    }
    uint8_t blk[210];
    if (max_abs_scale < kGroupMaxEps) {
        for (int i = 0; i < 210; ++i) y[i] = 0;
        return;
    }
    const float iscale = -128.f / max_scale;
    const uint16_t dh = f16bits(1 / iscale);
    int8_t *sc = (int8_t *) (blk + 192);
    for (int ib = 0; ib < 16; ++ib) sc[ib] = (int8_t) min(127, nearest(iscale * scl[ib]));
    for (int j = 0; j < 16; ++j) {
        const float d = f16val(dh) * sc[j];
        if (!d) continue;
        for (int ii = 0; ii < 16; ++ii) L[16 * j + ii] = (int8_t) (clampi(nearest(x[16 * j + ii] / d), -32, 31) + 32);
    }
    uint8_t *ql = blk, *qh = blk + 128;
    for (int j = 0; j < 256; j += 128, ql += 64, qh += 32) {
        for (int l = 0; l < 32; ++l) {
            const uint8_t q1 = L[j + l] & 0xF, q2 = L[j + l + 32] & 0xF, q3 = L[j + l + 64] & 0xF, q4 = L[j + l + 96] & 0xF;
            ql[l] = (uint8_t) (q1 | (q3 << 4));
            ql[l + 32] = (uint8_t) (q2 | (q4 << 4));
            qh[l] = (uint8_t) ((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) | ((L[j + l + 64] >> 4) << 4) |
                               ((L[j + l + 96] >> 4) << 6));
        }
    }
    blk[208] = dh & 0xff;
    blk[209] = dh >> 8;
    for (int i = 0; i < 210; ++i) y[i] = blk[i];
}

// ggml make_q3_quants with rmse refinement, 16 values, nmax 4; returns L = l + nmax.
__device__ float q3_16(const float *x, int8_t *L) {
    constexpr int nmax = 4;
    float mx = 0, amax = 0;
    for (int i = 0; i < 16; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; mx = x[i]; }
    }
    if (amax < kGroupMaxEps) {
        for (int i = 0; i < 16; ++i) L[i] = 0;
        return 0.0f;
    }
    const float iscale = -nmax / mx;
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < 16; ++i) {
        const int l = clampi(nearest(iscale * x[i]), -nmax, nmax - 1);
        L[i] = (int8_t) l;
        const float w = x[i] * x[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    for (int itry = 0; itry < 5; ++itry) {
        int n_changed = 0;
        for (int i = 0; i < 16; ++i) {
            const float w = x[i] * x[i];
            float slx = sumlx - w * x[i] * L[i];
            if (slx > 0) {
                float sl2 = suml2 - w * L[i] * L[i];
                const int new_l = clampi(nearest(x[i] * sl2 / slx), -nmax, nmax - 1);
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
    for (int i = 0; i < 16; ++i) L[i] = (int8_t) (L[i] + nmax);
    return sumlx / suml2;
}

__device__ void quant_q3_K(const float *x, uint8_t *y) {
    int8_t L[256];
    float scl[16], xs[16];
    float max_scale = 0, amax = 0;
    for (int j = 0; j < 16; ++j) {
        for (int i = 0; i < 16; ++i) xs[i] = x[16 * j + i];
        scl[j] = q3_16(xs, L + 16 * j);
        const float s = fabsf(scl[j]);
        if (s > amax) { amax = s; max_scale = scl[j]; }
    }
    uint8_t blk[110];
    uint8_t *hmask = blk, *qs = blk + 32, *scales = blk + 96;
    for (int j = 0; j < 12; ++j) scales[j] = 0;
    uint16_t dh = 0;
    if (max_scale) {
        const float iscale = -32.f / max_scale;
        for (int j = 0; j < 16; ++j) {
            int l = clampi(nearest(iscale * scl[j]), -32, 31) + 32;
            if (j < 8) scales[j] = (uint8_t) (l & 0xF);
            else scales[j - 8] |= (uint8_t) ((l & 0xF) << 4);
            l >>= 4;
            scales[j % 4 + 8] |= (uint8_t) (l << (2 * (j / 4)));
        }
        dh = f16bits(1 / iscale);
    }
    for (int j = 0; j < 16; ++j) {
        int sc = j < 8 ? scales[j] & 0xF : scales[j - 8] >> 4;
        sc = (sc | (((scales[8 + j % 4] >> (2 * (j / 4))) & 3) << 4)) - 32;
        const float d = f16val(dh) * sc;
        if (!d) continue;
        for (int ii = 0; ii < 16; ++ii) L[16 * j + ii] = (int8_t) (clampi(nearest(x[16 * j + ii] / d), -4, 3) + 4);
    }
    for (int j = 0; j < 32; ++j) hmask[j] = 0;
    int m = 0;
    uint8_t hm = 1;
    for (int j = 0; j < 256; ++j) {
        if (L[j] > 3) {
            hmask[m] |= hm;
            L[j] = (int8_t) (L[j] - 4);
        }
        if (++m == 32) {
            m = 0;
            hm = (uint8_t) (hm << 1);
        }
    }
    for (int j = 0; j < 256; j += 128)
        for (int l = 0; l < 32; ++l)
            qs[j / 4 + l] = (uint8_t) (L[j + l] | (L[j + l + 32] << 2) | (L[j + l + 64] << 4) | (L[j + l + 96] << 6));
    blk[108] = dh & 0xff;
    blk[109] = dh >> 8;
    for (int i = 0; i < 110; ++i) y[i] = blk[i];
}

// ggml quantize_row_q8_0_ref over 8 consecutive blocks of 32: d = amax / 127, q = roundf(x / d) (x * (1/d), as ggml).
__device__ void quant_q8_0(const float *x, uint8_t *y) {
    for (int b = 0; b < 8; ++b) {
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(x[32 * b + i]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint32_t dh = float_to_half(d);
        y[34 * b] = dh & 0xff;
        y[34 * b + 1] = dh >> 8;
        for (int i = 0; i < 32; ++i) y[34 * b + 2 + i] = (uint8_t) (int8_t) roundf(x[32 * b + i] * id);
    }
}

template <int T>
__global__ __launch_bounds__(64) void k_quantize_blocks(const float *__restrict__ x, uint8_t *__restrict__ y,
                                                        int64_t nblocks) {
    const int64_t b = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const float *xb = x + b * 256;
    uint8_t *yb = y + b * block_bytes(T);
    if constexpr (T == T_Q4_K) quant_q4_K(xb, yb);
    if constexpr (T == T_Q5_K) quant_q5_K(xb, yb);
    if constexpr (T == T_Q6_K) quant_q6_K(xb, yb);
    if constexpr (T == T_Q3_K) quant_q3_K(xb, yb);
    if constexpr (T == T_Q8_0) quant_q8_0(xb, yb);
}

}  // namespace

namespace impl {

int fill_normal(float *out, int64_t n, uint64_t seed, uint64_t offset, float mean, float std, hipStream_t st) {
    if (!out || n < 0 || offset % 4) return host::set_error(host::ERR_SHAPE, "fill_normal: bad arguments (offset % 4)");
    if (n == 0) return host::OK;
    const int64_t nthreads = (n + 3) / 4;
    hipLaunchKernelGGL(k_fill_normal, dim3((unsigned) ((nthreads + 255) / 256)), dim3(256), 0, st, out, n, seed,
                       offset, mean, std);
    return host::check_launch("fill_normal");
}

int quantize_weights(int type, const float *x, void *out, int64_t nrows, int64_t ncols, hipStream_t st) {
    if (!host::is_kquant(type) && type != T_Q8_0)
        return host::set_error(host::ERR_TYPE, "quantize_weights: type %d not supported", type);
    if (!x || !out || nrows < 0 || ncols <= 0 || ncols % 256)
        return host::set_error(host::ERR_SHAPE, "quantize_weights: ncols must be a positive multiple of 256");
    const int64_t nb = nrows * (ncols / 256);
    if (nb == 0) return host::OK;
    const dim3 g((unsigned) ((nb + 63) / 64));
    switch (type) {
        case T_Q3_K: hipLaunchKernelGGL(k_quantize_blocks<T_Q3_K>, g, dim3(64), 0, st, x, (uint8_t *) out, nb); break;
        case T_Q4_K: hipLaunchKernelGGL(k_quantize_blocks<T_Q4_K>, g, dim3(64), 0, st, x, (uint8_t *) out, nb); break;
        case T_Q5_K: hipLaunchKernelGGL(k_quantize_blocks<T_Q5_K>, g, dim3(64), 0, st, x, (uint8_t *) out, nb); break;
        case T_Q6_K: hipLaunchKernelGGL(k_quantize_blocks<T_Q6_K>, g, dim3(64), 0, st, x, (uint8_t *) out, nb); break;
        case T_Q8_0: hipLaunchKernelGGL(k_quantize_blocks<T_Q8_0>, g, dim3(64), 0, st, x, (uint8_t *) out, nb); break;
    }
    return host::check_launch("quantize_weights");
}

}  // namespace impl

}  // namespace fns
