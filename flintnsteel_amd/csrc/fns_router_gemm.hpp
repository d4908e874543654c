// Batch router GEMM on fp32 MFMA, shared by the router kernel and the prefill kernel that also builds the activation
// image (reference src/prefill_kernels.cu:217-233).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace fns {
namespace {

__device__ __forceinline__ float bf16_to_float(uint16_t b) { return __builtin_bit_cast(float, (uint32_t) b << 16); }

// y[t][e] = sum_i W[e][i] x[t][i] (+ bias[e]) with v_mfma_f32_16x16x4_f32. A 512-thread workgroup computes 16 tokens x
// 16 experts (tile (bx, by)); its 8 waves split the columns in chunks of 64 and add their partial tiles in wave
// order through LDS. In the operand layout lane (i = lane % 16, kk = lane / 16) holds, for columns k0 + 16 u + 4 kk
// .. +3, a float4 of x row i and of W row i, and MFMA m of the step takes element m of both (the same permutation of
// k on both operands). BF16: W is bf16 and x is rounded to bf16 first (the reference's cuBLAS BF16 path).
typedef float v4f __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld4_guard(const float *row, int k, int ncols) {
    if (k + 3 < ncols) return *(const float4 *) (row + k);
    float v[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) v[m] = k + m < ncols ? row[k + m] : 0.0f;
    return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ float4 ld4_bf16(const uint16_t *p) {
    const uint2 v = *(const uint2 *) p;
    return make_float4(__builtin_bit_cast(float, v.x << 16), __builtin_bit_cast(float, v.x & 0xffff0000u),
                       __builtin_bit_cast(float, v.y << 16), __builtin_bit_cast(float, v.y & 0xffff0000u));
}
__device__ __forceinline__ float4 ld4_bf16_guard(const uint16_t *row, int k, int ncols) {
    float v[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) v[m] = k + m < ncols ? bf16_to_float(row[k + m]) : 0.0f;
    return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ float round_bf16(float v) {
    uint32_t b = __builtin_bit_cast(uint32_t, v);
    b = (b + 0x7fffu + ((b >> 16) & 1u)) & 0xffff0000u;
    return __builtin_bit_cast(float, b);
}
// FULL: ncols is a multiple of 64, so every chunk is whole and the loads need no guard (a guarded load is a branch,
// and the compiler then waits for each load before issuing the next).
template <bool BF16, bool FULL>
__device__ __forceinline__ void router_gemm_tile(const void *__restrict__ w, const float *__restrict__ bias,
                                                 const float *__restrict__ x, float *__restrict__ y, int ncols,
                                                 int nrows, int n_tok, int bx, int by) {
    // 16 tokens x 16 experts per workgroup; the 8 waves split the columns (wave w: chunks of 64 columns w, w + 8, ...,
    // the next chunk's loads in flight while one is multiplied) and their partial tiles are added in wave order
    // through LDS.
    constexpr int NW = 8;
    __shared__ v4f part[NW][64];
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64, il = lane % 16, kk = lane / 16;
    const int t0 = bx * 16, e0 = by * 16;
    const int ta = min(t0 + il, n_tok - 1), ea = min(e0 + il, nrows - 1);  // clamped rows (results discarded)
    const float *xr = x + (size_t) ta * ncols;
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    float4 a[4], b[4];
    auto load = [&](int k0) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int k = k0 + 16 * u + 4 * kk;
            if constexpr (FULL) {
                a[u] = *(const float4 *) (xr + k);
                if constexpr (BF16) b[u] = ld4_bf16((const uint16_t *) w + (size_t) ea * ncols + k);
                else b[u] = *(const float4 *) ((const float *) w + (size_t) ea * ncols + k);
            } else {
                a[u] = ld4_guard(xr, k, ncols);
                if constexpr (BF16) b[u] = ld4_bf16_guard((const uint16_t *) w + (size_t) ea * ncols, k, ncols);
                else b[u] = ld4_guard((const float *) w + (size_t) ea * ncols, k, ncols);
            }
        }
    };
    if constexpr (FULL) {
        // Coalesced loads, each instruction covering 4 whole 256-byte row pieces of the chunk (8 full cache lines
        // instead of 16 half lines in the MFMA operand layout), through a wave-private padded LDS tile back into
        // that layout. Same chunk order and products as the direct loop below.
        __shared__ __align__(16) float tile[NW][2][16][68];
        float (*xs)[68] = tile[wave][0], (*wsh)[68] = tile[wave][1];
        const int lr = lane / 16, lc = 4 * (lane % 16);
        // element offsets of this lane's four rows (clamped rows: results discarded)
        const int xo0 = min(t0 + lr, n_tok - 1) * ncols + lc, xo1 = min(t0 + 4 + lr, n_tok - 1) * ncols + lc;
        const int xo2 = min(t0 + 8 + lr, n_tok - 1) * ncols + lc, xo3 = min(t0 + 12 + lr, n_tok - 1) * ncols + lc;
        const int wo0 = min(e0 + lr, nrows - 1) * ncols + lc, wo1 = min(e0 + 4 + lr, nrows - 1) * ncols + lc;
        const int wo2 = min(e0 + 8 + lr, nrows - 1) * ncols + lc, wo3 = min(e0 + 12 + lr, nrows - 1) * ncols + lc;
        auto ldw = [&](int off) {
            if constexpr (BF16) return ld4_bf16((const uint16_t *) w + off);
            else return *(const float4 *) ((const float *) w + off);
        };
        float4 ga0, ga1, ga2, ga3, gb0, gb1, gb2, gb3;
        int k0 = wave * 64;
        if (k0 < ncols) {
            ga0 = *(const float4 *) (x + xo0 + k0), ga1 = *(const float4 *) (x + xo1 + k0);
            ga2 = *(const float4 *) (x + xo2 + k0), ga3 = *(const float4 *) (x + xo3 + k0);
            gb0 = ldw(wo0 + k0), gb1 = ldw(wo1 + k0), gb2 = ldw(wo2 + k0), gb3 = ldw(wo3 + k0);
        }
        for (; k0 < ncols; k0 += NW * 64) {
            // (the tile is wave-private: LDS accesses of one wave complete in order; the wave barriers keep the
            // compiler from moving the reads of one chunk across the writes of the next)
            __builtin_amdgcn_wave_barrier();
            *(float4 *) &xs[lr][lc] = ga0, *(float4 *) &xs[4 + lr][lc] = ga1;
            *(float4 *) &xs[8 + lr][lc] = ga2, *(float4 *) &xs[12 + lr][lc] = ga3;
            *(float4 *) &wsh[lr][lc] = gb0, *(float4 *) &wsh[4 + lr][lc] = gb1;
            *(float4 *) &wsh[8 + lr][lc] = gb2, *(float4 *) &wsh[12 + lr][lc] = gb3;
            const int kn = k0 + NW * 64;
            if (kn < ncols) {
                ga0 = *(const float4 *) (x + xo0 + kn), ga1 = *(const float4 *) (x + xo1 + kn);
                ga2 = *(const float4 *) (x + xo2 + kn), ga3 = *(const float4 *) (x + xo3 + kn);
                gb0 = ldw(wo0 + kn), gb1 = ldw(wo1 + kn), gb2 = ldw(wo2 + kn), gb3 = ldw(wo3 + kn);
            }
            __builtin_amdgcn_wave_barrier();
            float4 ca[4], cb[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                ca[u] = *(const float4 *) &xs[il][16 * u + 4 * kk];
                cb[u] = *(const float4 *) &wsh[il][16 * u + 4 * kk];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float av[4] = {ca[u].x, ca[u].y, ca[u].z, ca[u].w}, bv[4] = {cb[u].x, cb[u].y, cb[u].z, cb[u].w};
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const float xa = BF16 ? round_bf16(av[m]) : av[m];
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa, bv[m], acc, 0, 0, 0);
                }
            }
        }
    } else {
    int k0 = wave * 64;
    if (k0 < ncols) load(k0);
    for (; k0 < ncols; k0 += NW * 64) {
        float av[4][4], bv[4][4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            av[u][0] = a[u].x, av[u][1] = a[u].y, av[u][2] = a[u].z, av[u][3] = a[u].w;
            bv[u][0] = b[u].x, bv[u][1] = b[u].y, bv[u][2] = b[u].z, bv[u][3] = b[u].w;
        }
        if (k0 + NW * 64 < ncols) load(k0 + NW * 64);
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const float xa = BF16 ? round_bf16(av[u][m]) : av[u][m];
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa, bv[u][m], acc, 0, 0, 0);
            }
    }
    }
    part[wave][lane] = acc;
    __syncthreads();
    if (wave == 0) {
        v4f s = part[0][lane];
#pragma unroll
        for (int w2 = 1; w2 < NW; ++w2) s += part[w2][lane];
        const int e = e0 + il;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = t0 + 4 * kk + r;
            if (t < n_tok && e < nrows) y[(size_t) t * nrows + e] = bias ? s[r] + bias[e] : s[r];
        }
    }
}

}  // namespace
}  // namespace fns
