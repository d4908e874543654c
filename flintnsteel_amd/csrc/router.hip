// router.hip - router logits (fp32 / bf16 GEMV and batch GEMM), gating + top-k + renormalisation, weighted combine
// and the routing histogram, for MI355X gfx950.
//
// Reference: src/kernels.cu:452-514 (gemv_bf16, route_topk), :579-586 (moe_combine), :955-962 (count_routes);
// src/prefill_kernels.cu:133-183,217-242 (batch router, route_topk_batch, moe_combine_batch). Gating is
// generalised to softmax (the configs, llama.cpp build_moe_ffn) or sigmoid (the Flint model), any expert count up to
// 256 and k up to 16; the reference hard-codes sigmoid, 256 experts and k <= 8.
#include <algorithm>
#include "fns/kernels.h"
#include "fns_common.hpp"
#include "fns_host.hpp"
#include "fns_internal.hpp"
#include "fns_route.hpp"
#include "fns_router_gemm.hpp"

namespace fns {

using namespace fns::dev;

namespace {

// One workgroup (256 lanes) per output row r; COLS input columns share the row read.
template <int COLS, bool BF16>
__global__ __launch_bounds__(256) void k_gemv_router(const void *__restrict__ w, const float *__restrict__ x,
                                                     float *__restrict__ y, int ncols, int nrows) {
    __shared__ float red[4][COLS];
    const int r = blockIdx.x;
    float s[COLS];
#pragma unroll
    for (int c = 0; c < COLS; ++c) s[c] = 0.0f;
    if (ncols % 4 == 0) {
        for (int i = threadIdx.x; i < ncols / 4; i += 256) {
            float4 wv;
            if constexpr (BF16) {
                const uint2 pk = ((const uint2 *) ((const uint16_t *) w + (size_t) r * ncols))[i];
                wv = make_float4(bf16_to_float(pk.x & 0xffff), bf16_to_float(pk.x >> 16), bf16_to_float(pk.y & 0xffff),
                                 bf16_to_float(pk.y >> 16));
            } else {
                wv = ((const float4 *) ((const float *) w + (size_t) r * ncols))[i];
            }
#pragma unroll
            for (int c = 0; c < COLS; ++c) {
                const float4 xv = ((const float4 *) (x + (size_t) c * ncols))[i];
                s[c] += wv.x * xv.x + wv.y * xv.y + wv.z * xv.z + wv.w * xv.w;
            }
        }
    } else {
        for (int i = threadIdx.x; i < ncols; i += 256) {
            const float wv = BF16 ? bf16_to_float(((const uint16_t *) w)[(size_t) r * ncols + i])
                                  : ((const float *) w)[(size_t) r * ncols + i];
#pragma unroll
            for (int c = 0; c < COLS; ++c) s[c] += wv * x[(size_t) c * ncols + i];
        }
    }
#pragma unroll
    for (int c = 0; c < COLS; ++c) {
        const float v = lanes_sum<64>(s[c]);
        if (threadIdx.x % 64 == 0) red[threadIdx.x / 64][c] = v;
    }
    __syncthreads();
    if (threadIdx.x < COLS)
        y[(size_t) threadIdx.x * nrows + r] =
            (red[0][threadIdx.x] + red[1][threadIdx.x]) + (red[2][threadIdx.x] + red[3][threadIdx.x]);
}

template <bool BF16, bool FULL>
__global__ __launch_bounds__(512) void k_gemm_router(const void *__restrict__ w, const float *__restrict__ bias,
                                                     const float *__restrict__ x, float *__restrict__ y, int ncols,
                                                     int nrows, int n_tok) {
    router_gemm_tile<BF16, FULL>(w, bias, x, y, ncols, nrows, n_tok, blockIdx.x, blockIdx.y);
}

}  // namespace

namespace {

// One token per 256-thread workgroup: the rank-based block top-k (same probabilities, same selection and weights as
// route_topk_wave, bit for bit), without the k dependent argmax rounds of a single wave.
constexpr int kRouteThreads = 256;
template <int NT>
__global__ __launch_bounds__(NT) void k_route_topk(const float *__restrict__ logits, int32_t *__restrict__ ids,
                                                   float *__restrict__ w, int n_expert, int k, int gating, int norm) {
    __shared__ __align__(16) uint64_t s_key[kTopkScratch];
    __shared__ int s_sel[16];
    __shared__ float s_pv[16];
    PF_MARK(1, 0);
    const int t = blockIdx.x;
    route_topk_block<NT>((int) threadIdx.x, logits + (size_t) t * n_expert, n_expert, k, gating, s_key, s_sel, s_pv);
    if ((int) threadIdx.x < k) {
        ids[(size_t) t * k + threadIdx.x] = s_sel[threadIdx.x];
        w[(size_t) t * k + threadIdx.x] = route_weight(s_pv, k, norm, threadIdx.x);
    }
    PF_MARK(1, 1);
}

__global__ void k_moe_combine(const float *__restrict__ dexp, const float *__restrict__ escale,
                              const float *__restrict__ w, const float *__restrict__ sh, const float *x_in, float *out,
                              int n, int k) {
    const int t = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float *d = dexp + (size_t) t * k * n;
    const float *e = escale ? escale + (size_t) t * k : nullptr;
    const float *ww = w + (size_t) t * k;
    float moe = (d[i] * (e ? e[0] : 1.0f)) * ww[0];
    for (int j = 1; j < k; ++j) moe = moe + (d[(size_t) j * n + i] * (e ? e[j] : 1.0f)) * ww[j];
    const float s = sh ? sh[(size_t) t * n + i] : 0.0f;
    out[(size_t) t * n + i] = (moe + s) + (x_in ? x_in[(size_t) t * n + i] : 0.0f);
}

// Four adjacent columns per thread and the k expert rows unrolled, every load issued before the sums; the same
// arithmetic and order per column as k_moe_combine.
template <int K>
__global__ void k_moe_combine4(const float *__restrict__ dexp, const float *__restrict__ escale,
                               const float *__restrict__ w, const float *__restrict__ sh, const float *x_in, float *out,
                               int n) {
    PF_MARK(4, 0);
    const int t = blockIdx.y;
    const int i = 4 * (blockIdx.x * blockDim.x + threadIdx.x);
    if (i >= n) return;
    const float *d = dexp + (size_t) t * K * n + i;
    float4 dv[K];
#pragma unroll
    for (int j = 0; j < K; ++j) dv[j] = *(const float4 *) (d + (size_t) j * n);
    const float4 s = sh ? *(const float4 *) (sh + (size_t) t * n + i) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float4 xv = x_in ? *(const float4 *) (x_in + (size_t) t * n + i) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float ws[K], es[K];
#pragma unroll
    for (int j = 0; j < K; ++j) {
        ws[j] = w[(size_t) t * K + j];
        es[j] = escale ? escale[(size_t) t * K + j] : 1.0f;
    }
    auto col = [&](auto get) {
        float moe = (get(dv[0]) * es[0]) * ws[0];
#pragma unroll
        for (int j = 1; j < K; ++j) moe = moe + (get(dv[j]) * es[j]) * ws[j];
        return moe;
    };
    float4 o;
    o.x = (col([](float4 v) { return v.x; }) + s.x) + xv.x;
    o.y = (col([](float4 v) { return v.y; }) + s.y) + xv.y;
    o.z = (col([](float4 v) { return v.z; }) + s.z) + xv.z;
    o.w = (col([](float4 v) { return v.w; }) + s.w) + xv.w;
    *(float4 *) (out + (size_t) t * n + i) = o;
    PF_MARK(4, 1);
}

__global__ void k_count_routes(const int32_t *ids, uint32_t *counts, int k) {
    if ((int) threadIdx.x < k) atomicAdd(&counts[ids[threadIdx.x]], 1u);
}

template <bool BF16> int launch_gemv(const void *w, const float *x, float *y, int ncols, int nrows, int cols,
                                     hipStream_t st) {
    const dim3 g((unsigned) nrows);
    switch (cols) {
        case 1: hipLaunchKernelGGL((k_gemv_router<1, BF16>), g, dim3(256), 0, st, w, x, y, ncols, nrows); break;
        case 2: hipLaunchKernelGGL((k_gemv_router<2, BF16>), g, dim3(256), 0, st, w, x, y, ncols, nrows); break;
        case 3: hipLaunchKernelGGL((k_gemv_router<3, BF16>), g, dim3(256), 0, st, w, x, y, ncols, nrows); break;
        case 4: hipLaunchKernelGGL((k_gemv_router<4, BF16>), g, dim3(256), 0, st, w, x, y, ncols, nrows); break;
        case 5: hipLaunchKernelGGL((k_gemv_router<5, BF16>), g, dim3(256), 0, st, w, x, y, ncols, nrows); break;
        case 6: hipLaunchKernelGGL((k_gemv_router<6, BF16>), g, dim3(256), 0, st, w, x, y, ncols, nrows); break;
        case 7: hipLaunchKernelGGL((k_gemv_router<7, BF16>), g, dim3(256), 0, st, w, x, y, ncols, nrows); break;
        default: hipLaunchKernelGGL((k_gemv_router<8, BF16>), g, dim3(256), 0, st, w, x, y, ncols, nrows); break;
    }
    return host::check_launch("gemv_router");
}

}  // namespace

namespace impl {

int gemv_router(int dtype, const void *w, const float *x, float *y, int ncols, int nrows, int cols, hipStream_t st) {
    if (cols < 1 || cols > 8) return host::set_error(host::ERR_SHAPE, "gemv: expected 1 to 8 columns");
    if (!w || !x || !y || ncols <= 0 || nrows <= 0) return host::set_error(host::ERR_SHAPE, "gemv: bad arguments");
    if (dtype == T_BF16) return launch_gemv<true>(w, x, y, ncols, nrows, cols, st);
    if (dtype == 0) return launch_gemv<false>(w, x, y, ncols, nrows, cols, st);
    return host::set_error(host::ERR_TYPE, "gemv: router dtype %d not supported (f32 = 0, bf16 = 30)", dtype);
}

int gemm_router_bias(int dtype, const void *w, const float *bias, const float *x, float *y, int ncols, int nrows,
                     int n_tok, hipStream_t st) {
    if (!w || !x || !y || ncols <= 0 || nrows <= 0 || n_tok < 0)
        return host::set_error(host::ERR_SHAPE, "gemm_router: bad arguments");
    if (n_tok == 0) return host::OK;
    const dim3 g((unsigned) ((n_tok + 15) / 16), (unsigned) ((nrows + 15) / 16));
    if (dtype != T_BF16 && dtype != 0)
        return host::set_error(host::ERR_TYPE, "gemm_router: dtype %d not supported", dtype);
    // Whole 64-column chunks on 16-byte (f32) / 8-byte (bf16) aligned rows, with 32-bit element offsets, take the
    // unguarded loads.
    const bool full = ncols % 64 == 0 && (int64_t) ncols * std::max(n_tok, nrows) < ((int64_t) 1 << 31) && ((uintptr_t) x & 15) == 0 && ((uintptr_t) w & (dtype == T_BF16 ? 7 : 15)) == 0;
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, g, dim3(512), 0, st, w, bias, x, y, ncols, nrows, n_tok); };
    if (dtype == T_BF16) full ? go(k_gemm_router<true, true>) : go(k_gemm_router<true, false>);
    else full ? go(k_gemm_router<false, true>) : go(k_gemm_router<false, false>);
    return host::check_launch("gemm_router");
}

int gemm_router(int dtype, const void *w, const float *x, float *y, int ncols, int nrows, int n_tok, hipStream_t st) {
    return gemm_router_bias(dtype, w, nullptr, x, y, ncols, nrows, n_tok, st);
}

int route_topk(const float *logits, int32_t *ids, float *w, int n_expert, int k, int n_tok, int gating, int norm,
               hipStream_t st) {
    if (!logits || !ids || !w || n_expert < 1 || n_expert > 256 || k < 1 || k > 16 || k > n_expert || n_tok < 0 ||
        (gating != 0 && gating != 1))
        return host::set_error(host::ERR_SHAPE, "route_topk: expected 1 <= k <= min(16, n_expert), n_expert <= 256");
    if (n_tok == 0) return host::OK;
    // a few tokens (decode, verify): 1024 threads per token, the rank phase in one pass (1.0-1.5 us less per call at
    // one token); many tokens (prefill): 256, no faster at 1024. Same selection and weights either way.
    if (n_tok <= 64)
        hipLaunchKernelGGL(k_route_topk<1024>, dim3((unsigned) n_tok), dim3(1024), 0, st, logits, ids, w, n_expert, k,
                           gating, norm);
    else
        hipLaunchKernelGGL(k_route_topk<kRouteThreads>, dim3((unsigned) n_tok), dim3(kRouteThreads), 0, st, logits, ids, w,
                       n_expert, k, gating, norm);
    return host::check_launch("route_topk");
}

int moe_combine(const float *dexp, const float *escale, const float *w, const float *sh, const float *x_in, float *out,
                int n, int k, int n_tok, hipStream_t st) {
    if (!dexp || !w || !out || n < 0 || k < 1 || n_tok < 0)
        return host::set_error(host::ERR_SHAPE, "moe_combine: bad arguments");
    if (n == 0 || n_tok == 0) return host::OK;
    const bool vec = n % 4 == 0 && k <= 8 && (((uintptr_t) dexp | (uintptr_t) out | (uintptr_t) (sh ? sh : out) |
                                                (uintptr_t) (x_in ? x_in : out)) & 15) == 0;
    if (vec) {
        const dim3 g((unsigned) ((n / 4 + 255) / 256), (unsigned) n_tok);
        switch (k) {
#define FNS_COMBINE4(K) \
    case K: hipLaunchKernelGGL(k_moe_combine4<K>, g, dim3(256), 0, st, dexp, escale, w, sh, x_in, out, n); break;
            FNS_COMBINE4(1) FNS_COMBINE4(2) FNS_COMBINE4(3) FNS_COMBINE4(4)
            FNS_COMBINE4(5) FNS_COMBINE4(6) FNS_COMBINE4(7) FNS_COMBINE4(8)
#undef FNS_COMBINE4
        }
    } else {
        hipLaunchKernelGGL(k_moe_combine, dim3((unsigned) ((n + 255) / 256), (unsigned) n_tok), dim3(256), 0, st, dexp,
                           escale, w, sh, x_in, out, n, k);
    }
    return host::check_launch("moe_combine");
}

int count_routes(const int32_t *ids, uint32_t *counts, int k, hipStream_t st) {
    if (!ids || !counts || k < 1 || k > 64) return host::set_error(host::ERR_SHAPE, "count_routes: bad arguments");
    hipLaunchKernelGGL(k_count_routes, dim3(1), dim3(64), 0, st, ids, counts, k);
    return host::check_launch("count_routes");
}

}  // namespace impl

namespace k {

void gemv_bf16(const void *w, const float *x, float *y, int ncols, int nrows, int cols, hipStream_t st) {
    host::abort_on_error(impl::gemv_router(T_BF16, w, x, y, ncols, nrows, cols, st), "gemv_bf16");
}
void gemv_f32(const float *w, const float *x, float *y, int ncols, int nrows, int cols, hipStream_t st) {
    host::abort_on_error(impl::gemv_router(0, w, x, y, ncols, nrows, cols, st), "gemv_f32");
}
void route_topk(const float *logits, int32_t *ids, float *w, int n_expert, int k, hipStream_t st, Gating gating,
                bool norm) {
    host::abort_on_error(impl::route_topk(logits, ids, w, n_expert, k, 1, gating, norm, st), "route_topk");
}
void route_topk_batch(const float *logits, int32_t *ids, float *w, int n_expert, int k, int n_tok, hipStream_t st,
                      Gating gating, bool norm) {
    host::abort_on_error(impl::route_topk(logits, ids, w, n_expert, k, n_tok, gating, norm, st), "route_topk_batch");
}
void count_routes(const int32_t *ids, uint32_t *counts, int k, hipStream_t st) {
    host::abort_on_error(impl::count_routes(ids, counts, k, st), "count_routes");
}
void moe_combine(const float *dexp, const float *escale, const float *w, const float *sh, float *x, int n, int k,
                 hipStream_t st) {
    host::abort_on_error(impl::moe_combine(dexp, escale, w, sh, x, x, n, k, 1, st), "moe_combine");
}
void moe_combine_batch(const float *dexp, const float *escale, const float *w, const float *sh, float *x, int n,
                       int k, int n_tok, hipStream_t st) {
    host::abort_on_error(impl::moe_combine(dexp, escale, w, sh, x, x, n, k, n_tok, st), "moe_combine_batch");
}
void gemm_bf16_batch(void *, const void *w, const float *x, void *, float *y, int ncols, int nrows, int n_tok,
                     hipStream_t st) {
    host::abort_on_error(impl::gemm_router(T_BF16, w, x, y, ncols, nrows, n_tok, st), "gemm_bf16_batch");
}
void gemm_f32_batch(const float *w, const float *x, float *y, int ncols, int nrows, int n_tok, hipStream_t st) {
    host::abort_on_error(impl::gemm_router(0, w, x, y, ncols, nrows, n_tok, st), "gemm_f32_batch");
}

}  // namespace k

}  // namespace fns
