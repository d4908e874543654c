// quantize.hip - Q8_1 activation quantisation (plain, fused with RMSNorm, fused with the F16 guard), the F16 guard,
// and the SwiGLU epilogues, for MI355X gfx950.
//
// Q8_1 op order (bit-exact with the reference): one value per lane, a 32-value block on 32 consecutive lanes of the
// 64-lane wave; amax and sum by xor butterfly with offsets 16, 8, 4, 2, 1; d = amax / 127 (IEEE division);
// q = amax == 0 ? 0 : (int8) roundf(x / d); ds = (f16(d), f16(sum)) rounded to nearest even.
// Reference: src/kernels.cu:150-159 (rms_norm_q8_1), :552-577 (amax_guard_q8_1), src/ggml/ggml_mmvq.cu:17-21
// (quantize_q8_1, rows padded to 512 columns with zeros).
#include "fns/ggml_kernels.h"
#include "fns/kernels.h"
#include "fns_common.hpp"
#include "fns_host.hpp"
#include "fns_internal.hpp"

namespace fns {

using namespace fns::dev;

namespace {

// Quantises one value per lane; lanes 32k .. 32k+31 form block `blk` of the row `y` (reference 36-byte layout).
__device__ __forceinline__ void q8_1_store(float v, uint8_t *__restrict__ y, int blk, int i32) {
    const Q8Lane r = q8_1_lane(v);
    uint8_t *b = y + (size_t) blk * 36;
    b[4 + i32] = (uint8_t) (int8_t) r.q;
    if (i32 == 0) *(uint32_t *) b = float_to_half(r.d) | (float_to_half(r.sum) << 16);
}

__global__ __launch_bounds__(256) void k_quantize_q8_1(const float *__restrict__ x, uint8_t *__restrict__ xq,
                                                        int64_t ncols, int64_t row_bytes) {
    const int64_t r = blockIdx.y;
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    const float v = i < ncols ? x[r * ncols + i] : 0.0f;
    q8_1_store(v, xq + r * row_bytes, (int) (i / 32), (int) (i % 32));
}

// RMSNorm of one row (any n that is a multiple of 32) then Q8_1 of the result; one workgroup per row.
__global__ __launch_bounds__(256) void k_rms_norm_q8_1(const float *__restrict__ x, const float *__restrict__ w,
                                                       float *__restrict__ out, uint8_t *__restrict__ xq, int n,
                                                       float eps, int64_t row_bytes) {
    __shared__ float red[4];
    const float *xr = x + (size_t) blockIdx.x * n;
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) s += xr[i] * xr[i];
    s = lanes_sum<64>(s);
    if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = s;
    __syncthreads();
    s = (red[0] + red[1]) + (red[2] + red[3]);
    const float scale = 1.0f / sqrtf(s / n + eps);
    const int npad = (n + 511) / 512 * 512;
    uint8_t *y = xq + (size_t) blockIdx.x * row_bytes;
    for (int i = threadIdx.x; i < npad; i += 256) {
        float xi = 0.0f;
        if (i < n) {
            xi = scale * xr[i] * w[i];
            out[(size_t) blockIdx.x * n + i] = xi;
        }
        q8_1_store(xi, y, i / 32, i % 32);
    }
}

// F16 guard scale of a row with the fp32 sequence of the reference (src/kernels.cu:544-551).
__device__ __forceinline__ float guard_scale(float amax) {
    // amax <= 1024 (the common case): the sequence below gives exactly 1 (log <= 0, ceil <= 0, clamped to 0, exp(0))
    if (amax <= 1024.0f) return 1.0f;
    float e = amax * (1.0f / 1024.0f);
    e = logf(e);
    e = e * 1.4426950408889634f;
    e = ceilf(e);
    e = fminf(fmaxf(e, 0.0f), 127.0f);
    e = e * 0.6931471805599453f;
    return expf(e);
}

__device__ __forceinline__ float block_max256(float m, float *red) {
    m = lanes_max<64>(m);
    __syncthreads();
    if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = m;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__global__ __launch_bounds__(256) void k_amax_guard(float *__restrict__ act, float *__restrict__ escale, int n) {
    __shared__ float red[4];
    float *r = act + (size_t) blockIdx.x * n;
    float m = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) m = fmaxf(m, fabsf(r[i]));
    const float e = guard_scale(block_max256(m, red));
    for (int i = threadIdx.x; i < n; i += 256) r[i] = r[i] / e;
    if (threadIdx.x == 0) escale[blockIdx.x] = e;
}

__global__ __launch_bounds__(256) void k_amax_guard_q8_1(const float *__restrict__ act, float *__restrict__ escale,
                                                         uint8_t *__restrict__ xq, int n, int64_t row_bytes) {
    __shared__ float red[4];
    const float *r = act + (size_t) blockIdx.x * n;
    float m = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) m = fmaxf(m, fabsf(r[i]));
    const float e = guard_scale(block_max256(m, red));
    if (threadIdx.x == 0) escale[blockIdx.x] = e;
    const int npad = (n + 511) / 512 * 512;
    uint8_t *y = xq + (size_t) blockIdx.x * row_bytes;
    for (int i = threadIdx.x; i < npad; i += 256) {
        const float xi = i < n ? r[i] / e : 0.0f;
        q8_1_store(xi, y, i / 32, i % 32);
    }
}

// The same for rows of at most 256 C padded columns: each thread's C values are loaded once, all in flight together
// (clamped, unconditional loads), and quantised from registers; same operations, same bits.
template <int C>
__global__ __launch_bounds__(256) void k_amax_guard_q8_1_reg(const float *__restrict__ act, float *__restrict__ escale,
                                                             uint8_t *__restrict__ xq, int n, int64_t row_bytes) {
    __shared__ float red[4];
    const float *r = act + (size_t) blockIdx.x * n;
    float v[C];
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int i = threadIdx.x + 256 * c;
        const float x = r[min(i, n - 1)];
        v[c] = i < n ? x : 0.0f;
    }
    float m = 0.0f;
#pragma unroll
    for (int c = 0; c < C; ++c) m = fmaxf(m, fabsf(v[c]));
    const float e = guard_scale(block_max256(m, red));
    if (threadIdx.x == 0) escale[blockIdx.x] = e;
    uint8_t *y = xq + (size_t) blockIdx.x * row_bytes;
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int i = threadIdx.x + 256 * c;
        q8_1_store(i < n ? v[c] / e : 0.0f, y, i / 32, i % 32);
    }
}

__global__ void k_swiglu(const float *__restrict__ g, const float *__restrict__ u, float *__restrict__ act,
                         int64_t total) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const float x = g[i];
    act[i] = x / (1.0f + fns_expf(-x)) * u[i];
}

// out = x + ((p_0 + p_1) + ...) over n_parts partial sums of n values each (in part order), one element per thread
__global__ void k_add_parts(const float *x, const float *parts, int n_parts, float *out, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float s = parts[i];
    for (int p = 1; p < n_parts; ++p) s = s + parts[(size_t) p * n + i];
    out[i] = x[i] + s;
}

// out = x + y, one element per thread (any alignment)
__global__ void k_add1(const float *x, const float *y, float *out, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = x[i] + y[i];
}
// out = x + y, four elements per thread (n4 = n / 4 float4s; 16-byte aligned arrays), then the tail
__global__ void k_add(const float *x, const float *y, float *out, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t n4 = n / 4;
    if (i < n4) {
        const float4 a = ((const float4 *) x)[i], b = ((const float4 *) y)[i];
        ((float4 *) out)[i] = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
    } else if (i < n4 + n % 4) {
        const int64_t j = 4 * n4 + (i - n4);
        out[j] = x[j] + y[j];
    }
}

__global__ void k_glu_mmvq(const float *__restrict__ g, const float *u, float *act, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float result = u[i];
    result += 0.0f;
    result *= silu(g[i] + 0.0f);
    act[i] = result;
}

}  // namespace

namespace impl {

int quantize_q8_1(const float *x, void *xq, int64_t ncols, int64_t nrows, hipStream_t st) {
    if (!x || !xq || ncols <= 0 || nrows < 0 || nrows > 65535)
        return host::set_error(host::ERR_SHAPE, "quantize_q8_1: bad arguments (ncols %lld nrows %lld)",
                               (long long) ncols, (long long) nrows);
    if (nrows == 0) return host::OK;
    const int64_t npad = host::pad512(ncols);
    hipLaunchKernelGGL(k_quantize_q8_1, dim3((unsigned) (npad / 256), (unsigned) nrows), dim3(256), 0, st, x,
                       (uint8_t *) xq, ncols, host::q8_1_row_bytes(ncols));
    return host::check_launch("quantize_q8_1");
}

int rms_norm_q8_1(const float *x, const float *w, float *out, void *xq, int n, float eps, int rows, hipStream_t st) {
    if (!x || !w || !out || !xq || n <= 0 || n % 32 || rows < 0)
        return host::set_error(host::ERR_SHAPE, "rms_norm_q8_1: n must be a positive multiple of 32");
    if (rows == 0) return host::OK;
    hipLaunchKernelGGL(k_rms_norm_q8_1, dim3((unsigned) rows), dim3(256), 0, st, x, w, out, (uint8_t *) xq, n, eps,
                       host::q8_1_row_bytes(n));
    return host::check_launch("rms_norm_q8_1");
}

int amax_guard(float *act, float *escale, int n, int rows, hipStream_t st) {
    if (!act || !escale || n <= 0 || rows < 0) return host::set_error(host::ERR_SHAPE, "amax_guard: bad arguments");
    if (rows == 0) return host::OK;
    hipLaunchKernelGGL(k_amax_guard, dim3((unsigned) rows), dim3(256), 0, st, act, escale, n);
    return host::check_launch("amax_guard");
}

int amax_guard_q8_1(const float *act, float *escale, void *xq, int n, int rows, hipStream_t st) {
    if (!act || !escale || !xq || n <= 0 || rows < 0)
        return host::set_error(host::ERR_SHAPE, "amax_guard_q8_1: bad arguments");
    if (rows == 0) return host::OK;
    const int64_t npad = host::pad512(n), rb = host::q8_1_row_bytes(n);
    if (npad <= 512)
        hipLaunchKernelGGL(k_amax_guard_q8_1_reg<2>, dim3((unsigned) rows), dim3(256), 0, st, act, escale, (uint8_t *) xq, n, rb);
    else if (npad <= 1024)
        hipLaunchKernelGGL(k_amax_guard_q8_1_reg<4>, dim3((unsigned) rows), dim3(256), 0, st, act, escale, (uint8_t *) xq, n, rb);
    else if (npad <= 2048)
        hipLaunchKernelGGL(k_amax_guard_q8_1_reg<8>, dim3((unsigned) rows), dim3(256), 0, st, act, escale, (uint8_t *) xq, n, rb);
    else
        hipLaunchKernelGGL(k_amax_guard_q8_1, dim3((unsigned) rows), dim3(256), 0, st, act, escale, (uint8_t *) xq, n, rb);
    return host::check_launch("amax_guard_q8_1");
}

int swiglu(const float *g, const float *u, float *act, int n, int rows, hipStream_t st) {
    const int64_t total = (int64_t) n * rows;
    if (!g || !u || !act || n < 0 || rows < 0) return host::set_error(host::ERR_SHAPE, "swiglu: bad arguments");
    if (total == 0) return host::OK;
    hipLaunchKernelGGL(k_swiglu, dim3((unsigned) ((total + 255) / 256)), dim3(256), 0, st, g, u, act, total);
    return host::check_launch("swiglu");
}

int add_parts(const float *x, const float *parts, int n_parts, float *out, int64_t n, hipStream_t st) {
    if (!x || !parts || !out || n < 0 || n_parts < 1) return host::set_error(host::ERR_SHAPE, "add_parts: bad arguments");
    if (n == 0) return host::OK;
    hipLaunchKernelGGL(k_add_parts, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, st, x, parts, n_parts, out, n);
    return host::check_launch("add_parts");
}

int add(const float *x, const float *y, float *out, int64_t n, hipStream_t st) {
    if (!x || !y || !out || n < 0) return host::set_error(host::ERR_SHAPE, "add: bad arguments");
    if (n == 0) return host::OK;
    if (((uintptr_t) x | (uintptr_t) y | (uintptr_t) out) % 16) {
        hipLaunchKernelGGL(k_add1, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, st, x, y, out, n);
        return host::check_launch("add");
    }
    const int64_t threads = n / 4 + n % 4;
    hipLaunchKernelGGL(k_add, dim3((unsigned) ((threads + 255) / 256)), dim3(256), 0, st, x, y, out, n);
    return host::check_launch("add");
}

int glu_mmvq(const float *g, const float *u, float *act, int n, hipStream_t st) {
    if (!g || !u || !act || n < 0) return host::set_error(host::ERR_SHAPE, "glu_mmvq: bad arguments");
    if (n == 0) return host::OK;
    hipLaunchKernelGGL(k_glu_mmvq, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, st, g, u, act, n);
    return host::check_launch("glu_mmvq");
}

}  // namespace impl

void quantize_q8_1(const float *x, void *xq, int64_t ncols, int64_t nrows, hipStream_t stream) {
    host::abort_on_error(impl::quantize_q8_1(x, xq, ncols, nrows, stream), "quantize_q8_1");
}

namespace k {
void rms_norm_q8_1(const float *x, const float *w, float *out, void *xq, int n, float eps, int rows, hipStream_t st) {
    host::abort_on_error(impl::rms_norm_q8_1(x, w, out, xq, n, eps, rows, st), "rms_norm_q8_1");
}
void amax_guard(float *act, float *escale, int n, int rows, hipStream_t st) {
    host::abort_on_error(impl::amax_guard(act, escale, n, rows, st), "amax_guard");
}
void amax_guard_q8_1(const float *act, float *escale, void *xq, int n, int rows, hipStream_t st) {
    host::abort_on_error(impl::amax_guard_q8_1(act, escale, xq, n, rows, st), "amax_guard_q8_1");
}
void swiglu(const float *g, const float *u, float *act, int n, int rows, hipStream_t st) {
    host::abort_on_error(impl::swiglu(g, u, act, n, rows, st), "swiglu");
}
void glu_mmvq(const float *g, const float *u, float *act, int n, hipStream_t st) {
    host::abort_on_error(impl::glu_mmvq(g, u, act, n, st), "glu_mmvq");
}
}  // namespace k

}  // namespace fns
