// include/fns/kernels.h - MoE glue kernels of the engine for MI355X (gfx950): router GEMV, gating + top-k, SwiGLU,
// F16 guard, fused guard + Q8_1, weighted combine, routing histogram, and the fused decode layer. Drop-in for the
// MoE subset of the reference's src/kernels.cuh (namespace fns::k), generalised over the expert count, top-k, gating
// function (the reference hard-codes 256 experts, sigmoid, k <= 8: src/kernels.cu:911-918) and the router dtype.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "fns/ggml_kernels.h"

namespace fns::k {

enum Gating : int { GATING_SOFTMAX = 0, GATING_SIGMOID = 1 };

// rms_norm of `rows` rows of n, times w, then quantize_q8_1 of each output row into xq (rows of q8_1_row_bytes(n)).
// Reference: src/kernels.cuh:29-32, src/kernels.cu:128-161 (n = 2048 there; any multiple of 32 here).
void rms_norm_q8_1(const float *x, const float *w, float *out, void *xq, int n, float eps, int rows, hipStream_t st);

// y[c][r] = sum_i W[r][i] x[c][i] in fp32, c < cols (1..8). Reference: src/kernels.cuh:90-91, src/kernels.cu:452-482.
void gemv_bf16(const void *w, const float *x, float *y, int ncols, int nrows, int cols, hipStream_t st);
// Same with fp32 router weights (the configs' router).
void gemv_f32(const float *w, const float *x, float *y, int ncols, int nrows, int cols, hipStream_t st);

// Gating p = softmax(logits) or sigmoid(logits); k rounds of argmax (ties to the lower index); w = p_sel / max(sum,
// 6.103515625e-5) when norm. n_expert <= 256, k <= 16. Reference: src/kernels.cuh:93-94, src/kernels.cu:484-514.
void route_topk(const float *logits, int32_t *ids, float *w, int n_expert, int k, hipStream_t st,
                Gating gating = GATING_SIGMOID, bool norm = true);
// One token per wave. Reference: src/kernels.cuh:155, src/prefill_kernels.cu:138-169,235-242.
void route_topk_batch(const float *logits, int32_t *ids, float *w, int n_expert, int k, int n_tok, hipStream_t st,
                      Gating gating = GATING_SIGMOID, bool norm = true);

// counts[ids[j]] += 1, j < k. Reference: src/kernels.cuh:96-97, src/kernels.cu:955-962.
void count_routes(const int32_t *ids, uint32_t *counts, int k, hipStream_t st);

// act[r][i] = silu(g[r][i]) * u[r][i]. Reference: src/kernels.cuh:99-100, src/kernels.cu:516-521.
void swiglu(const float *g, const float *u, float *act, int n, int rows, hipStream_t st);

// act[i] = (u[i] + 0) * silu(g[i] + 0): the fused-GLU epilogue of the MMVQs. Reference: src/kernels.cuh:102-104.
void glu_mmvq(const float *g, const float *u, float *act, int n, hipStream_t st);

// F16 guard: e_r = 2^clamp(ceil(log2(amax_r/1024)), 0, 127); act_r /= e_r; escale[r] = e_r.
// Reference: src/kernels.cuh:106-108, src/kernels.cu:534-552.
void amax_guard(float *act, float *escale, int n, int rows, hipStream_t st);
// amax_guard (act unmodified) then quantize_q8_1 of the scaled rows into xq [rows][q8_1_row_bytes(n)].
// Reference: src/kernels.cuh:110-111, src/kernels.cu:554-577 (n = 512 there; any multiple of 32 here).
void amax_guard_q8_1(const float *act, float *escale, void *xq, int n, int rows, hipStream_t st);

// x[i] = (sum_j (dexp_j[i] * e_j) * w_j + sh[i]) + x[i], j in order 0..k-1 (escale and sh may be null: 1 and 0).
// Reference: src/kernels.cuh:113-115, src/kernels.cu:579-586.
void moe_combine(const float *dexp, const float *escale, const float *w, const float *sh, float *x, int n, int k,
                 hipStream_t st);
// Per token t < n_tok. Reference: src/kernels.cuh:156, src/prefill_kernels.cu:171-183.
void moe_combine_batch(const float *dexp, const float *escale, const float *w, const float *sh, float *x, int n,
                       int k, int n_tok, hipStream_t st);

// Batch router y [n_tok][nrows] = W . x[t] with f32 accumulation (the reference goes through cuBLAS BF16 with a
// bf16 workspace xb: src/kernels.cuh:150-153, src/prefill_kernels.cu:217-233). `handle` is unused (kept for the
// drop-in signature); xb may be null.
void gemm_bf16_batch(void *handle, const void *w, const float *x, void *xb, float *y, int ncols, int nrows, int n_tok,
                     hipStream_t st);
void gemm_f32_batch(const float *w, const float *x, float *y, int ncols, int nrows, int n_tok, hipStream_t st);

}  // namespace fns::k
