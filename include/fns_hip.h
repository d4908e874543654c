/* include/fns_hip.h - C ABI of libfns_hip.so, the MI355X (gfx950) MoE FFN hot path of FlintNSteel.
 *
 * Plain pointers and sizes only: every buffer argument is a device pointer (hipMalloc'd or otherwise GPU-visible)
 * unless stated; `stream` is a hipStream_t passed as void* (NULL = the null stream). Every call is asynchronous on
 * `stream`, allocates nothing, and returns 0 on success or a negative FNS_ERR_* code; fns_hip_last_error() then
 * describes the failure (thread-local). The C++ API of include/fns/ggml_kernels.h and include/fns/kernels.h wraps
 * the same implementations and aborts on error, as the reference does.
 *
 * Each entry point names the reference interface it replaces (paths under the reference repository).
 */
#ifndef FNS_HIP_H
#define FNS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FNS_OK 0
#define FNS_ERR_TYPE (-1)
#define FNS_ERR_SHAPE (-2)
#define FNS_ERR_LAUNCH (-3)
#define FNS_ERR_NOMEM (-4)

/* ggml type ids accepted by the quantized entry points (ggml.h numbering); router dtypes: 0 = f32, 30 = bf16. */
#define FNS_TYPE_F32 0
#define FNS_TYPE_Q8_1 9
#define FNS_TYPE_Q3_K 11
#define FNS_TYPE_Q4_K 12
#define FNS_TYPE_Q5_K 13
#define FNS_TYPE_Q6_K 14
#define FNS_TYPE_BF16 30

#define FNS_GATING_SOFTMAX 0
#define FNS_GATING_SIGMOID 1

int fns_hip_abi_version(void);
const char *fns_hip_last_error(void);

/* --- ggml_kernels.h (reference include/fns/ggml_kernels.h) --- */

/* include/fns/ggml_kernels.h:13-14 q8_1_row_bytes */
size_t fns_hip_q8_1_row_bytes(int64_t ncols);
/* include/fns/ggml_kernels.h:16-17 quantize_q8_1 */
int fns_hip_quantize_q8_1(const float *x, void *xq, int64_t ncols, int64_t nrows, void *stream);
/* include/fns/ggml_kernels.h:19-22 mmvq */
int fns_hip_mmvq(int type, const void *w, int64_t ncols, int64_t nrows, const void *xq, float *dst, int64_t n_cols,
                 void *stream);
/* include/fns/ggml_kernels.h:24-27 mmvq_ids */
int fns_hip_mmvq_ids(int type, const void *w, int64_t ncols, int64_t nrows, int64_t n_mats, const void *xq,
                     int64_t n_xq, const int32_t *ids, int64_t n_ids, float *dst, void *stream);
/* include/fns/ggml_kernels.h:29-31 mmvq_swiglu */
int fns_hip_mmvq_swiglu(int type, const void *w_gate, const void *w_up, int64_t ncols, int64_t nrows, const void *xq,
                        float *dst, void *stream);
/* include/fns/ggml_kernels.h:33-37 mmvq_ids_swiglu_shared (sh_* may be NULL: no shared expert) */
int fns_hip_mmvq_ids_swiglu_shared(int type, const void *w_gate, const void *w_up, int64_t ncols, int64_t nrows,
                                   int64_t n_mats, const void *xq, const int32_t *ids, int64_t n_ids, float *dst,
                                   const void *sh_gate, const void *sh_up, float *sh_dst, void *stream);
/* include/fns/ggml_kernels.h:44-46 mmvq_experts_swiglu; table: device array of expert base pointers */
int fns_hip_mmvq_experts_swiglu(int type, const void *const *table, size_t gate_off, size_t up_off, int64_t ncols,
                                int64_t nrows, const void *xq, int64_t n_xq, const int32_t *ids, int64_t n_ids,
                                float *dst, void *stream);
/* include/fns/ggml_kernels.h:47-48 mmvq_experts */
int fns_hip_mmvq_experts(int type, const void *const *table, size_t off, int64_t ncols, int64_t nrows, const void *xq,
                         int64_t n_xq, const int32_t *ids, int64_t n_ids, float *dst, void *stream);
/* include/fns/ggml_kernels.h:79-80 mmvq_supports */
int fns_hip_mmvq_supports(int type);

/* --- kernels.cuh MoE subset (reference src/kernels.cuh, namespace fns::k) --- */

/* src/kernels.cuh:29-32 rms_norm_q8_1 (n any multiple of 32) */
int fns_hip_rms_norm_q8_1(const float *x, const float *w, float *out, void *xq, int n, float eps, int rows,
                          void *stream);
/* src/kernels.cuh:90-91 gemv_bf16, generalised to dtype 0 (f32) or 30 (bf16); cols 1..8 */
int fns_hip_gemv_router(int dtype, const void *w, const float *x, float *y, int ncols, int nrows, int cols,
                        void *stream);
/* src/kernels.cuh:150-153 gemm_bf16_batch (no cuBLAS handle), dtype 0 or 30 */
int fns_hip_gemm_router(int dtype, const void *w, const float *x, float *y, int ncols, int nrows, int n_tok,
                        void *stream);
/* src/kernels.cuh:93-94 route_topk and :155 route_topk_batch; gating FNS_GATING_*, norm 0/1 */
int fns_hip_route_topk(const float *logits, int32_t *ids, float *w, int n_expert, int k, int n_tok, int gating,
                       int norm, void *stream);
/* src/kernels.cuh:96-97 count_routes */
int fns_hip_count_routes(const int32_t *ids, uint32_t *counts, int k, void *stream);
/* src/kernels.cuh:99-100 swiglu */
int fns_hip_swiglu(const float *g, const float *u, float *act, int n, int rows, void *stream);
/* src/kernels.cuh:102-104 glu_mmvq */
int fns_hip_glu_mmvq(const float *g, const float *u, float *act, int n, void *stream);
/* src/kernels.cuh:106-108 amax_guard */
int fns_hip_amax_guard(float *act, float *escale, int n, int rows, void *stream);
/* src/kernels.cuh:110-111 amax_guard_q8_1 (n any multiple of 32) */
int fns_hip_amax_guard_q8_1(const float *act, float *escale, void *xq, int n, int rows, void *stream);
/* src/kernels.cuh:113-115 moe_combine and :156 moe_combine_batch, out-of-place:
 * out[t] = (sum_j (dexp[t][j] * escale[t][j]) * w[t][j] + sh[t]) + x_in[t]; escale, sh, x_in may be NULL;
 * out may alias x_in (the reference's in-place form). */
int fns_hip_moe_combine(const float *dexp, const float *escale, const float *w, const float *sh, const float *x_in,
                        float *out, int n, int k, int n_tok, void *stream);

#ifdef __cplusplus
}
#endif
#endif
