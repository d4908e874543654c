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
#define FNS_ERR_IO (-5) /* a GGUF file that cannot be opened or is malformed */

/* ggml type ids accepted by the quantized entry points (ggml.h numbering); router dtypes: 0 = f32, 30 = bf16. */
#define FNS_TYPE_F32 0
#define FNS_TYPE_Q8_1 9
#define FNS_TYPE_Q3_K 11
#define FNS_TYPE_Q4_K 12
#define FNS_TYPE_Q5_K 13
#define FNS_TYPE_Q6_K 14
#define FNS_TYPE_IQ3_XXS 18
#define FNS_TYPE_IQ3_S 21
#define FNS_TYPE_IQ2_S 22
#define FNS_TYPE_IQ4_XS 23
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
/* No counterpart in the reference, whose ggml build compiles the IQ codebooks in: registers ggml's iq3xxs_grid[256],
 * iq3s_grid[512] and iq2s_grid[1024] (the engine's own copies) on the current device; call once per device before
 * any IQ3_XXS / IQ3_S / IQ2_S product. Until then mmvq_supports rejects those three types (IQ4_XS needs no table).
 * Every codebook byte must be 1..127, as ggml's are. Synchronous (hipMemcpyToSymbol); not graph-capturable. */
int fns_hip_set_iq_grids(const uint32_t *iq3xxs, const uint32_t *iq3s, const uint64_t *iq2s);

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

/* --- fused MoE FFN layer: decode (n_tok = 1) and speculative verify (n_tok <= 4) ---
 * The MoE section of the reference's Engine::ffn_block (src/engine.cu:655-696: router gemv_bf16, route_topk,
 * mmvq_experts_swiglu, amax_guard_q8_1, mmvq_experts, moe_combine) as one call of three kernels:
 *   out[t] = sum_j w[t][j] * e[t][j] * down_{e_j}(q8_1(act[t][j] / e[t][j])) (+ x_resid[t]),
 *   act[t][j] = up_{e_j} . q8_1(x[t]) * silu(gate_{e_j} . q8_1(x[t])), (ids, w) = top-k of gating(router . x[t]).
 * Expert e's slot is table[e] (device array) with gate/up/down matrices at the byte offsets below (GGUF blocks).
 * For n_tok > 1 the selected experts are compacted: each distinct expert's weights are read once per call.
 * workspace: fns_hip_moe_workspace_layout() bytes, device memory, zero-filled once before its first use (it holds an
 * arrival counter that the library keeps consistent from call to call), sections (byte offsets in offsets[6]):
 *   0 logits f32 [n_tok][n_expert], 1 xq Q8_1 [n_tok][q8_1_row_bytes(hidden)], 2 ids i32 [n_tok][k],
 *   3 w f32 [n_tok][k], 4 act f32 [n_tok*k][inter], 5 escale f32 [n_tok*k]. */
typedef struct FnsMoeLayer {
    int hidden, inter, n_expert, k;
    int gating;       /* FNS_GATING_SOFTMAX or FNS_GATING_SIGMOID */
    int norm_w;       /* 1: w = p / max(sum p, 6.103515625e-5) */
    int guard;        /* 1: F16 guard of act before down (reference src/kernels.cu:534-577) */
    int router_dtype; /* FNS_TYPE_F32 or FNS_TYPE_BF16 */
    const void *router_w; /* [n_expert][hidden] */
    int gu_type, down_type;
    const void *const *table;
    size_t gate_off, up_off, down_off;
    const float *router_bias; /* NULL or f32 [n_expert], added to the logits before gating (selection and weights) */
    /* The rest of the reference's Engine::ffn_block (src/engine.cu:655-696; prefill src/engine.cu:331-357); all zero:
     * absent. With ffn_norm the layer input x is the residual stream: h = RMSNorm(x) * ffn_norm (eps norm_eps, as
     * rms_norm_q8_1) feeds the router and the experts. With a shared expert (shexp_inter > 0) its output
     * sh = down_sh . q8_1(up_sh . q8_1(h) * silu(gate_sh . q8_1(h))) joins the combine as the reference's:
     * out = (sum_j w_j e_j dexp_j + sh) + x_resid. */
    const float *ffn_norm;     /* NULL or f32 [hidden] */
    float norm_eps;
    int shexp_inter;           /* 0 or the shared expert's width (a positive multiple of 256) */
    int shexp_gu_type, shexp_down_type;  /* K-quant types of the shared expert's gate/up and down (0: gu_type / down_type) */
    const void *shexp_gate, *shexp_up;   /* [shexp_inter][hidden] blocks */
    const void *shexp_down;              /* [hidden][shexp_inter] blocks */
    /* No counterpart in the reference: a read-ahead hint. NULL, or device bytes the next call will read first
     * (normally the next layer's router_w, prefetch_bytes = its size): the decode router kernel reads them along with
     * its own work so that they sit in the memory-side cache (MI355X Infinity Cache) when the next layer's router
     * reads them. Results do not depend on it. */
    const void *prefetch;
    size_t prefetch_bytes;
} FnsMoeLayer;

int fns_hip_moe_workspace_layout(const FnsMoeLayer *layer, int n_tok, size_t *offsets, size_t *total_bytes);
int fns_hip_moe_layer(const FnsMoeLayer *layer, const float *x, const float *x_resid, float *out, int n_tok,
                      void *workspace, size_t workspace_bytes, void *stream);
/* Same, recording events[0..3] (hipEvent_t, any may be NULL) on `stream` before the router kernel, before the
 * gate/up kernel, before the down kernel and after it: per-kernel durations for measurement. */
int fns_hip_moe_layer_profiled(const FnsMoeLayer *layer, const float *x, const float *x_resid, float *out, int n_tok,
                               void *workspace, size_t workspace_bytes, void *const *events, void *stream);
/* No counterpart in the reference: the same layer as fns_hip_moe_layer for callers that cannot allocate (code under HIP
 * graph capture, serving loops or harnesses that forbid hipMalloc). The workspace is a device array inside the
 * library, fns_hip_moe_noalloc_max_bytes() bytes (4 MiB) per GPU, held until the process ends; a layer whose
 * fns_hip_moe_workspace_layout total exceeds it is rejected with FNS_ERR_NOMEM. The call allocates nothing. Every call
 * on one GPU shares that array and leaves its intermediates there (as fns_hip_moe_layer leaves them in its
 * workspace): calls that overlap on one GPU race, so order them (one stream). The first call on a device clears the
 * array with a kernel on `stream`. */
int fns_hip_moe_layer_noalloc(const FnsMoeLayer *layer, const float *x, const float *x_resid, float *out, int n_tok,
                              void *stream);
size_t fns_hip_moe_noalloc_max_bytes(void);
/* No counterpart in the reference (its kernels have no cross-workgroup wait). The decode kernel's workgroups exchange
 * the act rows through a bounded wait in device memory; a workgroup that gives up (its producers were never
 * scheduled, e.g. other work held the CUs) writes NaN to its output rows and sets FNS_STATUS_EXCHANGE_TIMEOUT in the
 * workspace's status word. The word is sticky across calls (the engine can check once per token or graph replay):
 * this call waits for the stream's work so far, stores the word in *status and, with clear = 1, zeroes it (a kernel
 * on `stream`). workspace NULL: the no-allocation array of the current device. Not graph-capturable (it
 * synchronises). */
#define FNS_STATUS_EXCHANGE_TIMEOUT 1u
int fns_hip_moe_layer_status(const FnsMoeLayer *layer, int n_tok, void *workspace, int clear, uint32_t *status,
                             void *stream);
/* No counterpart in the reference: the graph-capturable form of fns_hip_moe_layer_status for engines that replay a
 * graph per token. Enqueues one single-thread kernel on `stream` that, when the workspace's status word is non-zero,
 * ORs it into *dst (device memory or host memory from hipHostMalloc; the caller zeroes it) and clears the word; a
 * zero word leaves *dst untouched. Layers that share one workspace share its word, so one collect per token covers
 * them. workspace NULL: the no-allocation array of the current device. */
int fns_hip_moe_layer_status_collect(const FnsMoeLayer *layer, int n_tok, void *workspace, uint32_t *dst,
                                     void *stream);
/* Test hook, no counterpart in the reference: the decode kernel's poll limit (0: the default, 65536 polls) and a
 * number of producer arrivals to withhold (> 0: the exchange never completes, every workgroup gives up after
 * spin_limit polls) for the calls that follow; the failure path is then exercised with every kernel exiting normally.
 * Process-wide; set it only while no other thread launches layers. */
int fns_hip_moe_set_test_hooks(int spin_limit, int withhold_arrivals);
/* No counterpart in the reference: how many kernels a call of this layer at n_tok tokens launches on the current
 * device - 2 (n_tok = 1 and a shape the fused kernel holds, all its workgroups resident: router kernel + fused layer
 * kernel) or 3 (router, gate/up, down). Both give the same results bit for bit. */
int fns_hip_moe_layer_kernels(const FnsMoeLayer *layer, int n_tok, int *kernels);
/* Test hook, no counterpart in the reference: restricts the decode path for the calls that follow (0: automatic,
 * 1: never the fused kernel - the three-kernel path). Process-wide, like fns_hip_moe_set_test_hooks. */
int fns_hip_moe_set_path(int path);
/* One of the three kernels of fns_hip_moe_layer (stage 0 router + Q8_1 of x, 1 routing + gate/up + SwiGLU,
 * 2 F16 guard + Q8_1 of act + down + combine), each reading what the previous stage left in the workspace:
 * per-stage tracing (the reference's FNS_TRACE nodes, src/engine.cu:590-599) and per-kernel timing. A call that takes
 * the fused kernel (fns_hip_moe_layer_kernels = 2) launches it at stage 1; stage 2 then launches nothing. */
int fns_hip_moe_layer_stage(const FnsMoeLayer *layer, int stage, const float *x, const float *x_resid, float *out,
                            int n_tok, void *workspace, size_t workspace_bytes, void *stream);

/* --- prefill / batched expert GEMM (MMQ) ---
 * Q8_1 activation rows for the MMQ path are kept as "split images" (q8 * d8 as two f16 halves per value, then the
 * per-32 scaled sums as f16 halves: 4.125 bytes per value): fns_hip_mmq_q8_1_bytes(ncols, nrows) bytes hold nrows
 * of them plus 4096 bytes of slack (mmq_experts keeps its group lists there). */
/* include/fns/ggml_kernels.h:53-54 mmq_q8_1_bytes */
size_t fns_hip_mmq_q8_1_bytes(int64_t ncols, int64_t nrows);
/* bytes of the expert_bounds buffer of fns_hip_mmq_compact for n_expert experts (bounds + tile-group prefix) */
size_t fns_hip_mmq_bounds_bytes(int64_t n_expert);
/* include/fns/ggml_kernels.h:56-58 mmq: dst[t][nrows] = W . q8_1(x[t]), x f32 [n_tok][ncols]; xq scratch of
 * fns_hip_mmq_q8_1_bytes(ncols, n_tok) bytes. ncols a multiple of 256, nrows of 64. Types (the reference's MMQ set,
 * src/ggml/ggml_mmq.cu:59-66, plus Q3_K): the K-quants and IQ4_XS / IQ3_XXS / IQ3_S / IQ2_S (the last three once
 * their codebooks are registered) on the tiled MFMA GEMM; Q8_0 (any nrows) on the GEMV kernels, a few token columns
 * per weight pass. */
int fns_hip_mmq(int type, const void *w, int64_t ncols, int64_t nrows, const float *x, int64_t n_tok, void *xq,
                float *dst, void *stream);
/* include/fns/ggml_kernels.h:60-69 MmqIdsScratch + mmq_experts: dst[t][j][nrows] = W_e . q8_1(x[t][j % x_rows_per_tok]),
 * e = ids[t][j]; expert e's matrix at table[e] + off. Scratch (the reference's MmqIdsScratch sizing): ids_src1 /
 * ids_dst n_tok * n_used int32, expert_bounds n_expert + 1 int32, xq fns_hip_mmq_q8_1_bytes(ncols, n_tok * x_rows_per_tok)
 * bytes. */
int fns_hip_mmq_experts(int type, const void *const *table, size_t off, int64_t ncols, int64_t nrows, int64_t n_expert,
                        const float *x, int64_t x_rows_per_tok, int64_t n_tok, const int32_t *ids, int64_t n_used,
                        int32_t *ids_src1, int32_t *ids_dst, int32_t *expert_bounds, void *xq, float *dst, void *stream);
/* Expert-id compaction alone (ggml mm_ids_helper semantics; reference src/ggml/ggml_mmq.cu:110-111): pairs
 * p = t * n_used + j sorted by expert, stable; ids_dst[q] = p, ids_src1[q] = (x_rows_per_tok == 1 ? t : p),
 * expert_bounds[e] = first sorted position of expert e (e <= n_expert), followed by the tile-group prefix
 * (fns_hip_mmq_bounds_bytes(n_expert) bytes in all). */
int fns_hip_mmq_compact(const int32_t *ids, int64_t n_tok, int64_t n_used, int64_t n_expert, int64_t x_rows_per_tok,
                        int32_t *ids_src1, int32_t *ids_dst, int32_t *expert_bounds, void *stream);

/* Prefill MoE layer for n_tok tokens (n_tok * k <= 65536): the MoE section of the reference's Engine::prefill_chunk
 * (src/engine.cu:340-357: batch router, route_topk_batch, mmq_experts gate / up, swiglu, amax_guard, mmq_experts down,
 * moe_combine_batch), out[t] = sum_j w[t][j] * e[t][j] * down_e(q8_1(act[t][j] / e[t][j])) (+ x_resid[t]).
 * workspace: fns_hip_moe_prefill_workspace() bytes; sections (byte offsets in offsets[6]): 0 logits f32 [n_tok][n_expert],
 * 1 ids i32 [n_tok][k], 2 w f32 [n_tok][k], 3 x images, 4 act images [n_tok * k], 5 down outputs f32 [n_tok][k][hidden]. */
int fns_hip_moe_prefill_workspace(const FnsMoeLayer *layer, int64_t n_tok, size_t *offsets, size_t *total_bytes);
/* Byte offset and size of any workspace section of fns_hip_moe_prefill (the six above, then 6 ids_src1, 7 ids_dst,
 * 8 expert bounds, group prefix, arrival counters and the status word, 9 f32 act [n_tok * k][inter] (F16 guard
 * only, after the division), 10 guard scales [n_tok * k],
 * 11 RMSNorm output, 12 its Q8_1 blocks, 13 shared-expert act images, 14 shared-expert output). Inspection and tests;
 * the image layouts are internal. */
int fns_hip_moe_prefill_section(const FnsMoeLayer *layer, int64_t n_tok, int section, size_t *offset, size_t *bytes);
int fns_hip_moe_prefill(const FnsMoeLayer *layer, const float *x, const float *x_resid, float *out, int64_t n_tok,
                        void *workspace, size_t workspace_bytes, void *stream);
/* No counterpart in the reference. Without the F16 guard and for gate/up and down types from {Q3_K, Q4_K}, gate/up
 * and down run as one launch whose down workgroups wait (bounded) for their row group's gate/up
 * workgroups; one that gives up writes NaN to its output rows and sets FNS_STATUS_EXCHANGE_TIMEOUT in the workspace's
 * status word (section 8, which the workspace must hold zeroed when first used). As fns_hip_moe_layer_status: waits
 * for the stream's work so far, stores the word in *status and, with clear = 1, zeroes it. The poll limit and
 * withheld arrivals of fns_hip_moe_set_test_hooks apply to this wait too. Not graph-capturable (it synchronises). */
int fns_hip_moe_prefill_status(const FnsMoeLayer *layer, int64_t n_tok, void *workspace, int clear, uint32_t *status,
                               void *stream);
/* No counterpart in the reference: the graph-capturable form of fns_hip_moe_prefill_status, with the behaviour of
 * fns_hip_moe_layer_status_collect. */
int fns_hip_moe_prefill_status_collect(const FnsMoeLayer *layer, int64_t n_tok, void *workspace, uint32_t *dst,
                                       void *stream);

/* --- dense FFN layer (the reference model's leading dense blocks) ---
 * The dense branch of the reference's Engine::ffn_block (src/engine.cu:655-667: rms_norm_q8_1, dense_glu
 * (src/engine.cu:644-653: mmvq_swiglu at one column, else two mmvq and glu_mmvq), gemv of ffn_down (quantize_q8_1 +
 * mmvq, src/engine.cu:585-588), add_inplace) and of Engine::prefill_chunk (src/engine.cu:331-337: rms_norm_mul, mmq of
 * ffn_gate and ffn_up, swiglu, mmq of ffn_down, add_inplace):
 *   out[t] = x[t] + down . q8_1(silu(gate . q8_1(h[t])) * (up . q8_1(h[t]))), h = RMSNorm(x) * ffn_norm (or x).
 * Matrices are GGUF blocks: gate and up [inter][hidden], down [hidden][inter]; any type of the GEMV kernels
 * (fns_hip_mmvq_supports) for the decode form, any type of fns_hip_mmq for the prefill form. out may alias x. */
typedef struct FnsDenseFfn {
    int hidden, inter;                 /* positive multiples of 256 */
    int gate_type, up_type, down_type; /* ggml types */
    const void *gate, *up, *down;
    const float *ffn_norm;             /* NULL or f32 [hidden] */
    float norm_eps;
} FnsDenseFfn;
/* Device bytes of the workspace of either form at n_tok tokens (no zero-fill needed). */
int fns_hip_dense_ffn_workspace(const FnsDenseFfn *ffn, int64_t n_tok, size_t *total_bytes);
/* Decode / verify form (the reference's forward at cols_ = n_tok columns). */
int fns_hip_dense_ffn(const FnsDenseFfn *ffn, const float *x, float *out, int64_t n_tok, void *workspace,
                      size_t workspace_bytes, void *stream);
/* Prefill form (the MMQ GEMMs). */
int fns_hip_dense_ffn_prefill(const FnsDenseFfn *ffn, const float *x, float *out, int64_t n_tok, void *workspace,
                              size_t workspace_bytes, void *stream);
/* src/kernels.cuh:119 add_inplace, out-of-place: out[i] = x[i] + y[i]; out may alias x. */
int fns_hip_add(const float *x, const float *y, float *out, int64_t n, void *stream);

/* --- GGUF checkpoints: reader and fully resident MoE layers ---
 * Replaces the reference's loader (src/model.cpp:30-136: gguf header and tensor table, the file mapped without copying)
 * and expert placement (src/engine.cu:375-471: slots [gate | up | down] 256-byte aligned with 4096 zero bytes after the
 * last, a device table of slot pointers); every expert is resident in HBM. The reader is host code (no GPU needed);
 * fns_hip_moe_layer_from_gguf copies with hipMemcpy on the current device. C++ interface: include/fns/gguf.h. */
typedef struct FnsGguf FnsGguf;
typedef struct FnsGgufTensorInfo {
    int type;        /* ggml_type */
    int n_dims;
    int64_t ne[4];   /* ggml order: ne[0] contiguous */
    size_t nbytes;
    size_t offset;   /* from the start of the data section */
    const void *data; /* host pointer into the mapping (valid until fns_hip_gguf_close) */
} FnsGgufTensorInfo;
/* Opens and maps `path`; FNS_ERR_IO (with the reason in fns_hip_last_error) on a missing or malformed file. */
int fns_hip_gguf_open(const char *path, FnsGguf **out);
void fns_hip_gguf_close(FnsGguf *file);
int fns_hip_gguf_info(const FnsGguf *file, uint32_t *version, int64_t *n_tensors, int64_t *n_kv, size_t *data_offset);
/* Tensor by name (FNS_ERR_SHAPE when absent) or by index; *name (optional) points into the reader. */
int fns_hip_gguf_tensor(const FnsGguf *file, const char *name, FnsGgufTensorInfo *info);
int fns_hip_gguf_tensor_at(const FnsGguf *file, int64_t index, FnsGgufTensorInfo *info, const char **name);
/* gguf_get_val_u32 / f32 / bool / str of the reference's loader (src/model.cpp:19-26): FNS_ERR_SHAPE when the key is
 * absent or of another type. *value of _str points into the reader. */
int fns_hip_gguf_get_u32(const FnsGguf *file, const char *key, uint32_t *value);
int fns_hip_gguf_get_f32(const FnsGguf *file, const char *key, float *value);
int fns_hip_gguf_get_bool(const FnsGguf *file, const char *key, int *value);
int fns_hip_gguf_get_str(const FnsGguf *file, const char *key, const char **value);
/* MoE layer `layer` of the file made resident in HBM (blk.N.ffn_{gate,up,down}_exps.weight, ffn_gate_inp.weight,
 * optional exp_probs_b.bias, ffn_norm.weight and ffn_{gate,up,down}_shexp.weight; metadata
 * <arch>.expert_used_count, expert_weights_norm, expert_gating_func (1 softmax, 2 sigmoid; default sigmoid for
 * "flint", the reference's gating), attention.layer_norm_rms_epsilon). Fills *desc for fns_hip_moe_layer /
 * fns_hip_moe_prefill (guard = 1 for "flint", whose blocks apply the F16 guard, else 0); the device memory it points
 * to is owned by *resident. */
typedef struct FnsMoeResident FnsMoeResident;
int fns_hip_moe_layer_from_gguf(const FnsGguf *file, int layer, FnsMoeResident **resident, FnsMoeLayer *desc);
void fns_hip_moe_resident_free(FnsMoeResident *resident);
/* Dense FFN layer `layer` of the file made resident in HBM (reference src/model.cpp:120-125,193-196:
 * blk.N.ffn_{gate,up,down}.weight and ffn_norm.weight, metadata attention.layer_norm_rms_epsilon). Fills *desc for
 * fns_hip_dense_ffn / fns_hip_dense_ffn_prefill; the device memory it points to is owned by *resident. */
typedef struct FnsDenseResident FnsDenseResident;
int fns_hip_dense_ffn_from_gguf(const FnsGguf *file, int layer, FnsDenseResident **resident, FnsDenseFfn *desc);
void fns_hip_dense_resident_free(FnsDenseResident *resident);

/* --- seeded synthetic data on the device (benchmarks and large tests) ---
 * out[i] = mean + std * N(0,1), Philox-4x32-10 counter (offset + i) / 4 and Box-Muller; offset % 4 == 0. */
int fns_hip_fill_normal(float *out, int64_t n, uint64_t seed, uint64_t offset, float mean, float std, void *stream);
/* ggml's reference K-quant quantisers (quantize_row_q{3,4,5,6}_K_ref) on the device: x f32 [nrows][ncols] -> out. */
int fns_hip_quantize_weights(int type, const float *x, void *out, int64_t nrows, int64_t ncols, void *stream);

/* Device self-test of the DPP / lane-permute exchanges the kernels use: writes a bit mask of failing checks to
 * *bad_mask (device int, zero it first); 0 means every exchange matched the LDS-crossbar shuffle. */
int fns_hip_selftest_lanes(int *bad_mask, void *stream);

#ifdef __cplusplus
}
#endif
#endif
