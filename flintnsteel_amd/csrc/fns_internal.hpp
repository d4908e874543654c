// fns_internal.hpp - status-returning implementations behind the C ABI (include/fns_hip.h) and the C++ API
// (include/fns/ggml_kernels.h, include/fns/kernels.h). Every function validates its arguments, launches on `st`
// and returns fns::host::Status.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "fns_hip.h"

namespace fns::impl {

int quantize_q8_1(const float *x, void *xq, int64_t ncols, int64_t nrows, hipStream_t st);
int rms_norm_q8_1(const float *x, const float *w, float *out, void *xq, int n, float eps, int rows, hipStream_t st);
int amax_guard(float *act, float *escale, int n, int rows, hipStream_t st);
int amax_guard_q8_1(const float *act, float *escale, void *xq, int n, int rows, hipStream_t st);
int swiglu(const float *g, const float *u, float *act, int n, int rows, hipStream_t st);
int glu_mmvq(const float *g, const float *u, float *act, int n, hipStream_t st);
int add(const float *x, const float *y, float *out, int64_t n, hipStream_t st);

int mmvq(int type, const void *w, int64_t ncols, int64_t nrows, const void *xq, float *dst, int64_t n_cols,
         hipStream_t st);
int mmvq_ids(int type, const void *w, int64_t ncols, int64_t nrows, int64_t n_mats, const void *xq, int64_t n_xq,
             const int32_t *ids, int64_t n_ids, float *dst, hipStream_t st);
int mmvq_swiglu(int type, const void *w_gate, const void *w_up, int64_t ncols, int64_t nrows, const void *xq,
                float *dst, hipStream_t st);
int mmvq_ids_swiglu_shared(int type, const void *w_gate, const void *w_up, int64_t ncols, int64_t nrows,
                           int64_t n_mats, const void *xq, const int32_t *ids, int64_t n_ids, float *dst,
                           const void *sh_gate, const void *sh_up, float *sh_dst, hipStream_t st);
int mmvq_experts_swiglu(int type, const char *const *table, size_t gate_off, size_t up_off, int64_t ncols,
                        int64_t nrows, const void *xq, int64_t n_xq, const int32_t *ids, int64_t n_ids, float *dst,
                        hipStream_t st);
int mmvq_experts(int type, const char *const *table, size_t off, int64_t ncols, int64_t nrows, const void *xq,
                 int64_t n_xq, const int32_t *ids, int64_t n_ids, float *dst, hipStream_t st);
// as mmvq_experts, id i reading activation row (i / x_div) % n_xq
int mmvq_experts_div(int type, const char *const *table, size_t off, int64_t ncols, int64_t nrows, const void *xq,
                     int64_t n_xq, int64_t x_div, const int32_t *ids, int64_t n_ids, float *dst, hipStream_t st);

int gemv_router(int dtype, const void *w, const float *x, float *y, int ncols, int nrows, int cols, hipStream_t st);
int gemm_router_bias(int dtype, const void *w, const float *bias, const float *x, float *y, int ncols, int nrows,
                     int n_tok, hipStream_t st);
int gemm_router(int dtype, const void *w, const float *x, float *y, int ncols, int nrows, int n_tok, hipStream_t st);
int route_topk(const float *logits, int32_t *ids, float *w, int n_expert, int k, int n_tok, int gating, int norm,
               hipStream_t st);
int moe_combine(const float *dexp, const float *escale, const float *w, const float *sh, const float *x_in, float *out,
                int n, int k, int n_tok, hipStream_t st);
int count_routes(const int32_t *ids, uint32_t *counts, int k, hipStream_t st);

int moe_workspace_layout(const FnsMoeLayer *L, int n_tok, size_t *offsets, size_t *total);
int moe_layer(const FnsMoeLayer *L, const float *x, const float *x_resid, float *out, int n_tok, void *ws,
              size_t ws_bytes, hipStream_t st, void *const *events = nullptr);
int moe_layer_noalloc(const FnsMoeLayer *L, const float *x, const float *x_resid, float *out, int n_tok, hipStream_t st);
size_t moe_noalloc_max_bytes();
// Each translation unit that decodes IQ blocks keeps its own device copy of the codebooks.
int iq_grids_upload_mmvq(const void *grids);
int iq_grids_upload_layer(const void *grids);
int iq_grids_upload_mmq(const void *grids);
int moe_layer_stage(const FnsMoeLayer *L, int stage, const float *x, const float *x_resid, float *out, int n_tok,
                    void *ws, size_t ws_bytes, hipStream_t st);

size_t mmq_image_bytes(int64_t ncols);
size_t mmq_q8_1_bytes(int64_t ncols, int64_t nrows);
size_t mmq_bounds_bytes(int64_t n_expert);
int mmq_quant_image(const float *x, int64_t ncols, int64_t rows, void *xpack, hipStream_t st);
int mmq_quant_image_scaled(const float *x, const float *escale, int64_t ncols, int64_t rows, void *xpack, int64_t stride,
                           hipStream_t st);
int mmq_compact(const int32_t *ids, int64_t n_tok, int64_t k, int64_t n_expert, int64_t x_rows_per_tok,
                int32_t *ids_src1, int32_t *ids_dst, int32_t *bounds, int32_t *gprefix, hipStream_t st,
                int32_t *gdone = nullptr, int n_gdone = 0);
int mmq_gemm_experts(int type, const char *const *table, size_t off_a, size_t off_b, bool glu, int64_t ncols,
                     int64_t nrows, int64_t n_expert, const void *xpack, int64_t n_pairs, const int32_t *ids_src1,
                     const int32_t *ids_dst, const int32_t *bounds, const int32_t *gprefix, float *dst, void *out_pack,
                     float *act_out, hipStream_t st);
int mmq(int type, const void *w, int64_t ncols, int64_t nrows, const float *x, int64_t n_tok, void *xq, float *dst,
        hipStream_t st);
int mmq_dense_glu(int type, const void *gate, const void *up, int64_t ncols, int64_t nrows, const void *ximg,
                  int64_t n_tok, void *act_img, hipStream_t st);
int mmq_dense_parts(int type, const void *w, int64_t ncols, int64_t nrows, const void *ximg, int64_t n_tok, float *dst,
                    int ksplit, hipStream_t st);
bool mmq_tiled(int type, int64_t ncols, int64_t nrows);  // the tiled GEMM takes this type and shape
int add_parts(const float *x, const float *parts, int n_parts, float *out, int64_t n, hipStream_t st);
int mmq_experts(int type, const char *const *table, size_t off, int64_t ncols, int64_t nrows, int64_t n_expert,
                const float *x, int64_t x_rows_per_tok, int64_t n_tok, const int32_t *ids, int64_t n_used,
                int32_t *ids_src1, int32_t *ids_dst, int32_t *bounds, void *xq, float *dst, hipStream_t st);
int moe_set_test_hooks(int spin_limit, int withhold);
void moe_test_hooks(int *spin_limit, int *withhold);  // the values set by moe_set_test_hooks
int moe_set_path(int path);
int moe_layer_kernels(const FnsMoeLayer *L, int n_tok, int *kernels);
int moe_layer_status(const FnsMoeLayer *L, int n_tok, void *ws, int clear, uint32_t *status, hipStream_t st);
int moe_layer_status_collect(const FnsMoeLayer *L, int n_tok, void *ws, uint32_t *dst, hipStream_t st);
int status_collect(uint32_t *word, uint32_t *dst, hipStream_t st);
int moe_prefill_workspace(const FnsMoeLayer *L, int64_t n_tok, size_t *offsets, size_t *total);
int moe_prefill_section(const FnsMoeLayer *L, int64_t n_tok, int section, size_t *offset, size_t *bytes);
int moe_prefill_status(const FnsMoeLayer *L, int64_t n_tok, void *ws, int clear, uint32_t *status, hipStream_t st);
int moe_prefill_status_collect(const FnsMoeLayer *L, int64_t n_tok, void *ws, uint32_t *dst, hipStream_t st);
int moe_prefill(const FnsMoeLayer *L, const float *x, const float *x_resid, float *out, int64_t n_tok, void *ws,
                size_t ws_bytes, hipStream_t st);

int dense_ffn_workspace(const FnsDenseFfn *D, int64_t n_tok, size_t *total);
int dense_ffn(const FnsDenseFfn *D, const float *x, float *out, int64_t n_tok, void *ws, size_t ws_bytes, bool prefill,
              hipStream_t st);

int fill_normal(float *out, int64_t n, uint64_t seed, uint64_t offset, float mean, float std, hipStream_t st);
int quantize_weights(int type, const float *x, void *out, int64_t nrows, int64_t ncols, hipStream_t st);

int selftest_lanes(int *bad_mask_device, hipStream_t st);

}  // namespace fns::impl
