// capi.cpp - extern "C" entry points of libfns_hip.so (include/fns_hip.h): thin forwards to fns::impl.
#include "fns_hip.h"
#include "fns/ggml_kernels.h"

#include <cstring>

#include "fns_host.hpp"
#include "fns_internal.hpp"

using namespace fns;

static inline hipStream_t S(void *s) { return (hipStream_t) s; }

extern "C" {

int fns_hip_abi_version(void) { return 1; }
const char *fns_hip_last_error(void) { return host::last_error(); }

size_t fns_hip_q8_1_row_bytes(int64_t ncols) { return (size_t) host::q8_1_row_bytes(ncols); }

int fns_hip_quantize_q8_1(const float *x, void *xq, int64_t ncols, int64_t nrows, void *stream) {
    return impl::quantize_q8_1(x, xq, ncols, nrows, S(stream));
}

int fns_hip_mmvq(int type, const void *w, int64_t ncols, int64_t nrows, const void *xq, float *dst, int64_t n_cols,
                 void *stream) {
    return impl::mmvq(type, w, ncols, nrows, xq, dst, n_cols, S(stream));
}

int fns_hip_mmvq_ids(int type, const void *w, int64_t ncols, int64_t nrows, int64_t n_mats, const void *xq,
                     int64_t n_xq, const int32_t *ids, int64_t n_ids, float *dst, void *stream) {
    return impl::mmvq_ids(type, w, ncols, nrows, n_mats, xq, n_xq, ids, n_ids, dst, S(stream));
}

int fns_hip_mmvq_swiglu(int type, const void *w_gate, const void *w_up, int64_t ncols, int64_t nrows, const void *xq,
                        float *dst, void *stream) {
    return impl::mmvq_swiglu(type, w_gate, w_up, ncols, nrows, xq, dst, S(stream));
}

int fns_hip_mmvq_ids_swiglu_shared(int type, const void *w_gate, const void *w_up, int64_t ncols, int64_t nrows,
                                   int64_t n_mats, const void *xq, const int32_t *ids, int64_t n_ids, float *dst,
                                   const void *sh_gate, const void *sh_up, float *sh_dst, void *stream) {
    return impl::mmvq_ids_swiglu_shared(type, w_gate, w_up, ncols, nrows, n_mats, xq, ids, n_ids, dst, sh_gate, sh_up,
                                        sh_dst, S(stream));
}

int fns_hip_mmvq_experts_swiglu(int type, const void *const *table, size_t gate_off, size_t up_off, int64_t ncols,
                                int64_t nrows, const void *xq, int64_t n_xq, const int32_t *ids, int64_t n_ids,
                                float *dst, void *stream) {
    return impl::mmvq_experts_swiglu(type, (const char *const *) table, gate_off, up_off, ncols, nrows, xq, n_xq, ids,
                                     n_ids, dst, S(stream));
}

int fns_hip_mmvq_experts(int type, const void *const *table, size_t off, int64_t ncols, int64_t nrows, const void *xq,
                         int64_t n_xq, const int32_t *ids, int64_t n_ids, float *dst, void *stream) {
    return impl::mmvq_experts(type, (const char *const *) table, off, ncols, nrows, xq, n_xq, ids, n_ids, dst,
                              S(stream));
}

int fns_hip_mmvq_supports(int type) { return host::is_supported(type) ? 1 : 0; }

int fns_hip_set_iq_grids(const uint32_t *iq3xxs, const uint32_t *iq3s, const uint64_t *iq2s) {
    if (!iq3xxs || !iq3s || !iq2s) return host::set_error(host::ERR_SHAPE, "set_iq_grids: null table");
    struct {
        uint32_t a[256];
        uint32_t b[512];
        uint64_t c[1024];
    } g;
    static_assert(sizeof g == 256 * 4 + 512 * 4 + 1024 * 8, "packed like dev::IqGrids");
    std::memcpy(g.a, iq3xxs, sizeof g.a);
    std::memcpy(g.b, iq3s, sizeof g.b);
    std::memcpy(g.c, iq2s, sizeof g.c);
    // the decoders negate a codebook byte as (g ^ 0xff) + 1 within its byte: every value must be non-zero
    const uint8_t *bytes = (const uint8_t *) &g;
    for (size_t i = 0; i < sizeof g; ++i)
        if (bytes[i] == 0 || bytes[i] > 127)
            return host::set_error(host::ERR_SHAPE, "set_iq_grids: codebook byte %zu is %d (values must be 1..127)", i,
                                   bytes[i]);
    FNS_TRY(impl::iq_grids_upload_mmvq(&g));
    FNS_TRY(impl::iq_grids_upload_layer(&g));
    FNS_TRY(impl::iq_grids_upload_mmq(&g));
    host::set_iq_grids_ready();
    return host::OK;
}

int fns_hip_rms_norm_q8_1(const float *x, const float *w, float *out, void *xq, int n, float eps, int rows,
                          void *stream) {
    return impl::rms_norm_q8_1(x, w, out, xq, n, eps, rows, S(stream));
}

int fns_hip_gemv_router(int dtype, const void *w, const float *x, float *y, int ncols, int nrows, int cols,
                        void *stream) {
    return impl::gemv_router(dtype, w, x, y, ncols, nrows, cols, S(stream));
}

int fns_hip_gemm_router(int dtype, const void *w, const float *x, float *y, int ncols, int nrows, int n_tok,
                        void *stream) {
    return impl::gemm_router(dtype, w, x, y, ncols, nrows, n_tok, S(stream));
}

int fns_hip_route_topk(const float *logits, int32_t *ids, float *w, int n_expert, int k, int n_tok, int gating,
                       int norm, void *stream) {
    return impl::route_topk(logits, ids, w, n_expert, k, n_tok, gating, norm, S(stream));
}

int fns_hip_count_routes(const int32_t *ids, uint32_t *counts, int k, void *stream) {
    return impl::count_routes(ids, counts, k, S(stream));
}

int fns_hip_swiglu(const float *g, const float *u, float *act, int n, int rows, void *stream) {
    return impl::swiglu(g, u, act, n, rows, S(stream));
}

int fns_hip_glu_mmvq(const float *g, const float *u, float *act, int n, void *stream) {
    return impl::glu_mmvq(g, u, act, n, S(stream));
}

int fns_hip_amax_guard(float *act, float *escale, int n, int rows, void *stream) {
    return impl::amax_guard(act, escale, n, rows, S(stream));
}

int fns_hip_amax_guard_q8_1(const float *act, float *escale, void *xq, int n, int rows, void *stream) {
    return impl::amax_guard_q8_1(act, escale, xq, n, rows, S(stream));
}

int fns_hip_moe_combine(const float *dexp, const float *escale, const float *w, const float *sh, const float *x_in,
                        float *out, int n, int k, int n_tok, void *stream) {
    return impl::moe_combine(dexp, escale, w, sh, x_in, out, n, k, n_tok, S(stream));
}

int fns_hip_moe_workspace_layout(const FnsMoeLayer *layer, int n_tok, size_t *offsets, size_t *total_bytes) {
    return impl::moe_workspace_layout(layer, n_tok, offsets, total_bytes);
}

int fns_hip_moe_layer(const FnsMoeLayer *layer, const float *x, const float *x_resid, float *out, int n_tok,
                      void *workspace, size_t workspace_bytes, void *stream) {
    return impl::moe_layer(layer, x, x_resid, out, n_tok, workspace, workspace_bytes, S(stream));
}

int fns_hip_moe_layer_profiled(const FnsMoeLayer *layer, const float *x, const float *x_resid, float *out, int n_tok,
                               void *workspace, size_t workspace_bytes, void *const *events, void *stream) {
    return impl::moe_layer(layer, x, x_resid, out, n_tok, workspace, workspace_bytes, S(stream), events);
}

int fns_hip_moe_layer_noalloc(const FnsMoeLayer *layer, const float *x, const float *x_resid, float *out, int n_tok,
                              void *stream) {
    return impl::moe_layer_noalloc(layer, x, x_resid, out, n_tok, S(stream));
}

size_t fns_hip_moe_noalloc_max_bytes(void) { return impl::moe_noalloc_max_bytes(); }

int fns_hip_moe_layer_status(const FnsMoeLayer *layer, int n_tok, void *workspace, int clear, uint32_t *status,
                             void *stream) {
    return impl::moe_layer_status(layer, n_tok, workspace, clear, status, S(stream));
}

int fns_hip_moe_layer_status_collect(const FnsMoeLayer *layer, int n_tok, void *workspace, uint32_t *dst, void *stream) {
    return impl::moe_layer_status_collect(layer, n_tok, workspace, dst, S(stream));
}

int fns_hip_moe_set_path(int path) { return impl::moe_set_path(path); }

int fns_hip_moe_layer_kernels(const FnsMoeLayer *layer, int n_tok, int *kernels) {
    return impl::moe_layer_kernels(layer, n_tok, kernels);
}

int fns_hip_moe_set_test_hooks(int spin_limit, int withhold_arrivals) {
    return impl::moe_set_test_hooks(spin_limit, withhold_arrivals);
}

int fns_hip_moe_layer_stage(const FnsMoeLayer *layer, int stage, const float *x, const float *x_resid, float *out,
                            int n_tok, void *workspace, size_t workspace_bytes, void *stream) {
    return impl::moe_layer_stage(layer, stage, x, x_resid, out, n_tok, workspace, workspace_bytes, S(stream));
}

int fns_hip_fill_normal(float *out, int64_t n, uint64_t seed, uint64_t offset, float mean, float std, void *stream) {
    return impl::fill_normal(out, n, seed, offset, mean, std, S(stream));
}

int fns_hip_quantize_weights(int type, const float *x, void *out, int64_t nrows, int64_t ncols, void *stream) {
    return impl::quantize_weights(type, x, out, nrows, ncols, S(stream));
}

int fns_hip_selftest_lanes(int *bad_mask, void *stream) { return impl::selftest_lanes(bad_mask, S(stream)); }


size_t fns_hip_mmq_q8_1_bytes(int64_t ncols, int64_t nrows) { return impl::mmq_q8_1_bytes(ncols, nrows); }
size_t fns_hip_mmq_bounds_bytes(int64_t n_expert) { return impl::mmq_bounds_bytes(n_expert); }

int fns_hip_mmq(int type, const void *w, int64_t ncols, int64_t nrows, const float *x, int64_t n_tok, void *xq,
                float *dst, void *stream) {
    return impl::mmq(type, w, ncols, nrows, x, n_tok, xq, dst, S(stream));
}

int fns_hip_mmq_experts(int type, const void *const *table, size_t off, int64_t ncols, int64_t nrows, int64_t n_expert,
                        const float *x, int64_t x_rows_per_tok, int64_t n_tok, const int32_t *ids, int64_t n_used,
                        int32_t *ids_src1, int32_t *ids_dst, int32_t *expert_bounds, void *xq, float *dst, void *stream) {
    return impl::mmq_experts(type, (const char *const *) table, off, ncols, nrows, n_expert, x, x_rows_per_tok, n_tok,
                             ids, n_used, ids_src1, ids_dst, expert_bounds, xq, dst, S(stream));
}

int fns_hip_mmq_compact(const int32_t *ids, int64_t n_tok, int64_t n_used, int64_t n_expert, int64_t x_rows_per_tok,
                        int32_t *ids_src1, int32_t *ids_dst, int32_t *expert_bounds, void *stream) {
    return impl::mmq_compact(ids, n_tok, n_used, n_expert, x_rows_per_tok, ids_src1, ids_dst, expert_bounds,
                             expert_bounds + n_expert + 1, S(stream));
}

int fns_hip_moe_prefill_workspace(const FnsMoeLayer *layer, int64_t n_tok, size_t *offsets, size_t *total_bytes) {
    return impl::moe_prefill_workspace(layer, n_tok, offsets, total_bytes);
}

int fns_hip_moe_prefill_section(const FnsMoeLayer *layer, int64_t n_tok, int section, size_t *offset, size_t *bytes) {
    return impl::moe_prefill_section(layer, n_tok, section, offset, bytes);
}

int fns_hip_add(const float *x, const float *y, float *out, int64_t n, void *stream) {
    return impl::add(x, y, out, n, S(stream));
}

int fns_hip_dense_ffn_workspace(const FnsDenseFfn *ffn, int64_t n_tok, size_t *total_bytes) {
    return impl::dense_ffn_workspace(ffn, n_tok, total_bytes);
}

int fns_hip_dense_ffn(const FnsDenseFfn *ffn, const float *x, float *out, int64_t n_tok, void *workspace,
                      size_t workspace_bytes, void *stream) {
    return impl::dense_ffn(ffn, x, out, n_tok, workspace, workspace_bytes, false, S(stream));
}

int fns_hip_dense_ffn_prefill(const FnsDenseFfn *ffn, const float *x, float *out, int64_t n_tok, void *workspace,
                              size_t workspace_bytes, void *stream) {
    return impl::dense_ffn(ffn, x, out, n_tok, workspace, workspace_bytes, true, S(stream));
}

int fns_hip_moe_prefill_status(const FnsMoeLayer *layer, int64_t n_tok, void *workspace, int clear, uint32_t *status,
                               void *stream) {
    return impl::moe_prefill_status(layer, n_tok, workspace, clear, status, S(stream));
}

int fns_hip_moe_prefill_status_collect(const FnsMoeLayer *layer, int64_t n_tok, void *workspace, uint32_t *dst,
                                       void *stream) {
    return impl::moe_prefill_status_collect(layer, n_tok, workspace, dst, S(stream));
}

int fns_hip_moe_prefill(const FnsMoeLayer *layer, const float *x, const float *x_resid, float *out, int64_t n_tok,
                        void *workspace, size_t workspace_bytes, void *stream) {
    return impl::moe_prefill(layer, x, x_resid, out, n_tok, workspace, workspace_bytes, S(stream));
}
}  // extern "C"

// C++ API form (include/fns/ggml_kernels.h): aborts on bad tables, as the reference's API aborts on errors.
namespace fns {
void set_iq_grids(const uint32_t *iq3xxs, const uint32_t *iq3s, const uint64_t *iq2s) {
    host::abort_on_error(fns_hip_set_iq_grids(iq3xxs, iq3s, iq2s), "set_iq_grids");
}
}  // namespace fns
