/* fns_oracle.h - CPU restatement of the MoE FFN hot path of FlintNSteel (TEST INFRASTRUCTURE ONLY).
 *
 * This library is the checker, never the product: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it. The product path (flintnsteel_amd/, libfns_hip.so) never links or calls it.
 *
 * What it restates (reference = /root/reference, ggml = llama.cpp 19ab5a5e65736a35437e6b1c0ccd6562fed01b1b, MIT;
 * ggml is not vendored in the reference, its published algorithms are restated here):
 *   - GGUF K-quant block formats Q3_K/Q4_K/Q5_K/Q6_K (+ Q8_0) and their dequantisation (ggml-common.h /
 *     ggml-quants.c dequantize_row_*); block sizes pinned by static asserts.
 *   - ggml's reference weight quantisers quantize_row_q{3,4,5,6}_K_ref (make_qkx2_quants, make_qx_quants,
 *     make_q3_quants). Restated from the published algorithm; bit-identity with ggml's own output is NOT pinned
 *     (no ggml available) - parity never depends on it because both sides consume the same blocks.
 *   - Q8_1 activation quantisation with the GPU op order of the reference: src/kernels.cu:150-159 and
 *     :568-576 (d = amax/127, q = roundf(x/d), ds = half2(d, sum) with the xor-butterfly 16..1 sum),
 *     row padding to 512 columns (src/ggml/ggml_mmvq.cu:13-21).
 *   - Router logits (fp32 weights, float64 accumulation), softmax / sigmoid gating, top-k with ties to the lower
 *     index, renormalisation w = p / max(sum, 6.103515625e-5) (src/kernels.cu:484-514).
 *   - Expert GEMV (mmvq) = dequant(W) . dequant(xq) in float64 (the quantity tests/kernel_parity.py:80-88 checks).
 *   - SwiGLU epilogue act = up * silu(gate) (src/ggml/ggml_mmvq.cu:240-247), F16 guard (src/kernels.cu:534-577),
 *     weighted combine in slot order (src/kernels.cu:579-586).
 *   - Expert-id compaction with the invariants of ggml's mm_ids_helper (src/ggml/ggml_mmq.cu:110-111).
 */
#ifndef FNS_ORACLE_H
#define FNS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (public ggml.h numbering). */
enum { OR_Q8_0 = 8, OR_Q8_1 = 9, OR_Q3_K = 11, OR_Q4_K = 12, OR_Q5_K = 13, OR_Q6_K = 14,
       OR_IQ3_XXS = 18, OR_IQ3_S = 21, OR_IQ2_S = 22, OR_IQ4_XS = 23 };
int or_is_iq(int type);
/* The IQ3_XXS / IQ3_S / IQ2_S codebooks (ggml's iq3xxs_grid[256], iq3s_grid[512], iq2s_grid[1024]; not in this
 * container): registered by the caller before any IQ call. */
void or_set_iq_grids(const uint32_t *iq3xxs, const uint32_t *iq3s, const uint64_t *iq2s);

uint16_t or_f32_to_f16(float f);   /* IEEE binary16, round to nearest even */
float or_f16_to_f32(uint16_t h);
float or_expf(float x);            /* the exp used by the gating (same op sequence as the HIP kernels) */

size_t or_block_bytes(int type);   /* bytes per block */
int or_block_elems(int type);      /* weights per block */
size_t or_row_bytes(int type, int64_t ncols);

/* Quantise nrows x ncols fp32 into ggml blocks (ggml reference quantisers). Returns 0 or -1 (bad type/shape). */
int or_quantize(int type, const float *x, void *out, int64_t nrows, int64_t ncols, int nthreads);
/* Dequantise to float64 (exact: every block value is d*int or d*int - dmin*int with f16 d). */
int or_dequantize(int type, const void *in, double *out, int64_t nrows, int64_t ncols);

/* Q8_1 with the reference GPU op order: xq [nrows][or_q8_1_row_bytes(ncols)]. */
size_t or_q8_1_row_bytes(int64_t ncols);
void or_quantize_q8_1(const float *x, void *xq, int64_t ncols, int64_t nrows);
/* Dequantised Q8_1 values q*half(d), float64, ncols per row. */
void or_dequantize_q8_1(const void *xq, double *out, int64_t ncols, int64_t nrows);

/* logits[t][e] = sum_i W[e][i] x[t][i], float64 accumulation, rounded to fp32. */
void or_router_f32(const float *w, const float *x, float *logits, int64_t ncols, int64_t n_expert, int64_t n_tok);
/* Gating + top-k + renormalisation, exact fp32 op order of the HIP kernel. gating: 0 softmax, 1 sigmoid.
 * margin (optional, per token): p[k-1] - p[k] of the sorted probabilities (0 if k == n_expert). */
int or_route_topk(const float *logits, int32_t *ids, float *w, float *probs, float *margin, int n_expert, int k,
                  int n_tok, int gating, int norm);

/* dst[c][r] = W_{ids[c]}[r] . deq(xq row (c / x_div) % n_xq), float64. table[e] points at expert e's matrix. */
int or_mmvq_experts(int type, const void *const *table, int64_t ncols, int64_t nrows, const void *xq, int64_t n_xq,
                    int64_t x_div, const int32_t *ids, int64_t n_ids, double *dst);
/* act = up * silu(gate), float64. */
void or_swiglu(const double *gate, const double *up, double *act, int64_t n);
/* F16 guard e = 2^clamp(ceil(log2(amax/1024)), 0, 127) with the fp32 sequence of src/kernels.cu:544-551. */
float or_amax_guard_scale(const float *row, int64_t n);
/* out[t][i] = (sum_j (dexp[t][j][i] * e[t][j]) * w[t][j] (j in order) + sh[t][i]) + x[t][i], fp32 in order. */
void or_moe_combine(const float *dexp, const float *escale, const float *w, const float *sh, const float *x, float *out,
                    int64_t n, int k, int64_t n_tok);

/* Expert compaction: sort (token, slot) pairs by expert, stable in (token, slot) order.
 * bounds[n_expert+1], src[T*K] = t*x_rows_per_tok + (x_rows_per_tok == 1 ? 0 : j), dst[T*K] = t*K + j.
 * Returns the number of distinct experts. */
int or_compact_ids(const int32_t *ids, int64_t n_tok, int k, int n_expert, int x_rows_per_tok, int32_t *bounds,
                   int32_t *src, int32_t *dst);

/* CPU baseline (not ggml): one batch-1 MoE layer with int8 x K-quant integer dot products, OpenMP over rows. */
int or_cpu_moe_layer(int gu_type, int down_type, const float *router_w, const void *const *table, size_t gate_off,
                     size_t up_off, size_t down_off, const float *x, float *out, int64_t hidden, int64_t inter,
                     int n_expert, int k, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
