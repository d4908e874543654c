// include/fns/ggml_kernels.h - quantized expert GEMV (MMVQ), Q8_1 activation quantisation and prefill grouped GEMM
// (MMQ) for MI355X (gfx950). Drop-in for the reference header of the same name (/root/reference/
// include/fns/ggml_kernels.h:1-82): same namespace, names, argument lists and semantics, with hipStream_t for
// cudaStream_t and an own ggml_type enum carrying ggml's numeric values. Implemented by libfns_hip.so
// (flintnsteel_amd/csrc/*.hip); the C ABI over the same entry points is include/fns_hip.h.
//
// Errors follow the reference: a launch failure or an unsupported type/shape prints a message and aborts the process
// (reference src/ggml/ggml_mmvq.cu:385, src/ggml/ggml_cuda_host.cu:14-17). The C ABI returns error codes instead.
// Every function is asynchronous on `stream`, allocates nothing and is capturable in a HIP graph.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#ifndef FNS_GGML_TYPE_DEFINED
#define FNS_GGML_TYPE_DEFINED
// ggml_type values of public ggml.h (the subset this path uses). Reference: include/fns/ggml_kernels.h:4 includes ggml.h.
enum ggml_type : int {
    GGML_TYPE_F32 = 0,
    GGML_TYPE_F16 = 1,
    GGML_TYPE_Q8_0 = 8,
    GGML_TYPE_Q8_1 = 9,
    GGML_TYPE_Q3_K = 11,
    GGML_TYPE_Q4_K = 12,
    GGML_TYPE_Q5_K = 13,
    GGML_TYPE_Q6_K = 14,
    GGML_TYPE_IQ3_XXS = 18,
    GGML_TYPE_IQ3_S = 21,
    GGML_TYPE_IQ2_S = 22,
    GGML_TYPE_IQ4_XS = 23,
    GGML_TYPE_BF16 = 30,
};
#endif

namespace fns {

// Bytes of one row of `ncols` activations quantized to Q8_1, padded to a multiple of 512 columns.
// Reference: include/fns/ggml_kernels.h:13-14, src/ggml/ggml_mmvq.cu:13-15.
size_t q8_1_row_bytes(int64_t ncols);

// x [nrows][ncols] f32 -> xq [nrows][q8_1_row_bytes(ncols)]: d = amax/127, q = roundf(x/d), ds = (d, sum x) in f16,
// both reductions over 32 lanes by xor butterfly. Reference: include/fns/ggml_kernels.h:16-17, src/ggml/ggml_mmvq.cu:17-21.
void quantize_q8_1(const float *x, void *xq, int64_t ncols, int64_t nrows, hipStream_t stream);

// dst[c][nrows] = W[nrows][ncols] . x[c], c < n_cols, launches of at most 4 columns; each column has the bits of a
// single-column call. Reference: include/fns/ggml_kernels.h:19-22, src/ggml/ggml_mmvq.cu:23-38.
void mmvq(ggml_type type, const void *w, int64_t ncols, int64_t nrows, const void *xq, float *dst, int64_t n_cols,
          hipStream_t stream);

// MUL_MAT_ID for one token: dst[c][nrows] = W[ids[c]] . xq[c % n_xq], c < n_ids, W [n_mats][nrows][ncols].
// Reference: include/fns/ggml_kernels.h:24-27, src/ggml/ggml_mmvq.cu:40-52.
void mmvq_ids(ggml_type type, const void *w, int64_t ncols, int64_t nrows, int64_t n_mats, const void *xq,
              int64_t n_xq, const int32_t *ids, int64_t n_ids, float *dst, hipStream_t stream);

// dst[r] = (W_up . x)[r] * silu((W_gate . x)[r]), x read once. Reference: include/fns/ggml_kernels.h:29-31,
// src/ggml/ggml_mmvq.cu:54-66.
void mmvq_swiglu(ggml_type type, const void *w_gate, const void *w_up, int64_t ncols, int64_t nrows, const void *xq,
                 float *dst, hipStream_t stream);

// Routed experts (one shared input row) with SwiGLU, optionally the shared expert in the same launch.
// Reference: include/fns/ggml_kernels.h:33-37, src/ggml/ggml_mmvq.cu:68-89.
void mmvq_ids_swiglu_shared(ggml_type type, const void *w_gate, const void *w_up, int64_t ncols, int64_t nrows,
                            int64_t n_mats, const void *xq, const int32_t *ids, int64_t n_ids, float *dst,
                            const void *sh_gate, const void *sh_up, float *sh_dst, hipStream_t stream);

// Expert pointer tables: expert e's matrix [nrows][ncols] starts at table[e] + off (table in device memory).
// Bit-identical to mmvq_ids_swiglu_shared / mmvq_ids on the contiguous tensor.
//   swiglu: dst[c] = up_e . x[c / (n_ids / n_xq)] * silu(gate_e . x[...]), e = ids[c]
//   simple: dst[c] = W_e . xq[c % n_xq]
// Reference: include/fns/ggml_kernels.h:39-50, src/ggml/ggml_mmvq.cu:159-401.
void mmvq_experts_swiglu(ggml_type type, const char *const *table, size_t gate_off, size_t up_off, int64_t ncols,
                         int64_t nrows, const void *xq, int64_t n_xq, const int32_t *ids, int64_t n_ids, float *dst,
                         hipStream_t stream);
void mmvq_experts(ggml_type type, const char *const *table, size_t off, int64_t ncols, int64_t nrows, const void *xq,
                  int64_t n_xq, const int32_t *ids, int64_t n_ids, float *dst, hipStream_t stream);

// --- Batched prefill (MMQ) ---
// Bytes of the MMQ activation buffer for nrows rows of ncols activations (Q8_1 rows, padding included).
// Reference: include/fns/ggml_kernels.h:53-54, src/ggml/ggml_mmq.cu:74-78.
size_t mmq_q8_1_bytes(int64_t ncols, int64_t nrows);

// dst[t][r] = (W . x[t])[r], t < n_tok; x f32 [n_tok][ncols]; xq: mmq_q8_1_bytes(ncols, n_tok) bytes of scratch.
// Types: the reference's MMQ set (src/ggml/ggml_mmq.cu:59-66: Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS, IQ3_S, IQ3_XXS, IQ2_S)
// and Q3_K. Reference: include/fns/ggml_kernels.h:56-58, src/ggml/ggml_mmq.cu:80-96.
void mmq(ggml_type type, const void *w, int64_t ncols, int64_t nrows, const float *x, int64_t n_tok, void *xq,
         float *dst, hipStream_t stream);

// Scratch of the expert path for at most n_tok tokens and n_used experts per token: ids_src1 and ids_dst
// n_tok*n_used (+128) int32, expert_bounds n_expert+1 int32, xq mmq_q8_1_bytes(ncols_max, n_tok*n_used) bytes (its
// slack also holds the GEMM's tile-group prefix). Reference: include/fns/ggml_kernels.h:60-65, src/engine.cu:228-231.
struct MmqIdsScratch {
    int32_t *ids_src1 = nullptr, *ids_dst = nullptr, *expert_bounds = nullptr;
    void *xq = nullptr;
};
// Bytes of the bounds buffer of the standalone compaction (fns_hip_mmq_compact: n_expert + 1 bounds + tile prefix).
size_t mmq_bounds_bytes(int64_t n_expert);

// dst[t][j][r] = (W_e . x[t][j % x_rows_per_tok])[r], e = ids[t][j], j < n_used; expert e's matrix at table[e] + off.
// x_rows_per_tok = 1 (gate/up) or n_used (down). Reference: include/fns/ggml_kernels.h:67-69, src/ggml/ggml_mmq.cu:98-129.
void mmq_experts(ggml_type type, const char *const *table, size_t off, int64_t ncols, int64_t nrows, int64_t n_expert,
                 const float *x, int64_t x_rows_per_tok, int64_t n_tok, const int32_t *ids, int64_t n_used,
                 MmqIdsScratch &s, float *dst, hipStream_t stream);

// FlashAttention over a prefill chunk: declared with the reference's signature so that Engine::prefill_chunk, which
// includes this header, keeps compiling; attention is not part of the MoE FFN path and libfns_hip.so does NOT define
// it: the engine keeps linking its own implementation (the reference's src/ggml/ggml_fattn.cu).
// out[t][h] = softmax(scale * q[t][h] . K^T + mask[t]; sink_h) . V. Reference: include/fns/ggml_kernels.h:71-77.
void flash_attn_prefill(const float *q, const void *kc, const void *vc, const void *mask, const float *sinks,
                        float *out, int n_tok, int n_kv, int n_head, int n_head_kv, int head_dim, float scale,
                        hipStream_t stream);

// Quantized types this path accepts: Q8_0 and the K-quants (Q3_K added for the configs' UD-Q3_K_XL-like mix).
// Reference: include/fns/ggml_kernels.h:79-80, src/ggml/ggml_mmvq.cu:403-411.
bool mmvq_supports(ggml_type type);

// No counterpart in the reference (its ggml build compiles the IQ codebooks in): registers ggml's iq3xxs_grid[256],
// iq3s_grid[512] and iq2s_grid[1024] on the current device, once per device, before IQ3_XXS / IQ3_S / IQ2_S products;
// mmvq_supports rejects those types until then. Aborts on bad tables (every byte must be 1..127).
void set_iq_grids(const uint32_t *iq3xxs, const uint32_t *iq3s, const uint64_t *iq2s);

}  // namespace fns
