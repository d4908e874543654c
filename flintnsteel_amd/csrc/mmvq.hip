// mmvq.hip - quantized GEMV over GGUF K-quant matrices (dense, MUL_MAT_ID, expert pointer tables, fused SwiGLU,
// shared expert) for MI355X gfx950.
//
// Reference semantics: src/ggml/ggml_mmvq.cu:23-89 (ggml MMVQ entry points) and :159-401 (pointer-table expert
// kernels). This is a new wave64 design, not a transcription of ggml's warp-32 mul_mat_vec_q:
//   - a row is split into 16-byte "slots" of packed quants (8 per 256-value block for Q4_K/Q5_K/Q6_K, 4 for Q3_K);
//   - LPR lanes (a power of two dividing the slot count, up to the whole wave) own one row; each lane reads its slots
//     with 16-byte loads issued up front (RPG rows per lane group), so one wave keeps 2-4 KB in flight;
//   - the Q8_1 activation row is staged once per workgroup in LDS (int8 values, per-32 scales and per-16 scaled
//     sums for the K-quant min term) and read by every lane group of the workgroup;
//   - per-lane partials are reduced over the LPR lanes by an xor butterfly.
// Each output element depends only on its own row, channel and activation row, never on how many channels or columns
// share the launch: the table path is bit-identical to the contiguous path, and column c of a multi-column call is
// bit-identical to a single-column call (the invariants of reference tests/expert_parity.cu:1-8 and
// src/ggml/ggml_mmvq.cu:25-27).
#include "fns/ggml_kernels.h"
#include "fns_common.hpp"
#include "fns_quarter.hpp"
#include "fns_host.hpp"
#include "fns_internal.hpp"

namespace fns {

using namespace fns::dev;

namespace {

struct MmvqParams {
    const char *const *table;  // expert table (device) or null
    const uint8_t *base;       // matrices base + e * mat_stride when table is null
    int64_t mat_stride;
    int64_t off_a, off_b;  // A: plain matrix or `up`; B: `gate` (GLU)
    const int32_t *ids;    // channel -> expert (null: expert 0)
    int n_ids;             // channel n_ids is the shared expert when sh_a is set
    const uint8_t *sh_a, *sh_b;
    float *sh_dst;
    const uint8_t *xq;
    int64_t xq_row_bytes;
    int n_xq, x_div;
    int ncol_dense;  // > 0: one channel, columns j < ncol_dense read x row j and write dst row j
    float *dst;
    int ncols, nrows;
};

// Channel c -> its matrices (A; B = gate for GLU), live columns, activation rows and output rows.
template <int NC>
__device__ __forceinline__ void channel_of(const MmvqParams &p, int c, const uint8_t *&wa, const uint8_t *&wb,
                                           int &ncol, int (&xrow)[NC], float *(&out)[NC]) {
    if (p.ncol_dense > 0) {
        wa = p.base + p.off_a;
        wb = p.base + p.off_b;
        ncol = p.ncol_dense;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            xrow[j] = j;
            out[j] = p.dst + (size_t) j * p.nrows;
        }
    } else if (p.sh_a && c == p.n_ids) {
        wa = p.sh_a;
        wb = p.sh_b;
        ncol = 1;
        xrow[0] = 0;
        out[0] = p.sh_dst;
    } else {
        const int e = p.ids ? p.ids[c] : 0;
        const uint8_t *m = p.table ? (const uint8_t *) p.table[e] : p.base + (size_t) e * p.mat_stride;
        wa = m + p.off_a;
        wb = m + p.off_b;
        ncol = 1;
        xrow[0] = (c / p.x_div) % p.n_xq;
        out[0] = p.dst + (size_t) c * p.nrows;
    }
}

// rows per lane group: whole-wave rows (LPR = 64) one per group, the most workgroups (at one token, 2 rows per group
// measured 0.6-1.1 us slower per gate/up + down pair, 4 rows 1.6 us slower); 32-lane rows two
template <int LPR> constexpr int rows_per_group() { return LPR == 32 ? 2 : 1; }

template <int T, int LPR, int SPL, int NC, bool GLU>
__global__ __launch_bounds__(256) void k_mmvq(const MmvqParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int SPB = Traits<T>::slots;
    constexpr int BB = Traits<T>::bytes;
    constexpr int G = 256 / LPR;
    constexpr int RPG = rows_per_group<LPR>();
    constexpr int SPLX = SPL > 0 ? SPL : 1;
    const int tid = threadIdx.x;
    const int c = blockIdx.y;

    const uint8_t *wa, *wb;
    int ncol;
    int xrow[NC];
    float *out[NC];
    channel_of<NC>(p, c, wa, wb, ncol, xrow, out);

    const int nblk = p.ncols / 256;
    const int nslots = nblk * SPB;
    const int64_t row_bytes = (int64_t) nblk * BB;
    const int lane = tid % LPR, grp = tid / LPR;
    const int row0 = blockIdx.x * (G * RPG) + grp;

    // 1. weight fragments: issued before the activation staging so both are in flight together
    Frag fa[RPG][SPLX], fb[RPG][GLU ? SPLX : 1];
    if constexpr (SPL > 0) {
#pragma unroll
        for (int r = 0; r < RPG; ++r) {
            const int row = row0 + r * G;
#pragma unroll
            for (int s = 0; s < SPL; ++s) {
                const int sl = lane + s * LPR;
                if (row < p.nrows && sl < nslots) {
                    const uint8_t *blk = wa + row * row_bytes + (int64_t) (sl / SPB) * BB;
                    slot_load<T>(blk, sl % SPB, fa[r][s]);
                    if constexpr (GLU) slot_load<T>(wb + row * row_bytes + (int64_t) (sl / SPB) * BB, sl % SPB, fb[r][s]);
                }
            }
        }
    }

    // 2. activation rows -> LDS
    const int npad = (int) ((p.ncols + 511) / 512 * 512);
    ActView av[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        uint8_t *base = smem + j * act_lds_bytes(npad);
        int8_t *q = (int8_t *) base;
        float *d = (float *) (base + npad);
        float *s16 = d + npad / 32;
        av[j] = ActView{q, d, s16};
        if (j < ncol) stage_q8_1_row(p.xq + (int64_t) xrow[j] * p.xq_row_bytes, npad / 32, q, d, s16, tid, 256);
    }
    __syncthreads();

    // 3. dot products
    float acc[RPG][NC], accg[RPG][NC];
#pragma unroll
    for (int r = 0; r < RPG; ++r)
#pragma unroll
        for (int j = 0; j < NC; ++j) acc[r][j] = accg[r][j] = 0.0f;

#pragma unroll
    for (int r = 0; r < RPG; ++r) {
        const int row = row0 + r * G;
        if (row >= p.nrows) continue;
        if constexpr (SPL > 0) {
#pragma unroll
            for (int s = 0; s < SPL; ++s) {
                const int sl = lane + s * LPR;
                if (sl < nslots) {
#pragma unroll
                    for (int j = 0; j < NC; ++j) {
                        if (j < ncol) {
                            acc[r][j] += slot_dot<T>(fa[r][s], sl % SPB, (sl / SPB) * 256, av[j]);
                            if constexpr (GLU) accg[r][j] += slot_dot<T>(fb[r][s], sl % SPB, (sl / SPB) * 256, av[j]);
                        }
                    }
                }
            }
        } else {
            for (int sl = lane; sl < nslots; sl += LPR) {
                Frag f, g;
                slot_load<T>(wa + row * row_bytes + (int64_t) (sl / SPB) * BB, sl % SPB, f);
                if constexpr (GLU) slot_load<T>(wb + row * row_bytes + (int64_t) (sl / SPB) * BB, sl % SPB, g);
#pragma unroll
                for (int j = 0; j < NC; ++j) {
                    if (j < ncol) {
                        acc[r][j] += slot_dot<T>(f, sl % SPB, (sl / SPB) * 256, av[j]);
                        if constexpr (GLU) accg[r][j] += slot_dot<T>(g, sl % SPB, (sl / SPB) * 256, av[j]);
                    }
                }
            }
        }
    }

    // 4. reduce over the LPR lanes of each row and write
#pragma unroll
    for (int r = 0; r < RPG; ++r) {
        const int row = row0 + r * G;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            float v = group_sum<LPR>(acc[r][j]);
            if constexpr (GLU) {
                const float gsum = group_sum<LPR>(accg[r][j]);
                // fused-GLU epilogue with zero biases (reference src/ggml/ggml_mmvq.cu:240-247)
                v += 0.0f;
                v *= silu(gsum + 0.0f);
            }
            if (lane == 0 && j < ncol && row < p.nrows) out[j][row] = v;
        }
    }
}

template <int T, int LPR, int SPL, int NC, bool GLU>
int launch_shape(const MmvqParams &p, int n_chan, hipStream_t st) {
    constexpr int RPB = (256 / LPR) * rows_per_group<LPR>();
    const dim3 grid((unsigned) ((p.nrows + RPB - 1) / RPB), (unsigned) n_chan);
    const int npad = (int) host::pad512(p.ncols);
    const size_t lds = (size_t) NC * act_lds_bytes(npad);
    if (lds > 160 * 1024) return host::set_error(host::ERR_SHAPE, "mmvq: ncols %d too large for LDS staging", p.ncols);
    hipLaunchKernelGGL((k_mmvq<T, LPR, SPL, NC, GLU>), grid, dim3(256), lds, st, p);
    return host::check_launch("mmvq");
}

template <int T, int NC, bool GLU> int launch_nc(const MmvqParams &p, int n_chan, hipStream_t st) {
    const host::Shape s = host::pick_shape(p.ncols / 256 * Traits<T>::slots);
    if (s.lpr == 64 && s.spl == 1) return launch_shape<T, 64, 1, NC, GLU>(p, n_chan, st);
    if (s.lpr == 64 && s.spl == 2) return launch_shape<T, 64, 2, NC, GLU>(p, n_chan, st);
    if (s.lpr == 64 && s.spl == 3) return launch_shape<T, 64, 3, NC, GLU>(p, n_chan, st);
    if (s.lpr == 32) return launch_shape<T, 32, 1, NC, GLU>(p, n_chan, st);
    if (s.lpr == 16) return launch_shape<T, 16, 1, NC, GLU>(p, n_chan, st);
    if (s.lpr == 8) return launch_shape<T, 8, 3, NC, GLU>(p, n_chan, st);
    if (s.lpr == 4) return launch_shape<T, 4, 3, NC, GLU>(p, n_chan, st);
    return launch_shape<T, 64, 0, NC, GLU>(p, n_chan, st);
}


// Quarter-block form, for the types without slot decoders (Q8_0): LPR lanes per row (16 or 32), lane l takes the
// 64-value quarters l, l + LPR, ... of its row; the activation rows are staged in LDS as row images (fns_block.hpp
// layout, built from the Q8_1 blocks). Per (row, column) the arithmetic does not depend on the launch shape.
__device__ __forceinline__ void stage_q8_1_img(const uint8_t *__restrict__ src, int npad, uint8_t *img, int tid,
                                               int nthreads) {
    float *d = (float *) (img + img_q_bytes(npad)), *s16 = d + npad / 32, *s32 = s16 + npad / 16;
    for (int b = tid; b < npad / 32; b += nthreads) {
        const uint32_t *w = (const uint32_t *) (src + (size_t) b * 36);
        uint32_t v[9];
#pragma unroll
        for (int i = 0; i < 9; ++i) v[i] = w[i];
        const float db = half_to_float(v[0] & 0xffffu);
        int sa = 0, sb = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) sa = dot4((int) v[1 + i], 0x01010101, sa);
#pragma unroll
        for (int i = 0; i < 4; ++i) sb = dot4((int) v[5 + i], 0x01010101, sb);
        uint4 *dq = (uint4 *) (img + img_q_index(32 * b));
        dq[0] = make_uint4(v[1], v[2], v[3], v[4]);
        dq[1] = make_uint4(v[5], v[6], v[7], v[8]);
        d[b] = db;
        s16[2 * b] = db * (float) sa;
        s16[2 * b + 1] = db * (float) sb;
        s32[b] = db * (float) (sa + sb);
    }
}

template <int T, int LPR, int NC, bool GLU>
__global__ __launch_bounds__(256) void k_mmvq_q(const MmvqParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int BB = Traits<T>::bytes;
    const int tid = threadIdx.x;
    const uint8_t *wa, *wb;
    int ncol;
    int xrow[NC];
    float *out[NC];
    channel_of<NC>(p, blockIdx.y, wa, wb, ncol, xrow, out);
    const int npad = (p.ncols + 511) / 512 * 512, ib = img_bytes(npad);
    ActImg img[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        img[j] = act_img(smem + j * ib, npad);
        if (j < ncol) stage_q8_1_img(p.xq + (int64_t) xrow[j] * p.xq_row_bytes, npad, smem + j * ib, tid, 256);
    }
    iq_grids_to_lds<T>(tid, 256);  // (visible after the barrier)
    __syncthreads();
    const int nblk = p.ncols / 256, lane = tid % LPR;
    const int row = blockIdx.x * (256 / LPR) + tid / LPR;
    const int64_t row_bytes = (int64_t) nblk * BB;
    float acc[NC], accg[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) acc[j] = accg[j] = 0.0f;
    if (row < p.nrows) {
        for (int qi = lane; qi < 4 * nblk; qi += LPR) {
            const int bb = qi >> 2, qt = qi & 3;
            const uint8_t *ba = wa + row * row_bytes + (int64_t) bb * BB;
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                if (j < ncol) {
                    acc[j] += quarter_dot<T, Any2>(ba, img[j], bb, qt);
                    if constexpr (GLU) accg[j] += quarter_dot<T, Any2>(wb + row * row_bytes + (int64_t) bb * BB, img[j], bb, qt);
                }
            }
        }
    }
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        float v = lanes_sum<LPR>(acc[j]);
        if constexpr (GLU) {
            const float gsum = lanes_sum<LPR>(accg[j]);
            v += 0.0f;  // fused-GLU epilogue with zero biases (reference src/ggml/ggml_mmvq.cu:240-247)
            v *= silu(gsum + 0.0f);
        }
        if (lane == 0 && j < ncol && row < p.nrows) out[j][row] = v;
    }
}

template <int T, int NC, bool GLU> int launch_q(const MmvqParams &p, int n_chan, hipStream_t st) {
    const int npad = (int) host::pad512(p.ncols);
    const size_t lds = (size_t) NC * img_bytes(npad);
    if (lds > 160 * 1024) return host::set_error(host::ERR_SHAPE, "mmvq: ncols %d too large for LDS staging", p.ncols);
    if (p.ncols / 256 * 4 <= 16) {
        hipLaunchKernelGGL((k_mmvq_q<T, 16, NC, GLU>), dim3((unsigned) ((p.nrows + 15) / 16), (unsigned) n_chan),
                           dim3(256), lds, st, p);
    } else {
        hipLaunchKernelGGL((k_mmvq_q<T, 32, NC, GLU>), dim3((unsigned) ((p.nrows + 7) / 8), (unsigned) n_chan),
                           dim3(256), lds, st, p);
    }
    return host::check_launch("mmvq (quarters)");
}

template <int NC, bool GLU> int launch_type(int type, const MmvqParams &p, int n_chan, hipStream_t st) {
    switch (type) {
        case T_Q3_K: return launch_nc<T_Q3_K, NC, GLU>(p, n_chan, st);
        case T_Q4_K: return launch_nc<T_Q4_K, NC, GLU>(p, n_chan, st);
        case T_Q5_K: return launch_nc<T_Q5_K, NC, GLU>(p, n_chan, st);
        case T_Q6_K: return launch_nc<T_Q6_K, NC, GLU>(p, n_chan, st);
        case T_Q8_0: return launch_q<T_Q8_0, NC, GLU>(p, n_chan, st);
        case T_IQ4_XS: return launch_q<T_IQ4_XS, NC, GLU>(p, n_chan, st);
        case T_IQ3_XXS: return launch_q<T_IQ3_XXS, NC, GLU>(p, n_chan, st);
        case T_IQ3_S: return launch_q<T_IQ3_S, NC, GLU>(p, n_chan, st);
        case T_IQ2_S: return launch_q<T_IQ2_S, NC, GLU>(p, n_chan, st);
        default: return host::set_error(host::ERR_TYPE, "mmvq: ggml type %d not supported", type);
    }
}

int check_shape(int type, int64_t ncols, int64_t nrows) {
    if (!host::is_supported(type)) return host::set_error(host::ERR_TYPE, "mmvq: ggml type %d not supported", type);
    if (ncols <= 0 || ncols % 256 || nrows <= 0 || ncols > (1 << 20) || nrows > (1 << 24))
        return host::set_error(host::ERR_SHAPE, "mmvq: ncols %lld must be a positive multiple of 256, nrows %lld > 0",
                               (long long) ncols, (long long) nrows);
    return host::OK;
}

}  // namespace

namespace impl {

int mmvq(int type, const void *w, int64_t ncols, int64_t nrows, const void *xq, float *dst, int64_t n_cols,
         hipStream_t st) {
    FNS_TRY(check_shape(type, ncols, nrows));
    if (!w || !xq || !dst || n_cols < 0) return host::set_error(host::ERR_SHAPE, "mmvq: null buffer");
    const int64_t xrb = host::q8_1_row_bytes(ncols);
    for (int64_t c0 = 0; c0 < n_cols; c0 += 4) {
        const int n = (int) std::min<int64_t>(4, n_cols - c0);
        MmvqParams p{};
        p.base = (const uint8_t *) w;
        p.xq = (const uint8_t *) xq + c0 * xrb;
        p.xq_row_bytes = xrb;
        p.n_xq = 1;
        p.x_div = 1;
        p.ncol_dense = n;
        p.dst = dst + c0 * nrows;
        p.ncols = (int) ncols;
        p.nrows = (int) nrows;
        FNS_TRY(n == 1 ? launch_type<1, false>(type, p, 1, st) : launch_type<4, false>(type, p, 1, st));
    }
    return host::OK;
}

int mmvq_ids(int type, const void *w, int64_t ncols, int64_t nrows, int64_t n_mats, const void *xq, int64_t n_xq,
             const int32_t *ids, int64_t n_ids, float *dst, hipStream_t st) {
    FNS_TRY(check_shape(type, ncols, nrows));
    if (!w || !xq || !ids || !dst || n_mats < 1 || n_xq < 1 || n_ids < 0 || n_ids > 65535)
        return host::set_error(host::ERR_SHAPE, "mmvq_ids: bad arguments");
    if (n_ids == 0) return host::OK;
    MmvqParams p{};
    p.base = (const uint8_t *) w;
    p.mat_stride = nrows * (ncols / 256) * host::kquant_block_bytes(type);
    p.ids = ids;
    p.n_ids = (int) n_ids;
    p.xq = (const uint8_t *) xq;
    p.xq_row_bytes = host::q8_1_row_bytes(ncols);
    p.n_xq = (int) n_xq;
    p.x_div = 1;
    p.dst = dst;
    p.ncols = (int) ncols;
    p.nrows = (int) nrows;
    return launch_type<1, false>(type, p, (int) n_ids, st);
}

int mmvq_swiglu(int type, const void *w_gate, const void *w_up, int64_t ncols, int64_t nrows, const void *xq,
                float *dst, hipStream_t st) {
    FNS_TRY(check_shape(type, ncols, nrows));
    if (!w_gate || !w_up || !xq || !dst) return host::set_error(host::ERR_SHAPE, "mmvq_swiglu: null buffer");
    MmvqParams p{};
    p.base = (const uint8_t *) w_up;
    p.off_b = (const uint8_t *) w_gate - (const uint8_t *) w_up;
    p.xq = (const uint8_t *) xq;
    p.xq_row_bytes = host::q8_1_row_bytes(ncols);
    p.n_xq = 1;
    p.x_div = 1;
    p.ncol_dense = 1;
    p.dst = dst;
    p.ncols = (int) ncols;
    p.nrows = (int) nrows;
    return launch_type<1, true>(type, p, 1, st);
}

int mmvq_ids_swiglu_shared(int type, const void *w_gate, const void *w_up, int64_t ncols, int64_t nrows,
                           int64_t n_mats, const void *xq, const int32_t *ids, int64_t n_ids, float *dst,
                           const void *sh_gate, const void *sh_up, float *sh_dst, hipStream_t st) {
    FNS_TRY(check_shape(type, ncols, nrows));
    if (!w_gate || !w_up || !xq || !ids || !dst || n_mats < 1 || n_ids < 0 || n_ids > 65535)
        return host::set_error(host::ERR_SHAPE, "mmvq_ids_swiglu_shared: bad arguments");
    if (sh_dst && (!sh_gate || !sh_up))
        return host::set_error(host::ERR_SHAPE, "mmvq_ids_swiglu_shared: shared expert needs sh_gate and sh_up");
    MmvqParams p{};
    p.base = (const uint8_t *) w_up;
    p.mat_stride = nrows * (ncols / 256) * host::kquant_block_bytes(type);
    p.off_b = (const uint8_t *) w_gate - (const uint8_t *) w_up;
    p.ids = ids;
    p.n_ids = (int) n_ids;
    if (sh_dst) {
        p.sh_a = (const uint8_t *) sh_up;
        p.sh_b = (const uint8_t *) sh_gate;
        p.sh_dst = sh_dst;
    }
    p.xq = (const uint8_t *) xq;
    p.xq_row_bytes = host::q8_1_row_bytes(ncols);
    p.n_xq = 1;
    p.x_div = 1;
    p.dst = dst;
    p.ncols = (int) ncols;
    p.nrows = (int) nrows;
    const int n_chan = (int) n_ids + (sh_dst ? 1 : 0);
    if (n_chan == 0) return host::OK;
    return launch_type<1, true>(type, p, n_chan, st);
}

int mmvq_experts_swiglu(int type, const char *const *table, size_t gate_off, size_t up_off, int64_t ncols,
                        int64_t nrows, const void *xq, int64_t n_xq, const int32_t *ids, int64_t n_ids, float *dst,
                        hipStream_t st) {
    FNS_TRY(check_shape(type, ncols, nrows));
    if (!table || !xq || !ids || !dst || n_xq < 1 || n_ids < 0 || n_ids > 65535 || (n_ids && n_ids % n_xq))
        return host::set_error(host::ERR_SHAPE, "mmvq_experts_swiglu: bad arguments (n_ids must be a multiple of n_xq)");
    if (n_ids == 0) return host::OK;
    MmvqParams p{};
    p.table = table;
    p.off_a = (int64_t) up_off;
    p.off_b = (int64_t) gate_off;
    p.ids = ids;
    p.n_ids = (int) n_ids;
    p.xq = (const uint8_t *) xq;
    p.xq_row_bytes = host::q8_1_row_bytes(ncols);
    p.n_xq = (int) n_xq;
    p.x_div = (int) (n_ids / n_xq);
    p.dst = dst;
    p.ncols = (int) ncols;
    p.nrows = (int) nrows;
    return launch_type<1, true>(type, p, (int) n_ids, st);
}

int mmvq_experts(int type, const char *const *table, size_t off, int64_t ncols, int64_t nrows, const void *xq,
                 int64_t n_xq, const int32_t *ids, int64_t n_ids, float *dst, hipStream_t st) {
    return mmvq_experts_div(type, table, off, ncols, nrows, xq, n_xq, 1, ids, n_ids, dst, st);
}

int mmvq_experts_div(int type, const char *const *table, size_t off, int64_t ncols, int64_t nrows, const void *xq,
                     int64_t n_xq, int64_t x_div, const int32_t *ids, int64_t n_ids, float *dst, hipStream_t st) {
    FNS_TRY(check_shape(type, ncols, nrows));
    if (!table || !xq || !ids || !dst || n_xq < 1 || x_div < 1 || x_div > 65535 || n_ids < 0 || n_ids > 65535)
        return host::set_error(host::ERR_SHAPE, "mmvq_experts: bad arguments");
    if (n_ids == 0) return host::OK;
    MmvqParams p{};
    p.table = table;
    p.off_a = (int64_t) off;
    p.ids = ids;
    p.n_ids = (int) n_ids;
    p.xq = (const uint8_t *) xq;
    p.xq_row_bytes = host::q8_1_row_bytes(ncols);
    p.n_xq = (int) n_xq;
    p.x_div = (int) x_div;
    p.dst = dst;
    p.ncols = (int) ncols;
    p.nrows = (int) nrows;
    return launch_type<1, false>(type, p, (int) n_ids, st);
}

}  // namespace impl

// ---- C++ API (reference names; abort on error) ----
size_t q8_1_row_bytes(int64_t ncols) { return (size_t) host::q8_1_row_bytes(ncols); }

void mmvq(ggml_type type, const void *w, int64_t ncols, int64_t nrows, const void *xq, float *dst, int64_t n_cols,
          hipStream_t stream) {
    host::abort_on_error(impl::mmvq(type, w, ncols, nrows, xq, dst, n_cols, stream), "mmvq");
}
void mmvq_ids(ggml_type type, const void *w, int64_t ncols, int64_t nrows, int64_t n_mats, const void *xq,
              int64_t n_xq, const int32_t *ids, int64_t n_ids, float *dst, hipStream_t stream) {
    host::abort_on_error(impl::mmvq_ids(type, w, ncols, nrows, n_mats, xq, n_xq, ids, n_ids, dst, stream), "mmvq_ids");
}
void mmvq_swiglu(ggml_type type, const void *w_gate, const void *w_up, int64_t ncols, int64_t nrows, const void *xq,
                 float *dst, hipStream_t stream) {
    host::abort_on_error(impl::mmvq_swiglu(type, w_gate, w_up, ncols, nrows, xq, dst, stream), "mmvq_swiglu");
}
void mmvq_ids_swiglu_shared(ggml_type type, const void *w_gate, const void *w_up, int64_t ncols, int64_t nrows,
                            int64_t n_mats, const void *xq, const int32_t *ids, int64_t n_ids, float *dst,
                            const void *sh_gate, const void *sh_up, float *sh_dst, hipStream_t stream) {
    host::abort_on_error(impl::mmvq_ids_swiglu_shared(type, w_gate, w_up, ncols, nrows, n_mats, xq, ids, n_ids, dst,
                                                      sh_gate, sh_up, sh_dst, stream),
                         "mmvq_ids_swiglu_shared");
}
void mmvq_experts_swiglu(ggml_type type, const char *const *table, size_t gate_off, size_t up_off, int64_t ncols,
                         int64_t nrows, const void *xq, int64_t n_xq, const int32_t *ids, int64_t n_ids, float *dst,
                         hipStream_t stream) {
    host::abort_on_error(impl::mmvq_experts_swiglu(type, table, gate_off, up_off, ncols, nrows, xq, n_xq, ids, n_ids,
                                                   dst, stream),
                         "mmvq_experts_swiglu");
}
void mmvq_experts(ggml_type type, const char *const *table, size_t off, int64_t ncols, int64_t nrows, const void *xq,
                  int64_t n_xq, const int32_t *ids, int64_t n_ids, float *dst, hipStream_t stream) {
    host::abort_on_error(impl::mmvq_experts(type, table, off, ncols, nrows, xq, n_xq, ids, n_ids, dst, stream),
                         "mmvq_experts");
}
bool mmvq_supports(ggml_type type) { return host::is_supported((int) type); }

namespace impl {
// This translation unit's copy of the IQ codebooks (fns_quarter.hpp g_iq_grids), on the current device.
int iq_grids_upload_mmvq(const void *grids) {
    const hipError_t e = dev::upload_iq_grids((const dev::IqGrids *) grids);
    return e == hipSuccess ? host::OK : host::set_error(host::ERR_LAUNCH, "set_iq_grids: %s", hipGetErrorString(e));
}
}  // namespace impl

}  // namespace fns
