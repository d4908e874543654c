// mmq.hip - prefill / batched expert GEMM (MMQ) over GGUF K-quant weights for MI355X gfx950: expert-id compaction,
// split Q8_1 activation images, and an f16-MFMA grouped GEMM with the SwiGLU + Q8_1 of act fused into the gate/up pass.
//
// Reference semantics: src/ggml/ggml_mmq.cu:74-129 (mmq_q8_1_bytes, mmq, mmq_experts: mm_ids_helper sorts the
// (token, slot) pairs by expert, the activations are quantised once per source row, the GEMM writes each row back to
// its (token, slot) position), include/fns/ggml_kernels.h:50-69. This is a new CDNA4 design, not ggml's mmq.cuh:
//
//   * The K-quant scales change every 32 (Q4_K, Q5_K) or 16 (Q6_K, Q3_K) columns and the Q8_1 scale d8 every 32, so an
//     int8 MFMA per sub-block needs a convert + scale + add per output element per sub-block: VALU-bound. Here the
//     scales are folded into the operands instead, exactly: A = q8 * d8 as two f16 halves (hi + lo, see the image
//     layout below), B = integer code * integer sub-block scale as f16 (|B| <= 2048: exact; Q6_K's 8-bit scales are
//     split in two operands). v_mfma_f32_32x32x16_f16 then accumulates a whole 256-column superblock, and only the
//     superblock's float scales d (and dmin times one more MFMA of the min term) touch the accumulators.
//     Every product is exact; the sums are fp32.
//   * A = 32 activation rows (tokens) x 16 columns, B = 16 columns x 32 weight rows: the lane that owns output
//     (token i, weight row j) holds weight row j = lane % 32 for 16 tokens and decodes row j's codes and scales
//     itself. The 32x32 shape moves half the operand bytes (LDS reads, decode VALU) per product of the 16x16 one.
//   * A workgroup (4 waves) owns two 32-row weight streams per wave - gate and up of the same 128 rows (GLU), or 256
//     rows - and up to 64 of the expert's routed activation rows (2 tiles of 32): each weight byte is read from HBM
//     once per 64 routed rows. Activations are staged per half superblock in LDS by LDS-DMA, double-buffered (66 KB:
//     two workgroups per CU); weights go straight to VGPRs, half a superblock ahead.
//   * Gate/up: both matrices in one pass, then act = up * silu(gate) and its Q8_1 blocks (32 consecutive rows = 32
//     consecutive act columns) written straight into the split image rows the down pass reads.
//
// Outputs match the float64 oracle (oracle/fns_oracle.c) on the same Q8_1 activations within the fp32 tolerance of
// the tests.
#include <algorithm>
#include "fns_block.hpp"
#include "fns_common.hpp"
#include "fns_host.hpp"
#include "fns_internal.hpp"
#include "fns_lanes.hpp"
#include "fns_quarter.hpp"
#include "fns_router_gemm.hpp"

#include "fns/ggml_kernels.h"

namespace fns {

using namespace fns::dev;

namespace {

constexpr int kMmqThreads = 256;   // 4 waves
constexpr int kMmqWaves = kMmqThreads / 64;
constexpr int kMmqRows = 64;       // row granularity of the weight matrices
constexpr int kMmqTok = 64;        // activation rows per workgroup (2 MFMA tiles of 32)
constexpr int kCompactThreads = 1024;

// ---- scratch layout of the expert path --------------------------------------------------------------------------
// bounds[n_expert + 1] (sorted-row offset of each expert); the GEMM's group prefixes gprefix[2][n_expert + 1]: the
// 64-row groups of each expert (n_e / 64 full ones, and the remainder if it is > 32 rows; two 32-row MFMA tiles), and
// the remainder groups of <= 32 rows (one tile).
inline size_t bounds_bytes(int64_t n_expert) { return (size_t) 3 * (n_expert + 1) * 4; }
inline size_t gprefix_bytes(int64_t n_expert) { return (size_t) 2 * (n_expert + 1) * 4; }

// ---- compaction (ggml mm_ids_helper semantics, stable) ------------------------------------------------------------
// ids [n_tok][k] -> pairs p = t k + j sorted by expert, ties in p order: ids_dst[q] = p, ids_src1[q] = the activation
// row of p (t when x_rows_per_tok = 1, p when x_rows_per_tok = k), bounds[e] = first sorted position of expert e.
// One workgroup; wave w owns a contiguous chunk of the pairs (its first 8 ids per lane kept in registers): per-wave
// histograms (LDS atomics), one prefix over (expert, wave) in that order, then each wave walks its chunk again in
// order, ranking the lanes that share an expert by ballots on the expert id bits, and advances its own running
// positions - two passes over the ids, four barriers.
// Workgroup barrier for LDS data only: no global memory is produced and consumed inside the compaction kernel, so its
// barriers need not wait for the id loads and the output stores still in flight (__syncthreads' fence would).
__device__ __forceinline__ void lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// Exclusive prefix of the per-expert counts cnt[0..ne) (ne <= 256) by one wave (lane = its lane): cnt[e] becomes the
// expert's first sorted position; bounds[0..ne], and the group prefixes gprefix[0..ne] of the 64-row groups
// (n_e / 64 full ones, and the remainder if it is > 32 rows) and gprefix[ne + 1 .. 2 ne + 1] of the <= 32-row
// remainders are written. 4 experts per lane, then a lane scan.
__device__ __forceinline__ void expert_prefix_wave(int lane, int *cnt, int ne, int32_t *bounds, int32_t *gprefix) {
    int v[4], g[4], g2[4], s = 0, sg = 0, sg2 = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = 4 * lane + j, r = (e < ne ? cnt[e] : 0) % kMmqTok;
        v[j] = e < ne ? cnt[e] : 0;
        g[j] = v[j] / kMmqTok + (r > kMmqTok / 2);
        g2[j] = r > 0 && r <= kMmqTok / 2;
        s += v[j];
        sg += g[j];
        sg2 += g2[j];
    }
    int incl = s, inclg = sg, inclg2 = sg2;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(incl, o, 64), tg = __shfl_up(inclg, o, 64), tg2 = __shfl_up(inclg2, o, 64);
        if (lane >= o) {
            incl += t;
            inclg += tg;
            inclg2 += tg2;
        }
    }
    int run = incl - s, rung = inclg - sg, rung2 = inclg2 - sg2;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = 4 * lane + j;
        if (e < ne) {
            cnt[e] = run;  // the expert's first sorted position (its count is no longer needed)
            bounds[e] = run;
            gprefix[e] = rung;
            gprefix[ne + 1 + e] = rung2;
        }
        run += v[j];
        rung += g[j];
        rung2 += g2[j];
    }
    if (lane == 63) {
        bounds[ne] = incl;
        gprefix[ne] = inclg;
        gprefix[2 * ne + 1] = inclg2;
    }
}

__global__ __launch_bounds__(kCompactThreads) void k_mmq_compact(const int32_t *__restrict__ ids, int n, int k, int ne,
                                                                 int x_rows_per_tok, int32_t *__restrict__ ids_src1,
                                                                 int32_t *__restrict__ ids_dst, int32_t *bounds,
                                                                 int32_t *gprefix, int32_t *gdone, int n_gdone) {
    constexpr int NW = kCompactThreads / kWave;
    __shared__ int cnt[256];
    __shared__ int wpos[NW][256];  // per-wave counts, then each wave's next sorted position per expert
    PF_MARK(2, 0);
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    for (int i = tid; i < NW * 256; i += kCompactThreads) (&wpos[0][0])[i] = 0;
    for (int i = tid; i < n_gdone; i += kCompactThreads) gdone[i] = 0;  // the next fused GEMM launch's arrivals
    lds_sync();
    PF_MARK(2, 2);
    const int chunk = (n + NW * kWave - 1) / (NW * kWave) * kWave;  // pairs per wave, a multiple of 64
    const int p0 = wave * chunk, p1 = min(n, p0 + chunk);
    // the first kCache ids of each lane stay in registers for the second pass; their loads are clamped into the
    // array and unconditional (under the uniform n > 0: an empty batch still writes the bounds), so they are all in
    // flight together
    constexpr int kCache = 8;
    int ev[kCache];
#pragma unroll
    for (int it = 0; it < kCache; ++it) {
        const int p = p0 + lane + kWave * it;
        const int v = n > 0 ? ids[min(p, n - 1)] : -1;
        ev[it] = kWave * it < chunk && p < p1 ? v : -1;
    }
    auto id_at = [&](int p) { return p < p1 ? ids[p] : -1; };
#pragma unroll
    for (int it = 0; it < kCache; ++it) {
        const int e = ev[it];
        if (e >= 0 && e < ne) atomicAdd(&wpos[wave][e], 1);
    }
    for (int p = p0 + lane + kWave * kCache; p < p0 + chunk; p += kWave) {  // wave-uniform trip count
        const int e = id_at(p);
        if (e >= 0 && e < ne) atomicAdd(&wpos[wave][e], 1);
    }
    lds_sync();
    PF_MARK(2, 3);
    if (tid < ne) {
        int c = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) c += wpos[w][tid];
        cnt[tid] = c;
    }
    lds_sync();
    PF_MARK(2, 4);
    if (wave == 0) expert_prefix_wave(lane, cnt, ne, bounds, gprefix);
    lds_sync();
    PF_MARK(2, 5);
    if (tid < ne) {  // the expert's sorted positions, split over the waves in wave order
        int pos = cnt[tid];
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const int c = wpos[w][tid];
            wpos[w][tid] = pos;
            pos += c;
        }
    }
    lds_sync();
    PF_MARK(2, 6);
    for (int it = 0, p = p0 + lane; p < p0 + chunk; ++it, p += kWave) {
        int e = -1;
#pragma unroll
        for (int c = 0; c < kCache; ++c)
            if (it == c) e = ev[c];
        if (it >= kCache) e = id_at(p);
        const bool live = e >= 0 && e < ne;
        // lanes with the same expert id: intersect the ballots of each id bit (and of liveness)
        uint64_t same = __ballot(live);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const uint64_t m = __ballot(live && ((e >> b) & 1));
            same &= ((e >> b) & 1) ? m : ~m;
        }
        if (!live) same = 0;
        const int rank = __popcll(same & ((1ull << lane) - 1ull));
        if (live) {
            const int pos = wpos[wave][e] + rank;
            ids_dst[pos] = p;
            ids_src1[pos] = x_rows_per_tok == 1 ? p / k : p;
        }
        // (this wave's reads above complete before its write below: one wave, LDS accesses in order)
        if (live && rank == 0) wpos[wave][e] += __popcll(same);
    }
    PF_MARK(2, 1);
}

// ---- split activation images --------------------------------------------------------------------------------------
// The GEMM's A operand is the Q8_1 activation q8 * d8 as an exact pair of halves (hi = f16(q8 d8), lo = f16(q8 d8 - hi):
// a 7-bit integer times an f16 scale has at most 18 significant bits, two halves hold 22). Row layout, per 256-column
// superblock kb: 1024 bytes at kb * 1024, two 128-column halves of [hi 128 f16][lo 128 f16]; then at nb * 1024 + 32 kb
// the min-term sums [S_hi 8 f16][S_lo 8 f16], S_s = d8_s * sum(q8 of sub-block s). Within every 8 columns (and every
// 4 sums) the stored order is 0 2 1 3 4 6 5 7: the order in which the weight decoders below emit their B operand.
// Magnitudes are those of the reference's f16 Q8_1 fields (|q8 d8| <= amax, S within the f16 sum's range).
constexpr int kSbMain = 1024, kSbMin = 32;
__host__ __device__ constexpr int64_t split_row_bytes(int64_t ncols) { return ncols / 256 * (kSbMain + kSbMin); }
__device__ __forceinline__ int perm8(int k) { return (k & ~3) | ((k & 1) << 1) | ((k >> 1) & 1); }

// Q8_1 of 8 consecutive values per lane, 4 lanes per 32-value block (lanes 4j .. 4j + 3 of a quad, all active), into
// the split image row `row` at column col (a multiple of 8): d = amax / 127, q = roundf(v / d) - with an IEEE
// division per value (EXACT: the reference's arithmetic, bit for bit) or v * (1 / d). The max and the integer sum are
// exact in any order. Returns nothing; lane q = 0 of the block also stores its min-term sums.
struct Q8Split {
    _Float16 hi[8], lo[8];  // in the stored order
    _Float16 shi, slo;      // the block's min-term sum (lane q = 0 of the block stores it)
};
template <bool EXACT>
__device__ __forceinline__ Q8Split q8_split8_vals(const float (&v)[8]) {
    Q8Split r;
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) amax = fmaxf(amax, fabsf(v[k]));
    amax = lanes_max<4>(amax);
    const float d = amax / 127.0f;
    const float dh = half_to_float(float_to_half(d));
    const float id = amax == 0.0f ? 0.0f : 1.0f / d;
    int qsum = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int qk = amax == 0.0f ? 0 : (int) (int8_t) roundf(EXACT ? v[k] / d : v[k] * id);
        qsum += qk;
        const float x = (float) qk * dh;  // exact
        const _Float16 h = (_Float16) x;
        r.hi[perm8(k)] = h;
        r.lo[perm8(k)] = (_Float16) (x - (float) h);
    }
    qsum = lanes_sum_i<4>(qsum);
    const float sv = dh * (float) qsum;  // exact in fp32
    r.shi = (_Float16) sv;
    r.slo = (_Float16) (sv - (float) r.shi);
    return r;
}
// byte offsets within an image row of the 8 columns at col (hi; lo at + 256) and of the block's min-term sums (hi;
// lo at + 16)
__device__ __forceinline__ uint32_t img_col_off(int col) {
    return (uint32_t) ((col >> 8) * kSbMain + ((col >> 7) & 1) * 512 + ((col & 127) >> 3) * 16);
}
__device__ __forceinline__ uint32_t img_sum_off(int ncols, int col) {
    return (uint32_t) ((ncols >> 8) * kSbMain + (col >> 8) * kSbMin + 2 * perm8((col >> 5) & 7));
}
template <bool EXACT>
__device__ __forceinline__ void q8_split8(const float (&v)[8], uint8_t *row, int ncols, int col, bool store) {
    const Q8Split r = q8_split8_vals<EXACT>(v);
    if (!store) return;
    uint8_t *o = row + img_col_off(col);
    *(uint4 *) o = __builtin_bit_cast(uint4, r.hi);
    *(uint4 *) (o + 256) = __builtin_bit_cast(uint4, r.lo);
    if ((col & 31) == 0) {
        _Float16 *m = (_Float16 *) (row + img_sum_off(ncols, col));
        m[0] = r.shi;
        m[8] = r.slo;
    }
}

// x [rows][ncols] f32 -> split image rows with the reference's Q8_1 arithmetic; grid (ceil(ncols / 2048), rows), 256
// threads of 8 columns each (ncols % 256 == 0, so a block's 4 lanes are all in or all out).
__global__ __launch_bounds__(256) void k_quant_image(const float *__restrict__ x, int ncols, uint8_t *__restrict__ out,
                                                     int64_t img_row_bytes) {
    const int row = blockIdx.y, col = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (col >= ncols) return;
    const float *src = x + (size_t) row * ncols + col;
    const float4 x0 = *(const float4 *) src, x1 = *(const float4 *) (src + 4);
    const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    q8_split8<true>(v, out + (size_t) row * img_row_bytes, ncols, col, true);
}

// F16-guard form: only the rows whose guard scale is not 1 are re-quantised (the others already hold the image of
// the same values, written by the GEMM epilogue); grid as k_quant_image.
__global__ __launch_bounds__(256) void k_quant_image_scaled(const float *__restrict__ x, const float *__restrict__ escale,
                                                            int ncols, uint8_t *__restrict__ out, int64_t img_row_bytes) {
    const int row = blockIdx.y, col = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (escale[row] == 1.0f || col >= ncols) return;
    const float *src = x + (size_t) row * ncols + col;
    const float4 x0 = *(const float4 *) src, x1 = *(const float4 *) (src + 4);
    const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    q8_split8<true>(v, out + (size_t) row * img_row_bytes, ncols, col, true);
}

// Router GEMM tiles and the split activation image of the same rows in one launch (the two only read x): workgroups
// [0, n_rt) are router tiles (tile (id % tiles_x, id / tiles_x)), the rest quantise two 2048-column pieces of x each,
// as k_quant_image does, so the image is built on the CUs the router tiles leave free.
template <bool BF16>
__global__ __launch_bounds__(512) void k_router_image(const void *__restrict__ w, const float *__restrict__ bias,
                                                      const float *__restrict__ x, float *__restrict__ y, int ncols,
                                                      int nrows, int n_tok, int tiles_x, int n_rt,
                                                      uint8_t *__restrict__ img, int64_t img_row_bytes, int nxb) {
    PF_MARK(0, 0);
    const int id = blockIdx.x;
    if (id < n_rt) {
        router_gemm_tile<BF16, true>(w, bias, x, y, ncols, nrows, n_tok, id % tiles_x, id / tiles_x);
        PF_MARK(0, 1);
        return;
    }
    const int item = 2 * (id - n_rt) + (int) threadIdx.x / 256;
    const int row = item / nxb, col = ((item % nxb) * 256 + (int) threadIdx.x % 256) * 8;
    if (item < nxb * n_tok && col < ncols) {
        const float *src = x + (size_t) row * ncols + col;
        const float4 x0 = *(const float4 *) src, x1 = *(const float4 *) (src + 4);
        const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        q8_split8<true>(v, img + (size_t) row * img_row_bytes, ncols, col, true);
    }
    PF_MARK(0, 1);
}

// ---- grouped GEMM -------------------------------------------------------------------------------------------------
struct MmqArgs {
    const char *const *table;  // expert pointer table (null: dense, w_dense)
    const uint8_t *w_dense;
    int64_t off_a, off_b;      // byte offsets of the (gate) matrix and of the up matrix (GLU)
    int ncols, nrows;          // K (columns of W) and N (rows of W)
    int n_expert;
    const uint8_t *xpack;      // split activation image rows
    int64_t x_img;             // bytes per activation image row
    const int32_t *bounds;     // [n_expert + 1] (null: dense)
    const int32_t *gprefix;    // [2][n_expert + 1] group prefixes: 64-row groups, then the <= 32-row remainders
    int n_main;                // launch: groups of the 64-row list (then the remainder list up to n_groups)
    int n_groups, n_cb;        // launch: groups in both lists; weight row blocks per group
    const int32_t *src;        // sorted position -> activation image row (null: identity)
    const int32_t *dst_rows;   // sorted position -> output row (null: identity)
    int n_rows;                // dense: number of activation rows
    int dense_small;           // dense: 1 = groups of 32 activation rows (one tile), 0 = of 64
    int ksplit;                // dense, non-GLU: > 1 = the K range split into ksplit parts (blockIdx.y), part p's
    int64_t part_stride;       //   partial sums written at dst + p * part_stride floats
    float *dst;                // [out row][nrows] f32 (non-GLU)
    uint8_t *out_pack;         // GLU: act split image rows (by output row)
    int64_t out_img;
    float *act_out;            // GLU: optional f32 act [out row][nrows]
    int *gdone;                // fused launch: per-group arrival counts (zeroed by the compaction kernel)
    int gwait;                 // fused launch: arrivals a down item waits for (its group's gate/up items)
    int spin_limit;            // fused launch: polls before a down item gives up (its outputs are then NaN)
    uint32_t *status;          // fused launch: sticky status word, kStatusTimeout once a wait gave up
};

// Weight fragments of one 256-value block for one lane: the header (scales, d) and the codes of column groups
// kg = 2 h and 2 h + 1 (h = lane / 32) of every sub-block - 16 contiguous bytes per code array, one load each.
template <int T> struct WFrag;
template <> struct WFrag<T_Q4_K> { uint4 h; uint4 q[4]; };
template <> struct WFrag<T_Q5_K> { uint4 h; uint4 q[4]; uint4 qh; };
template <> struct WFrag<T_Q6_K> { uint4 ql[4]; uint4 qh[2]; uint4 sc; uint32_t d; };
template <> struct WFrag<T_Q3_K> { uint4 qs[2]; uint4 hm; uint4 tail; };
// Q8_0 (8 blocks of 34 bytes per 256 values): the 16 code bytes of column groups 2 h, 2 h + 1 and the f16 d of
// every block (low 16 bits)
template <> struct WFrag<T_Q8_0> { uint4 q[8]; uint32_t d[8]; };
// IQ formats (lane half h, its two column groups of every 32-value sub-block; see decode):
//   IQ4_XS : header (d, scales_h, scales_l) and qs bytes 8 h .. 8 h + 7 of each sub-block
//   IQ3_XXS: d, index bytes 4 h .. 4 h + 3 of each sub-block, the sub-block's aux word (signs, scale)
//   IQ3_S  : d, qh (8 bytes), scales (4 bytes), index bytes 4 h .. 4 h + 3 and sign bytes 2 h, 2 h + 1 per sub-block
//   IQ2_S  : d, qh, scales, the 16 index bytes and 16 sign bytes of each half block (lanes use 2 of every 4)
template <> struct WFrag<T_IQ4_XS> { uint2 h; uint2 q[8]; };
template <> struct WFrag<T_IQ3_XXS> { uint32_t d; uint32_t idx[8]; uint4 aux[2]; };
template <> struct WFrag<T_IQ3_S> { uint32_t d, sc; uint2 qh; uint32_t idx[8], sg[8]; };
template <> struct WFrag<T_IQ2_S> { uint32_t d; uint2 qh, sc; uint4 idx[2], sg[2]; };

// Buffer loads: a uniform base in a resource (SGPRs), a 32-bit per-lane offset and a uniform offset - no 64-bit
// address arithmetic per load. (Unaligned dword access is enabled on the platform, as for the plain global loads.)
typedef __amdgpu_buffer_rsrc_t Rsrc;
__device__ __forceinline__ Rsrc rsrc_of(const void *base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, 0x7FFFFFFF, 0x00020000);
}
__device__ __forceinline__ uint4 bload16(Rsrc r, uint32_t vo, uint32_t so) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint2 bload8(Rsrc r, uint32_t vo, uint32_t so) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, vo, so, 0);
    return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ uint32_t bload4(Rsrc r, uint32_t vo, uint32_t so) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, vo, so, 0);
}
__device__ __forceinline__ uint32_t bload2(Rsrc r, uint32_t vo, uint32_t so) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, vo, so, 0);
}

// Part P (compile time) of the fragment of the block at (vo + so) from r; vc = vo + 16 h selects the lane's code
// bytes. Part 0: the header and the codes of sub-blocks 0-3; part 1: the codes of sub-blocks 4-7.
template <int T, int P>
__device__ __forceinline__ void wfrag_load(Rsrc r, uint32_t vo, uint32_t vc, uint32_t so, WFrag<T> &f) {
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        constexpr int qoff = T == T_Q4_K ? 16 : 48;
        if constexpr (P == 0) {
            f.h = bload16(r, vo, so);
            if constexpr (T == T_Q5_K) f.qh = bload16(r, vc, so + 16);
        }
#pragma unroll
        for (int g = 2 * P; g < 2 * P + 2; ++g) f.q[g] = bload16(r, vc, so + qoff + 32 * g);
    } else if constexpr (T == T_Q6_K) {
        f.ql[2 * P] = bload16(r, vc, so + 64 * P);
        f.ql[2 * P + 1] = bload16(r, vc, so + 64 * P + 32);
        f.qh[P] = bload16(r, vc, so + 128 + 32 * P);
        if constexpr (P == 0) {
            f.sc = bload16(r, vo, so + 192);
            f.d = __builtin_amdgcn_raw_buffer_load_b16(r, vo, so + 208, 0);
        }
    } else if constexpr (T == T_Q3_K) {
        if constexpr (P == 0) {
            f.hm = bload16(r, vc, so);
            f.tail = bload16(r, vo, so + 94);  // scales[12] at +2, d at +14
        }
        f.qs[P] = bload16(r, vc, so + 32 + 32 * P);
    } else if constexpr (T == T_Q8_0) {  // block s at 34 s: d @0, qs @2 (vc - vo = 16 h selects the lane's 16 bytes)
#pragma unroll
        for (int b = 4 * P; b < 4 * P + 4; ++b) {
            f.q[b] = bload16(r, vc, so + 34 * b + 2);
            f.d[b] = bload2(r, vo, so + 34 * b);
        }
    } else if constexpr (T == T_IQ4_XS) {  // d @0, scales_h @2, scales_l @4, qs @8 (16 per sub-block)
        const uint32_t vq = vo + ((vc - vo) >> 1);  // + 8 h
        if constexpr (P == 0) f.h = bload8(r, vo, so);
#pragma unroll
        for (int ib = 4 * P; ib < 4 * P + 4; ++ib) f.q[ib] = bload8(r, vq, so + 8 + 16 * ib);
    } else if constexpr (T == T_IQ3_XXS) {  // d @0, index bytes @2 (8 per sub-block), aux words @66
        const uint32_t vq = vo + ((vc - vo) >> 2);  // + 4 h
        if constexpr (P == 0) f.d = bload2(r, vo, so);
#pragma unroll
        for (int ib = 4 * P; ib < 4 * P + 4; ++ib) f.idx[ib] = bload4(r, vq, so + 2 + 8 * ib);
        f.aux[P] = bload16(r, vo, so + 66 + 16 * P);
    } else if constexpr (T == T_IQ3_S) {  // d @0, qs @2 (8 per sub-block), qh @66, signs @74 (4 per sub-block), scales @106
        const uint32_t vq = vo + ((vc - vo) >> 2), vs = vo + ((vc - vo) >> 3);  // + 4 h, + 2 h
        if constexpr (P == 0) {
            f.d = bload2(r, vo, so);
            f.qh = bload8(r, vo, so + 66);
            f.sc = bload4(r, vo, so + 106);
        }
#pragma unroll
        for (int ib = 4 * P; ib < 4 * P + 4; ++ib) {
            f.idx[ib] = bload4(r, vq, so + 2 + 8 * ib);
            f.sg[ib] = bload2(r, vs, so + 74 + 4 * ib);
        }
    } else {  // IQ2_S: d @0, index bytes @2 (4 per sub-block), sign bytes @34 (4 per sub-block), qh @66, scales @74
        if constexpr (P == 0) {
            f.d = bload2(r, vo, so);
            f.qh = bload8(r, vo, so + 66);
            f.sc = bload8(r, vo, so + 74);
        }
        f.idx[P] = bload16(r, vo, so + 2 + 16 * P);
        f.sg[P] = bload16(r, vo, so + 34 + 16 * P);
    }
}
// vector loads issued by part P of wfrag_load for one stream
template <int T, int P> constexpr int wfrag_loads() {
    return T == T_Q4_K    ? (P ? 2 : 3)
           : T == T_Q5_K  ? (P ? 2 : 4)
           : T == T_Q6_K  ? (P ? 3 : 5)
           : T == T_Q3_K  ? (P ? 1 : 3)
           : T == T_Q8_0  ? 8
           : T == T_IQ4_XS ? (P ? 4 : 5)
           : T == T_IQ3_XXS ? (P ? 5 : 6)
           : T == T_IQ3_S ? (P ? 8 : 11)
                          : (P ? 2 : 5);  // IQ2_S
}
// the 8 code bytes of column group 2 h + p (p compile time) from a 16-byte code array
__device__ __forceinline__ uint2 half8(const uint4 &v, int p) { return p ? make_uint2(v.z, v.w) : make_uint2(v.x, v.y); }

typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ uint32_t as_u(h2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ h2 splat(_Float16 v) { return h2{v, v}; }
// bytes b0..b3 (< 1024 each) of w -> halves (1024 + b0, 1024 + b2) and (1024 + b1, 1024 + b3): 0x6400 is 1024.0
__device__ __forceinline__ h2 biased02(uint32_t w) { return as_h2(__builtin_amdgcn_perm(0x64646464u, w, 0x04020400u)); }
__device__ __forceinline__ h2 biased13(uint32_t w) { return as_h2(__builtin_amdgcn_perm(0x64646464u, w, 0x04030401u)); }
__device__ __forceinline__ h2 fma2(h2 a, h2 b, h2 c) { return __builtin_elementwise_fma(a, b, c); }
__device__ __forceinline__ v8h cat4(h2 a, h2 b, h2 c, h2 d) {
    return __builtin_bit_cast(v8h, make_uint4(as_u(a), as_u(b), as_u(c), as_u(d)));
}
// codes bytes (x = columns 0-3, y = columns 4-7 of the lane) times a scale: exact products (|code * scale| <= 2048)
__device__ __forceinline__ v8h scaled8(uint32_t x, uint32_t y, h2 sc, h2 bias) {  // (1024 + c) sc + bias, bias = -1024 sc
    return cat4(fma2(biased02(x), sc, bias), fma2(biased13(x), sc, bias), fma2(biased02(y), sc, bias),
                fma2(biased13(y), sc, bias));
}
__device__ __forceinline__ v8h centred8(uint32_t x, uint32_t y, h2 off, h2 sc) {  // ((1024 + c) - off) * sc
    return cat4((biased02(x) - off) * sc, (biased13(x) - off) * sc, (biased02(y) - off) * sc,
                (biased13(y) - off) * sc);
}

// B operand(s) of sub-block s, column group kg = 2 h + p (s, p compile time) for this lane: B[k][row] = integer code x
// integer scale as f16 (Q6_K: two operands, scale split as 16 (sc >> 4) + (sc & 15), each product exact). The block's
// float scale d (and dmin) are applied per superblock. on = (d != 0): a block with d = 0 contributes d * (...) = 0
// whatever its codes.
template <int T> constexpr int kNumB = T == T_Q6_K || T == T_IQ4_XS || T == T_Q8_0 ? 2 : 1;
template <int T> struct BOp { v8h b[kNumB<T>]; };
template <int T>
__device__ __forceinline__ BOp<T> decode(const WFrag<T> &f, int s, int p, int h, bool on, const uint32_t *grid);

// (sc_s, sc_s) as f16 and its bias -1024 sc_s for sub-block s (compile time) of a Q4_K / Q5_K block; on = 0: zeros.
// The 6-bit scales are unpacked four at a time (ggml get_scale_min_k4), byte s placed twice next to 0x64 (1024.0).
__device__ __forceinline__ void k4_scale2(const uint4 &h, int s, bool on, h2 &s2, h2 &bias) {
    const uint32_t w = s < 4 ? (h.y & 0x3F3F3F3Fu) : ((h.w & kLo4) | ((h.y >> 2) & 0x30303030u));
    const uint32_t i = (uint32_t) (s & 3);
    s2 = as_h2(__builtin_amdgcn_perm(0x64646464u, on ? w : 0u, 0x04000400u | (i << 16) | i)) - splat((_Float16) 1024.0f);
    bias = s2 * splat((_Float16) -1024.0f);
}
template <> __device__ __forceinline__ BOp<T_Q4_K> decode<T_Q4_K>(const WFrag<T_Q4_K> &f, int s, int p, int, bool on, const uint32_t *) {
    const uint2 q = half8(f.q[s >> 1], p);
    const int sh = 4 * (s & 1);
    h2 s2, bias;
    k4_scale2(f.h, s, on, s2, bias);
    BOp<T_Q4_K> r;
    r.b[0] = scaled8((q.x >> sh) & kLo4, (q.y >> sh) & kLo4, s2, bias);
    return r;
}
template <> __device__ __forceinline__ BOp<T_Q5_K> decode<T_Q5_K>(const WFrag<T_Q5_K> &f, int s, int p, int, bool on, const uint32_t *) {
    const uint2 q = half8(f.q[s >> 1], p), qh = half8(f.qh, p);
    const int sh = 4 * (s & 1);
    h2 s2, bias;
    k4_scale2(f.h, s, on, s2, bias);
    BOp<T_Q5_K> r;
    r.b[0] = scaled8(((q.x >> sh) & kLo4) | (((qh.x >> s) & 0x01010101u) << 4),
                     ((q.y >> sh) & kLo4) | (((qh.y >> s) & 0x01010101u) << 4), s2, bias);
    return r;
}
// Q6_K sub-block s: n = s / 4, qq = s % 4: ql[64 n + 32 (qq & 1) + l] nibble qq >> 1, qh[32 n + l] bits 2 qq,
// value - 32; int8 scale of group 8 n + 2 qq + (l >= 16), i.e. + h for column groups 2 h, 2 h + 1.
template <> __device__ __forceinline__ BOp<T_Q6_K> decode<T_Q6_K>(const WFrag<T_Q6_K> &f, int s, int p, int h, bool on, const uint32_t *) {
    const int n = s >> 2, qq = s & 3;
    const uint2 ql = half8(f.ql[2 * n + (qq & 1)], p), qh = half8(f.qh[n], p);
    const int shl = 4 * (qq >> 1), shh = 2 * qq;
    const uint32_t x = ((ql.x >> shl) & kLo4) | (((qh.x >> shh) & 0x03030303u) << 4);
    const uint32_t y = ((ql.y >> shl) & kLo4) | (((qh.y >> shh) & 0x03030303u) << 4);
    const int g0 = 8 * n + 2 * qq;  // even: both groups in one word
    const uint32_t w0 = word(f.sc, g0 >> 2);
    const int sc = on ? (int) (int8_t) ((w0 >> (8 * ((g0 & 3) + h))) & 0xffu) : 0;
    const h2 off = splat((_Float16) 1056.0f);
    BOp<T_Q6_K> r;
    r.b[0] = centred8(x, y, off, splat((_Float16) (16 * (sc >> 4))));
    r.b[1] = centred8(x, y, off, splat((_Float16) (sc & 15)));
    return r;
}
// Q3_K sub-block s: n = s / 4, j = s % 4: qs[32 n + l] bits 2 j, hmask[l] bit 4 n + j (clear: -4); scale groups
// 8 n + 2 j + (l >= 16), 6-bit value - 32 (low nibbles in scales[0..7], high bit pairs in scales[8..11]).
template <> __device__ __forceinline__ BOp<T_Q3_K> decode<T_Q3_K>(const WFrag<T_Q3_K> &f, int s, int p, int h, bool on, const uint32_t *) {
    const int n = s >> 2, j = s & 3;
    const uint2 q = half8(f.qs[n], p), hm = half8(f.hm, p);
    const int hs = 4 * n + j;
    const uint32_t x = ((q.x >> (2 * j)) & 0x03030303u) | (((hm.x >> hs) & 0x01010101u) << 2);
    const uint32_t y = ((q.y >> (2 * j)) & 0x03030303u) | (((hm.y >> hs) & 0x01010101u) << 2);
    // tail = block bytes 94..109: scales[i] is tail byte 2 + i
    const uint32_t hi_w = (f.tail.z >> 16) | (f.tail.w << 16);  // scales[8..11]
    int scv[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int g = 8 * n + 2 * j + u;
        const int lb = (g & 7) + 2;  // tail byte of scales[g & 7]
        const uint32_t lw = lb < 4 ? f.tail.x : lb < 8 ? f.tail.y : f.tail.z;
        const uint32_t b = (lw >> (8 * (lb & 3))) & 0xffu;
        const uint32_t lo4 = g < 8 ? (b & 0xFu) : (b >> 4);
        const uint32_t hi2 = (((hi_w >> (8 * (g & 3))) & 0xffu) >> (2 * (g >> 2))) & 3u;
        scv[u] = (int) (lo4 | (hi2 << 4)) - 32;
    }
    const int sc = on ? (h == 0 ? scv[0] : scv[1]) : 0;
    BOp<T_Q3_K> r;
    r.b[0] = centred8(x, y, splat((_Float16) 1028.0f), splat((_Float16) sc));
    return r;
}

// IQ formats: B = signed codebook value x integer sub-block scale, exact in f16 (|B| <= 2048, or split in two
// operands), the rest of the float scale in blk_d: IQ4_XS kv * (ls - 32) (split as 4 (s >> 2) + (s & 3)) with d;
// IQ3_XXS g * (2 ls + 1) with d / 4; IQ3_S g * (2 sc + 1) with d; IQ2_S g * (2 ls + 1) with d / 8 - the products of
// the dequantisers' scales (ggml-quants.c dequantize_row_iq*). Codebook entries come from the LDS copy `grid` of the
// format's table. Signed values are biased by 128 (byte ^ 0x80) for the 1024 + byte conversion.
__device__ __forceinline__ v8h signed_scaled8(uint32_t x, uint32_t y, int sc, bool on) {  // x, y: 4 int8 each
    const _Float16 s = (_Float16) (on ? sc : 0);
    return scaled8(x ^ 0x80808080u, y ^ 0x80808080u, splat(s), splat((_Float16) -1152.0f * s));
}
template <> __device__ __forceinline__ BOp<T_IQ4_XS> decode<T_IQ4_XS>(const WFrag<T_IQ4_XS> &f, int s, int p, int,
                                                                      bool on, const uint32_t *) {
    // column group p: the low (p = 0) or high (p = 1) nibbles of the lane's 8 bytes, values 8 h .. 8 h + 7 (+ 16 p)
    const uint32_t x = iq4nl_values((f.q[s].x >> (4 * p)) & kLo4), y = iq4nl_values((f.q[s].y >> (4 * p)) & kLo4);
    const int ls = (int) (((f.h.y >> (4 * s)) & 0xfu) | (((f.h.x >> (16 + 2 * s)) & 3u) << 4)) - 32;
    BOp<T_IQ4_XS> r;
    r.b[0] = signed_scaled8(x, y, 4 * (ls >> 2), on);
    r.b[1] = signed_scaled8(x, y, ls & 3, on);
    return r;
}
template <> __device__ __forceinline__ BOp<T_IQ3_XXS> decode<T_IQ3_XXS>(const WFrag<T_IQ3_XXS> &f, int s, int p, int h,
                                                                        bool on, const uint32_t *grid) {
    const int g = 2 * h + p;  // column group: index bytes 2 g, 2 g + 1; signs (aux >> 7 g) & 127
    const uint32_t aux = word(f.aux[s >> 2], s & 3), idx = f.idx[s] >> (16 * p);
    const uint32_t sg = ksigns((aux >> (7 * g)) & 127u);
    const int x = signed_grid(grid[idx & 0xffu], spread4(sg & 0xfu));
    const int y = signed_grid(grid[(idx >> 8) & 0xffu], spread4(sg >> 4));
    BOp<T_IQ3_XXS> r;
    r.b[0] = signed_scaled8((uint32_t) x, (uint32_t) y, 2 * (int) (aux >> 28) + 1, on);
    return r;
}
template <> __device__ __forceinline__ BOp<T_IQ3_S> decode<T_IQ3_S>(const WFrag<T_IQ3_S> &f, int s, int p, int h,
                                                                    bool on, const uint32_t *grid) {
    const int g = 2 * h + p;  // codebook entries 2 g, 2 g + 1 of the sub-block (9-bit indices), sign byte g
    const uint32_t qh = (s < 4 ? f.qh.x : f.qh.y) >> (8 * (s & 3)), idx = f.idx[s] >> (16 * p);
    const uint32_t i0 = (idx & 0xffu) | (((qh >> (2 * g)) & 1u) << 8);
    const uint32_t i1 = ((idx >> 8) & 0xffu) | (((qh >> (2 * g + 1)) & 1u) << 8);
    const uint32_t sb = (f.sg[s] >> (8 * p)) & 0xffu;
    const int x = signed_grid(grid[i0], spread4(sb & 0xfu)), y = signed_grid(grid[i1], spread4(sb >> 4));
    BOp<T_IQ3_S> r;
    r.b[0] = signed_scaled8((uint32_t) x, (uint32_t) y, 2 * (int) ((f.sc >> (4 * s)) & 0xfu) + 1, on);
    return r;
}
template <> __device__ __forceinline__ BOp<T_IQ2_S> decode<T_IQ2_S>(const WFrag<T_IQ2_S> &f, int s, int p, int h,
                                                                    bool on, const uint32_t *grid) {
    const int g = 2 * h + p;  // codebook entry g of the sub-block (10-bit index, 8 values), sign byte g
    const uint32_t idx = word(f.idx[s >> 2], s & 3), sgw = word(f.sg[s >> 2], s & 3);
    const uint32_t qh = (s < 4 ? f.qh.x : f.qh.y) >> (8 * (s & 3)), sc = (s < 4 ? f.sc.x : f.sc.y) >> (8 * (s & 3));
    const uint32_t gi = ((idx >> (8 * g)) & 0xffu) | (((qh >> (2 * g)) & 3u) << 8);
    const uint32_t sb = (sgw >> (8 * g)) & 0xffu;
    const int x = signed_grid(grid[2 * gi], spread4(sb & 0xfu)), y = signed_grid(grid[2 * gi + 1], spread4(sb >> 4));
    BOp<T_IQ2_S> r;
    r.b[0] = signed_scaled8((uint32_t) x, (uint32_t) y, 2 * (int) ((sc >> (4 * h)) & 0xfu) + 1, on);
    return r;
}

// Q8_0: B = code * d split into two f16 operands, hi = f16(code d) and lo = f16(code d - hi) (an fma in f16): code d
// has at most 19 significant bits and hi + lo holds 22, so the pair is the product exactly when lo is a normal f16
// (|code d| >= 2^-3); for smaller products lo is rounded to a multiple of 2^-24 (an absolute error of at most 2^-25
// per weight). The block scale is then inside the operands and the superblock unit is 1. Codes are signed bytes:
// (1024 + (c ^ 0x80)) - 1152. Weights must stay below the f16 range (|code d| <= 65504), as they do in a Q8_0 block.
template <> __device__ __forceinline__ BOp<T_Q8_0> decode<T_Q8_0>(const WFrag<T_Q8_0> &f, int s, int p, int, bool, const uint32_t *) {
    const uint2 q = half8(f.q[s], p);
    const uint32_t x = q.x ^ 0x80808080u, y = q.y ^ 0x80808080u;
    const h2 off = splat((_Float16) 1152.0f), d2 = as_h2((f.d[s] & 0xffffu) * 0x10001u);
    const h2 c[4] = {biased02(x) - off, biased13(x) - off, biased02(y) - off, biased13(y) - off};
    h2 hi[4], lo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        hi[i] = c[i] * d2;
        lo[i] = fma2(c[i], d2, -hi[i]);
    }
    BOp<T_Q8_0> r;
    r.b[0] = cat4(hi[0], hi[1], hi[2], hi[3]);
    r.b[1] = cat4(lo[0], lo[1], lo[2], lo[3]);
    return r;
}

// Per-superblock float scales of this lane's row: d, and dmin for Q4_K / Q5_K.
template <int T> __device__ __forceinline__ float blk_d(const WFrag<T> &f) {
    if constexpr (T == T_Q4_K || T == T_Q5_K) return half_to_float(f.h.x & 0xffffu);
    else if constexpr (T == T_Q8_0) return 1.0f;  // the block scales are inside the B operands
    else if constexpr (T == T_Q6_K) return half_to_float(f.d);
    else if constexpr (T == T_Q3_K) return half_to_float(f.tail.w >> 16);
    else if constexpr (T == T_IQ4_XS) return half_to_float(f.h.x & 0xffffu);
    else if constexpr (T == T_IQ3_XXS) return 0.25f * half_to_float(f.d & 0xffffu);
    else if constexpr (T == T_IQ3_S) return half_to_float(f.d & 0xffffu);
    else return 0.125f * half_to_float(f.d & 0xffffu);  // IQ2_S
}
// The A piece (8 columns, 16 bytes of a half-superblock chunk row) of step i for lane half hh: sub-block i / 2,
// column group 2 hh + i % 2 (the decoders above emit those), or for IQ4_XS group 2 (i % 2) + hh (its lane half reads
// 8 bytes of both nibbles: values 8 hh .. 8 hh + 7 and 16 + 8 hh ..).
template <int T> __device__ __forceinline__ int a_piece(int i, int hh) {
    return T == T_IQ4_XS ? 4 * (i >> 1) + 2 * (i & 1) + hh : 4 * (i >> 1) + 2 * hh + (i & 1);
}
// LDS words of the format's codebook (IQ2_S: two words per entry)
template <int T> constexpr int kGridWords = T == T_IQ3_XXS ? 256 : T == T_IQ3_S ? 512 : T == T_IQ2_S ? 2048 : 0;
// Q4_K / Q5_K min term operand: B[k][row] = m_s against the A operand [S_hi 8 | S_lo 8] (lane half h holds k = 8 h ..
// 8 h + 7), both halves the 8 mins in the stored sum order 0 2 1 3 4 6 5 7.
template <int T> __device__ __forceinline__ v8h min_b(const WFrag<T> &f) {
    const uint32_t m_lo = f.h.z & 0x3F3F3F3Fu;                                         // m[0..3]
    const uint32_t m_hi = ((f.h.w >> 4) & kLo4) | ((f.h.z >> 2) & 0x30303030u);       // m[4..7]
    const h2 off = splat((_Float16) 1024.0f);
    return cat4(biased02(m_lo) - off, biased13(m_lo) - off, biased02(m_hi) - off, biased13(m_hi) - off);
}

// LDS of one workgroup (static, distinct objects, so the compiler can tell the chunk being filled by LDS-DMA from the
// one being read and puts no wait between them): the half-superblock activation chunks [rows][512] (hi, lo)
// double-buffered, with the 16-byte pieces of row r stored at piece index p ^ (r % 16) so that the 16 rows of an
// A-fragment read quarter hit distinct banks; the superblock min-term sums [rows][32]. 66 KB for 64 rows: two
// workgroups per CU.
constexpr int kRowA = 512, kRowS = 32;

// 1 / (1 + e^-g); 0 for g -> -inf (the exponential saturates to +inf), 1 for g -> +inf
__device__ __forceinline__ float silu_rcp(float g) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f));
}

__device__ __forceinline__ v16f mfma32(v8h a, v8h b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Workgroup barrier for LDS filled by LDS-DMA: the DMA data is complete once this wave's vmcnt wait before it retires
// (waits placed by the caller: __syncthreads' fence would also wait for the weight loads still in flight). This
// wave's own LDS reads must have returned (lgkmcnt 0) before the next DMA into the buffer may start, and the asm's
// memory clobber keeps the compiler from moving LDS accesses across it (the s_barrier builtin is not a memory op).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

typedef __attribute__((address_space(3))) void *LdsPtr;
// 16 bytes per lane from r at (vo + so) into LDS at dst + 16 lane (dst wave-uniform); CPOL: cache-policy bits
template <int CPOL = 0>
__device__ __forceinline__ void dma16(Rsrc r, void *dst, uint32_t vo, uint32_t so) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LdsPtr) dst, 16, vo, so, 0, CPOL);
}

// ---- the fused gate/up + down launch: per-group arrivals --------------------------------------------------------
// A gate/up item stores its act image rows device-coherent (sc1: written through to memory, so no other XCD's L2 can
// serve an older copy), waits for the stores to complete and then counts its arrival on the group's counter; a down
// item of the group polls the counter (device-scope loads) until every gate/up item of the group has arrived and then
// reads the act rows with device-scope (sc1) loads. No fence is involved: the order comes from the completed stores
// before the arrival, as in the decode layer's exchange.
constexpr int kCpolDevice = 16;           // sc1
constexpr uint32_t kStatusTimeout = 1u;   // FNS_STATUS_EXCHANGE_TIMEOUT
__device__ __forceinline__ void q8_split8_dev(const float (&v)[8], Rsrc r, uint32_t row_off, int ncols, int col,
                                              bool store) {
    const Q8Split q = q8_split8_vals<true>(v);
    if (!store) return;
    const uint32_t o = row_off + img_col_off(col);
    const uint4 hi = __builtin_bit_cast(uint4, q.hi), lo = __builtin_bit_cast(uint4, q.lo);
    typedef uint32_t v4u __attribute__((ext_vector_type(4)));
    __builtin_amdgcn_raw_buffer_store_b128(v4u{hi.x, hi.y, hi.z, hi.w}, r, o, 0, kCpolDevice);
    __builtin_amdgcn_raw_buffer_store_b128(v4u{lo.x, lo.y, lo.z, lo.w}, r, o + 256, 0, kCpolDevice);
    if ((col & 31) == 0) {
        const uint32_t m = row_off + img_sum_off(ncols, col);
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, q.shi), r, m, 0, kCpolDevice);
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, q.slo), r, m + 16, 0, kCpolDevice);
    }
}
// thread 0 polls the group's arrival count (bounded); true for every thread when the wait gave up
__device__ __forceinline__ bool wait_group(const MmqArgs &a, int slot, int *flag) {
    if (threadIdx.x == 0) {
        int spins = 0, fail = 0;
        while (__hip_atomic_load(a.gdone + slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < a.gwait) {
            if (++spins > a.spin_limit) {
                fail = 1;
                __hip_atomic_fetch_or(a.status, kStatusTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        *flag = fail;
    }
    __syncthreads();
    return __builtin_amdgcn_readfirstlane(*flag) != 0;
}

// One workgroup = 4 waves x two 32-row weight streams x up to 32 NT routed activation rows of one expert (NT = 2: the
// 64-row groups and remainders > 32 rows; NT = 1: remainders <= 32 rows). GLU: stream 0 is the gate row, stream 1 the
// same up row (128 rows per workgroup); otherwise the streams are rows r and r + 128 (256).
// v_mfma_f32_32x32x16_f16: A = 32 activation rows x 16 columns, B = 16 columns x 32 weight rows; the lane that owns
// weight row j = lane % 32 decodes row j's codes and scales itself (column groups 2 h, 2 h + 1 of each sub-block,
// h = lane / 32), and holds the outputs of row j for 16 of the 32 tokens.
// LDS of one workgroup, sized for the 64-row groups (the 32-row groups use the first half of each array).
struct MmqLds {
    uint8_t (&a0)[kMmqTok * kRowA];
    uint8_t (&a1)[kMmqTok * kRowA];
    uint8_t (&s)[kMmqTok * kRowS];
    int (&src)[kMmqTok];
    int (&dst)[kMmqTok];
    int (&grp)[4];  // the group's expert, first sorted row and row count
    uint32_t *grid;  // IQ3_XXS / IQ3_S / IQ2_S: the codebook (kGridWords words)
};

// Group g of the launch's list (NT = 2: the 64-row groups and remainders > 32 rows; NT = 1: the expert's <= 32-row
// remainder), weight row block wb. DEV: an item of the fused launch (gate/up items count their arrival, down items
// wait for their group's).
template <int T, bool GLU, int NT, bool DEV>
__device__ __forceinline__ void mmq_group(const MmqArgs &a, int g, int wb, const MmqLds &L) {
    constexpr int ROWS = 32 * NT;  // activation rows of the workgroup
    constexpr int WROWS = GLU ? 128 : 256;  // weight rows of the workgroup
    auto &sh_a0 = L.a0;
    auto &sh_a1 = L.a1;
    auto &sh_s = L.s;
    auto &sh_src = L.src;
    auto &sh_dst = L.dst;
    constexpr int BB = Traits<T>::bytes, NB = kNumB<T>;
    constexpr bool MIN = T == T_Q4_K || T == T_Q5_K;
    // (the wave index as a scalar: the LDS-DMA destinations derived from it are wave-uniform M0 values)
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / kWave), lane = tid % kWave;
    const int hh = lane / 32, jl = lane % 32;

    if constexpr (kGridWords<T> > 0) {  // the codebook into LDS (visible after the barriers below)
        const uint4 *src = (const uint4 *) (T == T_IQ3_XXS ? (const void *) g_iq_grids.iq3xxs
                                            : T == T_IQ3_S ? (const void *) g_iq_grids.iq3s
                                                           : (const void *) g_iq_grids.iq2s);
        for (int i = tid; i < kGridWords<T> / 4; i += kMmqThreads) ((uint4 *) L.grid)[i] = src[i];
    }
    // which expert / rows of activations: thread t < n_expert tests whether group g is expert t's (gp[t] <= g <
    // gp[t + 1]); all the prefix loads are independent, one round trip, and the one match publishes through LDS
    int e = 0, seg = 0, cnt = 0;
    if (a.bounds) {
        const int32_t *gp = NT == 2 ? a.gprefix : a.gprefix + a.n_expert + 1;
        if (g >= gp[a.n_expert]) return;
        if (tid < a.n_expert) {
            const int g0 = gp[tid], g1 = gp[tid + 1], b0 = a.bounds[tid], b1 = a.bounds[tid + 1];
            if (g0 <= g && g < g1) {
                int c, sg;
                if constexpr (NT == 1) {  // the expert's last rows: n_e % 64 of them
                    c = (b1 - b0) % kMmqTok;
                    sg = b1 - c;
                } else {
                    sg = b0 + (g - g0) * kMmqTok;
                    c = min(kMmqTok, b1 - sg);
                }
                L.grp[0] = tid;
                L.grp[1] = sg;
                L.grp[2] = c;
            }
        }
        __syncthreads();
        e = __builtin_amdgcn_readfirstlane(L.grp[0]);
        seg = __builtin_amdgcn_readfirstlane(L.grp[1]);
        cnt = __builtin_amdgcn_readfirstlane(L.grp[2]);
    } else {
        seg = g * ROWS;
        cnt = min(ROWS, a.n_rows - seg);
    }
    if (cnt <= 0) return;
    MMQ_MARK(0);
    MMQ_NOTE(NT * 1000 + cnt);
    for (int i = tid; i < ROWS; i += kMmqThreads) {
        const int q = seg + min(i, cnt - 1);
        sh_src[i] = a.src ? a.src[q] : q;
        sh_dst[i] = a.dst_rows ? a.dst_rows[q] : q;
    }

    // (the expert's base as a scalar, so the weight buffer resources stay in SGPRs)
    const uint8_t *wbase = a.table ? (const uint8_t *) gload<const char *>((const uint8_t *) (a.table + e)) : a.w_dense;
    {
        const uint64_t wb64 = (uint64_t) wbase;
        wbase = (const uint8_t *) (((uint64_t) __builtin_amdgcn_readfirstlane((uint32_t) (wb64 >> 32)) << 32) |
                                   (uint32_t) __builtin_amdgcn_readfirstlane((uint32_t) wb64));
    }
    const int nb = a.ncols / 256;
    const int64_t row_bytes = (int64_t) nb * BB;
    // weight rows past nrows (nrows % WROWS != 0) are computed from the last row and not stored
    const int row0 = wb * WROWS + wave * 32 + jl;
    const int ra = min(row0, a.nrows - 1), rb = GLU ? ra : min(row0 + 128, a.nrows - 1);
    const Rsrc r0 = rsrc_of(wbase + a.off_a), r1 = rsrc_of(wbase + (GLU ? a.off_b : a.off_a)), rx = rsrc_of(a.xpack);
    const uint32_t v0 = (uint32_t) (ra * row_bytes), v1 = (uint32_t) (rb * row_bytes);
    const uint32_t c0 = v0 + 16 * hh, c1 = v1 + 16 * hh;
    __syncthreads();  // sh_src / sh_dst

    // LDS-DMA of chunk (kb, h) - columns 256 kb + 128 h .. + 127, hi and lo: 512 bytes per row - by instruction u of
    // wave w: rows 8 u + 2 w, + 1 (one per 32 lanes; lane piece i of row r reads image piece i ^ (r % 16))
    constexpr int NU = ROWS / 8;
    uint32_t qo[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        const int r = 8 * u + 2 * wave + lane / 32;
        qo[u] = (uint32_t) ((size_t) sh_src[r] * a.x_img + 16 * ((lane % 32) ^ (r % 16)));
    }
    // min-term sums of superblock kb: rows 32 w' + lane / 2 (2 pieces per row), w' = wave % (ROWS / 32)
    const int srow = 32 * (wave % (ROWS / 32));
    const uint32_t so = (uint32_t) ((size_t) sh_src[srow + lane / 2] * a.x_img + (size_t) nb * kSbMain + 16 * (lane & 1));
    // (unconditional: a fixed number of loads in flight keeps the compiler's wait counts exact; rows past cnt read
    // the last routed row again)
    constexpr int CPOL = DEV && !GLU ? kCpolDevice : 0;  // the fused down items read this launch's act rows
    auto dma_chunk = [&](uint8_t *buf, int kb, int h) __attribute__((always_inline)) {
        const uint32_t soff = (uint32_t) (kb * kSbMain + h * 512);
#pragma unroll
        for (int u = 0; u < NU; ++u) dma16<CPOL>(rx, buf + (8 * u + 2 * wave) * kRowA, qo[u], soff);
    };
    auto dma_sums = [&](int kb) __attribute__((always_inline)) {  // the waves past ROWS / 32 repeat the first ones
        if constexpr (MIN) dma16<CPOL>(rx, sh_s + srow * kRowS, so, (uint32_t) (kb * kSbMin));
    };

    // the superblocks [kb0, kb_end) of this item: all of them, or part blockIdx.y of a split K range
    int kb0 = 0, kb_end = nb, part = 0;
    if constexpr (!GLU && !DEV) {
        if (a.ksplit > 1) {
            part = (int) blockIdx.y;
            kb0 = part * nb / a.ksplit;
            kb_end = (part + 1) * nb / a.ksplit;
        }
    }
    WFrag<T> f0, f1, n0, n1;
    bool failed = false;
    if constexpr (DEV && !GLU) {  // the first weights in flight, then the wait for the group's act rows
        wfrag_load<T, 0>(r0, v0, c0, 0, f0);
        wfrag_load<T, 0>(r1, v1, c1, 0, f1);
        failed = wait_group(a, NT == 2 ? g : a.n_main + g, &L.grp[3]);
        dma_chunk(sh_a0, 0, 0);
        dma_sums(0);
    } else {
        dma_chunk(sh_a0, kb0, 0);
        dma_sums(kb0);
        wfrag_load<T, 0>(r0, v0, c0, (uint32_t) (kb0 * BB), f0);
        wfrag_load<T, 0>(r1, v1, c1, (uint32_t) (kb0 * BB), f1);
    }
    dma_wait();
    lds_barrier();
    MMQ_MARK(1);

    // acc[t][m] is kept in units of the current superblock's d (per lane: its row's d, 1 if d = 0), so the MFMAs
    // accumulate into it directly; between superblocks it is rescaled and the min term added (fp32 rounding).
    // All tiles are computed whatever cnt (rows past it hold stale LDS data and are never stored).
    v16f acc[NT][2];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][0][r] = acc[t][1][r] = 0.0f;
    float ds0 = blk_d<T>(f0), ds1 = blk_d<T>(f1);
    bool on0 = ds0 != 0.0f, on1 = ds1 != 0.0f;
    ds0 = on0 ? ds0 : 1.0f;
    ds1 = on1 ? ds1 : 1.0f;

    // eight 16-column steps of one half from LDS chunk buf (step i: sub-block 4 h + i / 2, column group 2 hh + i % 2):
    // acc[t][m] += A (hi, lo) x B (integer-scaled codes). Software-pipelined: while the MFMAs of step i issue, the A
    // fragments of step i + 1 are read from LDS and its B operands decoded (VALU); the compiler interleaves them
    // (pinning one MFMA to a fixed number of VALU instructions with scheduling-group barriers measured 2% slower).
    auto load_a = [&](const uint8_t *buf, int i, v8h (&av)[2][NT]) __attribute__((always_inline)) {
        const int piece = a_piece<T>(i, hh);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const uint8_t *ap = buf + (t * 32 + jl) * kRowA;
            av[0][t] = *(const v8h *) (ap + 16 * (piece ^ (jl & 15)));
            av[1][t] = *(const v8h *) (ap + 16 * ((16 + piece) ^ (jl & 15)));
        }
    };
    auto load_a1 = [&](const uint8_t *buf, int i, int x, v8h (&av)[NT]) __attribute__((always_inline)) {
        const int piece = 16 * x + a_piece<T>(i, hh);
#pragma unroll
        for (int t = 0; t < NT; ++t) av[t] = *(const v8h *) (buf + (t * 32 + jl) * kRowA + 16 * (piece ^ (jl & 15)));
    };
    auto half_pass = [&](const uint8_t *buf, auto hc, const WFrag<T> &f0, const WFrag<T> &f1) __attribute__((always_inline)) {
        constexpr int h = decltype(hc)::value;
        v8h av[2][NT];
        const uint32_t *grid = L.grid;
        BOp<T> b0 = decode<T>(f0, 4 * h, 0, hh, on0, grid), b1 = decode<T>(f1, 4 * h, 0, hh, on1, grid), d0, d1;
        load_a(buf, 0, av);
        if constexpr (NB == 1) {
            // One B operand per stream: the hi fragments of step i + 1 are read into the registers of step i's as soon
            // as its hi MFMAs have issued, the lo ones after its lo MFMAs (no second set of A registers).
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                __builtin_amdgcn_sched_barrier(0);
                if (i < 7) {
                    d0 = decode<T>(f0, 4 * h + (i + 1) / 2, (i + 1) & 1, hh, on0, grid);
                    d1 = decode<T>(f1, 4 * h + (i + 1) / 2, (i + 1) & 1, hh, on1, grid);
                }
#pragma unroll
                for (int x = 0; x < 2; ++x) {
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        acc[t][0] = mfma32(av[x][t], b0.b[0], acc[t][0]);
                        acc[t][1] = mfma32(av[x][t], b1.b[0], acc[t][1]);
                    }
                    if (i < 7) load_a1(buf, i + 1, x, av[x]);
                }
                if (i < 7) {
                    b0 = d0;
                    b1 = d1;
                }
            }
        } else {
            v8h an[2][NT];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                __builtin_amdgcn_sched_barrier(0);
                if (i < 7) {
                    load_a(buf, i + 1, an);
                    d0 = decode<T>(f0, 4 * h + (i + 1) / 2, (i + 1) & 1, hh, on0, grid);
                    d1 = decode<T>(f1, 4 * h + (i + 1) / 2, (i + 1) & 1, hh, on1, grid);
                }
                // hi for every (tile, stream), then lo: dependent MFMAs 2 NT issues apart
#pragma unroll
                for (int g = 0; g < NB; ++g)
#pragma unroll
                    for (int x = 0; x < 2; ++x)
#pragma unroll
                        for (int t = 0; t < NT; ++t) {
                            acc[t][0] = mfma32(av[x][t], b0.b[g], acc[t][0]);
                            acc[t][1] = mfma32(av[x][t], b1.b[g], acc[t][1]);
                        }
                if (i < 7) {
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        av[0][t] = an[0][t];
                        av[1][t] = an[1][t];
                    }
                    b0 = d0;
                    b1 = d1;
                }
            }
        }
    };

    // The scheduling barriers (sched_barrier 0) between the phases below are load-bearing: they keep the compiler from
    // moving instructions across the explicit vmcnt waits that stand for the DMA and fragment loads (removing them
    // all fails the GEMM tests).
    // one superblock with fragments f0, f1 (current; their first part loaded) and n0, n1 (next, first part loaded here)
    auto superblock = [&](int kb, WFrag<T> &f0, WFrag<T> &f1, WFrag<T> &n0, WFrag<T> &n1)
                          __attribute__((always_inline)) {
        const bool more = kb + 1 < kb_end;
        const int kn = more ? kb + 1 : kb;  // the last superblock reloads itself: same load count every iteration
        dma_chunk(sh_a1, kb, 1);
        __builtin_amdgcn_sched_barrier(0);
        // Weights one half superblock ahead: this block's second-half codes now, the next block's header and
        // first-half codes during the second half. Each part has half a superblock of compute to land, and only
        // about one and a half fragments per stream are live at a time.
        wfrag_load<T, 1>(r0, v0, c0, kb * BB, f0);
        wfrag_load<T, 1>(r1, v1, c1, kb * BB, f1);
        __builtin_amdgcn_sched_barrier(0);
        half_pass(sh_a0, std::integral_constant<int, 0>{}, f0, f1);
        __builtin_amdgcn_sched_barrier(0);
        // chunk (kb, 1) landed (only the weight loads issued after it may still be in flight)
        constexpr int kPend = 2 * wfrag_loads<T, 1>();  // s_waitcnt vmcnt(kPend): vmcnt bits 3:0 and 15:14
        __builtin_amdgcn_s_waitcnt(0x0F70 | (kPend & 0xF) | ((kPend >> 4) << 14));
        lds_barrier();  // chunk (kb, 1) visible; chunk buffer 0 free

        dma_chunk(sh_a0, kn, 0);
        wfrag_load<T, 0>(r0, v0, c0, kn * BB, n0);
        wfrag_load<T, 0>(r1, v1, c1, kn * BB, n1);
        __builtin_amdgcn_sched_barrier(0);
        half_pass(sh_a1, std::integral_constant<int, 1>{}, f0, f1);
        __builtin_amdgcn_sched_barrier(0);
        // superblock done: acc <- (acc ds - dmin (m . S)) / ds_next, ds_next = 1 after the last superblock
        float nd0 = 1.0f, nd1 = 1.0f;
        bool non0 = true, non1 = true;
        dma_wait();  // the next weights (and chunk (kb + 1, 0))
        if (more) {
            nd0 = blk_d<T>(n0);
            nd1 = blk_d<T>(n1);
            non0 = nd0 != 0.0f;
            non1 = nd1 != 0.0f;
            nd0 = non0 ? nd0 : 1.0f;
            nd1 = non1 ? nd1 : 1.0f;
        }
        const float inv0 = __builtin_amdgcn_rcpf(nd0), inv1 = __builtin_amdgcn_rcpf(nd1);
        const float k0 = ds0 * inv0, k1 = ds1 * inv1;
        float km0 = 0.0f, km1 = 0.0f;
        v8h bm0, bm1;
        if constexpr (MIN) {
            km0 = -half_to_float(f0.h.x >> 16) * inv0;
            km1 = -half_to_float(f1.h.x >> 16) * inv1;
            bm0 = min_b<T>(f0);
            bm1 = min_b<T>(f1);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if constexpr (MIN) {
                // one min-term product at a time (each is 16 registers)
                v16f z;
#pragma unroll
                for (int r = 0; r < 16; ++r) z[r] = 0.0f;
                const v8h am = *(const v8h *) (sh_s + (t * 32 + jl) * kRowS + 16 * hh);
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    const v16f mt = mfma32(am, m ? bm1 : bm0, z);
                    const float k = m ? k1 : k0, km = m ? km1 : km0;
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[t][m][r] = fmaf_(acc[t][m][r], k, km * mt[r]);
                    __builtin_amdgcn_sched_barrier(0);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    acc[t][0][r] *= k0;
                    acc[t][1][r] *= k1;
                }
            }
        }
        ds0 = nd0;
        ds1 = nd1;
        on0 = non0;
        on1 = non1;
        lds_barrier();  // chunk (kb + 1, 0) visible; chunk buffer 1 and the sums free
        dma_sums(kn);  // read at the end of superblock kb + 1, after its first barrier
        MMQ_MARK(2 + kb);
    };
    // the fragment sets swap roles every superblock
    for (int kb = kb0; kb < kb_end; kb += 2) {
        superblock(kb, f0, f1, n0, n1);
        if (kb + 1 < kb_end) superblock(kb + 1, n0, n1, f0, f1);
    }

    dma_wait();  // the last (unused) sums load
    // output (token i, weight row row0) of acc[t][m][r]: i = 32 t + 8 (r / 4) + 4 hh + r % 4
    if constexpr (!GLU) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int i = t * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
                if (i < cnt) {
                    float *o = a.dst + (size_t) part * a.part_stride + (size_t) sh_dst[i] * a.nrows;
                    if (row0 < a.nrows) o[row0] = failed ? __builtin_nanf("") : acc[t][0][r];
                    if (row0 + 128 < a.nrows) o[row0 + 128] = failed ? __builtin_nanf("") : acc[t][1][r];
                }
            }
    } else {
        // act = up * silu(gate) (reference src/ggml/ggml_mmvq.cu:240-247 epilogue with zero biases; silu(g) =
        // g / (1 + e^-g) from the hardware exp2 and reciprocal, about 2 ulp), staged as [token][64 rows] f32 per wave
        // pair (waves 0-1 in chunk buffer 0, waves 2-3 in buffer 1; row stride 68 floats: 16-byte aligned rows),
        // then the Q8_1 blocks (token, 32 rows) into the act split image rows: 4 lanes per block, 8 values per lane
        constexpr int kAct = 68;
        static_assert(ROWS * kAct * 4 <= ROWS * kRowA, "act tile fits a chunk buffer");
        float *act = (float *) (wave < 2 ? sh_a0 : sh_a1);
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int i = t * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
                const float g = acc[t][0][r] + 0.0f;
                act[i * kAct + (wave & 1) * 32 + jl] = (acc[t][1][r] + 0.0f) * (g * silu_rcp(g));
            }
        __syncthreads();
        for (int p0 = wave * 16; p0 < 4 * cnt; p0 += 16 * kMmqWaves) {  // wave-uniform trip count
            const int p = p0 + lane / 4, q = lane % 4;
            const int i = p < 4 * cnt ? p / 4 : 0, blk = p % 4;
            const int col = wb * WROWS + 32 * blk + 8 * q;
            const bool live = p < 4 * cnt && col < a.nrows;  // the same for the 4 lanes of a block
            const float *src = (const float *) (blk < 2 ? sh_a0 : sh_a1) + i * kAct + 32 * (blk & 1) + 8 * q;
            const float4 x0 = *(const float4 *) src, x1 = *(const float4 *) (src + 4);
            const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            // the reference's Q8_1 arithmetic (q = roundf(v / d), IEEE division): the same codes as the quantiser of
            // the f32 act rows would give
            if constexpr (DEV)
                q8_split8_dev(v, rsrc_of(a.out_pack), (uint32_t) ((size_t) sh_dst[i] * a.out_img), a.nrows, col, live);
            else
                q8_split8<true>(v, a.out_pack + (size_t) sh_dst[i] * a.out_img, a.nrows, col, live);
            if (live && a.act_out) {
                float *ao = a.act_out + (size_t) sh_dst[i] * a.nrows + col;
                *(float4 *) ao = x0;
                *(float4 *) (ao + 4) = x1;
            }
        }
        if constexpr (DEV) {  // every act store of the workgroup has completed: count the arrival
            dma_wait();
            __syncthreads();
            if (tid == 0)
                __hip_atomic_fetch_add(a.gdone + (NT == 2 ? g : a.n_main + g), 1, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    MMQ_MARK(12);
}

// One launch runs both lists, the 64-row groups first (g < n_main) and then the experts' <= 32-row remainders, so the
// smaller workgroups fill the machine while the last large ones finish. The grid is one-dimensional and XCD-aware:
// workgroup L runs on XCD L % 8 (the hardware's round-robin dispatch), and the n_cb weight row blocks of a group are
// consecutive items of one XCD, so the group's activation rows are fetched into that XCD's L2 once, not once per
// row block; groups go to the XCDs in turn (group u on XCD u % 8) in increasing order.
// (SPX mode: one partition of all 8 XCDs. In a partitioned mode the mapping is a performance assumption only.)
constexpr int kXcds = 8;  // MI355X: 8 XCDs, each with its own L2
template <int T, bool GLU>
__global__ __launch_bounds__(kMmqThreads) __attribute__((amdgpu_waves_per_eu(2, 4))) void k_mmq(const MmqArgs a) {
    __shared__ __align__(16) uint8_t sh_a0[kMmqTok * kRowA];
    __shared__ __align__(16) uint8_t sh_a1[kMmqTok * kRowA];
    __shared__ __align__(16) uint8_t sh_s[(T == T_Q4_K || T == T_Q5_K) ? kMmqTok * kRowS : 16];
    __shared__ __align__(16) uint32_t sh_grid[kGridWords<T> > 0 ? kGridWords<T> : 4];
    __shared__ int sh_src[kMmqTok], sh_dst[kMmqTok], sh_grp[4];
    const MmqLds L{sh_a0, sh_a1, *(uint8_t (*)[kMmqTok * kRowS]) sh_s, sh_src, sh_dst, sh_grp, sh_grid};
    const int lid = blockIdx.x, r = lid / kXcds;
    int j = (r / a.n_cb) * kXcds + lid % kXcds;
    const int wb = r % a.n_cb;
    if (a.bounds) {
        // expert path: the groups that exist in this call (the device-side counts of the 64-row list and of the
        // remainder list) take the first workgroups; the rest of the grid (sized for the upper bound) returns at once
        const int nm = a.gprefix[a.n_expert], nr = a.gprefix[2 * (a.n_expert + 1) - 1];
        if (j >= nm + nr) return;
        if (j < nm) mmq_group<T, GLU, 2, false>(a, j, wb, L);
        else mmq_group<T, GLU, 1, false>(a, j - nm, wb, L);
        return;
    }
    if (j >= a.n_groups) return;
    if (a.dense_small) mmq_group<T, GLU, 1, false>(a, j, wb, L);
    else mmq_group<T, GLU, 2, false>(a, j, wb, L);
}

// Gate/up (with SwiGLU and the Q8_1 of act) and down of the expert path in one launch. The gate/up items come first,
// in the order and XCD mapping of k_mmq (group g's weight row blocks on XCD g % 8), then the down items with the same
// mapping; a down item first waits for its group's gate/up items (arrival counts, see above). Workgroups are
// dispatched in index order on each XCD and every gate/up item precedes every down item, so a waiting down item never
// holds a slot that a gate/up item it waits for still needs: the wait always ends. The gate/up tail and the first
// down items overlap instead of being separated by a launch. (A persistent variant that takes items from per-XCD
// queues measured no faster.)
struct MoeArgs {
    const char *const *table;
    int64_t gate_off, up_off, down_off;
    int hidden, inter, n_expert, n_main;  // n_main: the 64-row list's upper bound
    int n_cb_gu, n_cb_dn, gwait, spin_limit;
    const uint8_t *ximg;                  // x split images [n_tok][x_img]
    uint8_t *aimg;                        // act split images [n_tok * k][a_img]
    int64_t x_img, a_img;
    const int32_t *bounds, *gprefix, *src1, *dstr;
    float *dexp;
    int *gdone;
    uint32_t *status;
};
template <int TGU, int TDN>
__global__ __launch_bounds__(kMmqThreads) __attribute__((amdgpu_waves_per_eu(2, 4))) void k_mmq_moe(const MoeArgs m) {
    constexpr bool MIN = TGU == T_Q4_K || TGU == T_Q5_K || TDN == T_Q4_K || TDN == T_Q5_K;
    __shared__ __align__(16) uint8_t sh_a0[kMmqTok * kRowA];
    __shared__ __align__(16) uint8_t sh_a1[kMmqTok * kRowA];
    __shared__ __align__(16) uint8_t sh_s[MIN ? kMmqTok * kRowS : 16];
    __shared__ int sh_src[kMmqTok], sh_dst[kMmqTok], sh_grp[4];
    const MmqLds L{sh_a0, sh_a1, *(uint8_t (*)[kMmqTok * kRowS]) sh_s, sh_src, sh_dst, sh_grp, nullptr};
    PF_MARK(3, 0);
    // The groups that exist in this call (the device-side counts of the two lists: the 64-row groups, then the <= 32-row
    // remainders) are numbered j = 0 .. R - 1 and take the first workgroups of the grid; the workgroups past them (the
    // grid is sized for the upper bound) return at once, after every real item has been dispatched.
    const int nm = m.gprefix[m.n_expert], nr = m.gprefix[2 * (m.n_expert + 1) - 1];
    const int R = nm + nr, rounds = (R + kXcds - 1) / kXcds;
    const int items_gu = m.n_cb_gu * kXcds * rounds;  // a multiple of kXcds
    const bool is_gu = (int) blockIdx.x < items_gu;
    const int cb = is_gu ? m.n_cb_gu : m.n_cb_dn;
    const int lid = is_gu ? (int) blockIdx.x : (int) blockIdx.x - items_gu, r = lid / kXcds;
    const int j = (r / cb) * kXcds + lid % kXcds, wb = r % cb;
    if (j >= R) return;
    const int g = j < nm ? j : m.n_main + (j - nm);
    MmqArgs a{};
    a.table = m.table;
    a.n_expert = m.n_expert;
    a.bounds = m.bounds;
    a.gprefix = m.gprefix;
    a.n_main = m.n_main;
    a.dst_rows = m.dstr;
    a.gdone = m.gdone;
    if (is_gu) {
        a.off_a = m.gate_off;
        a.off_b = m.up_off;
        a.ncols = m.hidden;
        a.nrows = m.inter;
        a.xpack = m.ximg;
        a.x_img = m.x_img;
        a.src = m.src1;
        a.out_pack = m.aimg;
        a.out_img = m.a_img;
        if (g < m.n_main) mmq_group<TGU, true, 2, true>(a, g, wb, L);
        else mmq_group<TGU, true, 1, true>(a, g - m.n_main, wb, L);
    } else {
        a.off_a = m.down_off;
        a.ncols = m.inter;
        a.nrows = m.hidden;
        a.xpack = m.aimg;
        a.x_img = m.a_img;
        a.src = m.dstr;
        a.dst = m.dexp;
        a.gwait = m.gwait;
        a.spin_limit = m.spin_limit;
        a.status = m.status;
        if (g < m.n_main) mmq_group<TDN, false, 2, true>(a, g, wb, L);
        else mmq_group<TDN, false, 1, true>(a, g - m.n_main, wb, L);
    }
    PF_MARK(3, 1);
}

template <bool GLU> const void *mmq_kernel(int type) {
    switch (type) {
        case T_Q8_0: return (const void *) k_mmq<T_Q8_0, GLU>;
        case T_Q3_K: return (const void *) k_mmq<T_Q3_K, GLU>;
        case T_Q4_K: return (const void *) k_mmq<T_Q4_K, GLU>;
        case T_Q5_K: return (const void *) k_mmq<T_Q5_K, GLU>;
        case T_Q6_K: return (const void *) k_mmq<T_Q6_K, GLU>;
        case T_IQ4_XS: return (const void *) k_mmq<T_IQ4_XS, GLU>;
        case T_IQ3_XXS: return (const void *) k_mmq<T_IQ3_XXS, GLU>;
        case T_IQ3_S: return (const void *) k_mmq<T_IQ3_S, GLU>;
        case T_IQ2_S: return (const void *) k_mmq<T_IQ2_S, GLU>;
    }
    return nullptr;
}

// groups: upper bound of the 64-row list; expert path: of the 64-row list and the <= 32-row remainders together (the
// workgroups past the device-side counts return at once)
int launch_mmq(int type, bool glu, const MmqArgs &a, int groups, hipStream_t st) {
    const void *fn = glu ? mmq_kernel<true>(type) : mmq_kernel<false>(type);
    if (!fn) return host::set_error(host::ERR_TYPE, "mmq: type %d not supported", type);
    if (groups <= 0) return host::OK;
    MmqArgs arg = a;
    arg.n_main = groups;
    // expert path: n_expert + ceil(pairs / 64) (the 64-row list's bound) bounds both lists together, as expert e
    // has ceil(n_e / 64) groups in all
    int total = groups;
    void *args[] = {&arg};
    const int rows = glu ? 128 : 256;  // weight rows per workgroup
    arg.n_cb = (a.nrows + rows - 1) / rows;
    // dense: when even twice the workgroups of the 64-row groups fit one per CU, groups of 32 rows (one token tile:
    // more B decode per MFMA, but twice the workgroups; measured faster for 64 -> 128 workgroups, slower for
    // 192 -> 384)
    arg.dense_small = 0;
    const int ks = !glu && !a.bounds && a.ksplit > 1 ? a.ksplit : 1;
    if (ks > 1 && (a.ncols / 256 < ks || ks > 8)) return host::set_error(host::ERR_SHAPE, "mmq: bad K split");
    arg.ksplit = ks;
    if (!a.bounds && a.n_rows > 32 && (int64_t) 2 * groups * arg.n_cb * ks <= 256) {
        arg.dense_small = 1;
        total = (a.n_rows + 31) / 32;
    }
    arg.n_groups = total;
    const int64_t items = (int64_t) arg.n_cb * kXcds * ((total + kXcds - 1) / kXcds);
    if (items > INT32_MAX) return host::set_error(host::ERR_SHAPE, "mmq: grid too large");
    const hipError_t e = hipLaunchKernel(fn, dim3((unsigned) items, (unsigned) ks), dim3(kMmqThreads), args, 0, st);
    if (e != hipSuccess) return host::set_error(host::ERR_LAUNCH, "mmq: %s", hipGetErrorString(e));
    return host::check_launch("mmq");
}

// The fused kernel for the type pairs whose register allocation does not spill (the Q5_K and Q6_K decoders push the
// combined kernel past 256 registers); the other pairs take two launches.
template <int TGU> const void *mmq_moe_kernel_dn(int tdn) {
    switch (tdn) {
        case T_Q3_K: return (const void *) k_mmq_moe<TGU, T_Q3_K>;
        case T_Q4_K: return (const void *) k_mmq_moe<TGU, T_Q4_K>;
    }
    return nullptr;
}
const void *mmq_moe_kernel(int tgu, int tdn) {
    switch (tgu) {
        case T_Q3_K: return mmq_moe_kernel_dn<T_Q3_K>(tdn);
        case T_Q4_K: return mmq_moe_kernel_dn<T_Q4_K>(tdn);
    }
    return nullptr;
}

// The fused launch (the arrival counters zero: the compaction kernel clears them).
int launch_mmq_moe(int tgu, int tdn, MoeArgs m, hipStream_t st) {
    const void *fn = mmq_moe_kernel(tgu, tdn);
    if (!fn) return host::set_error(host::ERR_TYPE, "mmq: types %d / %d not supported", tgu, tdn);
    if (m.n_main <= 0) return host::OK;
    m.n_cb_gu = (m.inter + 127) / 128;
    m.n_cb_dn = (m.hidden + 255) / 256;
    m.gwait += m.n_cb_gu;
    // n_main = n_expert + ceil(pairs / 64) bounds both lists together: expert e has ceil(n_e / 64) groups in all
    const int64_t total = m.n_main;
    const int64_t items = (int64_t) (m.n_cb_gu + m.n_cb_dn) * kXcds * ((total + kXcds - 1) / kXcds);
    if (items > INT32_MAX) return host::set_error(host::ERR_SHAPE, "mmq: grid too large");
    void *args[] = {&m};
    const hipError_t e = hipLaunchKernel(fn, dim3((unsigned) items), dim3(kMmqThreads), args, 0, st);
    if (e != hipSuccess) return host::set_error(host::ERR_LAUNCH, "mmq: %s", hipGetErrorString(e));
    return host::check_launch("mmq (gate/up + down)");
}

int check_mmq_shape(int type, int64_t ncols, int64_t nrows) {
    if (!host::is_kquant(type) && !host::is_iq(type) && type != T_Q8_0)
        return host::set_error(host::ERR_TYPE, "mmq: type %d not supported", type);
    if (host::iq_needs_grid(type) && !host::iq_grids_ready())
        return host::set_error(host::ERR_TYPE, "mmq: type %d needs the IQ codebooks (fns_hip_set_iq_grids)", type);
    if (ncols <= 0 || ncols % 256 || nrows <= 0 || nrows % kMmqRows || ncols > 65536)
        return host::set_error(host::ERR_SHAPE, "mmq: ncols must be a positive multiple of 256, nrows of 64");
    return host::OK;
}
}  // namespace

namespace impl {

// This translation unit's copy of the IQ codebooks (fns_quarter.hpp g_iq_grids), on the current device.
int iq_grids_upload_mmq(const void *grids) {
    const hipError_t e = dev::upload_iq_grids((const dev::IqGrids *) grids);
    return e == hipSuccess ? host::OK : host::set_error(host::ERR_LAUNCH, "set_iq_grids: %s", hipGetErrorString(e));
}

size_t mmq_image_bytes(int64_t ncols) { return (size_t) split_row_bytes(ncols); }
size_t mmq_q8_1_bytes(int64_t ncols, int64_t nrows) { return (size_t) nrows * mmq_image_bytes(ncols) + 4096; }
size_t mmq_bounds_bytes(int64_t n_expert) { return bounds_bytes(n_expert); }

int mmq_quant_image(const float *x, int64_t ncols, int64_t rows, void *xpack, hipStream_t st) {
    if (!x || !xpack || ncols <= 0 || ncols % 256 || ncols > 65536 || rows < 0 || rows > 65535)
        return host::set_error(host::ERR_SHAPE, "mmq quantize: bad arguments");
    if (rows == 0) return host::OK;
    hipLaunchKernelGGL(k_quant_image, dim3((unsigned) ((ncols + 2047) / 2048), (unsigned) rows), dim3(256), 0, st, x, (int) ncols,
                       (uint8_t *) xpack, (int64_t) mmq_image_bytes(ncols));
    return host::check_launch("mmq quantize");
}

int mmq_quant_image_scaled(const float *x, const float *escale, int64_t ncols, int64_t rows, void *xpack,
                           int64_t stride, hipStream_t st) {
    if (!x || !escale || !xpack || ncols <= 0 || ncols % 256 || ncols > 65536 || rows < 0 || rows > 65535)
        return host::set_error(host::ERR_SHAPE, "mmq quantize: bad arguments");
    if (rows == 0) return host::OK;
    hipLaunchKernelGGL(k_quant_image_scaled, dim3((unsigned) ((ncols + 2047) / 2048), (unsigned) rows), dim3(256), 0, st,
                       x, escale, (int) ncols, (uint8_t *) xpack, stride);
    return host::check_launch("mmq quantize (guarded rows)");
}

int mmq_compact(const int32_t *ids, int64_t n_tok, int64_t k, int64_t n_expert, int64_t x_rows_per_tok,
                int32_t *ids_src1, int32_t *ids_dst, int32_t *bounds, int32_t *gprefix, hipStream_t st, int32_t *gdone,
                int n_gdone) {
    // an empty batch (n_tok = 0) may pass null id arrays: it only writes zero bounds
    const bool any = n_tok > 0;
    if ((any && (!ids || !ids_src1 || !ids_dst)) || !bounds || !gprefix || n_tok < 0 || k < 1 || n_expert < 1 || n_expert > 256 ||
        n_tok * k > (1 << 20) || (x_rows_per_tok != 1 && x_rows_per_tok != k))
        return host::set_error(host::ERR_SHAPE, "mmq compaction: bad arguments");
    hipLaunchKernelGGL(k_mmq_compact, dim3(1), dim3(kCompactThreads), 0, st, ids, (int) (n_tok * k), (int) k,
                       (int) n_expert, (int) x_rows_per_tok, ids_src1, ids_dst, bounds, gprefix, gdone, gdone ? n_gdone : 0);
    return host::check_launch("mmq compaction");
}

// Bytes per act image row in the prefill workspace: the image rounded up to whole 128-byte lines, so that no cache
// line holds parts of two rows. The fused launch depends on it: rows of different groups are written and read by
// different workgroups at different times, and a line read for one row must never carry another row's older bytes.
int64_t act_stride(int64_t ncols) { return ((int64_t) mmq_image_bytes(ncols) + 127) / 128 * 128; }

// the 64-row list's upper bound for n_pairs sorted rows over n_expert experts: sum_e (n_e / 64 + (n_e % 64 > 32))
int64_t main_groups(int64_t n_expert, int64_t n_pairs) { return n_expert + (n_pairs + kMmqTok - 1) / kMmqTok; }

// x_stride / out_stride: bytes per activation / act image row (0: the image's own size)
int expert_args(int type, const char *const *table, size_t off_a, size_t off_b, bool glu, int64_t ncols,
                int64_t nrows, int64_t n_expert, const void *xpack, const int32_t *ids_src1, const int32_t *ids_dst,
                const int32_t *bounds, const int32_t *gprefix, float *dst, void *out_pack, float *act_out, MmqArgs &a,
                int64_t x_stride = 0, int64_t out_stride = 0) {
    FNS_TRY(check_mmq_shape(type, ncols, nrows));
    if (!table || !xpack || !bounds || !gprefix || (!glu && !dst) || (glu && !out_pack) || n_expert < 1 || n_expert > 256)
        return host::set_error(host::ERR_SHAPE, "mmq_experts: bad arguments");
    a = MmqArgs{};
    a.table = table;
    a.off_a = (int64_t) off_a;
    a.off_b = (int64_t) off_b;
    a.ncols = (int) ncols;
    a.nrows = (int) nrows;
    a.n_expert = (int) n_expert;
    a.xpack = (const uint8_t *) xpack;
    a.x_img = x_stride ? x_stride : (int64_t) mmq_image_bytes(ncols);
    a.bounds = bounds;
    a.gprefix = gprefix;
    a.src = ids_src1;
    a.dst_rows = ids_dst;
    a.dst = dst;
    a.out_pack = (uint8_t *) out_pack;
    a.out_img = out_stride ? out_stride : (int64_t) mmq_image_bytes(nrows);
    a.act_out = act_out;
    return host::OK;
}

int mmq_gemm_experts(int type, const char *const *table, size_t off_a, size_t off_b, bool glu, int64_t ncols,
                     int64_t nrows, int64_t n_expert, const void *xpack, int64_t n_pairs, const int32_t *ids_src1,
                     const int32_t *ids_dst, const int32_t *bounds, const int32_t *gprefix, float *dst, void *out_pack,
                     float *act_out, hipStream_t st) {
    MmqArgs a;
    FNS_TRY(expert_args(type, table, off_a, off_b, glu, ncols, nrows, n_expert, xpack, ids_src1, ids_dst, bounds,
                        gprefix, dst, out_pack, act_out, a));
    return launch_mmq(type, glu, a, (int) main_groups(n_expert, n_pairs), st);
}

// Q8_0 (the reference's dense and output-head type, src/ggml/ggml_mmq.cu:59) takes the GEMV kernels, a few token
// columns per weight pass: each 32-value block is d_w * d8 * (integer dot) in both, so the results are those of a
// GEMM over the same Q8_1 activations; the bytes are re-read per column group (the tiled GEMM covers the expert
// K-quant and IQ formats, whose sub-block scales fold into exact f16 operands; Q8_0's float block scale does not).
int mmq(int type, const void *w, int64_t ncols, int64_t nrows, const float *x, int64_t n_tok, void *xq, float *dst,
        hipStream_t st) {
    if (type == T_Q8_0 && nrows % kMmqRows) {  // the GEMV kernels (any row count), a few token columns per pass
        if (!w || !x || !xq || !dst || n_tok < 0 || ncols <= 0 || ncols % 256 || nrows <= 0)
            return host::set_error(host::ERR_SHAPE, "mmq: bad arguments");
        if (n_tok == 0) return host::OK;
        FNS_TRY(quantize_q8_1(x, xq, ncols, n_tok, st));
        return mmvq(type, w, ncols, nrows, xq, dst, n_tok, st);
    }
    FNS_TRY(check_mmq_shape(type, ncols, nrows));
    if (!w || !x || !xq || !dst || n_tok < 0) return host::set_error(host::ERR_SHAPE, "mmq: bad arguments");
    if (n_tok == 0) return host::OK;
    FNS_TRY(mmq_quant_image(x, ncols, n_tok, xq, st));
    MmqArgs a{};
    a.w_dense = (const uint8_t *) w;
    a.ncols = (int) ncols;
    a.nrows = (int) nrows;
    a.xpack = (const uint8_t *) xq;
    a.x_img = (int64_t) mmq_image_bytes(ncols);
    a.n_rows = (int) n_tok;
    a.dst = dst;
    return launch_mmq(type, false, a, (int) ((n_tok + kMmqTok - 1) / kMmqTok), st);
}

int mmq_experts(int type, const char *const *table, size_t off, int64_t ncols, int64_t nrows, int64_t n_expert,
                const float *x, int64_t x_rows_per_tok, int64_t n_tok, const int32_t *ids, int64_t n_used,
                int32_t *ids_src1, int32_t *ids_dst, int32_t *bounds, void *xq, float *dst, hipStream_t st) {
    if (type == T_Q8_0 && nrows % kMmqRows) {  // the GEMV over every (token, slot), as mmq above; the sort is still written
        if (!x || !xq || !table || !ids || !dst || n_used < 1 || n_tok < 0 || ncols <= 0 || ncols % 256 ||
            (x_rows_per_tok != 1 && x_rows_per_tok != n_used))
            return host::set_error(host::ERR_SHAPE, "mmq_experts: bad arguments");
        if (n_tok == 0) return host::OK;
        const int64_t rows = n_tok * x_rows_per_tok;
        int32_t *gprefix = (int32_t *) ((uint8_t *) xq + (size_t) rows * host::q8_1_row_bytes(ncols));
        FNS_TRY(mmq_compact(ids, n_tok, n_used, n_expert, x_rows_per_tok, ids_src1, ids_dst, bounds, gprefix, st));
        FNS_TRY(quantize_q8_1(x, xq, ncols, rows, st));
        return mmvq_experts_div(type, table, off, ncols, nrows, xq, rows, x_rows_per_tok == 1 ? n_used : 1, ids,
                                n_tok * n_used, dst, st);
    }
    FNS_TRY(check_mmq_shape(type, ncols, nrows));
    if (!x || !xq || n_used < 1 || n_tok < 0) return host::set_error(host::ERR_SHAPE, "mmq_experts: bad arguments");
    if (n_tok == 0) return host::OK;
    // bounds holds n_expert + 1 ints (the reference's MmqIdsScratch sizing); the tile-group prefix of the GEMM goes in
    // the slack that mmq_q8_1_bytes adds after the activation images (4096 bytes >= 257 ints)
    const int64_t rows = n_tok * x_rows_per_tok;
    int32_t *gprefix = (int32_t *) ((uint8_t *) xq + (size_t) rows * mmq_image_bytes(ncols));
    FNS_TRY(mmq_compact(ids, n_tok, n_used, n_expert, x_rows_per_tok, ids_src1, ids_dst, bounds, gprefix, st));
    FNS_TRY(mmq_quant_image(x, ncols, rows, xq, st));
    return mmq_gemm_experts(type, table, off, 0, false, ncols, nrows, n_expert, xq, n_tok * n_used, ids_src1, ids_dst,
                            bounds, gprefix, dst, nullptr, nullptr, st);
}

// ---- prefill MoE layer ----------------------------------------------------------------------------------------
// The MoE section of the reference's Engine::prefill_chunk (src/engine.cu:340-357: gemm_bf16_batch, route_topk_batch,
// mmq_experts for gate and up, swiglu, amax_guard, mmq_experts for down, moe_combine_batch) for n_tok tokens, with the
// activations quantised once per token, gate and up in one pass with the SwiGLU and the Q8_1 of act fused, and the
// expert sort shared by both GEMMs.
namespace {
constexpr int kPrefillSections = 15;
void prefill_sizes(const FnsMoeLayer *L, int64_t T, size_t *sz) {
    const int64_t P = T * L->k;
    sz[0] = (size_t) T * L->n_expert * 4;                 // logits
    sz[1] = (size_t) P * 4;                               // ids
    sz[2] = (size_t) P * 4;                               // w
    sz[3] = (size_t) T * mmq_image_bytes(L->hidden);      // x images
    sz[4] = (size_t) P * act_stride(L->inter);            // act images
    sz[5] = (size_t) P * L->hidden * 4;                   // per-(token, slot) down outputs
    sz[6] = (size_t) P * 4;                               // ids_src1
    sz[7] = (size_t) P * 4;                               // ids_dst
    // bounds + group prefix, arrival counters, status word
    sz[8] = bounds_bytes(L->n_expert) + 4 * (size_t) (main_groups(L->n_expert, P) + L->n_expert) + 4;
    sz[9] = L->guard ? (size_t) P * L->inter * 4 : 0;     // f32 act (F16 guard only)
    sz[10] = (size_t) P * 4;                              // escale
    const int64_t fs = L->shexp_inter > 0 ? L->shexp_inter : 0;
    sz[11] = L->ffn_norm ? (size_t) T * L->hidden * 4 : 0;                         // RMSNorm output h
    sz[12] = L->ffn_norm ? (size_t) T * host::q8_1_row_bytes(L->hidden) : 0;      // its Q8_1 blocks (unused)
    sz[13] = fs ? (size_t) T * mmq_image_bytes(fs) : 0;                            // shared-expert act images
    sz[14] = fs ? (size_t) T * L->hidden * 4 : 0;                                  // shared-expert output
}
}  // namespace

int moe_prefill_section(const FnsMoeLayer *L, int64_t n_tok, int section, size_t *offset, size_t *bytes) {
    FNS_TRY(moe_prefill_workspace(L, n_tok, nullptr, nullptr));
    if (section < 0 || section >= kPrefillSections) return host::set_error(host::ERR_SHAPE, "moe_prefill: no section %d", section);
    size_t sz[kPrefillSections], off = 0;
    prefill_sizes(L, n_tok, sz);
    for (int i = 0; i < section; ++i) off += (sz[i] + 255) / 256 * 256;
    if (offset) *offset = off;
    if (bytes) *bytes = sz[section];
    return host::OK;
}

int moe_prefill_workspace(const FnsMoeLayer *L, int64_t n_tok, size_t *offsets, size_t *total) {
    if (!L || n_tok < 1 || n_tok * L->k > 65536)
        return host::set_error(host::ERR_SHAPE, "moe_prefill: 1 <= n_tok, n_tok * k <= 65536");
    size_t sz[kPrefillSections], off = 0;
    prefill_sizes(L, n_tok, sz);
    for (int i = 0; i < kPrefillSections; ++i) {
        if (offsets && i < 6) offsets[i] = off;
        off += (sz[i] + 255) / 256 * 256;
    }
    if (total) *total = off + 4096;
    return host::OK;
}

// The shared expert over the n_tok split-image rows of h: one GLU launch (gate and up, SwiGLU, Q8_1 of act into
// act_img) and the down launch into sh [n_tok][hidden]; both are the grouped GEMM over one dense matrix.
int mmq_dense_shared(const FnsMoeLayer *L, const void *ximg, int64_t n_tok, void *act_img, float *sh, hipStream_t st) {
    const int gt = L->shexp_gu_type ? L->shexp_gu_type : L->gu_type;
    const int dt = L->shexp_down_type ? L->shexp_down_type : L->down_type;
    FNS_TRY(check_mmq_shape(gt, L->hidden, L->shexp_inter));
    FNS_TRY(check_mmq_shape(dt, L->shexp_inter, L->hidden));
    const int groups = (int) ((n_tok + kMmqTok - 1) / kMmqTok);
    MmqArgs g{};
    g.w_dense = (const uint8_t *) L->shexp_gate;
    g.off_a = 0;
    g.off_b = (const uint8_t *) L->shexp_up - (const uint8_t *) L->shexp_gate;
    g.ncols = L->hidden;
    g.nrows = L->shexp_inter;
    g.xpack = (const uint8_t *) ximg;
    g.x_img = (int64_t) mmq_image_bytes(L->hidden);
    g.n_rows = (int) n_tok;
    g.out_pack = (uint8_t *) act_img;
    g.out_img = (int64_t) mmq_image_bytes(L->shexp_inter);
    FNS_TRY(launch_mmq(gt, true, g, groups, st));
    MmqArgs d{};
    d.w_dense = (const uint8_t *) L->shexp_down;
    d.ncols = L->shexp_inter;
    d.nrows = L->hidden;
    d.xpack = (const uint8_t *) act_img;
    d.x_img = (int64_t) mmq_image_bytes(L->shexp_inter);
    d.n_rows = (int) n_tok;
    d.dst = sh;
    return launch_mmq(dt, false, d, groups, st);
}

// Dense GEMMs on activation images already built (the dense FFN block): gate/up in one GLU launch (SwiGLU and the
// Q8_1 of act in the epilogue, act images out), and a plain launch whose K range may be split into ksplit parts
// (dst then holds ksplit partial sums, part_stride floats apart).
bool mmq_tiled(int type, int64_t ncols, int64_t nrows) {
    const bool t = host::is_kquant(type) || type == T_Q8_0 || (host::is_iq(type) && (!host::iq_needs_grid(type) ||
                                                                                      host::iq_grids_ready()));
    return t && ncols > 0 && ncols % 256 == 0 && ncols <= 65536 && nrows > 0 && nrows % kMmqRows == 0;
}

int mmq_dense_glu(int type, const void *gate, const void *up, int64_t ncols, int64_t nrows, const void *ximg,
                  int64_t n_tok, void *act_img, hipStream_t st) {
    FNS_TRY(check_mmq_shape(type, ncols, nrows));
    MmqArgs g{};
    g.w_dense = (const uint8_t *) gate;
    g.off_a = 0;
    g.off_b = (const uint8_t *) up - (const uint8_t *) gate;
    g.ncols = (int) ncols;
    g.nrows = (int) nrows;
    g.xpack = (const uint8_t *) ximg;
    g.x_img = (int64_t) mmq_image_bytes(ncols);
    g.n_rows = (int) n_tok;
    g.out_pack = (uint8_t *) act_img;
    g.out_img = (int64_t) mmq_image_bytes(nrows);
    return launch_mmq(type, true, g, (int) ((n_tok + kMmqTok - 1) / kMmqTok), st);
}

int mmq_dense_parts(int type, const void *w, int64_t ncols, int64_t nrows, const void *ximg, int64_t n_tok, float *dst,
                    int ksplit, hipStream_t st) {
    FNS_TRY(check_mmq_shape(type, ncols, nrows));
    MmqArgs d{};
    d.w_dense = (const uint8_t *) w;
    d.ncols = (int) ncols;
    d.nrows = (int) nrows;
    d.xpack = (const uint8_t *) ximg;
    d.x_img = (int64_t) mmq_image_bytes(ncols);
    d.n_rows = (int) n_tok;
    d.dst = dst;
    d.ksplit = ksplit;
    d.part_stride = n_tok * nrows;
    return launch_mmq(type, false, d, (int) ((n_tok + kMmqTok - 1) / kMmqTok), st);
}

namespace {
__global__ void k_zero_word(uint32_t *w) { *w = 0; }
}  // namespace

// The sticky status word of a prefill workspace (after the fused launch's arrival counters in section 8), read after
// the stream's work so far has completed; clear: zero it afterwards (a kernel on `st`).
int moe_prefill_status(const FnsMoeLayer *L, int64_t n_tok, void *ws, int clear, uint32_t *status, hipStream_t st) {
    if (!ws || !status) return host::set_error(host::ERR_SHAPE, "moe_prefill_status: null argument");
    size_t off;
    FNS_TRY(moe_prefill_section(L, n_tok, 8, &off, nullptr));
    const int64_t words = 3 * (L->n_expert + 1) + main_groups(L->n_expert, n_tok * L->k) + L->n_expert;
    uint32_t *word = (uint32_t *) ((uint8_t *) ws + off) + words;
    if (hipMemcpyAsync(status, word, 4, hipMemcpyDeviceToHost, st) != hipSuccess || hipStreamSynchronize(st) != hipSuccess)
        return host::set_error(host::ERR_LAUNCH, "moe_prefill_status: reading the status word failed");
    if (clear) {
        hipLaunchKernelGGL(k_zero_word, dim3(1), dim3(1), 0, st, word);
        FNS_TRY(host::check_launch("moe_prefill_status: clearing"));
    }
    return host::OK;
}

int moe_prefill_status_collect(const FnsMoeLayer *L, int64_t n_tok, void *ws, uint32_t *dst, hipStream_t st) {
    if (!ws || !dst) return host::set_error(host::ERR_SHAPE, "moe_prefill_status_collect: null argument");
    size_t off;
    FNS_TRY(moe_prefill_section(L, n_tok, 8, &off, nullptr));
    const int64_t words = 3 * (L->n_expert + 1) + main_groups(L->n_expert, n_tok * L->k) + L->n_expert;
    return status_collect((uint32_t *) ((uint8_t *) ws + off) + words, dst, st);
}

int moe_prefill(const FnsMoeLayer *L, const float *x, const float *x_resid, float *out, int64_t n_tok, void *ws,
                size_t ws_bytes, hipStream_t st) {
    if (!L || !x || !out || !ws || !L->router_w || !L->table) return host::set_error(host::ERR_SHAPE, "moe_prefill: null argument");
    size_t total;
    FNS_TRY(moe_prefill_workspace(L, n_tok, nullptr, &total));
    if (ws_bytes < total) return host::set_error(host::ERR_NOMEM, "moe_prefill: workspace %zu < %zu bytes", ws_bytes, total);
    if (L->k < 1 || L->k > 16 || L->k > L->n_expert || L->n_expert > 256)
        return host::set_error(host::ERR_SHAPE, "moe_prefill: 1 <= k <= min(16, n_expert), n_expert <= 256");
    FNS_TRY(check_mmq_shape(L->gu_type, L->hidden, L->inter));
    FNS_TRY(check_mmq_shape(L->down_type, L->inter, L->hidden));
    if (L->shexp_inter < 0 || (L->shexp_inter > 0 && (!L->shexp_gate || !L->shexp_up || !L->shexp_down)))
        return host::set_error(host::ERR_SHAPE, "moe_prefill: shared expert: gate, up and down given");
    size_t sz[kPrefillSections];
    prefill_sizes(L, n_tok, sz);
    uint8_t *sec[kPrefillSections];
    size_t off = 0;
    for (int i = 0; i < kPrefillSections; ++i) {
        sec[i] = (uint8_t *) ws + off;
        off += (sz[i] + 255) / 256 * 256;
    }
    float *logits = (float *) sec[0], *w = (float *) sec[2], *dexp = (float *) sec[5], *act = (float *) sec[9];
    float *escale = (float *) sec[10];
    int32_t *ids = (int32_t *) sec[1], *src1 = (int32_t *) sec[6], *dstr = (int32_t *) sec[7], *bounds = (int32_t *) sec[8];
    const int64_t P = n_tok * L->k;
    const char *const *table = (const char *const *) L->table;

    // RMSNorm first when the layer has one: the router and the experts read h (reference src/engine.cu:331)
    if (L->ffn_norm) {
        FNS_TRY(rms_norm_q8_1(x, L->ffn_norm, (float *) sec[11], sec[12], (int) L->hidden, L->norm_eps, (int) n_tok, st));
        x = (const float *) sec[11];
    }
    // the router GEMM and the activation image in one launch when the GEMM takes its unguarded path (whole 64-column
    // chunks, aligned rows, 32-bit offsets), else as two launches
    const int H = (int) L->hidden, NE = (int) L->n_expert;
    const bool bf = L->router_dtype == T_BF16;
    const bool one = (bf || L->router_dtype == 0) && H % 64 == 0 && (int64_t) H * std::max<int64_t>(n_tok, NE) < INT32_MAX &&
                     ((uintptr_t) x & 15) == 0 && ((uintptr_t) L->router_w & (bf ? 7 : 15)) == 0;
    if (one) {
        const int tiles_x = (int) ((n_tok + 15) / 16), n_rt = tiles_x * ((NE + 15) / 16);
        const int nxb = (H + 2047) / 2048;
        const int64_t n_img = (nxb * n_tok + 1) / 2;
        if (n_rt + n_img > INT32_MAX) return host::set_error(host::ERR_SHAPE, "prefill: grid too large");
        const dim3 g((unsigned) (n_rt + n_img));
        if (bf)
            hipLaunchKernelGGL(k_router_image<true>, g, dim3(512), 0, st, L->router_w, L->router_bias, x, logits, H, NE,
                               (int) n_tok, tiles_x, n_rt, (uint8_t *) sec[3], (int64_t) mmq_image_bytes(H), nxb);
        else
            hipLaunchKernelGGL(k_router_image<false>, g, dim3(512), 0, st, L->router_w, L->router_bias, x, logits, H,
                               NE, (int) n_tok, tiles_x, n_rt, (uint8_t *) sec[3], (int64_t) mmq_image_bytes(H), nxb);
        FNS_TRY(host::check_launch("prefill router + image"));
    } else {
        FNS_TRY(gemm_router_bias(L->router_dtype, L->router_w, L->router_bias, x, logits, L->hidden, L->n_expert,
                                 (int) n_tok, st));
        FNS_TRY(mmq_quant_image(x, L->hidden, n_tok, sec[3], st));
    }
    FNS_TRY(route_topk(logits, ids, w, L->n_expert, L->k, (int) n_tok, L->gating, L->norm_w, st));
    // gate/up (SwiGLU and the Q8_1 of act fused) and down: act image rows padded to whole cache lines; one launch
    // unless the F16 guard's whole-row amax has to sit between them (or the type pair has no fused kernel)
    const int groups = (int) main_groups(L->n_expert, P);
    const int64_t astride = act_stride(L->inter);
    int32_t *gdone = bounds + 3 * (L->n_expert + 1);
    uint32_t *status = (uint32_t *) (gdone + groups + L->n_expert);
    const bool fused = !L->guard && mmq_moe_kernel(L->gu_type, L->down_type) && P * astride < INT32_MAX;
    FNS_TRY(mmq_compact(ids, n_tok, L->k, L->n_expert, 1, src1, dstr, bounds, bounds + L->n_expert + 1, st,
                        fused ? gdone : nullptr, groups + (int) L->n_expert));
    // down: one act row per (token, slot), in the same expert order as gate/up: the sorted rows are the pairs
    // themselves (activation row = output row = p), so the gate/up sort is reused with ids_dst as the source list
    MmqArgs gu, dn;
    FNS_TRY(expert_args(L->gu_type, table, L->gate_off, L->up_off, true, L->hidden, L->inter, L->n_expert, sec[3], src1,
                        dstr, bounds, bounds + L->n_expert + 1, nullptr, sec[4], L->guard ? act : nullptr, gu, 0,
                        astride));
    FNS_TRY(expert_args(L->down_type, table, L->down_off, 0, false, L->inter, L->hidden, L->n_expert, sec[4], dstr,
                        dstr, bounds, bounds + L->n_expert + 1, dexp, nullptr, nullptr, dn, astride));
    if (fused) {
        MoeArgs m{};
        m.table = table;
        m.gate_off = (int64_t) L->gate_off;
        m.up_off = (int64_t) L->up_off;
        m.down_off = (int64_t) L->down_off;
        m.hidden = (int) L->hidden;
        m.inter = (int) L->inter;
        m.n_expert = (int) L->n_expert;
        m.n_main = groups;
        m.ximg = sec[3];
        m.x_img = (int64_t) mmq_image_bytes(L->hidden);
        m.aimg = sec[4];
        m.a_img = astride;
        m.bounds = bounds;
        m.gprefix = bounds + L->n_expert + 1;
        m.src1 = src1;
        m.dstr = dstr;
        m.dexp = dexp;
        m.gdone = gdone;
        m.status = status;
        moe_test_hooks(&m.spin_limit, &m.gwait);  // withheld arrivals; + the gate/up row blocks per group
        FNS_TRY(launch_mmq_moe(L->gu_type, L->down_type, m, st));
    } else {
        FNS_TRY(launch_mmq(L->gu_type, true, gu, groups, st));
        if (L->guard) {  // whole-row amax: a second pass over the f32 act rows (reference src/kernels.cu:534-552)
            FNS_TRY(amax_guard(act, escale, L->inter, (int) P, st));
            FNS_TRY(mmq_quant_image_scaled(act, escale, L->inter, P, sec[4], astride, st));
        }
        FNS_TRY(launch_mmq(L->down_type, false, dn, groups, st));
    }
    float *sh = nullptr;
    if (L->shexp_inter > 0) {  // shared expert (reference src/engine.cu:351-355): dense gate/up + SwiGLU, then down
        sh = (float *) sec[14];
        FNS_TRY(mmq_dense_shared(L, sec[3], n_tok, sec[13], sh, st));
    }
    return moe_combine(dexp, L->guard ? escale : nullptr, w, sh, x_resid, out, L->hidden, L->k, (int) n_tok, st);
}

}  // namespace impl

// ---- C++ API (reference names; abort on error) ----
size_t mmq_q8_1_bytes(int64_t ncols, int64_t nrows) { return impl::mmq_q8_1_bytes(ncols, nrows); }
size_t mmq_bounds_bytes(int64_t n_expert) { return impl::mmq_bounds_bytes(n_expert); }

void mmq(ggml_type type, const void *w, int64_t ncols, int64_t nrows, const float *x, int64_t n_tok, void *xq,
         float *dst, hipStream_t stream) {
    host::abort_on_error(impl::mmq(type, w, ncols, nrows, x, n_tok, xq, dst, stream), "mmq");
}

void mmq_experts(ggml_type type, const char *const *table, size_t off, int64_t ncols, int64_t nrows, int64_t n_expert,
                 const float *x, int64_t x_rows_per_tok, int64_t n_tok, const int32_t *ids, int64_t n_used,
                 MmqIdsScratch &s, float *dst, hipStream_t stream) {
    host::abort_on_error(impl::mmq_experts(type, table, off, ncols, nrows, n_expert, x, x_rows_per_tok, n_tok, ids,
                                           n_used, s.ids_src1, s.ids_dst, s.expert_bounds, s.xq, dst, stream),
                         "mmq_experts");
}

}  // namespace fns
