// mmq.hip - prefill / batched expert GEMM (MMQ) over GGUF K-quant weights for MI355X gfx950: expert-id compaction,
// Q8_1 activation images, and an int8-MFMA grouped GEMM with the SwiGLU + Q8_1 of act fused into the gate/up pass.
//
// Reference semantics: src/ggml/ggml_mmq.cu:74-129 (mmq_q8_1_bytes, mmq, mmq_experts: mm_ids_helper sorts the
// (token, slot) pairs by expert, the activations are quantised once per source row, the GEMM writes each row back to
// its (token, slot) position), include/fns/ggml_kernels.h:50-69. This is a new CDNA4 design, not ggml's mmq.cuh:
//
//   * v_mfma_i32_16x16x32_i8: A = 16 activation rows (tokens) x 32 columns, B = 32 columns x 16 weight rows, so the
//     lane that owns output (token i, weight row j) holds one weight row j = lane % 16 for 4 tokens. The lane that
//     loads row j's bytes for the B operand is the one that applies row j's block scales: no scale exchange.
//   * One MFMA covers one 32-value sub-block (Q4_K / Q5_K) - the K-quant scale granularity - so its exact int32
//     result is scaled once: acc += float(I) * (d * sc_s * d8) - dmin * m_s * (d8 * sum q8). For the 16-value scale
//     groups of Q6_K / Q3_K the B operand is split in two masked halves (one MFMA per group); their zero points
//     (32, 4) are subtracted from the codes on the way into the int8 operand, so they need no activation sums.
//   * A workgroup (4 or 8 waves) owns 64 or 128 weight rows (16 per wave) of one expert and up to 64 of that expert's
//     rows of activations (4 tiles of 16): each weight byte is read from HBM once per 64 routed rows. Activations are staged
//     per 256-column superblock in LDS (LDS-DMA of the gathered Q8_1 image rows, 288-byte row stride so the 16 rows of
//     an A fragment read spread over the banks); weights go straight to VGPRs, one superblock ahead.
//   * Gate/up: both matrices in one pass (two accumulators per output), then act = up * silu(gate) and its Q8_1 blocks
//     (32 consecutive rows = 32 consecutive act columns) written straight into the act image rows the down pass reads.
//
// Integer products are exact; per sub-block results are accumulated in fp32 in sub-block order. Outputs match the
// float64 oracle (oracle/fns_oracle.c) on the same Q8_1 activations within the fp32 tolerance of the tests.
#include "fns_block.hpp"
#include "fns_common.hpp"
#include "fns_host.hpp"
#include "fns_internal.hpp"
#include "fns_lanes.hpp"

#include "fns/ggml_kernels.h"

namespace fns {

using namespace fns::dev;

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kMmqThreads = 256;   // gate/up launch: 4 waves
constexpr int kMmqRows = 64;       // gate/up launch: weight rows per workgroup (16 per wave)
constexpr int kMmqWavesWide = 8;   // plain launch (down / dense) when nrows allows: 8 waves, 128 rows per workgroup
constexpr int kMmqTok = 64;        // activation rows per workgroup (4 MFMA tiles of 16)
constexpr int kMmqTiles = kMmqTok / 16;
constexpr int kMmqStride = 288;    // LDS bytes per staged activation row (256 + 32: spreads the A-fragment reads)
constexpr int kCompactThreads = 1024;

// ---- scratch layout of the expert path --------------------------------------------------------------------------
// bounds[n_expert + 1] (sorted-row offset of each expert), then gprefix[n_expert + 1] (prefix of ceil(n_e / 64):
// the workgroup-group index of each expert's first tile group).
inline size_t bounds_bytes(int64_t n_expert) { return (size_t) 2 * (n_expert + 1) * 4; }

// ---- compaction (ggml mm_ids_helper semantics, stable) ------------------------------------------------------------
// ids [n_tok][k] -> pairs p = t k + j sorted by expert, ties in p order: ids_dst[q] = p, ids_src1[q] = the activation
// row of p (t when x_rows_per_tok = 1, p when x_rows_per_tok = k), bounds[e] = first sorted position of expert e.
// One workgroup: histogram and prefix in LDS, then rounds of 1024 pairs ranked within each wave by ballots on the
// expert id bits (lanes sharing an expert find each other without a loop), wave counts prefixed across the round.
__global__ __launch_bounds__(kCompactThreads) void k_mmq_compact(const int32_t *__restrict__ ids, int n, int k, int ne,
                                                                 int x_rows_per_tok, int32_t *__restrict__ ids_src1,
                                                                 int32_t *__restrict__ ids_dst, int32_t *bounds,
                                                                 int32_t *gprefix) {
    __shared__ int cnt[256], base[256];
    __shared__ int wcnt[kCompactThreads / kWave][256];
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    for (int e = tid; e < 256; e += kCompactThreads) cnt[e] = 0;
    __syncthreads();
    for (int p = tid; p < n; p += kCompactThreads) {
        const int e = ids[p];
        if (e >= 0 && e < ne) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    if (wave == 0) {  // exclusive prefix over <= 256 experts: 4 per lane, then a lane scan
        int v[4], g[4], s = 0, sg = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = 4 * lane + j;
            v[j] = e < ne ? cnt[e] : 0;
            g[j] = (v[j] + kMmqTok - 1) / kMmqTok;
            s += v[j];
            sg += g[j];
        }
        int incl = s, inclg = sg;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int t = __shfl_up(incl, o, 64), tg = __shfl_up(inclg, o, 64);
            if (lane >= o) {
                incl += t;
                inclg += tg;
            }
        }
        int run = incl - s, rung = inclg - sg;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = 4 * lane + j;
            if (e < ne) {
                base[e] = run;
                bounds[e] = run;
                gprefix[e] = rung;
            }
            run += v[j];
            rung += g[j];
        }
        if (lane == 63) {
            bounds[ne] = incl;
            gprefix[ne] = inclg;
        }
    }
    __syncthreads();
    for (int r0 = 0; r0 < n; r0 += kCompactThreads) {
        const int p = r0 + tid;
        const int e = p < n ? ids[p] : -1;
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
        for (int i = tid; i < (kCompactThreads / kWave) * 256; i += kCompactThreads) (&wcnt[0][0])[i] = 0;
        __syncthreads();
        if (live && rank == 0) wcnt[wave][e] = __popcll(same);
        __syncthreads();
        if (live) {
            int pos = base[e] + rank;
            for (int w = 0; w < wave; ++w) pos += wcnt[w][e];
            ids_dst[pos] = p;
            ids_src1[pos] = x_rows_per_tok == 1 ? p / k : p;
        }
        __syncthreads();
        for (int e2 = tid; e2 < ne; e2 += kCompactThreads) {
            int s = 0;
            for (int w = 0; w < kCompactThreads / kWave; ++w) s += wcnt[w][e2];
            base[e2] += s;
        }
        __syncthreads();
    }
}

// ---- Q8_1 activation images ---------------------------------------------------------------------------------------
// One value per lane, 32-lane blocks; the image layout of fns_block.hpp (int8 q with a 16-byte skew per 256 values,
// then d, d * sum16(q), d * sum32(q) in fp32). The Q8_1 arithmetic is the reference's (q8_1_lane).
__device__ __forceinline__ void img_store(uint8_t *img, int npad, int i, const Q8Lane &r) {
    const float dh = half_to_float(float_to_half(r.d));
    float *d = (float *) (img + img_q_bytes(npad));
    img[img_q_index(i)] = (uint8_t) (int8_t) r.q;
    if (i % 32 == 0) d[i / 32] = dh;
    if (i % 16 == 0) d[npad / 32 + i / 16] = dh * (float) r.qsum16;
    if (i % 32 == 0) d[npad / 32 + npad / 16 + i / 32] = dh * (float) r.qsum32;
}

// x [rows][ncols] f32 -> image rows; grid (ceil(npad / 256), rows), 256 threads.
__global__ __launch_bounds__(256) void k_quant_image(const float *__restrict__ x, int64_t ncols, uint8_t *__restrict__ out,
                                                     int64_t img_row_bytes) {
    const int npad = (int) ((ncols + 511) / 512 * 512);
    const int row = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    const float v = i < ncols ? x[(size_t) row * ncols + i] : 0.0f;
    const Q8Lane r = q8_1_lane(v);
    if (i < npad) img_store(out + (size_t) row * img_row_bytes, npad, i, r);
}

// ---- grouped GEMM -------------------------------------------------------------------------------------------------
struct MmqArgs {
    const char *const *table;  // expert pointer table (null: dense, w_dense)
    const uint8_t *w_dense;
    int64_t off_a, off_b;      // byte offsets of the (gate) matrix and of the up matrix (GLU)
    int ncols, nrows;          // K (columns of W) and N (rows of W)
    int n_expert;
    const uint8_t *xpack;      // activation image rows
    int64_t x_img;             // bytes per activation image row
    const int32_t *bounds;     // [n_expert + 1] (null: dense)
    const int32_t *gprefix;    // [n_expert + 1]
    const int32_t *src;        // sorted position -> activation image row (null: identity)
    const int32_t *dst_rows;   // sorted position -> output row (null: identity)
    int n_rows;                // dense: number of activation rows
    float *dst;                // [out row][nrows] f32 (non-GLU)
    uint8_t *out_pack;         // GLU: act image rows (by output row)
    int64_t out_img;
    float *act_out;            // GLU: optional f32 act [out row][nrows]
};

// Weight fragments of one 256-value block for one lane (row j, column group kg = lane / 16 of every sub-block).
template <int T> struct WFrag;
template <> struct WFrag<T_Q4_K> { uint4 h; uint2 q[4]; };
template <> struct WFrag<T_Q5_K> { uint4 h; uint2 q[4]; uint2 qh; };
template <> struct WFrag<T_Q6_K> { uint2 ql[4]; uint2 qh[2]; uint4 sc; uint32_t d; };
template <> struct WFrag<T_Q3_K> { uint2 qs[2]; uint2 hm; uint4 tail; };

__device__ __forceinline__ uint2 gload8a(const uint8_t *p) {  // 8 bytes at an 8-byte-aligned global address
    const uint64_t v = *(const __attribute__((address_space(1))) uint64_t *) p;
    return make_uint2((uint32_t) v, (uint32_t) (v >> 32));
}
__device__ __forceinline__ uint2 gload8u(const uint8_t *p) {  // 8 bytes at a 2-byte-aligned global address
    uint2 v;
    __builtin_memcpy(&v, (const __attribute__((address_space(1))) uint8_t *) p, 8);
    return v;
}

template <int T> __device__ __forceinline__ void wfrag_load(const uint8_t *blk, int kg, WFrag<T> &f);
template <> __device__ __forceinline__ void wfrag_load<T_Q4_K>(const uint8_t *blk, int kg, WFrag<T_Q4_K> &f) {
    f.h = gload<uint4>(blk);
#pragma unroll
    for (int g = 0; g < 4; ++g) f.q[g] = gload8a(blk + 16 + 32 * g + 8 * kg);
}
template <> __device__ __forceinline__ void wfrag_load<T_Q5_K>(const uint8_t *blk, int kg, WFrag<T_Q5_K> &f) {
    f.h = gload<uint4>(blk);
    f.qh = gload8a(blk + 16 + 8 * kg);
#pragma unroll
    for (int g = 0; g < 4; ++g) f.q[g] = gload8a(blk + 48 + 32 * g + 8 * kg);
}
template <> __device__ __forceinline__ void wfrag_load<T_Q6_K>(const uint8_t *blk, int kg, WFrag<T_Q6_K> &f) {
#pragma unroll
    for (int n = 0; n < 2; ++n) {
        f.ql[2 * n] = gload8u(blk + 64 * n + 8 * kg);
        f.ql[2 * n + 1] = gload8u(blk + 64 * n + 32 + 8 * kg);
        f.qh[n] = gload8u(blk + 128 + 32 * n + 8 * kg);
    }
    f.sc = gload16u(blk + 192);
    f.d = gload<uint16_t>(blk + 208);
}
template <> __device__ __forceinline__ void wfrag_load<T_Q3_K>(const uint8_t *blk, int kg, WFrag<T_Q3_K> &f) {
    f.hm = gload8u(blk + 8 * kg);
    f.qs[0] = gload8u(blk + 32 + 8 * kg);
    f.qs[1] = gload8u(blk + 64 + 8 * kg);
    f.tail = gload16u(blk + 94);  // scales[12] at +2, d at +14
}

__device__ __forceinline__ long pack_long(uint32_t lo, uint32_t hi) {
    return (long) (((uint64_t) hi << 32) | lo);
}

// Per sub-block s (32 values) of the block: the int8 B operand(s) and their float scales.
//   NG = 1 (Q4_K, Q5_K): b[0] all 32 columns; acc += I * (ws[0] * d8) - wm * (d8 * sum q8)
//   NG = 2 (Q6_K, Q3_K): b[0] columns 0-15 (other lanes' bytes zero), b[1] columns 16-31; acc += I_g * (ws[g] * d8)
template <int T> struct SubB {
    long b[2];
    float ws[2], wm;
};
template <int T> constexpr int groups_of() { return (T == T_Q6_K || T == T_Q3_K) ? 2 : 1; }

template <int T> __device__ __forceinline__ SubB<T> sub_b(const WFrag<T> &f, int s, int kg);

// Sub-block index s may be a runtime value: fragments and scale bytes are picked with selects and shifts (no
// dynamically indexed register arrays).
__device__ __forceinline__ uint2 sel4(uint2 a, uint2 b, uint2 c, uint2 d, int i) { return i == 0 ? a : i == 1 ? b : i == 2 ? c : d; }
__device__ __forceinline__ uint32_t byte_dyn(uint32_t w, int i) { return (w >> (8 * i)) & 0xffu; }

// 6-bit scale and min of sub-block s of a Q4_K / Q5_K block (ggml get_scale_min_k4); h.y, h.z, h.w = scales[0..11].
__device__ __forceinline__ void k4_sc_m(const uint4 &h, int s, int &sc, int &m) {
    const int i = s & 3;
    if (s < 4) {
        sc = (int) (byte_dyn(h.y, i) & 63u);
        m = (int) (byte_dyn(h.z, i) & 63u);
    } else {
        const uint32_t b8 = byte_dyn(h.w, i);
        sc = (int) ((b8 & 0xFu) | ((byte_dyn(h.y, i) >> 6) << 4));
        m = (int) ((b8 >> 4) | ((byte_dyn(h.z, i) >> 6) << 4));
    }
}

template <> __device__ __forceinline__ SubB<T_Q4_K> sub_b<T_Q4_K>(const WFrag<T_Q4_K> &f, int s, int kg) {
    SubB<T_Q4_K> r;
    const uint2 q = sel4(f.q[0], f.q[1], f.q[2], f.q[3], s >> 1);
    const int sh = 4 * (s & 1);
    r.b[0] = pack_long((q.x >> sh) & kLo4, (q.y >> sh) & kLo4);
    int sc, m;
    k4_sc_m(f.h, s, sc, m);
    r.ws[0] = half_to_float(f.h.x & 0xffffu) * (float) sc;
    r.wm = half_to_float(f.h.x >> 16) * (float) m;
    return r;
}
template <> __device__ __forceinline__ SubB<T_Q5_K> sub_b<T_Q5_K>(const WFrag<T_Q5_K> &f, int s, int kg) {
    SubB<T_Q5_K> r;
    const uint2 q = sel4(f.q[0], f.q[1], f.q[2], f.q[3], s >> 1);
    const int sh = 4 * (s & 1);
    r.b[0] = pack_long(((q.x >> sh) & kLo4) | (((f.qh.x >> s) & 0x01010101u) << 4),
                       ((q.y >> sh) & kLo4) | (((f.qh.y >> s) & 0x01010101u) << 4));
    int sc, m;
    k4_sc_m(f.h, s, sc, m);
    r.ws[0] = half_to_float(f.h.x & 0xffffu) * (float) sc;
    r.wm = half_to_float(f.h.x >> 16) * (float) m;
    return r;
}
// Q6_K sub-block s: n = s / 4, qq = s % 4: ql[64 n + 32 (qq & 1) + l] nibble qq >> 1, qh[32 n + l] bits 2 qq,
// value - 32; scale groups 8 n + 2 qq + (l >= 16).
template <> __device__ __forceinline__ SubB<T_Q6_K> sub_b<T_Q6_K>(const WFrag<T_Q6_K> &f, int s, int kg) {
    SubB<T_Q6_K> r;
    const int n = s >> 2, qq = s & 3;
    const uint2 ql = sel4(f.ql[0], f.ql[1], f.ql[2], f.ql[3], 2 * n + (qq & 1)), qh = n == 0 ? f.qh[0] : f.qh[1];
    const int shl = 4 * (qq >> 1), shh = 2 * qq;
    const uint32_t lo = bytes_sub<32>((int) (((ql.x >> shl) & kLo4) | (((qh.x >> shh) & 0x03030303u) << 4)));
    const uint32_t hi = bytes_sub<32>((int) (((ql.y >> shl) & kLo4) | (((qh.y >> shh) & 0x03030303u) << 4)));
    const long v = pack_long(lo, hi);
    r.b[0] = kg < 2 ? v : 0;
    r.b[1] = kg < 2 ? 0 : v;
    const float d = half_to_float(f.d);
    const int g0 = 8 * n + 2 * qq;  // even: both groups in one word
    const uint32_t w0 = word(f.sc, g0 >> 2);
    r.ws[0] = d * (float) (int8_t) byte_dyn(w0, g0 & 3);
    r.ws[1] = d * (float) (int8_t) byte_dyn(w0, (g0 & 3) + 1);
    r.wm = 0.0f;
    return r;
}
// Q3_K sub-block s: n = s / 4, j = s % 4: qs[32 n + l] bits 2 j, hmask[l] bit 4 n + j (clear: -4); scale groups
// 8 n + 2 j + (l >= 16), 6-bit value - 32 (low nibbles in scales[0..7], high bit pairs in scales[8..11]).
template <> __device__ __forceinline__ SubB<T_Q3_K> sub_b<T_Q3_K>(const WFrag<T_Q3_K> &f, int s, int kg) {
    SubB<T_Q3_K> r;
    const int n = s >> 2, j = s & 3;
    const uint2 q = n == 0 ? f.qs[0] : f.qs[1];
    const int hs = 4 * n + j;
    const uint32_t lo = bytes_sub<4>((int) (((q.x >> (2 * j)) & 0x03030303u) | (((f.hm.x >> hs) & 0x01010101u) << 2)));
    const uint32_t hi = bytes_sub<4>((int) (((q.y >> (2 * j)) & 0x03030303u) | (((f.hm.y >> hs) & 0x01010101u) << 2)));
    const long v = pack_long(lo, hi);
    r.b[0] = kg < 2 ? v : 0;
    r.b[1] = kg < 2 ? 0 : v;
    const float d = half_to_float(f.tail.w >> 16);
    // tail = block bytes 94..109: scales[i] is tail byte 2 + i
    const uint32_t hi_w = (f.tail.z >> 16) | (f.tail.w << 16);  // scales[8..11]
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int g = 8 * n + 2 * j + h;
        const int lb = (g & 7) + 2;  // tail byte of scales[g & 7]
        const uint32_t lw = lb < 4 ? f.tail.x : lb < 8 ? f.tail.y : f.tail.z;
        const uint32_t b = byte_dyn(lw, lb & 3);
        const uint32_t lo4 = g < 8 ? (b & 0xFu) : (b >> 4);
        const uint32_t hi2 = (byte_dyn(hi_w, g & 3) >> (2 * (g >> 2))) & 3u;
        r.ws[h] = d * (float) ((int) (lo4 | (hi2 << 4)) - 32);
    }
    r.wm = 0.0f;
    return r;
}

// -dmin * m_s of sub-blocks kg and kg + 4 of this lane's row (Q4_K / Q5_K): the B operand of the fp32 MFMAs that add
// the min term of a whole block at once.
template <int T> __device__ __forceinline__ void neg_min_pair(const WFrag<T> &f, int kg, float &m0, float &m1) {
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        int sc, m;
        const float dmin = half_to_float(f.h.x >> 16);
        k4_sc_m(f.h, kg, sc, m);
        m0 = -(dmin * (float) m);
        k4_sc_m(f.h, kg + 4, sc, m);
        m1 = -(dmin * (float) m);
    } else {
        m0 = m1 = 0.0f;
    }
}

// LDS of one workgroup: the activation superblock chunk [kMmqTok][kMmqStride] int8 and its per-sub-block d8 and
// d8 * sum(q8) transposed to [8][kMmqTok]; reused as the act tile [kMmqTok][rows] f32 by the GLU epilogue.
struct alignas(16) MmqLds {
    uint8_t q[2][kMmqTok * kMmqStride];  // double-buffered: chunk kb + 1 lands while chunk kb is computed
    float d8[2][8][kMmqTok];
    float s8[2][8][kMmqTok];
    int src[kMmqTok];
    int dst[kMmqTok];
};

template <int T, bool GLU, int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(GLU ? 3 : 1, GLU ? 4 : 8))) void k_mmq(const MmqArgs a) {
    constexpr int NT = NW * 64, ROWS = NW * 16;  // threads, weight rows per workgroup
    static_assert(sizeof(float) * kMmqTok * ROWS <= sizeof(MmqLds::q), "act tile fits the chunk buffers");
    extern __shared__ __align__(16) uint8_t smem_raw[];
    MmqLds &L = *(MmqLds *) smem_raw;
    constexpr int BB = Traits<T>::bytes, NG = groups_of<T>();
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const int kg = lane / 16, jl = lane % 16;

    // which expert / rows of activations
    int e = 0, seg = 0, cnt = 0;
    if (a.bounds) {
        const int g = blockIdx.x;
        if (g >= a.gprefix[a.n_expert]) return;
        int lo = 0, hi = a.n_expert;  // largest e with gprefix[e] <= g
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (a.gprefix[mid] <= g) lo = mid;
            else hi = mid;
        }
        e = lo;
        seg = a.bounds[e] + (g - a.gprefix[e]) * kMmqTok;
        cnt = min(kMmqTok, a.bounds[e + 1] - seg);
    } else {
        seg = blockIdx.x * kMmqTok;
        cnt = min(kMmqTok, a.n_rows - seg);
    }
    if (cnt <= 0) return;
    const int ntile = (cnt + 15) / 16;
    for (int i = tid; i < kMmqTok; i += NT) {
        const int q = seg + min(i, cnt - 1);
        L.src[i] = a.src ? a.src[q] : q;
        L.dst[i] = a.dst_rows ? a.dst_rows[q] : q;
    }

    const uint8_t *wbase = a.table ? (const uint8_t *) gload<const char *>((const uint8_t *) (a.table + e)) : a.w_dense;
    const int row = blockIdx.y * ROWS + wave * 16 + jl;  // this lane's weight row
    const int nb = a.ncols / 256;
    const int64_t row_bytes = (int64_t) nb * BB;
    const uint8_t *wa = wbase + a.off_a + (int64_t) row * row_bytes;
    const uint8_t *wb = GLU ? wbase + a.off_b + (int64_t) row * row_bytes : nullptr;
    const int npad = (a.ncols + 511) / 512 * 512;
    const int qbytes = img_q_bytes(npad);

    v4f acc[kMmqTiles], accu[kMmqTiles];
#pragma unroll
    for (int t = 0; t < kMmqTiles; ++t) acc[t] = accu[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    WFrag<T> fa, fb, na, nb2;
    wfrag_load<T>(wa, kg, fa);
    if constexpr (GLU) wfrag_load<T>(wb, kg, fb);
    __syncthreads();  // L.src / L.dst

    // staging of superblock chunk kb into buffer kb & 1 through registers (an LDS-DMA would make every LDS read of the
    // compute loop wait for the prefetch): 18 pieces of 16 bytes per row - the 256 q bytes + 32 bytes of padding read
    // from what follows them in the same image row - loaded by load_q, written by store_q after the compute; d8 and
    // d8 * sum(q8) of the chunk's 8 sub-blocks likewise (load_scales / store_scales, stored transposed)
    const int nrow = ntile * 16, npiece = nrow * (kMmqStride / 16);
    constexpr int kPieces = (kMmqTok * (kMmqStride / 16) + NT - 1) / NT;
    uint4 qv0, qv1, qv2, qv3, qv4;  // kPieces = 5 pieces per thread (named: keeps them out of scratch)
    static_assert(kPieces <= 5, "staging registers");
    // byte offset (from a.xpack) of each of this thread's staging pieces in chunk 0; chunk kb adds kb * kImgQRow
    uint32_t qo0 = 0, qo1 = 0, qo2 = 0, qo3 = 0, qo4 = 0;
    {
        uint32_t *qo[5] = {&qo0, &qo1, &qo2, &qo3, &qo4};
#pragma unroll
        for (int u = 0; u < kPieces; ++u) {
            const int p = tid + u * NT;
            if (p < npiece) {
                const int i = p / (kMmqStride / 16), o = 16 * (p % (kMmqStride / 16));
                *qo[u] = (uint32_t) ((size_t) L.src[i] * a.x_img + o);
            }
        }
    }
#define FNS_LOAD_Q(kb)                                                                                              \
    do {                                                                                                            \
        uint4 *dstv[5] = {&qv0, &qv1, &qv2, &qv3, &qv4};                                                            \
        const uint32_t offv[5] = {qo0, qo1, qo2, qo3, qo4};                                                         \
        _Pragma("unroll") for (int u = 0; u < kPieces; ++u) {                                                       \
            if (tid + u * NT < npiece)                                                                              \
                *dstv[u] = *(const uint4 *) (a.xpack + offv[u] + (kb) * kImgQRow);                                  \
        }                                                                                                           \
    } while (0)
#define FNS_STORE_Q(kb)                                                                                             \
    do {                                                                                                            \
        const uint4 srcv[5] = {qv0, qv1, qv2, qv3, qv4};                                                            \
        _Pragma("unroll") for (int u = 0; u < kPieces; ++u) {                                                       \
            const int p = tid + u * NT;                                                                             \
            if (p < npiece) *(uint4 *) (L.q[(kb) & 1] + 16 * p) = srcv[u];                                          \
        }                                                                                                           \
    } while (0)
    float sv[8];
    const float *sbase = nullptr;  // this thread's d8 (even) or d8 * sum(q8) (odd thread) row of its token
    if (tid < 2 * kMmqTok && (tid >> 1) < cnt)
        sbase = (const float *) (a.xpack + (size_t) L.src[tid >> 1] * a.x_img + qbytes) +
                ((tid & 1) ? npad / 32 + npad / 16 : 0);
    auto load_scales = [&](int kb) {
        if (tid < 2 * kMmqTok) {
            if (sbase) {
                const float *f = sbase + 8 * kb;
                const float4 v0 = *(const float4 *) f, v1 = *(const float4 *) (f + 4);
                sv[0] = v0.x, sv[1] = v0.y, sv[2] = v0.z, sv[3] = v0.w;
                sv[4] = v1.x, sv[5] = v1.y, sv[6] = v1.z, sv[7] = v1.w;
            } else {
#pragma unroll
                for (int s = 0; s < 8; ++s) sv[s] = 0.0f;
            }
        }
    };
    auto store_scales = [&](int kb) {
        if (tid < 2 * kMmqTok) {
            const int i = tid >> 1, which = tid & 1;
#pragma unroll
            for (int s = 0; s < 8; ++s) (which ? L.s8[kb & 1] : L.d8[kb & 1])[s][i] = sv[s];
        }
    };
    FNS_LOAD_Q(0);
    load_scales(0);
    FNS_STORE_Q(0);
    store_scales(0);
    // every load of the prologue (fa / fb included) complete before the loop: the compiler's wait analysis merges the
    // loop-entry state into every iteration, and a pending fa there would put a full wait in front of each sub-block
    dma_wait();
    __syncthreads();

    for (int kb = 0; kb < nb; ++kb) {
        const int cur = kb & 1;
        if (kb + 1 < nb) {  // next chunk and next block's weights in flight while this one is computed
            FNS_LOAD_Q(kb + 1);
            load_scales(kb + 1);
            wfrag_load<T>(wa + (int64_t) (kb + 1) * BB, kg, na);
            if constexpr (GLU) wfrag_load<T>(wb + (int64_t) (kb + 1) * BB, kg, nb2);
        }
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            if (s % 2 == 0) __builtin_amdgcn_sched_barrier(0);  // pairs of sub-blocks: bounded live ranges
            const SubB<T> ba = sub_b<T>(fa, s, kg);
            SubB<T> bu;
            if constexpr (GLU) bu = sub_b<T>(fb, s, kg);
#pragma unroll
            for (int t = 0; t < kMmqTiles; ++t) {
                if (t < ntile) {
                    const long av = *(const long *) (L.q[cur] + (t * 16 + jl) * kMmqStride + 32 * s + 8 * kg);
                    const float4 d8 = *(const float4 *) &L.d8[cur][s][t * 16 + 4 * kg];
                    const float dd[4] = {d8.x, d8.y, d8.z, d8.w};
#pragma unroll
                    for (int g = 0; g < NG; ++g) {
                        const v4i z = {0, 0, 0, 0};
                        const v4i ci = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, ba.b[g], z, 0, 0, 0);
                        v4i cu = z;
                        if constexpr (GLU) cu = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bu.b[g], z, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            acc[t][r] = fmaf_((float) ci[r], ba.ws[g] * dd[r], acc[t][r]);
                            if constexpr (GLU) accu[t][r] = fmaf_((float) cu[r], bu.ws[g] * dd[r], accu[t][r]);
                        }
                    }
                }
            }
        }
        if constexpr (NG == 1) {
            // min term of the whole block: acc[token][row] -= sum_s dmin m_s (d8 sum q8)_s as two fp32 MFMAs
            // (A = d8 sum q8 of sub-blocks kg, kg + 4 per token, B = -dmin m of the same sub-blocks per row)
            float ma0, ma1, mb0 = 0.0f, mb1 = 0.0f;
            neg_min_pair<T>(fa, kg, ma0, ma1);
            if constexpr (GLU) neg_min_pair<T>(fb, kg, mb0, mb1);
#pragma unroll
            for (int t = 0; t < kMmqTiles; ++t) {
                if (t < ntile) {
                    const float x0 = L.s8[cur][kg][t * 16 + jl], x1 = L.s8[cur][kg + 4][t * 16 + jl];
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(x0, ma0, acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(x1, ma1, acc[t], 0, 0, 0);
                    if constexpr (GLU) {
                        accu[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(x0, mb0, accu[t], 0, 0, 0);
                        accu[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(x1, mb1, accu[t], 0, 0, 0);
                    }
                }
            }
        }
        if (kb + 1 < nb) {
            FNS_STORE_Q(kb + 1);
            store_scales(kb + 1);
            fa = na;
            if constexpr (GLU) fb = nb2;
        }
        __syncthreads();  // chunk kb + 1 visible; buffer kb & 1 free for chunk kb + 2
    }

#undef FNS_LOAD_Q
#undef FNS_STORE_Q
    if constexpr (!GLU) {
#pragma unroll
        for (int t = 0; t < kMmqTiles; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = t * 16 + 4 * kg + r;
                if (t < ntile && i < cnt) a.dst[(size_t) L.dst[i] * a.nrows + row] = acc[t][r];
            }
    } else {
        // act = up * silu(gate) (reference src/ggml/ggml_mmvq.cu:240-247 epilogue with zero biases), staged as
        // [token][ROWS] f32, then one Q8_1 block per (token, 32 rows) into the act image rows.
        constexpr int NB = ROWS / 32;  // Q8_1 blocks per token
        float *act = (float *) &L.q[0][0];
#pragma unroll
        for (int t = 0; t < kMmqTiles; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = t * 16 + 4 * kg + r;
                if (t < ntile) {
                    float v = accu[t][r] + 0.0f;
                    v *= silu(acc[t][r] + 0.0f);
                    act[i * ROWS + wave * 16 + jl] = v;
                }
            }
        __syncthreads();
        const int fpad = (a.nrows + 511) / 512 * 512;
        for (int p0 = wave * 2; p0 < NB * cnt; p0 += 2 * NW) {  // wave-uniform trip count
            const int p = p0 + lane / 32;
            const bool live = p < NB * cnt;
            const int i = live ? p / NB : 0, blk = p % NB;
            const int col = blockIdx.y * ROWS + 32 * blk + lane % 32;
            const float v = live ? act[i * ROWS + 32 * blk + lane % 32] : 0.0f;
            const Q8Lane q = q8_1_lane(v);
            if (live) {
                img_store(a.out_pack + (size_t) L.dst[i] * a.out_img, fpad, col, q);
                if (a.act_out) a.act_out[(size_t) L.dst[i] * a.nrows + col] = v;
            }
        }
    }
}

template <bool GLU, int NW> const void *mmq_kernel(int type) {
    switch (type) {
        case T_Q3_K: return (const void *) k_mmq<T_Q3_K, GLU, NW>;
        case T_Q4_K: return (const void *) k_mmq<T_Q4_K, GLU, NW>;
        case T_Q5_K: return (const void *) k_mmq<T_Q5_K, GLU, NW>;
        case T_Q6_K: return (const void *) k_mmq<T_Q6_K, GLU, NW>;
    }
    return nullptr;
}

int launch_mmq(int type, bool glu, const MmqArgs &a, int groups, hipStream_t st) {
    // the plain launch takes 128 rows per workgroup when nrows allows: twice the weight rows per staged activation
    // (the gate/up launch stays at 4 waves: at 8 its register budget leaves one workgroup per CU - measured slower)
    const bool wide = !glu && a.nrows % (16 * kMmqWavesWide) == 0;
    const int nw = wide ? kMmqWavesWide : 4;
    const void *fn = glu ? mmq_kernel<true, 4>(type)
                         : (wide ? mmq_kernel<false, kMmqWavesWide>(type) : mmq_kernel<false, 4>(type));
    if (!fn) return host::set_error(host::ERR_TYPE, "mmq: type %d not supported", type);
    if (groups <= 0) return host::OK;
    MmqArgs arg = a;
    void *args[] = {&arg};
    const hipError_t e = hipLaunchKernel(fn, dim3((unsigned) groups, (unsigned) (a.nrows / (16 * nw))),
                                         dim3(64 * nw), args, sizeof(MmqLds), st);
    if (e != hipSuccess) return host::set_error(host::ERR_LAUNCH, "mmq: %s", hipGetErrorString(e));
    return host::check_launch("mmq");
}

int check_mmq_shape(int type, int64_t ncols, int64_t nrows) {
    if (!host::is_kquant(type)) return host::set_error(host::ERR_TYPE, "mmq: type %d not supported", type);
    if (ncols <= 0 || ncols % 256 || nrows <= 0 || nrows % kMmqRows || ncols > 65536)
        return host::set_error(host::ERR_SHAPE, "mmq: ncols must be a positive multiple of 256, nrows of 64");
    return host::OK;
}

}  // namespace

namespace impl {

size_t mmq_image_bytes(int64_t ncols) { return (size_t) img_bytes((int) host::pad512(ncols)); }
size_t mmq_q8_1_bytes(int64_t ncols, int64_t nrows) { return (size_t) nrows * mmq_image_bytes(ncols) + 4096; }
size_t mmq_bounds_bytes(int64_t n_expert) { return bounds_bytes(n_expert); }

int mmq_quant_image(const float *x, int64_t ncols, int64_t rows, void *xpack, hipStream_t st) {
    if (!x || !xpack || ncols <= 0 || rows < 0 || rows > 65535)
        return host::set_error(host::ERR_SHAPE, "mmq quantize: bad arguments");
    if (rows == 0) return host::OK;
    const int64_t npad = host::pad512(ncols);
    hipLaunchKernelGGL(k_quant_image, dim3((unsigned) (npad / 256), (unsigned) rows), dim3(256), 0, st, x, ncols,
                       (uint8_t *) xpack, (int64_t) mmq_image_bytes(ncols));
    return host::check_launch("mmq quantize");
}

int mmq_compact(const int32_t *ids, int64_t n_tok, int64_t k, int64_t n_expert, int64_t x_rows_per_tok,
                int32_t *ids_src1, int32_t *ids_dst, int32_t *bounds, int32_t *gprefix, hipStream_t st) {
    if (!ids || !ids_src1 || !ids_dst || !bounds || !gprefix || n_tok < 0 || k < 1 || n_expert < 1 || n_expert > 256 ||
        n_tok * k > (1 << 20) || (x_rows_per_tok != 1 && x_rows_per_tok != k))
        return host::set_error(host::ERR_SHAPE, "mmq compaction: bad arguments");
    hipLaunchKernelGGL(k_mmq_compact, dim3(1), dim3(kCompactThreads), 0, st, ids, (int) (n_tok * k), (int) k,
                       (int) n_expert, (int) x_rows_per_tok, ids_src1, ids_dst, bounds, gprefix);
    return host::check_launch("mmq compaction");
}

int mmq_gemm_experts(int type, const char *const *table, size_t off_a, size_t off_b, bool glu, int64_t ncols,
                     int64_t nrows, int64_t n_expert, const void *xpack, int64_t n_pairs, const int32_t *ids_src1,
                     const int32_t *ids_dst, const int32_t *bounds, const int32_t *gprefix, float *dst, void *out_pack,
                     float *act_out, hipStream_t st) {
    FNS_TRY(check_mmq_shape(type, ncols, nrows));
    if (!table || !xpack || !bounds || !gprefix || (!glu && !dst) || (glu && !out_pack) || n_expert < 1 || n_expert > 256)
        return host::set_error(host::ERR_SHAPE, "mmq_experts: bad arguments");
    MmqArgs a{};
    a.table = table;
    a.off_a = (int64_t) off_a;
    a.off_b = (int64_t) off_b;
    a.ncols = (int) ncols;
    a.nrows = (int) nrows;
    a.n_expert = (int) n_expert;
    a.xpack = (const uint8_t *) xpack;
    a.x_img = (int64_t) mmq_image_bytes(ncols);
    a.bounds = bounds;
    a.gprefix = gprefix;
    a.src = ids_src1;
    a.dst_rows = ids_dst;
    a.dst = dst;
    a.out_pack = (uint8_t *) out_pack;
    a.out_img = (int64_t) mmq_image_bytes(nrows);
    a.act_out = act_out;
    const int groups = (int) (n_expert + (n_pairs + kMmqTok - 1) / kMmqTok);  // >= sum_e ceil(n_e / 128)
    return launch_mmq(type, glu, a, groups, st);
}

int mmq(int type, const void *w, int64_t ncols, int64_t nrows, const float *x, int64_t n_tok, void *xq, float *dst,
        hipStream_t st) {
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
constexpr int kPrefillSections = 11;
void prefill_sizes(const FnsMoeLayer *L, int64_t T, size_t *sz) {
    const int64_t P = T * L->k;
    sz[0] = (size_t) T * L->n_expert * 4;                 // logits
    sz[1] = (size_t) P * 4;                               // ids
    sz[2] = (size_t) P * 4;                               // w
    sz[3] = (size_t) T * mmq_image_bytes(L->hidden);      // x images
    sz[4] = (size_t) P * mmq_image_bytes(L->inter);       // act images
    sz[5] = (size_t) P * L->hidden * 4;                   // per-(token, slot) down outputs
    sz[6] = (size_t) P * 4;                               // ids_src1
    sz[7] = (size_t) P * 4;                               // ids_dst
    sz[8] = bounds_bytes(L->n_expert);                    // bounds + group prefix
    sz[9] = L->guard ? (size_t) P * L->inter * 4 : 0;     // f32 act (F16 guard only)
    sz[10] = (size_t) P * 4;                              // escale
}
}  // namespace

int moe_prefill_workspace(const FnsMoeLayer *L, int64_t n_tok, size_t *offsets, size_t *total) {
    if (!L || n_tok < 1 || n_tok * L->k > 65536)
        return host::set_error(host::ERR_SHAPE, "moe_prefill: 1 <= n_tok, n_tok * k <= 65536");
    size_t sz[kPrefillSections], off = 0;
    prefill_sizes(L, n_tok, sz);
    for (int i = 0; i < kPrefillSections; ++i) {
        if (offsets && i < 6) offsets[i] = off;
        off += (sz[i] + 255) / 256 * 256;
    }
    if (total) *total = off + 4096;  // slack: the GEMM reads 32 bytes past a row's q values inside its image row
    return host::OK;
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

    FNS_TRY(gemm_router_bias(L->router_dtype, L->router_w, L->router_bias, x, logits, L->hidden, L->n_expert, (int) n_tok,
                             st));
    FNS_TRY(route_topk(logits, ids, w, L->n_expert, L->k, (int) n_tok, L->gating, L->norm_w, st));
    FNS_TRY(mmq_compact(ids, n_tok, L->k, L->n_expert, 1, src1, dstr, bounds, bounds + L->n_expert + 1, st));
    FNS_TRY(mmq_quant_image(x, L->hidden, n_tok, sec[3], st));
    FNS_TRY(mmq_gemm_experts(L->gu_type, table, L->gate_off, L->up_off, true, L->hidden, L->inter, L->n_expert, sec[3],
                             P, src1, dstr, bounds, bounds + L->n_expert + 1, nullptr, sec[4], L->guard ? act : nullptr,
                             st));
    if (L->guard) {  // whole-row amax: a second pass over the f32 act rows (reference src/kernels.cu:534-552)
        FNS_TRY(amax_guard(act, escale, L->inter, (int) P, st));
        FNS_TRY(mmq_quant_image(act, L->inter, P, sec[4], st));
    }
    // down: one act row per (token, slot), in the same expert order as gate/up: the sorted rows are the pairs
    // themselves (activation row = output row = p), so the gate/up sort is reused with ids_dst as the source list
    FNS_TRY(mmq_gemm_experts(L->down_type, table, L->down_off, 0, false, L->inter, L->hidden, L->n_expert, sec[4], P,
                             dstr, dstr, bounds, bounds + L->n_expert + 1, dexp, nullptr, nullptr, st));
    return moe_combine(dexp, L->guard ? escale : nullptr, w, nullptr, x_resid, out, L->hidden, L->k, (int) n_tok, st);
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
