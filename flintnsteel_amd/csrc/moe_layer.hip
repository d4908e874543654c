// moe_layer.hip - the MoE FFN decode / speculative-verify layer for MI355X gfx950.
//
// One token (n_tok = 1), two kernels per layer:
//   k_route_quant  : router logits (one workgroup per expert row, fp32 or bf16 weights) and Q8_1 of x (the reference's
//                    36-byte blocks, plus an unpacked copy laid out as the LDS image the GEMV code reads); zeroes the
//                    fused kernel's arrival counters.
//   k_layer_fused  : one workgroup per 8 output rows, all resident at once: every workgroup ranks the top-k itself,
//                    producers compute act = up . x * silu(gate . x) for 32 rows of one slot and publish its Q8_1
//                    block, a two-level arrival count releases every workgroup, which then applies the F16 guard,
//                    computes its 8 rows of down_e . act for every slot and combines them in slot order (reference
//                    src/kernels.cu:579-586). The kernel boundary before it is the logits exchange; the software
//                    exchange inside it replaces a second boundary (measured faster than three kernels).
// Several tokens (the speculative verify, n_tok <= 4), or a shape the fused kernel cannot hold, three kernels:
//   k_route_quant  : as above; for n_tok > 1 its last workgroup routes every token once and builds the channel table
//                    (distinct experts ascending, each with its (token, slot) columns).
//   k_gate_up_q    : act rows and their Q8_1 blocks for every channel (each distinct expert's weights read once).
//   k_down_q       : the down rows of every (token, slot), the F16 guard, the combine in slot order.
//
// Caller contract: the MoE section of the reference's Engine::ffn_block (src/engine.cu:655-696) - router, route_topk,
// mmvq_experts_swiglu, amax_guard_q8_1, mmvq_experts, moe_combine - in one call. Per-(token, row) arithmetic does not
// depend on the other tokens of the call: a verify column equals the batch-1 result bit for bit (reference
// src/engine.cu:601-603).
#include "fns_block.hpp"
#include "fns_common.hpp"
#include "fns_host.hpp"
#include "fns_internal.hpp"
#include "fns_lanes.hpp"
#include "fns_quarter.hpp"
#include "fns_route.hpp"

#include <algorithm>
#include <mutex>


#include <vector>

namespace fns {

using namespace fns::dev;


namespace {

constexpr int kMaxTok = 4;
constexpr int kMaxCh = kMaxTok * 16;
// Channel table entry (n_tok > 1): expert, number of (token, slot) columns, their token rows and output rows.
constexpr int kChanInts = 2 + 2 * kMaxTok;
constexpr int kDownRows = 8;  // output rows per down workgroup
constexpr size_t kLdsBudget = 150 * 1024;  // dynamic LDS per workgroup (gfx950: 160 KiB per CU)
// Fused-kernel synchronisation words, each on its own 256-byte line: 32 group counters, the count of complete groups,
// and 32 copies of the release flag (workgroups poll copy b % 32, so no line has more than 1/32 of the pollers).
// (16 groups: 16.29 us per config-0 layer against 16.21 with 32; one counter for every producer: 17.18.)
constexpr int kSyncStride = 64, kSyncGroups = 32, kSyncLines = 2 * kSyncGroups + 1;
// Decode path override (fns_hip_moe_set_path test hook): 0 automatic, 1 never the fused kernel.
int g_path_override = 0;

struct LayerArgs {
    int H, F, NE, K, T;
    int gating, norm, guard;
    int router_dtype;
    const void *router_w;
    const float *router_bias;  // [NE] or null: added to the logits
    const char *const *table;
    int64_t gate_off, up_off, down_off;
    const float *x;        // [T][H]
    const float *x_resid;  // [T][H] or null
    float *out;            // [T][H]
    // workspace
    float *logits;        // [T][NE]
    uint8_t *xq;          // [T][q8_1_row_bytes(H)]  reference Q8_1 blocks
    int32_t *ids;         // [T][K]
    float *w;             // [T][K]
    float *act;           // [T*K][F]
    float *escale;        // [T*K]
    uint8_t *xpack;       // [T][img_bytes(Hpad)]   Q8_1 of x, LDS image
    uint8_t *apack;       // [T*K][img_bytes(Fpad)] Q8_1 of act, LDS image
    float *blk_amax;      // [T*K][Fpad / 32]
    const uint8_t **dptr; // [T*K] down matrix of each (token, slot)
    int *sync;            // fused-kernel completion counters and flags, one per 256-byte line (zeroed by the router kernel)
    int *chan;            // n_tok > 1: [kMaxCh][kChanInts] channel table, then n_distinct, then the router arrival count
    int64_t xq_row_bytes;
    int fused;            // the shape fits the fused kernel (n_tok = 1)
    int dn_defer;         // fused kernel: 10-ns ticks a workgroup without gate/up rows defers its down-row fetch
    int spin_limit;       // fused kernel: polls of the release flag before a workgroup gives up
    int withhold;         // test hook: arrivals each producer group withholds (> 0: the release never comes)
    const float *sh;      // [T][H] shared-expert output added in the combine, or null
    const uint8_t *pf;    // bytes the router kernel reads ahead for the next call (the next layer's router), or null
    int64_t pf_bytes;
    const float *norm_w;  // [H] RMSNorm weights, or null: the router kernel normalises x first
    float norm_eps;
    // the shared expert inside the fused decode kernel (gate, up [Fs][H] and down [H][Fs] blocks of the routed
    // types; shd null: not fused)
    const uint8_t *shg, *shu, *shd;
    int Fs;
    // dense mode of the gate/up and down kernels (the shared expert outside the fused kernel): one channel holding
    // every token, gate and up at dense_gu + gate_off / + up_off, down at dense_down, weight 1, no guard
    const uint8_t *dense_gu, *dense_down;
    // host side only: the caller's x (x above is then the RMSNorm output), the shared expert's buffers
    const float *x_in;
    float *act_sh, *tmp_sh, *sh_out, *amax_sh;
    uint8_t *xq_sh, *apack_sh;
};

__device__ __forceinline__ float bf16f(uint16_t b) { return __builtin_bit_cast(float, (uint32_t) b << 16); }

// Writes one lane's Q8_1 value into the LDS-image row `pack` (npad columns) at column i; lanes of one block agree
// on d and the sums.
__device__ __forceinline__ void pack_store(uint8_t *pack, int npad, int i, const Q8Lane &r) {
    const float dh = half_to_float(float_to_half(r.d));
    float *d = (float *) (pack + img_q_bytes(npad));
    pack[img_q_index(i)] = (uint8_t) (int8_t) r.q;
    if (i % 32 == 0) d[i / 32] = dh;
    if (i % 16 == 0) d[npad / 32 + i / 16] = dh * (float) r.qsum16;
    if (i % 32 == 0) d[npad / 32 + npad / 16 + i / 32] = dh * (float) r.qsum32;
}

__device__ void route_all(const LayerArgs &a);

// ---- K1: router rows + Q8_1 of x ----------------------------------------------------------------------------------
// NT-thread workgroups: the first ceil(n_expert / (NT / 256)) each compute NT / 256 router rows (256 lanes per row),
// the rest quantise NT columns of one token row. One token (NT = 256): one row per workgroup, so the router's bytes
// are spread over as many CUs as there are rows; several tokens (NT = 1024): the last router workgroup to finish
// routes every token with one group of 256 threads per token (route_all).
constexpr int kK1Threads = 1024;

template <bool NORM, int NT>
__global__ __launch_bounds__(NT) void k_route_quant(const LayerArgs a) {
    constexpr int kK1Rows = NT / 256;
    __shared__ float red[kK1Rows][4][kMaxTok];
    __shared__ float s_nred[4], s_scale[kMaxTok], s_nq[kK1Rows][4][kMaxTok];
    const int H = a.H, T = a.T;
    const int n_router_wg = (a.NE + kK1Rows - 1) / kK1Rows;
    FNS_MARK(0, blockIdx.x, 0);
    // Read-ahead of the caller's next bytes (the next layer's router): two 16-byte loads per thread issued first and
    // folded into a value no one reads (stored only if it equals a constant, into the header's spare word), so the
    // lines are in the memory-side cache when the next call's router workgroups read them.
    const int64_t pf16 = a.pf ? a.pf_bytes / 16 : 0, pf_thr = (int64_t) gridDim.x * NT;
    const int64_t pf_j = (int64_t) blockIdx.x * NT + threadIdx.x;
    uint4 pfv[2] = {};
    if (pf16 > 0) {
#pragma unroll
        for (int u = 0; u < 2; ++u) pfv[u] = ((const uint4 *) a.pf)[min(pf_j + u * pf_thr, pf16 - 1)];
    }
    auto pf_done = [&]() __attribute__((always_inline)) {
        if (pf16 <= 0) return;
        uint32_t acc = pfv[0].x ^ pfv[1].x;
        for (int64_t j = pf_j + 2 * pf_thr; j < pf16; j += pf_thr) acc ^= ((const uint4 *) a.pf)[j].x;
        if (acc == 0x9E3779B9u) a.sync[kSyncLines * kSyncStride + 1] = (int) acc;
    };
    if (NORM && (int) blockIdx.x >= n_router_wg) {
        // RMSNorm scale of each token row, by threads 0-255 in the order of the rms_norm_q8_1 kernel (same bits):
        // the quantising workgroups then read h = (scale x) w where they would read x. (The router workgroups
        // accumulate x^2 beside their dot products and scale the logit at the end: same value up to fp32 rounding,
        // with no extra round trip before their loads.)
        for (int t = 0; t < T; ++t) {
            if (threadIdx.x < 256) {
                const float *xr = a.x + (size_t) t * H;
                float s = 0.0f;
                // eight values per lane per pass, every load issued first (clamped), summed in the same order
                for (int i0 = threadIdx.x; i0 < H; i0 += 8 * 256) {
                    float v[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) v[u] = xr[min(i0 + 256 * u, H - 1)];
#pragma unroll
                    for (int u = 0; u < 8; ++u)
                        if (i0 + 256 * u < H) s += v[u] * v[u];
                }
                s = lanes_sum<64>(s);
                if (threadIdx.x % 64 == 0) s_nred[threadIdx.x / 64] = s;
            }
            __syncthreads();
            if (threadIdx.x == 0) {
                const float s = (s_nred[0] + s_nred[1]) + (s_nred[2] + s_nred[3]);
                s_scale[t] = 1.0f / sqrtf(s / H + a.norm_eps);
            }
            __syncthreads();
        }
    }
    if (blockIdx.x == 0 && threadIdx.x < kSyncLines) a.sync[threadIdx.x * kSyncStride] = 0;  // ordered before the next kernel
    if ((int) blockIdx.x < n_router_wg) {
        const int sub = threadIdx.x / 256, t256 = threadIdx.x % 256;
        const int r = blockIdx.x * kK1Rows + sub;
        float s[kMaxTok] = {0.0f, 0.0f, 0.0f, 0.0f}, ssq[kMaxTok] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (r < a.NE) {
            // four 16-byte pieces of the row per lane per pass, every load of a pass issued before the first use
            for (int i0 = t256; i0 < H / 4; i0 += 4 * 256) {
                float4 wv[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int i = i0 + 256 * u;
                    if (i < H / 4) {
                        if (a.router_dtype == T_BF16) {
                            const uint2 pk = ((const uint2 *) ((const uint16_t *) a.router_w + (size_t) r * H))[i];
                            wv[u] = make_float4(bf16f(pk.x & 0xffff), bf16f(pk.x >> 16), bf16f(pk.y & 0xffff),
                                                bf16f(pk.y >> 16));
                        } else {
                            wv[u] = ((const float4 *) ((const float *) a.router_w + (size_t) r * H))[i];
                        }
                    } else {
                        wv[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    }
                }
#pragma unroll
                for (int t = 0; t < kMaxTok; ++t) {
                    if (t < T) {
                        float4 xv[4];
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            const int i = i0 + 256 * u;
                            xv[u] = i < H / 4 ? ((const float4 *) (a.x + (size_t) t * H))[i]
                                              : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                            if (NORM && i < H / 4) {  // x^2 for the scale; x w into the dot product
                                const float4 nw = ((const float4 *) a.norm_w)[i];
                                ssq[t] += xv[u].x * xv[u].x + xv[u].y * xv[u].y + xv[u].z * xv[u].z + xv[u].w * xv[u].w;
                                xv[u] = make_float4(xv[u].x * nw.x, xv[u].y * nw.y, xv[u].z * nw.z, xv[u].w * nw.w);
                            }
                        }
#pragma unroll
                        for (int u = 0; u < 4; ++u)
                            s[t] += wv[u].x * xv[u].x + wv[u].y * xv[u].y + wv[u].z * xv[u].z + wv[u].w * xv[u].w;
                    }
                }
            }
        }
#pragma unroll
        for (int t = 0; t < kMaxTok; ++t) {
            if (t < T) {
                const float v = lanes_sum<64>(s[t]);
                if (t256 % 64 == 0) red[sub][t256 / 64][t] = v;
                if (NORM) {
                    const float q = lanes_sum<64>(ssq[t]);
                    if (t256 % 64 == 0) s_nq[sub][t256 / 64][t] = q;
                }
            }
        }
        __syncthreads();
        if (t256 < T && r < a.NE) {
            float lg = (red[sub][0][t256] + red[sub][1][t256]) + (red[sub][2][t256] + red[sub][3][t256]);
            if (NORM) {
                const float q = (s_nq[sub][0][t256] + s_nq[sub][1][t256]) + (s_nq[sub][2][t256] + s_nq[sub][3][t256]);
                lg *= 1.0f / sqrtf(q / H + a.norm_eps);
            }
            const float v = a.router_bias ? lg + a.router_bias[r] : lg;
            if (T > 1) __hip_atomic_store(a.logits + (size_t) t256 * a.NE + r, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else a.logits[(size_t) t256 * a.NE + r] = v;
        }
        FNS_MARK(0, blockIdx.x, 3);
        if (NT == kK1Threads && T > 1) {  // the last router workgroup to finish routes every token (it resets the count)
            // the logits went out as device-coherent stores; the wait below makes them complete before the arrival
            __shared__ int s_last;
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            int *done = a.chan + kMaxCh * kChanInts + 1;
            if (threadIdx.x == 0)
                s_last = __hip_atomic_fetch_add(done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == n_router_wg - 1;
            __syncthreads();
            if (s_last) {
                FNS_MARK(0, blockIdx.x, 4);
                route_all(a);
                if (threadIdx.x == 0) __hip_atomic_store(done, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        pf_done();
        return;
    }
    const int npad = (H + 511) / 512 * 512;
    const int chunks = (npad + NT - 1) / NT;
    const int chunk = blockIdx.x - n_router_wg;
    const int t = chunk / chunks, i = (chunk % chunks) * NT + threadIdx.x;
    float v = i < H ? a.x[(size_t) t * H + i] : 0.0f;
    if (NORM && i < H) v = (s_scale[t] * v) * a.norm_w[i];
    const Q8Lane r = q8_1_lane(v);  // whole 32-lane blocks: the lanes past npad form whole blocks and store nothing
    if (i < npad) {
        uint8_t *b = a.xq + (size_t) t * a.xq_row_bytes + (size_t) (i / 32) * 36;
        b[4 + i % 32] = (uint8_t) (int8_t) r.q;
        if (i % 32 == 0) *(uint32_t *) b = float_to_half(r.d) | (float_to_half(r.sum) << 16);
        pack_store(a.xpack + (size_t) t * img_bytes(npad), npad, i, r);
    }
    pf_done();
}

// ---- K2: routing + gate/up + SwiGLU + Q8_1 of act ------------------------------------------------------------------
// NT threads per workgroup; LPR lanes per row; rows per workgroup RPB = max(32, NT / LPR) (whole Q8_1 blocks of act).

// LDS of the routing preamble.
struct alignas(16) RouteLds {
    uint64_t key[kTopkScratch];
    int ids[kMaxCh];
    float pv[16];
    int sel[16];
    int wave_cnt[16];
    int e, ncol, xrow[kMaxTok], orow[kMaxTok];
};

// Gating + top-k for every token (workgroup (0, 0) publishes ids, weights and down pointers), then channel
// blockIdx.y -> expert and its (token, slot) columns (rs.ncol, rs.xrow, rs.orow): slot order for n_tok = 1, distinct
// experts ascending for n_tok > 1 (compaction: channel c takes the c-th smallest selected id). Returns the expert, or
// -1 for an idle channel. Every thread of the workgroup must call it.
__device__ __forceinline__ void publish_route(const LayerArgs &a, const RouteLds &rs, int t, int j) {
    const int e = rs.sel[j];
    a.ids[t * a.K + j] = e;
    a.w[t * a.K + j] = route_weight(rs.pv, a.K, a.norm, j);
    a.dptr[t * a.K + j] = (const uint8_t *) gload<const char *>((const uint8_t *) (a.table + e)) + a.down_off;
}

template <int NT>
__device__ __forceinline__ int route_channel(const LayerArgs &a, RouteLds &rs) {
    const int tid = threadIdx.x, wave = tid / kWave, lane64 = tid % kWave;
    const int T = a.T, K = a.K;
    const bool pub = blockIdx.x == 0 && blockIdx.y == 0;
    if (a.dense_gu) {  // dense mode: every token, in order
        if (tid == 0) {
            rs.e = 0;
            rs.ncol = T;
            for (int i = 0; i < kMaxTok; ++i) rs.xrow[i] = rs.orow[i] = i < T ? i : 0;
        }
        __syncthreads();
        return 0;
    }
    if (T == 1) {
        if (tid == 0) {
            rs.ncol = 1;
            rs.xrow[0] = 0;
            rs.orow[0] = blockIdx.y;
        }
        route_topk_block<NT>((int) threadIdx.x, a.logits, a.NE, K, a.gating, rs.key, rs.sel, rs.pv);
        if (pub && tid < K) publish_route(a, rs, 0, tid);
        return rs.sel[blockIdx.y];
    }
    // n_tok > 1: routing and compaction were done once by the router kernel; read this channel's entry
    if (tid == 0) {
        const int n_distinct = a.chan[kMaxCh * kChanInts];
        const int c = blockIdx.y;
        if (c < n_distinct) {
            const int *en = a.chan + c * kChanInts;
            rs.e = en[0];
            rs.ncol = en[1];
            for (int i = 0; i < kMaxTok; ++i) {
                rs.xrow[i] = en[2 + i];
                rs.orow[i] = en[2 + kMaxTok + i];
            }
        } else {
            rs.e = -1;
            rs.ncol = 0;
        }
    }
    __syncthreads();
    (void) wave;
    (void) lane64;
    (void) pub;
    return rs.e;
}

// Routing of n_tok > 1 tokens, run once by the last router workgroup to finish (kK1Threads = 1024 threads): group t
// of 256 threads ranks token t with the block top-k (the batch-1 routing's probabilities and selection, so the same
// bits); the weights follow route_weight (slot-order sum). The distinct experts are listed in ascending order with
// their (token, slot) columns - the channel table the gate/up workgroups read (ggml mm_ids_helper-style compaction:
// each distinct expert's weights are read once per call) - and ids, weights and down pointers are published.
__device__ void route_all(const LayerArgs &a) {
    __shared__ int s_sel[kMaxTok][16];
    __shared__ float s_pv[kMaxTok][16];
    __shared__ int8_t s_col[256][kMaxTok];  // slot + 1 of expert e in token t's selection, 0 if not selected
    __shared__ int s_wcnt[kK1Threads / kWave];
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const int T = a.T, K = a.K, NE = a.NE;
    for (int i = tid; i < 256 * kMaxTok; i += kK1Threads) (&s_col[0][0])[i] = 0;
    // each token's logits into LDS (device-scope loads: other workgroups wrote them), then each group of 256 threads
    // ranks one token with the block top-k (the groups past T repeat the last token; their result is unused)
    __shared__ __align__(16) uint64_t s_tk[kMaxTok][kTopkScratch];
    __shared__ float s_lg[kMaxTok][256];
    __shared__ const uint8_t *s_tabp[256];  // the expert table, fetched with the logits (no dependent load later)
    const int grp = tid / 256, gt = tid % 256;
    if (grp < T && gt < NE)
        s_lg[grp][gt] = __hip_atomic_load(a.logits + (size_t) grp * NE + gt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid < NE) s_tabp[tid] = gload<const uint8_t *>((const uint8_t *) (a.table + tid));
    __syncthreads();
    route_topk_block<256>(gt, s_lg[grp < T ? grp : T - 1], NE, K, a.gating, s_tk[grp], s_sel[grp], s_pv[grp]);
    __syncthreads();
    FNS_MARK(0, blockIdx.x, 6);
    if (tid < T * K) {  // (token, slot): ids, weights, down pointers
        const int t = tid / K, j = tid % K, e = s_sel[t][j];
        a.ids[tid] = e;
        a.w[tid] = route_weight(s_pv[t], K, a.norm, j);
        a.dptr[tid] = s_tabp[e] + a.down_off;
        s_col[e][t] = (int8_t) (j + 1);
    }
    __syncthreads();
    FNS_MARK(0, blockIdx.x, 8);
    // distinct experts, ascending: expert ex = tid
    const int ex = tid;
    bool present = false;
    if (ex < NE)
        for (int t = 0; t < T; ++t) present |= s_col[ex][t] != 0;
    const uint64_t m = __ballot(present);
    if (lane == 0) s_wcnt[wave] = __popcll(m);
    __syncthreads();
    int rank = __popcll(m & ((1ull << lane) - 1ull));
    for (int w = 0; w < wave; ++w) rank += s_wcnt[w];
    if (present) {
        int *en = a.chan + rank * kChanInts;
        int n = 0;
        for (int t = 0; t < T; ++t)
            if (s_col[ex][t]) {
                en[2 + n] = t;
                en[2 + kMaxTok + n] = t * K + s_col[ex][t] - 1;
                ++n;
            }
        en[0] = ex;
        en[1] = n;
    }
    if (tid == 0) {
        int total = 0;
        for (int w = 0; w < kK1Threads / kWave; ++w) total += s_wcnt[w];
        a.chan[kMaxCh * kChanInts] = total;
    }
    FNS_MARK(0, blockIdx.x, 7);
}

// SwiGLU epilogue of one row (LPR-lane partial sums) and the Q8_1 of the workgroup's RPB act rows per column.
template <int LPR, int NC>
__device__ __forceinline__ void gate_up_epilogue(const LayerArgs &a, const RouteLds &rs, float *s_act, int RPB,
                                                 int lrow, int row, int lane, const float *acc, const float *accg) {
#pragma unroll
    for (int n = 0; n < NC; ++n) {
        float v = lanes_sum<LPR>(acc[n]);
        const float gs = lanes_sum<LPR>(accg[n]);
        v += 0.0f;  // fused-GLU epilogue with zero biases (reference src/ggml/ggml_mmvq.cu:240-247)
        v *= silu(gs + 0.0f);
        if (lane == 0 && (NC == 1 || n < rs.ncol)) {
            s_act[n * RPB + lrow] = v;
            a.act[(size_t) rs.orow[n] * a.F + row] = v;
        }
    }
}

template <int NT>
__device__ __forceinline__ void quant_act(const LayerArgs &a, const RouteLds &rs, const float *s_act, int RPB, int rowb) {
    const int wave = threadIdx.x / kWave, lane64 = threadIdx.x % kWave;
    const int fpad = (a.F + 511) / 512 * 512;
    const int fbytes = img_bytes(fpad);
    const int nqb = RPB / 32, ncol = rs.ncol;
    for (int p0 = wave * 2; p0 < ncol * nqb; p0 += 2 * (NT / kWave)) {  // uniform per wave: both halves run
        const int p = p0 + lane64 / 32;
        const bool live = p < ncol * nqb;
        const int n = live ? p / nqb : 0, qb = live ? p % nqb : 0;
        const int i = rowb + qb * 32 + lane64 % 32;  // act column (= gate/up row)
        const float v = live && i < a.F ? s_act[n * RPB + qb * 32 + lane64 % 32] : 0.0f;
        const Q8Lane r = q8_1_lane(v);
        const int c = rs.orow[n];
        if (live && i < fpad) pack_store(a.apack + (size_t) c * fbytes, fpad, i, r);
        if (live && i % 32 == 0 && i < fpad) a.blk_amax[(size_t) c * (fpad / 32) + i / 32] = r.amax;
    }
}

constexpr int kGuRows = 32;  // gate/up rows per workgroup (one Q8_1 block of act)

// Quarter-block form (the decode path): 1024 threads, 32 rows per workgroup, 32 lanes per row, each lane one or more
// 64-value quarters of the row's blocks. Waves 1-15 start the copy of the x images while wave 0 loads the logits;
// after routing, wave w moves its own two up rows and two gate rows into LDS and waits only for those (no workgroup
// barrier between the weight loads and the dot products), so waves whose data lands first compute first.
constexpr int kQThreads = 1024, kQWaves = kQThreads / kWave;

// NTH threads, 32 gate/up rows per workgroup: LPR = NTH / 32 lanes per row, each lane 32 / LPR quarters of it (all of
// its loads issued before the dot products). 1024 threads: one workgroup per CU; 256 threads (the verify step, whose
// hundreds of (expert, row block) workgroups then all fit on the device at once): four per CU.
template <int TQ, int NC, int NTH = kQThreads>
__global__ __launch_bounds__(NTH) void k_gate_up_q(const LayerArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ RouteLds rs;
    constexpr int BB = Traits<TQ>::bytes, NW = NTH / kWave, LPR = NTH / kGuRows;
    float *s_act = (float *) smem;  // [NC][32]
    uint8_t *s_x = smem + NC * kGuRows * 4;
    const int tid = threadIdx.x, wave = tid / kWave;
    const int T = a.T, H = a.H;
    const int npad = (H + 511) / 512 * 512;
    const int xbytes = img_bytes(npad);
    const int wgid = blockIdx.y * gridDim.x + blockIdx.x;
    FNS_MARK(1, wgid, 0);
    iq_grids_to_lds<TQ>(tid, NTH);  // the codebook (IQ3_XXS / IQ3_S), visible after the barriers before the dots

    __shared__ const uint8_t *s_tab[256];
    // waves 1..NW-1: the x images and the expert table (so the slot address is an LDS read once routing is done)
    if (wave != 0)
        for (int i = tid - kWave; i < a.NE; i += NTH - kWave)
            s_tab[i] = gload<const uint8_t *>((const uint8_t *) (a.table + i));
    dma_waves_from<NW>(s_x, a.xpack, T * xbytes, 1);
    if (wave != 0) dma_wait();
    const int e = route_channel<NTH>(a, rs);  // the x images and the table are complete after its first barrier
    FNS_MARK(1, wgid, 1);
    if (e < 0) return;
    const int ncol = rs.ncol;

    const int nblk = H / 256;
    const int row_bytes = nblk * BB;
    const int rowb = blockIdx.x * kGuRows;
    const uint8_t *slot = a.dense_gu ? a.dense_gu : s_tab[e];
    const uint8_t *wa = slot + a.up_off + (int64_t) rowb * row_bytes;
    const uint8_t *wb = slot + a.gate_off + (int64_t) rowb * row_bytes;
    // weights straight from global memory (each lane reads its own quarters; staging them through LDS cost an LDS
    // footprint of 74 KB and a DMA wait per workgroup), with 16-byte loads when the blocks are 16-byte aligned
    const bool al16 = (((uintptr_t) wa | (uintptr_t) wb | (uintptr_t) BB) & 15u) == 0;
    FNS_MARK(1, wgid, 2);

    const int lane = tid % LPR;
    const int rl = tid / LPR, row = rowb + rl;
    ActImg img[NC];
#pragma unroll
    for (int n = 0; n < NC; ++n) img[n] = act_img(s_x + (n < ncol ? rs.xrow[n] : 0) * xbytes, npad);
    float acc[NC], accg[NC];
#pragma unroll
    for (int n = 0; n < NC; ++n) acc[n] = accg[n] = 0.0f;
    // Lane `lane` stands for the V = 32 / LPR lanes lane + LPR m of the 32-lane form and sums in its order (each
    // virtual lane's quarters in sequence, then the xor butterfly's first steps), so the result is that form's bit for
    // bit: the verify columns equal their batch-1 results.
    constexpr int V = kGuRows * 32 / NTH;
    static_assert(V == 1 || V == 4, "1024 or 256 threads");
    float vu[V][NC], vg[V][NC];
#pragma unroll
    for (int m = 0; m < V; ++m)
#pragma unroll
        for (int n = 0; n < NC; ++n) vu[m][n] = vg[m][n] = 0.0f;
#pragma unroll
    for (int m = 0; m < V; ++m) {
        for (int qi = lane + LPR * m; qi < 4 * nblk; qi += 32) {
            const int bb = qi >> 2, qt = qi & 3;
            const int off = rl * row_bytes + bb * BB;
            if (al16) {
                quarter_dot_nc<TQ, Aligned16, NC>(wa + off, img, ncol, bb, qt, vu[m]);
                quarter_dot_nc<TQ, Aligned16, NC>(wb + off, img, ncol, bb, qt, vg[m]);
            } else {
                quarter_dot_nc<TQ, Any2, NC>(wa + off, img, ncol, bb, qt, vu[m]);
                quarter_dot_nc<TQ, Any2, NC>(wb + off, img, ncol, bb, qt, vg[m]);
            }
        }
    }
#pragma unroll
    for (int n = 0; n < NC; ++n) {
        if constexpr (V == 1) {
            acc[n] = vu[0][n];
            accg[n] = vg[0][n];
        } else {
            acc[n] = (vu[0][n] + vu[2][n]) + (vu[1][n] + vu[3][n]);
            accg[n] = (vg[0][n] + vg[2][n]) + (vg[1][n] + vg[3][n]);
        }
    }
    gate_up_epilogue<LPR, NC>(a, rs, s_act, kGuRows, rl, row, lane, acc, accg);
    __syncthreads();
    FNS_MARK(1, wgid, 3);
    quant_act<NTH>(a, rs, s_act, kGuRows, rowb);
    FNS_MARK(1, wgid, 4);
}

// ---- K3: (guard) + down GEMV + combine -------------------------------------------------------------------------------
__device__ __forceinline__ float guard_scale(float amax) {
    // amax <= 1024 (the common case): the sequence below gives exactly 1 (log <= 0, ceil <= 0, clamped to 0, exp(0))
    if (amax <= 1024.0f) return 1.0f;
    float e = amax * (1.0f / 1024.0f);
    e = logf(e);
    e = e * 1.4426950408889634f;
    e = ceilf(e);
    e = fminf(fmaxf(e, 0.0f), 127.0f);
    e = e * 0.6931471805599453f;
    return expf(e);
}

// Quarter-block form of the down projection + combine: 1024 threads; the work is 2 * n_chan groups of (channel, four
// of the workgroup's eight rows), group g taken by wave g % 16. Each wave copies its channel's act image and its four
// rows into a private LDS area, waits only for its own copies and computes its four rows with 16 lanes per row.
template <int TQ>
__global__ __launch_bounds__(kQThreads) void k_down_q(const LayerArgs a) {
    // the act images of every (token, slot) channel, staged once by the whole workgroup; the down weights are read
    // by each lane straight from global memory
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float s_e[kMaxCh], s_w[kMaxCh];
    __shared__ float s_dexp[kMaxCh][kDownRows];
    __shared__ const uint8_t *s_dp[kMaxCh];
    constexpr int BB = Traits<TQ>::bytes;
    const int tid = threadIdx.x, wave = tid / kWave, lane64 = tid % kWave;
    const int T = a.T, K = a.K, F = a.F, H = a.H;
    const int CH = T * K;
    const int fpad = (F + 511) / 512 * 512;
    const int fbytes = img_bytes(fpad);
    const int r0 = blockIdx.x * kDownRows;  // hidden is a multiple of 256: all 8 rows exist
    const int nblk = F / 256;
    const int row_bytes = nblk * BB;
    FNS_MARK(2, blockIdx.x, 0);
    iq_grids_to_lds<TQ>(tid, kQThreads);  // the codebook (IQ3_XXS / IQ3_S), visible after the barriers below

    dma_waves_from<kQWaves>(smem, a.apack, CH * fbytes, 0);
    if (tid < CH) {
        const uint8_t *dp = a.dense_down ? a.dense_down : gload<const uint8_t *>((const uint8_t *) (a.dptr + tid));
        s_dp[tid] = dp + (int64_t) r0 * row_bytes;
        s_w[tid] = a.dense_down ? 1.0f : a.w[tid];
    }
    dma_wait();
    __syncthreads();
    FNS_MARK(2, blockIdx.x, 1);
    // F16 guard: a channel whose scale is not 1 is divided and re-quantised (reference src/kernels.cu:554-577)
    for (int ch = wave; ch < CH; ch += kQWaves) {
        float esc = 1.0f;
        if (a.guard) {
            float m = 0.0f;
            for (int b = lane64; b < fpad / 32; b += kWave) m = fmaxf(m, a.blk_amax[(size_t) ch * (fpad / 32) + b]);
            m = lanes_max<64>(m);
            esc = guard_scale(m);
            if (esc != 1.0f) {
                const float *src = a.act + (size_t) ch * F;
                for (int i0 = 0; i0 < fpad; i0 += kWave) {
                    const int i = i0 + lane64;
                    const Q8Lane r = q8_1_lane(i < F ? src[i] / esc : 0.0f);
                    pack_store(smem + (size_t) ch * fbytes, fpad, i, r);
                }
            }
        }
        if (lane64 == 0) {
            s_e[ch] = esc;
            if (blockIdx.x == 0) a.escale[ch] = esc;
        }
    }
    __syncthreads();
    uintptr_t mis = (uintptr_t) BB;
    for (int c = 0; c < CH; ++c) mis |= (uintptr_t) s_dp[c];
    const bool al16 = (mis & 15u) == 0;
    const int sub = lane64 / 16, lane = tid % 16;
    // A wave's (channel, 4-row) groups in batches of kDnBatch, each group as before (its quarters in sequence, then
    // the 16-lane butterfly): the batch's weight loads are all in flight before its first dot product. Groups past
    // the last one repeat a valid group (clamped; their results are dropped).
    constexpr int kDnBatch = 4;
    for (int g0 = wave; g0 < 2 * CH; g0 += kDnBatch * kQWaves) {
        float acc[kDnBatch];
#pragma unroll
        for (int u = 0; u < kDnBatch; ++u) {
            const int g = min(g0 + u * kQWaves, 2 * CH - 1);
            const int ch = g >> 1, rr = 4 * (g & 1) + sub;  // rows 4 (g & 1) .. + 3 of the workgroup's eight
            const ActImg img = act_img(smem + (size_t) ch * fbytes, fpad);
            const uint8_t *wr = s_dp[ch] + rr * row_bytes;
            acc[u] = 0.0f;
            for (int qi = lane; qi < 4 * nblk; qi += 16) {
                const int bb = qi >> 2, qt = qi & 3;
                if (al16) acc[u] += quarter_dot<TQ, Aligned16>(wr + bb * BB, img, bb, qt);
                else acc[u] += quarter_dot<TQ, Any2>(wr + bb * BB, img, bb, qt);
            }
        }
#pragma unroll
        for (int u = 0; u < kDnBatch; ++u) {
            const int g = g0 + u * kQWaves;
            const float v = lanes_sum<16>(acc[u]);
            if (g < 2 * CH && lane == 0) s_dexp[g >> 1][4 * (g & 1) + sub] = v;
        }
    }
    __syncthreads();
    FNS_MARK(2, blockIdx.x, 3);
    // combine in slot order: out[t][r] = (sum_j (dexp * e_j) * w_j + sh) (+ x_resid), sh: shared expert or 0
    if (tid < T * kDownRows) {
        const int t = tid / kDownRows, rr = tid % kDownRows, r = r0 + rr;
        float moe = (s_dexp[t * K][rr] * s_e[t * K]) * s_w[t * K];
        for (int j = 1; j < K; ++j) moe = moe + (s_dexp[t * K + j][rr] * s_e[t * K + j]) * s_w[t * K + j];
        moe = moe + (a.sh ? a.sh[(size_t) t * H + r] : 0.0f);
        a.out[(size_t) t * H + r] = a.x_resid ? moe + a.x_resid[(size_t) t * H + r] : moe;
    }
    FNS_MARK(2, blockIdx.x, 4);
}

// ---- Fused decode layer (n_tok = 1): routing + gate/up + SwiGLU + down + combine in one kernel -------------------
// hidden / 8 workgroups of 1024 threads, all resident at once (one per CU; the host checks the occupancy).
//   producers b < k * inter / 32: gate/up rows [32 u, 32 u + 32) of slot c (b = c (inter / 32) + u), as k_gate_up_q,
//                                  and their Q8_1 block (the act image and block max, written device-coherent);
//   every workgroup              : down rows [8 b, 8 b + 8) of all k slots and their combine, as k_down_q.
// Right after routing each workgroup starts the LDS-DMA of its gate/up rows and its down rows together, so all of the
// layer's expert bytes are in flight at once. A producer counts its arrival once its act stores have completed (a
// two-level count: 32 group counters, then complete groups, the last of which raises 32 release flags) and every
// workgroup waits (bounded) on its flag before it reads the act images with device-scope loads. The router kernel
// zeroes the counters; a kernel boundary orders that before this kernel. Per-(row, slot) arithmetic is that of the
// two-kernel path, so results are the same bit for bit.
constexpr int kFusedRows = 8;
#ifndef FNS_DEFER_BYTES_PER_TICK
#define FNS_DEFER_BYTES_PER_TICK 50000
#endif
constexpr int64_t kDeferBytesPerTick = FNS_DEFER_BYTES_PER_TICK;  // 5 TB/s in bytes per 10-ns tick of s_memrealtime
constexpr int kSpinLimit = 1 << 16;
constexpr uint32_t kStatusTimeout = 1u;  // FNS_STATUS_EXCHANGE_TIMEOUT
constexpr int kCpolDevice = 16;  // cache-policy bits of a device-scope (sc1) load: not served from a stale L2 line

__device__ __forceinline__ void store_dev(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_dev(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One wave's LDS-DMA of blocks [b0, b1) of consecutive type-T blocks at src into LDS at dst with the staged stride
// kStageBytes<T>: verbatim when that is the block size; otherwise piece k of a block copies bytes 16 k .. 16 k + 15 and
// its last piece the block's last 16 bytes, so every piece lies inside its block.
template <int T>
__device__ __forceinline__ void dma_blocks(uint8_t *dst, const uint8_t *src, int b0, int b1) {
    constexpr int BB = Traits<T>::bytes, SB = kStageBytes<T>;
    if constexpr (SB == BB) {
        dma_wave(dst, src, b0 * BB, b1 * BB);
    } else {
        constexpr int NP = SB / 16;
        const int lane = threadIdx.x % kWave;
        for (int p0 = b0 * NP; p0 < b1 * NP; p0 += kWave) {
            const int p = p0 + lane;
            if (p < b1 * NP) {
                const int i = p / NP, k = p % NP;
                const uint8_t *g = src + i * BB + (k < NP - 1 ? 16 * k : BB - 16);
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *) g,
                                                 (__attribute__((address_space(3))) void *) (dst + 16 * p0), 16, 0, 0);
            }
        }
    }
}

template <int TGU, int TDN, bool SH>
__global__ __launch_bounds__(kQThreads) void k_layer_fused(const LayerArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ RouteLds rs;
    __shared__ const uint8_t *s_tab[256];
    __shared__ float s_dexp[16][kFusedRows];
    __shared__ float s_e[16], s_w[16], s_act[kGuRows], s_res[kFusedRows], s_sh[kFusedRows];
    __shared__ int s_fail, s_big;
    constexpr int BG = Traits<TGU>::bytes, BD = Traits<TDN>::bytes;
    const int tid = threadIdx.x, wave = tid / kWave, lane64 = tid % kWave;
    const int H = a.H, F = a.F, K = a.K;
    const int npad = (H + 511) / 512 * 512, xbytes = img_bytes(npad);
    const int fpad = (F + 511) / 512 * 512, fbytes = img_bytes(fpad);
    const int nbg = H / 256, rbg = nbg * BG;
    const int nbd = F / 256, rbd = nbd * BD;
    const int upc = F / kGuRows;                          // producers per slot
    // the shared expert (when fused) is slot K: its producers follow the routed ones, its act image and down rows
    // follow theirs, and its down output joins the combine with weight 1
    const int Fs = SH ? a.Fs : 0, fspad = (Fs + 511) / 512 * 512, fsbytes = SH ? img_bytes(fspad) : 0;
    const int nbd_s = Fs / 256, rbd_s = nbd_s * BD;
    const int nprod = K * upc + Fs / kGuRows;
    const bool producer = (int) blockIdx.x < nprod;
    const bool shared_p = SH && producer && (int) blockIdx.x >= K * upc;
    const int c = shared_p ? K : blockIdx.x / upc;
    const int u = shared_p ? blockIdx.x - K * upc : blockIdx.x % upc;  // meaningful for producers
    const int r0 = blockIdx.x * kFusedRows;
    // LDS images of the weight rows: blocks at the staged stride (Q6_K / Q3_K padded to 16-byte multiples)
    constexpr int SG = kStageBytes<TGU>, SD = kStageBytes<TDN>;
    const int lrbg = nbg * SG, lrbd = nbd * SD, lrbd_s = nbd_s * SD;
    const int gu_region = kGuRows * lrbg, dn_region = kFusedRows * lrbd;
    uint8_t *s_x = smem;
    uint8_t *s_a = s_x + xbytes;         // [K] act images, then the shared expert's
    uint8_t *s_gu = s_a + K * fbytes + fsbytes;  // [32 up rows | 32 gate rows]
    uint8_t *s_dn = s_gu + 2 * gu_region;  // [K][8 down rows], then the shared expert's 8 rows
    FNS_MARK(1, blockIdx.x, 0);
    // the codebooks (IQ3_XXS / IQ3_S) into LDS, visible after the routing's barriers
    iq_grids_to_lds<TGU>(tid, kQThreads);
    if constexpr (TDN != TGU) iq_grids_to_lds<TDN>(tid, kQThreads);

    // 1. waves 1-15: x image and expert table; wave 0: logits. Routing (all selected slots are needed here).
    if (wave != 0 && tid - kWave < a.NE)
        s_tab[tid - kWave] = gload<const uint8_t *>((const uint8_t *) (a.table + (tid - kWave)));
    // this workgroup's residual rows, read now rather than after the exchange (x_resid may alias out: each
    // workgroup reads and writes only its own rows)
    if (wave == kQWaves - 1 && lane64 < kFusedRows) {
        s_res[lane64] = a.x_resid ? a.x_resid[r0 + lane64] : 0.0f;
        s_sh[lane64] = a.sh ? a.sh[r0 + lane64] : 0.0f;  // the shared expert's output (an earlier kernel's)
    }
    if (tid == 0) s_fail = s_big = 0;
    dma_waves_from<kQWaves>(s_x, a.xpack, xbytes, 1);
    if (wave != 0) dma_wait();
    FNS_MARK(1, blockIdx.x, 4);
    route_topk_block<kQThreads>((int) threadIdx.x, a.logits, a.NE, K, a.gating, rs.key, rs.sel, rs.pv);
    if (blockIdx.x == 0 && tid < K) publish_route(a, rs, 0, tid);
    if (tid < K) s_w[tid] = route_weight(rs.pv, K, a.norm, tid);
    FNS_MARK(1, blockIdx.x, 1);

    // 2. weights: each wave its two gate/up rows (producers), then its share of the down rows
    const uint8_t *slot = s_tab[rs.sel[producer && !shared_p ? c : 0]];
    const uint8_t *wa = (shared_p ? a.shu : slot + a.up_off) + (int64_t) (u * kGuRows) * rbg;
    const uint8_t *wb = (shared_p ? a.shg : slot + a.gate_off) + (int64_t) (u * kGuRows) * rbg;
    uintptr_t mis = producer ? ((uintptr_t) wa | (uintptr_t) wb) : 0;
    for (int j = 0; j < K; ++j) mis |= (uintptr_t) (s_tab[rs.sel[j]] + a.down_off + (int64_t) r0 * rbd);
    if (SH) mis |= (uintptr_t) (a.shd + (int64_t) r0 * rbd_s);
    const bool staged = (mis & 15u) == 0;
    // down: waves 1-15 take equal shares of the flattened [K][dn_region] image. Wave 0 takes none: its thread 0 polls
    // the release flag, and a poll's value would wait for every earlier load of its wave, down rows included.
    auto dma_down = [&]() {
        constexpr int NWD = kQWaves - 1;
        const int wd = wave - 1;
        if (wd < 0) return;
        const int per = kFusedRows * nbd, total = K * per;  // blocks of the [K][8 rows] image
        const int bp = (total + NWD - 1) / NWD, b_lo = wd * bp, b_hi = min(total, b_lo + bp);
        for (int j = b_lo / per; j < K && j * per < b_hi; ++j) {
            const int lo = max(b_lo - j * per, 0), hi = min(b_hi - j * per, per);
            dma_blocks<TDN>(s_dn + j * dn_region, s_tab[rs.sel[j]] + a.down_off + (int64_t) r0 * rbd, lo, hi);
        }
        if (SH) {  // the shared expert's rows, split over the waves the same way
            const int ps = kFusedRows * nbd_s, sp = (ps + NWD - 1) / NWD;
            dma_blocks<TDN>(s_dn + K * dn_region, a.shd + (int64_t) r0 * rbd_s, min(wd * sp, ps),
                            min((wd + 1) * sp, ps));
        }
    };
    // Producers fetch their gate/up rows first and their down rows only once those are consumed: the gate/up bytes,
    // which the critical path waits for, then get the HBM to themselves, and the down bytes land during the exchange.
    if (staged) {
        if (producer) {
            dma_blocks<TGU>(s_gu, wa, 2 * wave * nbg, (2 * wave + 2) * nbg);
            dma_blocks<TGU>(s_gu + gu_region, wb, 2 * wave * nbg, (2 * wave + 2) * nbg);
        } else {
            // Defer the down rows by about the time the layer's gate/up bytes take at 5 TB/s: those bytes are on
            // the critical path (the exchange waits for them) and otherwise share the HBM with these from the start.
            // Timing only; the down rows land long before the exchange releases.
            const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
            while (__builtin_amdgcn_s_memrealtime() - t0 < (uint64_t) a.dn_defer) __builtin_amdgcn_s_sleep(8);
            dma_down();
        }
    }
    dma_wait();
    FNS_MARK(1, blockIdx.x, 2);

    // 3. producers: gate/up rows (32 lanes per row, as k_gate_up_q) -> act -> its Q8_1 block, stored device-coherent
    if (producer) {
        const int lane = tid % 32, rl = 2 * wave + lane64 / 32;
        const ActImg img = act_img(s_x, npad);
        float acc = 0.0f, accg = 0.0f;
        for (int qi = lane; qi < 4 * nbg; qi += 32) {
            const int bb = qi >> 2, qt = qi & 3;
            const int off = rl * rbg + bb * BG, loff = rl * lrbg + bb * SG;
            const ActQ xq = act_q(img, bb, qt);  // shared by the gate and the up row
            if (staged) {
                acc += quarter_dot_r<TGU, Padded>(s_gu + loff, xq, qt);
                accg += quarter_dot_r<TGU, Padded>(s_gu + gu_region + loff, xq, qt);
            } else {
                acc += quarter_dot_r<TGU, Any2>(wa + off, xq, qt);
                accg += quarter_dot_r<TGU, Any2>(wb + off, xq, qt);
            }
        }
        FNS_MARK(1, blockIdx.x, 5);
        float v = lanes_sum<32>(acc);
        const float gs = lanes_sum<32>(accg);
        v += 0.0f;  // fused-GLU epilogue with zero biases (reference src/ggml/ggml_mmvq.cu:240-247)
        v *= silu(gs + 0.0f);
        if (lane == 0) s_act[rl] = v;
        __syncthreads();
        FNS_MARK(1, blockIdx.x, 6);
        // Wave 0 alone stores the act values, so its own wait covers them and the other waves need not wait for
        // their down rows before the arrival is counted.
        if (wave != 0 && staged) dma_down();
        if (wave == 0) {  // the 32 rows form one Q8_1 block (lanes 0-31; lanes 32-63 quantise zeros, store nothing)
            const int i = u * kGuRows + lane64 % 32;
            const Q8Lane r = q8_1_lane(lane64 < 32 ? s_act[lane64] : 0.0f);
            if (lane64 < 32) {
                // (the shared expert's image follows the routed ones; it has no f32 act or guard)
                const int ip = shared_p ? fspad : fpad;
                if (!shared_p) store_dev(a.act + (size_t) c * F + i, s_act[lane64]);
                uint8_t *img_g = a.apack + (size_t) c * fbytes;
                const float dh = half_to_float(float_to_half(r.d));
                float *dg = (float *) (img_g + img_q_bytes(ip));
                // q: 32 bytes = 8 dwords; lane 4j stores dword j, gathered from lanes 4j .. 4j+3
                const uint32_t qb = (uint32_t) (uint8_t) (int8_t) r.q;
                uint32_t word = 0;
#pragma unroll
                for (int k = 0; k < 4; ++k) word |= (uint32_t) __shfl((int) qb, (lane64 & ~3) + k, 64) << (8 * k);
                if ((lane64 & 3) == 0) store_dev((uint32_t *) (img_g + img_q_index(i)), word);
                if (lane64 == 0) {
                    store_dev(dg + i / 32, dh);
                    store_dev(dg + ip / 32 + ip / 16 + i / 32, dh * (float) r.qsum32);
                    if (!shared_p) store_dev(a.blk_amax + (size_t) c * (fpad / 32) + i / 32, r.amax);
                }
                if (lane64 % 16 == 0) store_dev(dg + ip / 32 + i / 16, dh * (float) r.qsum16);
            }
        }
        FNS_MARK(1, blockIdx.x, 7);
    }
    if (producer && wave == 0) dma_wait();  // the act stores have completed
    FNS_MARK(1, blockIdx.x, 3);
    // 4. arrival (producers) and wait (everyone; bounded: a timeout poisons this workgroup's outputs with NaN)
    if (tid == 0) {
        int *sy = a.sync;
        if (producer) {
            const int g = blockIdx.x % kSyncGroups;
            const int members = (nprod - g + kSyncGroups - 1) / kSyncGroups + a.withhold;
            const int groups = nprod < kSyncGroups ? nprod : kSyncGroups;
            if (__hip_atomic_fetch_add(sy + g * kSyncStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                    members - 1 &&
                __hip_atomic_fetch_add(sy + kSyncGroups * kSyncStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                    groups - 1)
                for (int f = 0; f < kSyncGroups; ++f)
                    __hip_atomic_store(sy + (kSyncGroups + 1 + f) * kSyncStride, 1, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (tid == 0) {
        const int *sy = a.sync;
        const int *flag = sy + (kSyncGroups + 1 + blockIdx.x % kSyncGroups) * kSyncStride;
        int spins = 0;
        while (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0) {
            if (++spins > a.spin_limit) {  // give up: outputs NaN, the sticky status word says why
                s_fail = 1;
                __hip_atomic_fetch_or((unsigned *) (a.sync + kSyncLines * kSyncStride), kStatusTimeout, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(4);
        }
    }
    __syncthreads();
    FNS_MARK(1, blockIdx.x, 8);
    // 5. act images (device-scope LDS-DMA) and the F16 guard: a slot whose scale is not 1 is divided and re-quantised
    //    (reference src/kernels.cu:554-577)
    const int abytes = K * fbytes + fsbytes;
    for (int p = wave * 1024; p < abytes; p += kQThreads * 16)
        if (p + lane64 * 16 < abytes)
            __builtin_amdgcn_global_load_lds(
                (const __attribute__((address_space(1))) void *) (a.apack + p + lane64 * 16),
                (__attribute__((address_space(3))) void *) (s_a + p), 16, 0, kCpolDevice);
    // with the guard, the block maxima [K][fpad / 32] come along in the same wait, into the gate/up rows' LDS (consumed)
    float *s_bamax = (float *) s_gu;
    if (a.guard) {
        const int mbytes = K * fpad / 8;
        for (int p = wave * 1024; p < mbytes; p += kQThreads * 16)
            if (p + lane64 * 16 < mbytes)
                __builtin_amdgcn_global_load_lds(
                    (const __attribute__((address_space(1))) void *) ((const uint8_t *) a.blk_amax + p + lane64 * 16),
                    (__attribute__((address_space(3))) void *) ((uint8_t *) s_bamax + p), 16, 0, kCpolDevice);
    }
    dma_wait();
    __syncthreads();
    FNS_MARK(1, blockIdx.x, 9);
    if (a.guard) {
        // every block maximum <= 1024 (the common case): every slot's scale is exactly 1 (guard_scale), found with
        // one compare per value and one barrier instead of a cross-lane maximum per slot; otherwise (or NaN) the
        // per-slot maxima below
        for (int i = tid; i < K * (F / 32); i += kQThreads)
            if (!(s_bamax[(i / (F / 32)) * (fpad / 32) + i % (F / 32)] <= 1024.0f)) s_big = 1;
        __syncthreads();
    }
    if (a.guard && s_big) {
        for (int ch = wave; ch < K; ch += kQWaves) {
            float m = 0.0f;
            // (the F / 32 blocks the producers wrote: the padding blocks of act are zeros and never stored here)
            for (int bl = lane64; bl < F / 32; bl += kWave) m = fmaxf(m, s_bamax[ch * (fpad / 32) + bl]);
            m = lanes_max<64>(m);
            const float esc = guard_scale(m);
            if (lane64 == 0) {
                s_e[ch] = esc;
                if (blockIdx.x == 0) a.escale[ch] = esc;
            }
            if (esc != 1.0f) {
                for (int i0 = 0; i0 < fpad; i0 += kWave) {
                    const int i = i0 + lane64;
                    const float v = i < F ? __hip_atomic_load(a.act + (size_t) ch * F + i, __ATOMIC_RELAXED,
                                                              __HIP_MEMORY_SCOPE_AGENT)
                                          : 0.0f;
                    const Q8Lane r = q8_1_lane(v / esc);
                    pack_store(s_a + ch * fbytes, fpad, i, r);
                }
            }
        }
    } else if (tid < K) {
        s_e[tid] = 1.0f;
        if (blockIdx.x == 0) a.escale[tid] = 1.0f;
    }
    __syncthreads();
    FNS_MARK(1, blockIdx.x, 10);
    // 6. down rows (16 lanes per (row, slot) item, as k_down_q), then the combine in slot order
    const int lane16 = tid % 16;
    for (int it = tid / 16; it < kFusedRows * (K + (SH ? 1 : 0)); it += kQThreads / 16) {
        const int ch = it / kFusedRows, rr = it % kFusedRows;
        const bool shc = SH && ch == K;  // the shared expert's rows
        const ActImg img = act_img(s_a + ch * fbytes, shc ? fspad : fpad);
        const int nb_c = shc ? nbd_s : nbd, rb_c = shc ? rbd_s : rbd, lrb_c = shc ? lrbd_s : lrbd;
        const uint8_t *gsrc = (shc ? a.shd : s_tab[rs.sel[ch]] + a.down_off) + (int64_t) (r0 + rr) * rb_c;
        float acc = 0.0f;
        for (int qi = lane16; qi < 4 * nb_c; qi += 16) {
            const int bb = qi >> 2, qt = qi & 3;
            if (staged) acc += quarter_dot<TDN, Padded>(s_dn + ch * dn_region + rr * lrb_c + bb * SD, img, bb, qt);
            else acc += quarter_dot<TDN, Any2>(gsrc + bb * BD, img, bb, qt);
        }
        acc = lanes_sum<16>(acc);
        if (lane16 == 0) s_dexp[ch][rr] = acc;
    }
    FNS_MARK(1, blockIdx.x, 11);
    __syncthreads();
    FNS_MARK(1, blockIdx.x, 12);
    if (tid < kFusedRows) {
        const int r = r0 + tid;
        float moe = (s_dexp[0][tid] * s_e[0]) * s_w[0];
        for (int j = 1; j < K; ++j) moe = moe + (s_dexp[j][tid] * s_e[j]) * s_w[j];
        moe = moe + (SH ? s_dexp[K][tid] : s_sh[tid]);
        float o = a.x_resid ? moe + s_res[tid] : moe;
        if (s_fail) o = __builtin_nanf("");
        a.out[r] = o;
    }
    FNS_MARK(1, blockIdx.x, 13);
}

// Fixed header at the start of every workspace, whatever the layer's shape: the fused kernel's counters and flags
// (kSyncLines lines, zeroed by the router kernel each call), then the sticky status line (not cleared per call). A
// workspace (or the no-allocation scratch) shared by layers of different shapes keeps these words at the same places.
constexpr size_t kHdrSyncOff = 0, kHdrStatusOff = (size_t) kSyncLines * kSyncStride * 4;
constexpr size_t kHeaderBytes = (kHdrStatusOff + (size_t) kSyncStride * 4 + 255) / 256 * 256;

// Fused-kernel plan for one layer shape (n_tok = 1): LDS bytes, or 0 when the shape does not fit the scheme.
// Fs > 0: with the shared expert (width Fs, the routed types) as slot K.
// Bytes per block of the fused kernel's LDS weight images (kStageBytes of the type).
inline int stage_bytes_of(int t) { return t == T_Q6_K ? kStageBytes<T_Q6_K> : t == T_Q3_K ? kStageBytes<T_Q3_K> : block_bytes(t); }
inline size_t fused_lds(int H, int F, int K, int BG, int BD, int Fs = 0) {
    // every producer is a workgroup
    if (F % kGuRows || (int64_t) K * (F / kGuRows) + Fs / kGuRows > H / kFusedRows) return 0;
    if (K + (Fs > 0 ? 1 : 0) > 16) return 0;
    // the guard's block maxima are staged where the gate/up rows were
    if ((size_t) K * host::pad512(F) / 8 > 2 * (size_t) kGuRows * (H / 256) * BG) return 0;
    size_t lds = (size_t) img_bytes((int) host::pad512(H)) + (size_t) K * img_bytes((int) host::pad512(F)) +
                 2 * (size_t) kGuRows * (H / 256) * BG + (size_t) K * kFusedRows * (F / 256) * BD + 48;
    if (Fs > 0) lds += (size_t) img_bytes((int) host::pad512(Fs)) + (size_t) kFusedRows * (Fs / 256) * BD;
    return lds <= kLdsBudget ? lds : 0;
}

// Quarter forms: sized for kMaxTok tokens whatever the call's n_tok, so a verify call and a decode call of the same
// layer take the same kernels (and so the same arithmetic).
inline size_t gate_up_q_lds_bytes(int T, int H, int BB, int NC) {
    (void) BB;
    return (size_t) NC * kGuRows * 4 + (size_t) T * img_bytes((int) host::pad512(H)) + 16;
}
inline bool gate_up_q_fits(int H, int BB) { return gate_up_q_lds_bytes(kMaxTok, H, BB, kMaxTok) <= kLdsBudget; }
inline size_t down_q_lds_bytes(int CH, int F) { return (size_t) CH * img_bytes((int) host::pad512(F)) + 16; }
inline bool down_q_fits(int CH, int F) { return down_q_lds_bytes(CH, F) <= kLdsBudget; }
// The quarter kernels hold every shape moe_layer accepts: hidden <= 16384 keeps kMaxTok x images within the LDS budget
// of the gate/up kernel, and prepare() rejects n_tok * k act images beyond 64 KiB for the down kernel. The checks
// below only restate that.
template <int TQ> int dispatch_gate_up(const LayerArgs &a, hipStream_t st) {
    if (!gate_up_q_fits(a.H, Traits<TQ>::bytes))
        return host::set_error(host::ERR_SHAPE, "moe_layer: hidden %d too large for the gate/up kernel", a.H);
    const int n_chan = a.T == 1 ? a.K : std::min(a.T * a.K, a.NE);
    const dim3 grid((unsigned) (a.F / kGuRows), (unsigned) n_chan);
    if (a.T == 1)
        hipLaunchKernelGGL((k_gate_up_q<TQ, 1>), grid, dim3(kQThreads), gate_up_q_lds_bytes(1, a.H, Traits<TQ>::bytes, 1),
                           st, a);
    else
        hipLaunchKernelGGL((k_gate_up_q<TQ, kMaxTok, 256>), grid, dim3(256),
                           gate_up_q_lds_bytes(a.T, a.H, Traits<TQ>::bytes, kMaxTok), st, a);
    return host::check_launch("moe gate_up (quarters)");
}
template <int TQ> int dispatch_down(const LayerArgs &a, hipStream_t st) {
    if (!down_q_fits(a.T * a.K, a.F))
        return host::set_error(host::ERR_SHAPE, "moe_layer: n_tok * k * inter too large for the down kernel");
    hipLaunchKernelGGL((k_down_q<TQ>), dim3((unsigned) (a.H / kDownRows)), dim3(kQThreads),
                       down_q_lds_bytes(a.T * a.K, a.F), st, a);
    return host::check_launch("moe down_combine (quarters)");
}

template <int TGU, int TDN> const void *fused_fn(bool sh) {
    return sh ? (const void *) k_layer_fused<TGU, TDN, true> : (const void *) k_layer_fused<TGU, TDN, false>;
}

template <int TGU> const void *fused_fn_by_down(int tdn, bool sh) {
    switch (tdn) {
        case T_Q3_K: return fused_fn<TGU, T_Q3_K>(sh);
        case T_Q4_K: return fused_fn<TGU, T_Q4_K>(sh);
        case T_Q5_K: return fused_fn<TGU, T_Q5_K>(sh);
        case T_Q6_K: return fused_fn<TGU, T_Q6_K>(sh);
    }
    return nullptr;
}
const void *fused_kernel(int tgu, int tdn, bool sh) {
    if (tgu == T_Q8_0 || tdn == T_Q8_0) return tgu == tdn ? fused_fn<T_Q8_0, T_Q8_0>(sh) : nullptr;
    // IQ formats: the mixes of the reference's checkpoints (IQ3_XXS / IQ3_S / IQ2_S / IQ4_XS gate and up over an
    // IQ4_XS down); other mixes that involve them take the three-kernel path
    if (host::is_iq(tgu) || host::is_iq(tdn)) {
        if (tdn != T_IQ4_XS) return nullptr;
        switch (tgu) {
            case T_IQ4_XS: return fused_fn<T_IQ4_XS, T_IQ4_XS>(sh);
            case T_IQ3_XXS: return fused_fn<T_IQ3_XXS, T_IQ4_XS>(sh);
            case T_IQ3_S: return fused_fn<T_IQ3_S, T_IQ4_XS>(sh);
            case T_IQ2_S: return fused_fn<T_IQ2_S, T_IQ4_XS>(sh);
        }
        return nullptr;
    }
    switch (tgu) {
        case T_Q3_K: return fused_fn_by_down<T_Q3_K>(tdn, sh);
        case T_Q4_K: return fused_fn_by_down<T_Q4_K>(tdn, sh);
        case T_Q5_K: return fused_fn_by_down<T_Q5_K>(tdn, sh);
        case T_Q6_K: return fused_fn_by_down<T_Q6_K>(tdn, sh);
    }
    return nullptr;
}

struct ResidencyKey {
    int dev;
    const void *fn;
    size_t lds;
    int resident;  // workgroups that fit at once on the device
};
std::mutex g_res_mu;
std::vector<ResidencyKey> g_res;

int resident_groups(const void *fn, size_t lds) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    std::lock_guard<std::mutex> lk(g_res_mu);
    for (const ResidencyKey &k : g_res)
        if (k.dev == dev && k.fn == fn && k.lds == lds) return k.resident;
    int n_cu = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kQThreads, lds) != hipSuccess)
        return 0;
    g_res.push_back({dev, fn, lds, n_cu * per_cu});
    return n_cu * per_cu;
}

// True when this call (n_tok = 1, a shape that fits) takes the fused kernel.
bool use_fused(const FnsMoeLayer *L, const LayerArgs &a) {
    if (!a.fused || g_path_override == 1) return false;
    const size_t lds = fused_lds(a.H, a.F, a.K, stage_bytes_of(L->gu_type), stage_bytes_of(L->down_type), a.shd ? a.Fs : 0);
    const void *fn = fused_kernel(L->gu_type, L->down_type, a.shd != nullptr);
    return fn && resident_groups(fn, lds) >= a.H / kFusedRows;
}

int launch_fused(const FnsMoeLayer *L, const LayerArgs &a, hipStream_t st) {
    const size_t lds = fused_lds(a.H, a.F, a.K, stage_bytes_of(L->gu_type), stage_bytes_of(L->down_type), a.shd ? a.Fs : 0);
    LayerArgs arg = a;
    // non-producer workgroups defer their down rows by the gate/up bytes' time at 5 TB/s (50,000 bytes per 10 ns)
    const int64_t gu_bytes = ((int64_t) a.K * a.F + (a.shd ? a.Fs : 0)) * 2 * (a.H / 256) * block_bytes(L->gu_type);
    arg.dn_defer = (int) std::min<int64_t>(gu_bytes / kDeferBytesPerTick, 2000);
    void *args[] = {&arg};
    const hipError_t e = hipLaunchKernel(fused_kernel(L->gu_type, L->down_type, a.shd != nullptr),
                                         dim3((unsigned) (a.H / kFusedRows)),
                                         dim3(kQThreads), args, lds, st);
    if (e != hipSuccess) return host::set_error(host::ERR_LAUNCH, "moe fused layer: %s", hipGetErrorString(e));
    return host::check_launch("moe fused layer");
}

int by_type_gate_up(int t, const LayerArgs &a, hipStream_t st) {
    switch (t) {
        case T_Q3_K: return dispatch_gate_up<T_Q3_K>(a, st);
        case T_Q4_K: return dispatch_gate_up<T_Q4_K>(a, st);
        case T_Q5_K: return dispatch_gate_up<T_Q5_K>(a, st);
        case T_Q6_K: return dispatch_gate_up<T_Q6_K>(a, st);
        case T_Q8_0: return dispatch_gate_up<T_Q8_0>(a, st);
        case T_IQ4_XS: return dispatch_gate_up<T_IQ4_XS>(a, st);
        case T_IQ3_XXS: return dispatch_gate_up<T_IQ3_XXS>(a, st);
        case T_IQ3_S: return dispatch_gate_up<T_IQ3_S>(a, st);
        case T_IQ2_S: return dispatch_gate_up<T_IQ2_S>(a, st);
    }
    return host::set_error(host::ERR_TYPE, "moe_layer: gate/up type %d not supported", t);
}

int by_type_down(int t, const LayerArgs &a, hipStream_t st) {
    switch (t) {
        case T_Q3_K: return dispatch_down<T_Q3_K>(a, st);
        case T_Q4_K: return dispatch_down<T_Q4_K>(a, st);
        case T_Q5_K: return dispatch_down<T_Q5_K>(a, st);
        case T_Q6_K: return dispatch_down<T_Q6_K>(a, st);
        case T_Q8_0: return dispatch_down<T_Q8_0>(a, st);
        case T_IQ4_XS: return dispatch_down<T_IQ4_XS>(a, st);
        case T_IQ3_XXS: return dispatch_down<T_IQ3_XXS>(a, st);
        case T_IQ3_S: return dispatch_down<T_IQ3_S>(a, st);
        case T_IQ2_S: return dispatch_down<T_IQ2_S>(a, st);
    }
    return host::set_error(host::ERR_TYPE, "moe_layer: down type %d not supported", t);
}

size_t align256(size_t v) { return (v + 255) / 256 * 256; }
constexpr int kSections = 19;

// Byte sizes of the workspace sections: 0 logits, 1 xq, 2 ids, 3 w, 4 act, 5 escale (documented in fns_hip.h),
// then internal: 6 xpack, 7 apack, 8 blk_amax, 9 dptr, 10 sync, 11 channel table + arrival count (n_tok > 1),
// 12 (unused), 13 shared-expert act, 14 its gate (n_tok > 1), 15 Q8_1 of its act, 16 its output sh,
// 17 its act images, 18 their block maxima (the dense-mode kernels).
void section_sizes(const FnsMoeLayer *L, int n_tok, size_t *sizes) {
    const size_t hpad = (size_t) host::pad512(L->hidden), fpad = (size_t) host::pad512(L->inter);
    const size_t ch = (size_t) n_tok * L->k;
    sizes[0] = (size_t) n_tok * L->n_expert * 4;
    sizes[1] = (size_t) n_tok * host::q8_1_row_bytes(L->hidden);
    sizes[2] = ch * 4;
    sizes[3] = ch * 4;
    sizes[4] = ch * L->inter * 4;
    sizes[5] = ch * 4;
    sizes[6] = (size_t) n_tok * img_bytes((int) hpad);
    sizes[7] = ch * img_bytes((int) fpad) + (L->shexp_inter > 0 ? img_bytes((int) host::pad512(L->shexp_inter)) : 0);
    sizes[8] = ch * (fpad / 32) * 4;
    sizes[9] = ch * 8;
    sizes[10] = 0;  // (the synchronisation words live in the fixed header before section 0)
    sizes[11] = (size_t) (kMaxCh * kChanInts + 2) * 4;
    const size_t fs = L->shexp_inter > 0 ? (size_t) L->shexp_inter : 0;
    sizes[12] = 0;  // (unused: the router kernel applies the RMSNorm)
    sizes[13] = (size_t) n_tok * fs * 4;
    sizes[14] = n_tok > 1 ? (size_t) n_tok * fs * 4 : 0;
    sizes[15] = fs ? (size_t) n_tok * host::q8_1_row_bytes((int64_t) fs) : 0;
    sizes[16] = fs ? (size_t) n_tok * L->hidden * 4 : 0;
    sizes[17] = fs ? (size_t) n_tok * img_bytes((int) host::pad512((int64_t) fs)) : 0;
    sizes[18] = fs ? (size_t) n_tok * (host::pad512((int64_t) fs) / 32) * 4 : 0;
}

}  // namespace

namespace impl {

int moe_workspace_layout(const FnsMoeLayer *L, int n_tok, size_t *offsets, size_t *total) {
    if (!L || n_tok < 1 || n_tok > kMaxTok)
        return host::set_error(host::ERR_SHAPE, "moe_layer: 1 <= n_tok <= %d (larger batches use the MMQ path)", kMaxTok);
    if (L->k < 1 || L->k > 16 || L->hidden <= 0 || L->inter <= 0 || L->n_expert < 1)
        return host::set_error(host::ERR_SHAPE, "moe_layer: bad shape");
    size_t sizes[kSections];
    section_sizes(L, n_tok, sizes);
    size_t off = kHeaderBytes;
    for (int i = 0; i < kSections; ++i) {
        if (offsets && i < 6) offsets[i] = off;
        off += align256(sizes[i]);
    }
    if (total) *total = off;
    return host::OK;
}

// Test hooks (fns_hip_moe_set_test_hooks): the fused kernel's poll limit and withheld arrivals for the calls that
// follow. Set them only while no other thread launches layers.
static int g_spin_limit = kSpinLimit, g_withhold = 0;

int moe_set_test_hooks(int spin_limit, int withhold) {
    if (spin_limit < 0 || withhold < 0) return host::set_error(host::ERR_SHAPE, "moe_set_test_hooks: negative value");
    g_spin_limit = spin_limit ? spin_limit : kSpinLimit;
    g_withhold = withhold;
    return host::OK;
}
void moe_test_hooks(int *spin_limit, int *withhold) {
    *spin_limit = g_spin_limit;
    *withhold = g_withhold;
}

// Validates and fills the kernel arguments of one call.
static int prepare(const FnsMoeLayer *L, const float *x, const float *x_resid, float *out, int n_tok, void *ws,
                   size_t ws_bytes, LayerArgs &a) {
    if (!L || !x || !out || !ws || !L->router_w || !L->table)
        return host::set_error(host::ERR_SHAPE, "moe_layer: null argument");
    size_t total;
    FNS_TRY(moe_workspace_layout(L, n_tok, nullptr, &total));
    if (ws_bytes < total) return host::set_error(host::ERR_NOMEM, "moe_layer: workspace %zu < %zu bytes", ws_bytes, total);
    if (L->hidden % 256 || L->inter % 256 || L->hidden > 16384 || L->inter > 16384)
        return host::set_error(host::ERR_SHAPE, "moe_layer: hidden and inter must be positive multiples of 256 (<= 16384)");
    if (L->n_expert > 256 || L->k > L->n_expert)
        return host::set_error(host::ERR_SHAPE, "moe_layer: 1 <= k <= min(16, n_expert), n_expert <= 256");
    if (L->gating != 0 && L->gating != 1) return host::set_error(host::ERR_SHAPE, "moe_layer: bad gating");
    if (L->shexp_inter < 0 || L->shexp_inter % 256 || L->shexp_inter > 16384 ||
        (L->shexp_inter > 0 && (!L->shexp_gate || !L->shexp_up || !L->shexp_down)))
        return host::set_error(host::ERR_SHAPE, "moe_layer: shared expert: width a multiple of 256 (<= 16384), "
                                                "gate, up and down given");
    if (L->shexp_inter > 0 && ((L->shexp_gu_type && !host::is_supported(L->shexp_gu_type)) ||
                               (L->shexp_down_type && !host::is_supported(L->shexp_down_type))))
        return host::set_error(host::ERR_TYPE, "moe_layer: shared expert types %d/%d not supported", L->shexp_gu_type,
                               L->shexp_down_type);
    if (L->router_dtype != 0 && L->router_dtype != T_BF16)
        return host::set_error(host::ERR_TYPE, "moe_layer: router dtype %d not supported", L->router_dtype);
    if (!host::is_supported(L->gu_type) || !host::is_supported(L->down_type))
        return host::set_error(host::ERR_TYPE, "moe_layer: expert types %d/%d not supported", L->gu_type, L->down_type);
    const size_t lds_down = (size_t) n_tok * L->k * img_bytes((int) host::pad512(L->inter));
    if (lds_down > 64 * 1024)
        return host::set_error(host::ERR_SHAPE, "moe_layer: n_tok * k * inter too large for the down kernel's LDS");
    size_t sizes[kSections];
    section_sizes(L, n_tok, sizes);
    uint8_t *sec[kSections];
    size_t off = kHeaderBytes;
    for (int i = 0; i < kSections; ++i) {
        sec[i] = (uint8_t *) ws + off;
        off += align256(sizes[i]);
    }
    a = LayerArgs{};
    a.H = L->hidden;
    a.F = L->inter;
    a.NE = L->n_expert;
    a.K = L->k;
    a.T = n_tok;
    a.gating = L->gating;
    a.norm = L->norm_w;
    a.guard = L->guard;
    a.router_dtype = L->router_dtype;
    a.router_w = L->router_w;
    a.router_bias = L->router_bias;
    a.table = (const char *const *) L->table;
    a.gate_off = (int64_t) L->gate_off;
    a.up_off = (int64_t) L->up_off;
    a.down_off = (int64_t) L->down_off;
    a.x = x;
    a.x_resid = x_resid;
    a.out = out;
    a.logits = (float *) sec[0];
    a.xq = sec[1];
    a.ids = (int32_t *) sec[2];
    a.w = (float *) sec[3];
    a.act = (float *) sec[4];
    a.escale = (float *) sec[5];
    a.xpack = sec[6];
    a.apack = sec[7];
    a.blk_amax = (float *) sec[8];
    a.dptr = (const uint8_t **) sec[9];
    a.sync = (int *) ((uint8_t *) ws + kHdrSyncOff);  // the status word follows at kHdrStatusOff
    a.spin_limit = g_spin_limit;
    a.withhold = g_withhold;
    a.chan = (int *) sec[11];
    a.xq_row_bytes = host::q8_1_row_bytes(L->hidden);
    // the shared expert rides in the fused kernel when it has the routed types and the shape still fits
    const bool sh_same = L->shexp_inter > 0 && (!L->shexp_gu_type || L->shexp_gu_type == L->gu_type) &&
                         (!L->shexp_down_type || L->shexp_down_type == L->down_type);
    const int fs_fused = n_tok == 1 && sh_same &&
                                 fused_lds(a.H, a.F, a.K, stage_bytes_of(L->gu_type), stage_bytes_of(L->down_type),
                                           L->shexp_inter) > 0
                             ? L->shexp_inter
                             : 0;
    a.fused = n_tok == 1 && fused_lds(a.H, a.F, a.K, stage_bytes_of(L->gu_type), stage_bytes_of(L->down_type),
                                      L->shexp_inter > 0 ? fs_fused : 0) > 0 &&
              (L->shexp_inter == 0 || fs_fused > 0);
    a.x_in = x;
    a.norm_w = L->ffn_norm;  // the router kernel reads h = RMSNorm(x) in place of x
    a.norm_eps = L->norm_eps;
    a.pf = (const uint8_t *) L->prefetch;
    a.pf_bytes = L->prefetch ? (int64_t) L->prefetch_bytes : 0;
    if (L->shexp_inter > 0) {
        a.act_sh = (float *) sec[13];
        a.tmp_sh = (float *) sec[14];
        a.xq_sh = sec[15];
        a.sh_out = (float *) sec[16];
        a.apack_sh = sec[17];
        a.amax_sh = (float *) sec[18];
        a.sh = a.sh_out;
        if (a.fused) {  // candidate for the fused kernel; launch_stage falls back when it cannot be resident
            a.shg = (const uint8_t *) L->shexp_gate;
            a.shu = (const uint8_t *) L->shexp_up;
            a.shd = (const uint8_t *) L->shexp_down;
            a.Fs = L->shexp_inter;
        }
    }
    return host::OK;
}

// The shared expert of the reference's ffn_block (src/engine.cu:685-690, dense_glu then gemv): gate and up over the
// Q8_1 of h (one fused GLU launch for one column, else two GEMVs and the GLU), Q8_1 of act, down.
static int launch_shared(const FnsMoeLayer *L, const LayerArgs &a, hipStream_t st) {
    const int gt = L->shexp_gu_type ? L->shexp_gu_type : L->gu_type;
    const int dt = L->shexp_down_type ? L->shexp_down_type : L->down_type;
    const int64_t H = a.H, Fs = L->shexp_inter;
    if (gate_up_q_fits(a.H, block_bytes(gt)) && down_q_fits(a.T, (int) Fs)) {
        // The quarter kernels of the routed experts in dense mode: per (row, token) the arithmetic of the fused
        // kernel's shared expert, so a verify column equals its batch-1 result bit for bit.
        LayerArgs s = a;
        s.F = (int) Fs;
        s.K = 1;
        s.NE = 1;
        s.guard = 0;
        s.gate_off = 0;
        s.up_off = (const uint8_t *) L->shexp_up - (const uint8_t *) L->shexp_gate;
        s.dense_gu = (const uint8_t *) L->shexp_gate;
        s.dense_down = (const uint8_t *) L->shexp_down;
        s.act = a.act_sh;
        s.apack = a.apack_sh;
        s.blk_amax = a.amax_sh;
        s.out = a.sh_out;
        s.x_resid = nullptr;
        s.sh = nullptr;
        s.fused = 0;
        s.shd = nullptr;
        FNS_TRY(by_type_gate_up(gt, s, st));
        return by_type_down(dt, s, st);
    }
    if (a.T == 1) {
        FNS_TRY(mmvq_swiglu(gt, L->shexp_gate, L->shexp_up, H, Fs, a.xq, a.act_sh, st));
    } else {
        FNS_TRY(mmvq(gt, L->shexp_gate, H, Fs, a.xq, a.tmp_sh, a.T, st));
        FNS_TRY(mmvq(gt, L->shexp_up, H, Fs, a.xq, a.act_sh, a.T, st));
        FNS_TRY(glu_mmvq(a.tmp_sh, a.act_sh, a.act_sh, (int) (a.T * Fs), st));
    }
    FNS_TRY(quantize_q8_1(a.act_sh, a.xq_sh, Fs, a.T, st));
    return mmvq(dt, L->shexp_down, Fs, H, a.xq_sh, a.sh_out, a.T, st);
}

static int launch_stage(const FnsMoeLayer *L, const LayerArgs &a, int stage, hipStream_t st) {
    if (stage == 0) {  // [RMSNorm +] router + Q8_1 of x, [shared expert]
        const int nt = a.T == 1 ? 256 : kK1Threads, rows = nt / 256;
        const int chunks = (int) ((host::pad512(L->hidden) + nt - 1) / nt);
        const dim3 grid((unsigned) ((L->n_expert + rows - 1) / rows + chunks * a.T));
        if (a.T == 1) {
            if (a.norm_w) hipLaunchKernelGGL((k_route_quant<true, 256>), grid, dim3(256), 0, st, a);
            else hipLaunchKernelGGL((k_route_quant<false, 256>), grid, dim3(256), 0, st, a);
        } else {
            if (a.norm_w) hipLaunchKernelGGL((k_route_quant<true, kK1Threads>), grid, dim3(kK1Threads), 0, st, a);
            else hipLaunchKernelGGL((k_route_quant<false, kK1Threads>), grid, dim3(kK1Threads), 0, st, a);
        }
        FNS_TRY(host::check_launch("moe route_quant"));
        // (the shared expert runs inside the fused kernel when that takes the call)
        return L->shexp_inter > 0 && !(a.shd && use_fused(L, a)) ? launch_shared(L, a, st) : host::OK;
    }
    // n_tok = 1 shapes that fit take the fused kernel as stage 1; stage 2 then has nothing left to do
    if (stage == 1) return use_fused(L, a) ? launch_fused(L, a, st) : by_type_gate_up(L->gu_type, a, st);
    if (stage == 2) return use_fused(L, a) ? host::OK : by_type_down(L->down_type, a, st);
    return host::set_error(host::ERR_SHAPE, "moe_layer: stage must be 0 (router), 1 (gate/up) or 2 (down)");
}

int moe_layer(const FnsMoeLayer *L, const float *x, const float *x_resid, float *out, int n_tok, void *ws,
              size_t ws_bytes, hipStream_t st, void *const *events) {
    LayerArgs a;
    FNS_TRY(prepare(L, x, x_resid, out, n_tok, ws, ws_bytes, a));
    auto mark = [&](int i) -> int {
        if (!events || !events[i]) return host::OK;
        const hipError_t e = hipEventRecord((hipEvent_t) events[i], st);
        return e == hipSuccess ? host::OK : host::set_error(host::ERR_LAUNCH, "moe_layer: hipEventRecord failed");
    };
    for (int stage = 0; stage < 3; ++stage) {
        FNS_TRY(mark(stage));
        FNS_TRY(launch_stage(L, a, stage, st));
    }
    return mark(3);
}

// ---- no-allocation variant -------------------------------------------------------------------------------------------
// fns_hip_moe_layer_noalloc takes its workspace from this file-scope device array instead of a caller buffer, for
// callers that cannot allocate (HIP graph capture, serving loops that forbid hipMalloc). Each GPU the library runs on
// holds its own copy until the process ends. In host code `scratch` is only a stand-in symbol: its device address is
// looked up once per device with hipGetSymbolAddress and kept in g_scratch_ptr, and only that address reaches kernels.
// Every call on one GPU shares the array (calls that overlap on one GPU race; order them on one stream).
constexpr size_t kScratchBytes = (size_t) 4 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t *g_scratch_ptr[kMaxDevices];

__global__ void k_zero_words(uint32_t *p, size_t n) {
    for (size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t) gridDim.x * blockDim.x) p[i] = 0;
}

// The scratch address on the current device; the first call on a device also clears the array (a kernel on `st`,
// ordered before the call's own kernels; a fill kernel rather than a memset node, so a captured first call replays
// correctly). The layer kernels keep the arrival counter consistent from call to call after that.
int scratch_of_device(hipStream_t st, uint8_t **out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return host::set_error(host::ERR_LAUNCH, "moe_layer_noalloc: no current HIP device");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return host::set_error(host::ERR_LAUNCH, "moe_layer_noalloc: hipGetSymbolAddress(scratch): %s",
                                   hipGetErrorString(e));
        hipLaunchKernelGGL(k_zero_words, dim3(256), dim3(256), 0, st, (uint32_t *) ptr, kScratchBytes / 4);
        FNS_TRY(host::check_launch("moe_layer_noalloc: clearing the scratch"));
        g_scratch_ptr[dev] = (uint8_t *) ptr;
    }
    *out = g_scratch_ptr[dev];
    return host::OK;
}

int moe_layer_noalloc(const FnsMoeLayer *L, const float *x, const float *x_resid, float *out, int n_tok,
                      hipStream_t st) {
    size_t need = 0;
    FNS_TRY(moe_workspace_layout(L, n_tok, nullptr, &need));
    if (need > kScratchBytes)
        return host::set_error(host::ERR_NOMEM, "moe_layer_noalloc: the layer needs %zu workspace bytes, more than the "
                                                "%zu-byte device scratch", need, kScratchBytes);
    uint8_t *ws = nullptr;
    FNS_TRY(scratch_of_device(st, &ws));
    return moe_layer(L, x, x_resid, out, n_tok, ws, kScratchBytes, st);
}

size_t moe_noalloc_max_bytes() { return kScratchBytes; }

// This translation unit's copy of the IQ codebooks (fns_quarter.hpp g_iq_grids), on the current device.
int iq_grids_upload_layer(const void *grids) {
    const hipError_t e = dev::upload_iq_grids((const dev::IqGrids *) grids);
    return e == hipSuccess ? host::OK : host::set_error(host::ERR_LAUNCH, "set_iq_grids: %s", hipGetErrorString(e));
}

// The sticky status word of a workspace (ws null: this device's no-allocation scratch), read after the stream's work
// so far has completed; clear: zero it afterwards (a kernel on `st`).
int moe_layer_status(const FnsMoeLayer *L, int n_tok, void *ws, int clear, uint32_t *status, hipStream_t st) {
    if (!status) return host::set_error(host::ERR_SHAPE, "moe_layer_status: null status");
    FNS_TRY(moe_workspace_layout(L, n_tok, nullptr, nullptr));
    uint8_t *base = (uint8_t *) ws;
    if (!base) FNS_TRY(scratch_of_device(st, &base));
    uint32_t *word = (uint32_t *) (base + kHdrStatusOff);  // the fixed header: the same place for every shape
    if (hipMemcpyAsync(status, word, 4, hipMemcpyDeviceToHost, st) != hipSuccess || hipStreamSynchronize(st) != hipSuccess)
        return host::set_error(host::ERR_LAUNCH, "moe_layer_status: reading the status word failed");
    if (clear) {
        hipLaunchKernelGGL(k_zero_words, dim3(1), dim3(64), 0, st, word, (size_t) 1);
        FNS_TRY(host::check_launch("moe_layer_status: clearing"));
    }
    return host::OK;
}

// One thread: ORs the status word into *dst when it is non-zero (dst untouched otherwise, so host-pinned memory is read
// and written only after a failure) and clears the word. A kernel rather than copies and a memset, so that a HIP graph
// can hold it.
__global__ void k_status_collect(uint32_t *word, uint32_t *dst) {
    const uint32_t v = *word;
    if (v != 0) {
        *dst = *dst | v;
        *word = 0;
    }
}

int status_collect(uint32_t *word, uint32_t *dst, hipStream_t st) {
    hipLaunchKernelGGL(k_status_collect, dim3(1), dim3(1), 0, st, word, dst);
    return host::check_launch("status collect");
}

int moe_layer_status_collect(const FnsMoeLayer *L, int n_tok, void *ws, uint32_t *dst, hipStream_t st) {
    if (!dst) return host::set_error(host::ERR_SHAPE, "moe_layer_status_collect: null destination");
    FNS_TRY(moe_workspace_layout(L, n_tok, nullptr, nullptr));
    uint8_t *base = (uint8_t *) ws;
    if (!base) FNS_TRY(scratch_of_device(st, &base));
    return status_collect((uint32_t *) (base + kHdrStatusOff), dst, st);
}

int moe_set_path(int path) {
    if (path < 0 || path > 1) return host::set_error(host::ERR_SHAPE, "moe_set_path: path must be 0 or 1");
    g_path_override = path;
    return host::OK;
}

int moe_layer_kernels(const FnsMoeLayer *L, int n_tok, int *kernels) {
    if (!kernels) return host::set_error(host::ERR_SHAPE, "moe_layer_kernels: null result");
    FNS_TRY(moe_workspace_layout(L, n_tok, nullptr, nullptr));
    // prepare() needs real pointers only for its null checks: a dummy workspace of the right size stands in
    size_t total = 0;
    FNS_TRY(moe_workspace_layout(L, n_tok, nullptr, &total));
    LayerArgs a;
    static float dummy;
    FNS_TRY(prepare(L, &dummy, nullptr, &dummy, n_tok, (void *) &dummy, total, a));
    *kernels = use_fused(L, a) ? 2 : 3;
    return host::OK;
}

int moe_layer_stage(const FnsMoeLayer *L, int stage, const float *x, const float *x_resid, float *out, int n_tok,
                    void *ws, size_t ws_bytes, hipStream_t st) {
    LayerArgs a;
    FNS_TRY(prepare(L, x, x_resid, out, n_tok, ws, ws_bytes, a));
    return launch_stage(L, a, stage, st);
}

}  // namespace impl

}  // namespace fns

