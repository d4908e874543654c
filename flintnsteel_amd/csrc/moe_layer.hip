// moe_layer.hip - the fused MoE FFN decode / speculative-verify layer for MI355X gfx950: three kernels per layer.
//
//   K1 k_route_quant : router logits (one workgroup per expert row, fp32 or bf16 weights) and Q8_1 of the token rows.
//   K2 k_gate_up     : every workgroup runs gating + top-k for the n_tok tokens on one wave (the routing is ~1 us of
//                      ALU and is cheaper to repeat than to publish through a grid barrier), compacts the selected
//                      experts (distinct ids, ascending, for n_tok > 1; slot order for n_tok = 1), then computes
//                      act = up . x * silu(gate . x) for its rows of one expert and every token routed to it (ncols <= 4
//                      per expert: each expert's weights are read once per step).
//   K3 k_down_combine: stages act of all (token, slot) rows, applies the optional F16 guard and quantises to Q8_1 in
//                      LDS (bit-exact with amax_guard_q8_1), computes its output rows of down_e . act for every
//                      (token, slot) and combines them in slot order (reference src/kernels.cu:579-586).
// On this GPU a kernel boundary inside a HIP graph costs less than a software grid barrier across 256 CUs (measured),
// so the two global dependencies of the layer (all logits -> routing, all act rows -> down) are kernel boundaries.
//
// Caller contract: reference Engine::ffn_block (src/engine.cu:655-696) - rms_norm_q8_1 output (here: any fp32 x),
// router, route_topk, mmvq_experts_swiglu, amax_guard_q8_1, mmvq_experts, moe_combine - in one call.
// Per-(token, row) arithmetic does not depend on the other tokens of the step: a verify column equals the batch-1
// result bit for bit (reference src/engine.cu:601-603).
#include "fns_common.hpp"
#include "fns_host.hpp"
#include "fns_internal.hpp"
#include "fns_route.hpp"

namespace fns {

using namespace fns::dev;

namespace {

constexpr int kMaxTok = 4;

struct LayerArgs {
    // shapes
    int H, F, NE, K, T;
    int gating, norm, guard;
    // weights
    int router_dtype;
    const void *router_w;
    const char *const *table;
    int64_t gate_off, up_off, down_off;
    // activations / workspace
    const float *x;       // [T][H]
    const float *x_resid; // [T][H] or null
    float *out;           // [T][H]
    float *logits;        // [T][NE]
    uint8_t *xq;          // [T][q8_1_row_bytes(H)]
    int64_t xq_row_bytes;
    int32_t *ids;         // [T][K]
    float *w;             // [T][K]
    float *act;           // [T*K][F]
    float *escale;        // [T*K]
};

__device__ __forceinline__ float bf16f(uint16_t b) { return __builtin_bit_cast(float, (uint32_t) b << 16); }

// ---- K1: router rows + Q8_1 of x ----------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_route_quant(const LayerArgs a) {
    __shared__ float red[4][kMaxTok];
    const int H = a.H, T = a.T;
    if ((int) blockIdx.x < a.NE) {
        const int r = blockIdx.x;
        float s[kMaxTok] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int i = threadIdx.x; i < H / 4; i += 256) {
            float4 wv;
            if (a.router_dtype == T_BF16) {
                const uint2 pk = ((const uint2 *) ((const uint16_t *) a.router_w + (size_t) r * H))[i];
                wv = make_float4(bf16f(pk.x & 0xffff), bf16f(pk.x >> 16), bf16f(pk.y & 0xffff), bf16f(pk.y >> 16));
            } else {
                wv = ((const float4 *) ((const float *) a.router_w + (size_t) r * H))[i];
            }
#pragma unroll
            for (int t = 0; t < kMaxTok; ++t) {
                if (t < T) {
                    const float4 xv = ((const float4 *) (a.x + (size_t) t * H))[i];
                    s[t] += wv.x * xv.x + wv.y * xv.y + wv.z * xv.z + wv.w * xv.w;
                }
            }
        }
#pragma unroll
        for (int t = 0; t < kMaxTok; ++t) {
            float v = s[t];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
            if (threadIdx.x % 64 == 0) red[threadIdx.x / 64][t] = v;
        }
        __syncthreads();
        if ((int) threadIdx.x < T)
            a.logits[(size_t) threadIdx.x * a.NE + r] =
                (red[0][threadIdx.x] + red[1][threadIdx.x]) + (red[2][threadIdx.x] + red[3][threadIdx.x]);
        return;
    }
    // Q8_1 of x: chunk -> (token, 256 columns)
    const int npad = (H + 511) / 512 * 512;
    const int chunks = npad / 256;
    const int chunk = blockIdx.x - a.NE;
    const int t = chunk / chunks, i = (chunk % chunks) * 256 + threadIdx.x;
    const float v = i < H ? a.x[(size_t) t * H + i] : 0.0f;
    float amax = fabsf(v), sum = v;
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, o, kWave));
        sum += __shfl_xor(sum, o, kWave);
    }
    const float d = amax / 127.0f;
    uint8_t *b = a.xq + (size_t) t * a.xq_row_bytes + (size_t) (i / 32) * 36;
    b[4 + i % 32] = (uint8_t) (amax == 0.0f ? (int8_t) 0 : (int8_t) roundf(v / d));
    if (i % 32 == 0) *(uint32_t *) b = float_to_half(d) | (float_to_half(sum) << 16);
}

// ---- K2: routing + gate/up + SwiGLU -----------------------------------------------------------------------------
template <int T_, int LPR, int SPL, int NC>
__global__ __launch_bounds__(256) void k_gate_up(const LayerArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int s_ids[kMaxTok * 16];
    __shared__ int s_wave_cnt[4];
    __shared__ int s_e, s_ncol, s_xrow[kMaxTok], s_orow[kMaxTok];
    constexpr int SPB = Traits<T_>::slots, BB = Traits<T_>::bytes;
    constexpr int G = 256 / LPR;
    constexpr int RPG = LPR >= 32 ? 2 : 1;
    constexpr int SPLX = SPL > 0 ? SPL : 1;
    const int tid = threadIdx.x, wave = tid / kWave, lane64 = tid % kWave;
    const int T = a.T, K = a.K, H = a.H;
    const int npad = (H + 511) / 512 * 512;

    // 1. stage the Q8_1 rows of all tokens (independent of the routing)
    for (int t = 0; t < T; ++t) {
        uint8_t *base = smem + t * act_lds_bytes(npad);
        stage_q8_1_row(a.xq + (size_t) t * a.xq_row_bytes, npad / 32, (int8_t *) base, (float *) (base + npad),
                       (float *) (base + npad) + npad / 32, tid, 256);
    }
    // 2. routing on wave 0
    if (wave == 0) {
        const bool pub = blockIdx.x == 0 && blockIdx.y == 0;
        for (int t = 0; t < T; ++t)
            route_topk_wave(a.logits + (size_t) t * a.NE, a.NE, K, a.gating, a.norm, pub ? a.ids + t * K : nullptr,
                            pub ? a.w + t * K : nullptr, s_ids + t * K);
    }
    if (tid == 0) s_e = -1;
    __syncthreads();
    // 3. channel -> expert and its (token, slot) columns
    if (T == 1) {
        if (tid == 0) {
            s_e = s_ids[blockIdx.y];
            s_ncol = 1;
            s_xrow[0] = 0;
            s_orow[0] = blockIdx.y;
        }
    } else {
        bool present = false;
        if (tid < a.NE)
            for (int i = 0; i < T * K; ++i) present |= s_ids[i] == tid;
        const uint64_t m = __ballot(present);
        if (lane64 == 0) s_wave_cnt[wave] = __popcll(m);
        __syncthreads();
        int rank = __popcll(m & ((1ull << lane64) - 1ull));
        for (int wv = 0; wv < wave; ++wv) rank += s_wave_cnt[wv];
        if (present && rank == (int) blockIdx.y) {
            s_e = tid;
            int n = 0;
            for (int t = 0; t < T; ++t)
                for (int j = 0; j < K; ++j)
                    if (s_ids[t * K + j] == tid) {
                        s_xrow[n] = t;
                        s_orow[n] = t * K + j;
                        ++n;
                    }
            s_ncol = n;
        }
    }
    __syncthreads();
    const int e = s_e;
    if (e < 0) return;  // fewer distinct experts than channels: uniform exit of the whole workgroup
    const int ncol = s_ncol;

    const uint8_t *slot = (const uint8_t *) a.table[e];
    const uint8_t *wa = slot + a.up_off, *wb = slot + a.gate_off;
    const int nblk = H / 256, nslots = nblk * SPB;
    const int64_t row_bytes = (int64_t) nblk * BB;
    const int lane = tid % LPR, grp = tid / LPR;
    const int row0 = blockIdx.x * (G * RPG) + grp;

    Frag fa[RPG][SPLX], fb[RPG][SPLX];
    if constexpr (SPL > 0) {
#pragma unroll
        for (int r = 0; r < RPG; ++r) {
            const int row = row0 + r * G;
#pragma unroll
            for (int s = 0; s < SPL; ++s) {
                const int sl = lane + s * LPR;
                if (row < a.F && sl < nslots) {
                    slot_load<T_>(wa + row * row_bytes + (int64_t) (sl / SPB) * BB, sl % SPB, fa[r][s]);
                    slot_load<T_>(wb + row * row_bytes + (int64_t) (sl / SPB) * BB, sl % SPB, fb[r][s]);
                }
            }
        }
    }
    ActView av[NC];
#pragma unroll
    for (int n = 0; n < NC; ++n) {
        const uint8_t *base = smem + (n < ncol ? s_xrow[n] : 0) * act_lds_bytes(npad);
        av[n] = ActView{(const int8_t *) base, (const float *) (base + npad), (const float *) (base + npad) + npad / 32};
    }
    float acc[RPG][NC], accg[RPG][NC];
#pragma unroll
    for (int r = 0; r < RPG; ++r)
#pragma unroll
        for (int n = 0; n < NC; ++n) acc[r][n] = accg[r][n] = 0.0f;
#pragma unroll
    for (int r = 0; r < RPG; ++r) {
        const int row = row0 + r * G;
        if (row >= a.F) continue;
        if constexpr (SPL > 0) {
#pragma unroll
            for (int s = 0; s < SPL; ++s) {
                const int sl = lane + s * LPR;
                if (sl < nslots) {
#pragma unroll
                    for (int n = 0; n < NC; ++n) {
                        if (n < ncol) {
                            acc[r][n] += slot_dot<T_>(fa[r][s], sl % SPB, (sl / SPB) * 256, av[n]);
                            accg[r][n] += slot_dot<T_>(fb[r][s], sl % SPB, (sl / SPB) * 256, av[n]);
                        }
                    }
                }
            }
        } else {
            for (int sl = lane; sl < nslots; sl += LPR) {
                Frag f, g;
                slot_load<T_>(wa + row * row_bytes + (int64_t) (sl / SPB) * BB, sl % SPB, f);
                slot_load<T_>(wb + row * row_bytes + (int64_t) (sl / SPB) * BB, sl % SPB, g);
#pragma unroll
                for (int n = 0; n < NC; ++n) {
                    if (n < ncol) {
                        acc[r][n] += slot_dot<T_>(f, sl % SPB, (sl / SPB) * 256, av[n]);
                        accg[r][n] += slot_dot<T_>(g, sl % SPB, (sl / SPB) * 256, av[n]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RPG; ++r) {
        const int row = row0 + r * G;
#pragma unroll
        for (int n = 0; n < NC; ++n) {
            float v = group_sum<LPR>(acc[r][n]);
            const float gs = group_sum<LPR>(accg[r][n]);
            v += 0.0f;
            v *= silu(gs + 0.0f);
            if (lane == 0 && n < ncol && row < a.F) a.act[(size_t) s_orow[n] * a.F + row] = v;
        }
    }
}

// ---- K3: guard + Q8_1 of act, down GEMV, combine --------------------------------------------------------------------
constexpr int kDownRows = 8;  // output rows per workgroup

__device__ __forceinline__ float guard_scale(float amax) {
    float e = amax * (1.0f / 1024.0f);
    e = logf(e);
    e = e * 1.4426950408889634f;
    e = ceilf(e);
    e = fminf(fmaxf(e, 0.0f), 127.0f);
    e = e * 0.6931471805599453f;
    return expf(e);
}

template <int T_, int LPR, int SPL>
__global__ __launch_bounds__(256) void k_down_combine(const LayerArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int s_ids[kMaxTok * 16];
    __shared__ float s_w[kMaxTok * 16], s_e[kMaxTok * 16];
    __shared__ float s_dexp[kMaxTok * 16][kDownRows];
    constexpr int SPB = Traits<T_>::slots, BB = Traits<T_>::bytes;
    constexpr int G = 256 / LPR;
    const int tid = threadIdx.x, wave = tid / kWave, lane64 = tid % kWave;
    const int T = a.T, K = a.K, F = a.F, H = a.H;
    const int CH = T * K;
    const int fpad = (F + 511) / 512 * 512;
    const int r0 = blockIdx.x * kDownRows;

    if (tid < CH) {
        s_ids[tid] = a.ids[tid];
        s_w[tid] = a.w[tid];
    }
    // act rows -> (guard) -> Q8_1 in LDS; one wave per row
    for (int c = wave; c < CH; c += 4) {
        const float *src = a.act + (size_t) c * F;
        float m = 0.0f;
        for (int i = lane64; i < F; i += kWave) m = fmaxf(m, fabsf(src[i]));
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, kWave));
        const float e = a.guard ? guard_scale(m) : 1.0f;
        if (lane64 == 0) {
            s_e[c] = e;
            if (blockIdx.x == 0 && a.escale) a.escale[c] = e;
        }
        uint8_t *base = smem + c * act_lds_bytes(fpad);
        int8_t *q = (int8_t *) base;
        float *d = (float *) (base + fpad);
        float *s16 = d + fpad / 32;
        for (int i0 = 0; i0 < fpad; i0 += kWave) {
            const int i = i0 + lane64;
            const float v = i < F ? (a.guard ? src[i] / e : src[i]) : 0.0f;
            float amax = fabsf(v), sum = v;
#pragma unroll
            for (int o = 16; o > 0; o >>= 1) {
                amax = fmaxf(amax, __shfl_xor(amax, o, kWave));
                sum += __shfl_xor(sum, o, kWave);
            }
            const float dd = amax / 127.0f;
            const int qi = amax == 0.0f ? 0 : (int) (int8_t) roundf(v / dd);
            int qs = qi;
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) qs += __shfl_xor(qs, o, kWave);
            const float dh = half_to_float(float_to_half(dd));
            q[i] = (int8_t) qi;
            if (i % 32 == 0) d[i / 32] = dh;
            if (i % 16 == 0) s16[i / 16] = dh * (float) qs;
        }
    }
    __syncthreads();

    // (row, channel) items; a lane group of LPR lanes takes items grp, grp + G, ...
    const int nblk = F / 256, nslots = nblk * SPB;
    const int64_t row_bytes = (int64_t) nblk * BB;
    const int lane = tid % LPR, grp = tid / LPR;
    const int n_items = kDownRows * CH;
    for (int it0 = grp; it0 < n_items; it0 += 2 * G) {
        Frag f[2][SPL > 0 ? SPL : 1];
        int row_[2], ch_[2];
        bool ok[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int it = it0 + u * G;
            ch_[u] = it % CH;
            row_[u] = r0 + it / CH;
            ok[u] = it < n_items && row_[u] < H;
            if constexpr (SPL > 0) {
                const uint8_t *wm = (const uint8_t *) a.table[s_ids[ok[u] ? ch_[u] : 0]] + a.down_off;
#pragma unroll
                for (int s = 0; s < SPL; ++s) {
                    const int sl = lane + s * LPR;
                    if (ok[u] && sl < nslots)
                        slot_load<T_>(wm + row_[u] * row_bytes + (int64_t) (sl / SPB) * BB, sl % SPB, f[u][s]);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            float acc = 0.0f;
            const uint8_t *base = smem + (ok[u] ? ch_[u] : 0) * act_lds_bytes(fpad);
            const ActView av{(const int8_t *) base, (const float *) (base + fpad), (const float *) (base + fpad) + fpad / 32};
            if (ok[u]) {
                if constexpr (SPL > 0) {
#pragma unroll
                    for (int s = 0; s < SPL; ++s) {
                        const int sl = lane + s * LPR;
                        if (sl < nslots) acc += slot_dot<T_>(f[u][s], sl % SPB, (sl / SPB) * 256, av);
                    }
                } else {
                    const uint8_t *wm = (const uint8_t *) a.table[s_ids[ch_[u]]] + a.down_off;
                    for (int sl = lane; sl < nslots; sl += LPR) {
                        Frag g;
                        slot_load<T_>(wm + row_[u] * row_bytes + (int64_t) (sl / SPB) * BB, sl % SPB, g);
                        acc += slot_dot<T_>(g, sl % SPB, (sl / SPB) * 256, av);
                    }
                }
            }
            acc = group_sum<LPR>(acc);
            if (lane == 0 && ok[u]) s_dexp[ch_[u]][row_[u] - r0] = acc;
        }
    }
    __syncthreads();
    // combine in slot order: out[t][r] = (sum_j (dexp * e_j) * w_j + 0) + x_resid
    if (tid < T * kDownRows) {
        const int t = tid / kDownRows, rr = tid % kDownRows, r = r0 + rr;
        if (r < H) {
            float moe = (s_dexp[t * K][rr] * s_e[t * K]) * s_w[t * K];
            for (int j = 1; j < K; ++j) moe = moe + (s_dexp[t * K + j][rr] * s_e[t * K + j]) * s_w[t * K + j];
            moe = moe + 0.0f;
            a.out[(size_t) t * H + r] = a.x_resid ? moe + a.x_resid[(size_t) t * H + r] : moe;
        }
    }
}

template <int T_, int LPR, int SPL>
int launch_gate_up(const LayerArgs &a, hipStream_t st) {
    constexpr int RPB = (256 / LPR) * (LPR >= 32 ? 2 : 1);
    const int n_chan = a.T == 1 ? a.K : std::min(a.T * a.K, a.NE);
    const dim3 grid((unsigned) ((a.F + RPB - 1) / RPB), (unsigned) n_chan);
    const int npad = (int) host::pad512(a.H);
    const size_t lds = (size_t) a.T * act_lds_bytes(npad);
    if (a.T == 1) hipLaunchKernelGGL((k_gate_up<T_, LPR, SPL, 1>), grid, dim3(256), lds, st, a);
    else hipLaunchKernelGGL((k_gate_up<T_, LPR, SPL, kMaxTok>), grid, dim3(256), lds, st, a);
    return host::check_launch("moe gate_up");
}

template <int T_> int dispatch_gate_up(const LayerArgs &a, hipStream_t st) {
    const host::Shape s = host::pick_shape(a.H / 256 * Traits<T_>::slots);
    if (s.lpr == 64 && s.spl == 1) return launch_gate_up<T_, 64, 1>(a, st);
    if (s.lpr == 64 && s.spl == 2) return launch_gate_up<T_, 64, 2>(a, st);
    if (s.lpr == 64 && s.spl == 3) return launch_gate_up<T_, 64, 3>(a, st);
    if (s.lpr == 32) return launch_gate_up<T_, 32, 1>(a, st);
    if (s.lpr == 16) return launch_gate_up<T_, 16, 1>(a, st);
    if (s.lpr == 8) return launch_gate_up<T_, 8, 3>(a, st);
    if (s.lpr == 4) return launch_gate_up<T_, 4, 3>(a, st);
    return launch_gate_up<T_, 64, 0>(a, st);
}

template <int T_, int LPR, int SPL> int launch_down(const LayerArgs &a, hipStream_t st) {
    const dim3 grid((unsigned) ((a.H + kDownRows - 1) / kDownRows));
    const size_t lds = (size_t) a.T * a.K * act_lds_bytes((int) host::pad512(a.F));
    hipLaunchKernelGGL((k_down_combine<T_, LPR, SPL>), grid, dim3(256), lds, st, a);
    return host::check_launch("moe down_combine");
}

template <int T_> int dispatch_down(const LayerArgs &a, hipStream_t st) {
    const host::Shape s = host::pick_shape(a.F / 256 * Traits<T_>::slots);
    if (s.lpr == 64 && s.spl == 1) return launch_down<T_, 64, 1>(a, st);
    if (s.lpr == 64 && s.spl == 2) return launch_down<T_, 64, 2>(a, st);
    if (s.lpr == 64 && s.spl == 3) return launch_down<T_, 64, 3>(a, st);
    if (s.lpr == 32) return launch_down<T_, 32, 1>(a, st);
    if (s.lpr == 16) return launch_down<T_, 16, 1>(a, st);
    if (s.lpr == 8) return launch_down<T_, 8, 3>(a, st);
    if (s.lpr == 4) return launch_down<T_, 4, 3>(a, st);
    return launch_down<T_, 64, 0>(a, st);
}

int by_type_gate_up(int t, const LayerArgs &a, hipStream_t st) {
    switch (t) {
        case T_Q3_K: return dispatch_gate_up<T_Q3_K>(a, st);
        case T_Q4_K: return dispatch_gate_up<T_Q4_K>(a, st);
        case T_Q5_K: return dispatch_gate_up<T_Q5_K>(a, st);
        case T_Q6_K: return dispatch_gate_up<T_Q6_K>(a, st);
    }
    return host::set_error(host::ERR_TYPE, "moe_layer: gate/up type %d not supported", t);
}

int by_type_down(int t, const LayerArgs &a, hipStream_t st) {
    switch (t) {
        case T_Q3_K: return dispatch_down<T_Q3_K>(a, st);
        case T_Q4_K: return dispatch_down<T_Q4_K>(a, st);
        case T_Q5_K: return dispatch_down<T_Q5_K>(a, st);
        case T_Q6_K: return dispatch_down<T_Q6_K>(a, st);
    }
    return host::set_error(host::ERR_TYPE, "moe_layer: down type %d not supported", t);
}

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

}  // namespace

namespace impl {

// Workspace sections (byte offsets, 256-aligned): logits, xq, ids, w, act, escale.
int moe_workspace_layout(const FnsMoeLayer *L, int n_tok, size_t *offsets, size_t *total) {
    if (!L || n_tok < 1 || n_tok > kMaxTok)
        return host::set_error(host::ERR_SHAPE, "moe_layer: 1 <= n_tok <= %d (larger batches use the MMQ path)", kMaxTok);
    size_t off = 0;
    const size_t sizes[6] = {
        (size_t) n_tok * L->n_expert * 4,
        (size_t) n_tok * host::q8_1_row_bytes(L->hidden),
        (size_t) n_tok * L->k * 4,
        (size_t) n_tok * L->k * 4,
        (size_t) n_tok * L->k * L->inter * 4,
        (size_t) n_tok * L->k * 4,
    };
    for (int i = 0; i < 6; ++i) {
        if (offsets) offsets[i] = off;
        off += align256(sizes[i]);
    }
    if (total) *total = off;
    return host::OK;
}

// Validates and fills the kernel arguments of one call.
static int prepare(const FnsMoeLayer *L, const float *x, const float *x_resid, float *out, int n_tok, void *ws,
                   size_t ws_bytes, LayerArgs &a) {
    if (!L || !x || !out || !ws || !L->router_w || !L->table)
        return host::set_error(host::ERR_SHAPE, "moe_layer: null argument");
    size_t off[6], total;
    FNS_TRY(moe_workspace_layout(L, n_tok, off, &total));
    if (ws_bytes < total) return host::set_error(host::ERR_NOMEM, "moe_layer: workspace %zu < %zu bytes", ws_bytes, total);
    if (L->hidden <= 0 || L->hidden % 256 || L->inter <= 0 || L->inter % 256 || L->hidden > 16384 || L->inter > 16384)
        return host::set_error(host::ERR_SHAPE, "moe_layer: hidden and inter must be positive multiples of 256 (<= 16384)");
    if (L->n_expert < 1 || L->n_expert > 256 || L->k < 1 || L->k > 16 || L->k > L->n_expert)
        return host::set_error(host::ERR_SHAPE, "moe_layer: 1 <= k <= min(16, n_expert), n_expert <= 256");
    if (L->gating != 0 && L->gating != 1) return host::set_error(host::ERR_SHAPE, "moe_layer: bad gating");
    if (L->router_dtype != 0 && L->router_dtype != T_BF16)
        return host::set_error(host::ERR_TYPE, "moe_layer: router dtype %d not supported", L->router_dtype);
    if (!host::is_kquant(L->gu_type) || !host::is_kquant(L->down_type))
        return host::set_error(host::ERR_TYPE, "moe_layer: expert types %d/%d not supported", L->gu_type, L->down_type);
    const size_t lds_down = (size_t) n_tok * L->k * act_lds_bytes((int) host::pad512(L->inter));
    if (lds_down > 64 * 1024)
        return host::set_error(host::ERR_SHAPE, "moe_layer: n_tok * k * inter too large for the down kernel's LDS");
    uint8_t *w8 = (uint8_t *) ws;
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
    a.table = (const char *const *) L->table;
    a.gate_off = (int64_t) L->gate_off;
    a.up_off = (int64_t) L->up_off;
    a.down_off = (int64_t) L->down_off;
    a.x = x;
    a.x_resid = x_resid;
    a.out = out;
    a.logits = (float *) (w8 + off[0]);
    a.xq = w8 + off[1];
    a.xq_row_bytes = host::q8_1_row_bytes(L->hidden);
    a.ids = (int32_t *) (w8 + off[2]);
    a.w = (float *) (w8 + off[3]);
    a.act = (float *) (w8 + off[4]);
    a.escale = (float *) (w8 + off[5]);
    return host::OK;
}

static int launch_stage(const FnsMoeLayer *L, const LayerArgs &a, int stage, hipStream_t st) {
    if (stage == 0) {
        const int chunks = (int) (host::pad512(L->hidden) / 256);
        hipLaunchKernelGGL(k_route_quant, dim3((unsigned) (L->n_expert + chunks * a.T)), dim3(256), 0, st, a);
        return host::check_launch("moe route_quant");
    }
    if (stage == 1) return by_type_gate_up(L->gu_type, a, st);
    if (stage == 2) return by_type_down(L->down_type, a, st);
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

int moe_layer_stage(const FnsMoeLayer *L, int stage, const float *x, const float *x_resid, float *out, int n_tok,
                    void *ws, size_t ws_bytes, hipStream_t st) {
    LayerArgs a;
    FNS_TRY(prepare(L, x, x_resid, out, n_tok, ws, ws_bytes, a));
    return launch_stage(L, a, stage, st);
}

}  // namespace impl

}  // namespace fns
