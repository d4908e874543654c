// fns_route.hpp - gating + top-k + renormalisation for one token on one wave64 (device code shared by the
// standalone route_topk kernel and the fused decode layer).
// Reference: src/kernels.cu:484-514 (k_route_topk: warp argmax rounds, ties to the lower index,
// w = p / max(sum, 6.103515625e-5)); softmax gating per llama.cpp build_moe_ffn.
#pragma once

#include "fns_common.hpp"

namespace fns::dev {

// One xor-butterfly step of a (value, index) argmax; ties go to the lower index. The result is the same on every
// lane whatever the pairing order, so the exchange pattern is free.
template <int O> __device__ __forceinline__ void argmax_step(float &v, int &idx) {
    const float ov = xor_lane<O>(v);
    const int oi = xor_lane_i<O>(idx);
    if (ov > v || (ov == v && oi < idx)) {
        v = ov;
        idx = oi;
    }
}

// One wave per token. Lane l holds experts l + 64 j (j < 4); the CPU oracle (oracle/fns_oracle.c or_route_topk)
// restates exactly these fp32 operations.
__device__ __forceinline__ void route_topk_wave(const float *__restrict__ lg, int n_expert, int k, int gating, int norm,
                                int32_t *ids_out, float *w_out, int32_t *ids_lds) {
    const int lane = threadIdx.x % kWave;
    float p[4];
    if (gating == 0) {
        float v[4], m = -__builtin_inff();
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = lane + 64 * j;
            v[j] = e < n_expert ? lg[e] : -__builtin_inff();
            m = fmaxf(m, v[j]);
        }
        m = lanes_max<64>(m);
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            p[j] = lane + 64 * j < n_expert ? fns_expf(v[j] - m) : 0.0f;
            s = s + p[j];
        }
        s = lanes_sum<64>(s);
        const float inv = 1.0f / s;
#pragma unroll
        for (int j = 0; j < 4; ++j) p[j] = lane + 64 * j < n_expert ? p[j] * inv : -__builtin_inff();
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = lane + 64 * j;
            p[j] = e < n_expert ? 1.0f / (1.0f + fns_expf(-lg[e])) : -__builtin_inff();
        }
    }
    float sel_v = 0.0f, sum = 0.0f;
    int sel_i = 0;
    for (int r = 0; r < k; ++r) {
        float v = -__builtin_inff();
        int idx = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (p[j] > v) {
                v = p[j];
                idx = lane + 64 * j;
            }
        argmax_step<32>(v, idx);
        argmax_step<16>(v, idx);
        argmax_step<8>(v, idx);
        argmax_step<4>(v, idx);
        argmax_step<2>(v, idx);
        argmax_step<1>(v, idx);
        if (idx % 64 == lane) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (idx / 64 == j) p[j] = -__builtin_inff();
        }
        if (lane == r) {
            sel_v = v;
            sel_i = idx;
        }
        sum += v;
    }
    if (lane < k) {
        const float wv = norm ? sel_v / fmaxf(sum, 6.103515625e-5f) : sel_v;
        if (ids_out) ids_out[lane] = sel_i;
        if (w_out) w_out[lane] = wv;
        if (ids_lds) ids_lds[lane] = sel_i;
    }
}

// LDS scratch of route_topk_block, in 64-bit words: keys [0, 256), candidates [256, 384), group maxima [384, 416),
// the threshold and the candidate counts after them.
constexpr int kTopkScratch = 432;

// Group-maximum form (n_expert > 128 in route_topk_block): gating + top-k + renormalisation for one token by a whole
// workgroup of NT threads (n_expert <= 256). Wave 0
// computes the probabilities exactly as route_topk_wave (same fp32 operations, so the same bits) and stores for each
// expert the 64-bit key (bits(p) << 32) | ~e: p >= 0, so the keys order as (p descending, index ascending) and the
// live ones are distinct and non-zero. Then: the maxima of the 32 groups of 8 consecutive experts, and T0 = the k-th
// largest of them. At least k keys are >= T0 (those k group maxima), so the top k are all >= T0, and a key below T0
// exceeds none of them: the top k are the keys >= T0 ranked among themselves (at most 8k candidates, eight threads
// per candidate). The result is the same as k rounds of argmax with ties to the lower index. Must be called by every
// thread of the workgroup (it contains barriers). Results: sel[0..k) and their probabilities pv[0..k) in LDS, visible
// to the whole workgroup on return.
// gtid: the thread's index in its group of NT (NT = the workgroup, or one of its equal groups each ranking its own
// token: the barriers are the workgroup's, reached by every group in step).
// Sigmoid keys with one expert per thread (workgroups of 256 threads or more): elementwise, so the same operations
// and bits as the wave-0 loop of the forms below.
__device__ __forceinline__ void sigmoid_keys(int tid, const float *__restrict__ lg, int n_expert, uint64_t *s_key) {
    if (tid < 256) {
        const int e = tid;
        const float p = e < n_expert ? 1.0f / (1.0f + fns_expf(-lg[e])) : 0.0f;
        s_key[e] = e < n_expert ? ((uint64_t) __builtin_bit_cast(uint32_t, p) << 32) | (uint32_t) ~e : 0ull;
    }
}

template <int NT>
__device__ __forceinline__ void route_topk_filter(int gtid, const float *__restrict__ lg, int n_expert, int k,
                                                  int gating, uint64_t *scratch, int *sel, float *pv) {
    static_assert(NT >= 64 && NT % 64 == 0 && NT <= 1024, "whole waves");
    constexpr int P = 8;         // threads per candidate
    constexpr int CPP = NT / P;  // candidates per pass
    uint64_t *s_key = scratch, *s_cand = scratch + 256, *s_gm = scratch + 384, *s_t0 = scratch + 416;
    int *s_cnt = (int *) (scratch + 417);  // candidates per wave (16 at most)
    const int tid = gtid, lane = tid % kWave, wave = tid / kWave;
    const bool par_sig = NT >= 256 && gating != 0;
    if (par_sig) {
        sigmoid_keys(tid, lg, n_expert, s_key);
        if (tid == 0) *s_t0 = 0ull;
    } else if (tid < kWave) {
        float p[4];
        if (gating == 0) {
            float v[4], m = -__builtin_inff();
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = lane + 64 * j;
                v[j] = e < n_expert ? lg[e] : -__builtin_inff();
                m = fmaxf(m, v[j]);
            }
            m = lanes_max<64>(m);
            float ev[4], s = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                ev[j] = lane + 64 * j < n_expert ? fns_expf(v[j] - m) : 0.0f;
                s = s + ev[j];
            }
            s = lanes_sum<64>(s);
            const float inv = 1.0f / s;
#pragma unroll
            for (int j = 0; j < 4; ++j) p[j] = ev[j] * inv;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = lane + 64 * j;
                p[j] = e < n_expert ? 1.0f / (1.0f + fns_expf(-lg[e])) : 0.0f;
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = lane + 64 * j;
            s_key[e] = e < n_expert ? ((uint64_t) __builtin_bit_cast(uint32_t, p[j]) << 32) | (uint32_t) ~e : 0ull;
        }
        if (lane == 0) *s_t0 = 0ull;  // kept when fewer than k groups are live: every live key is a candidate
    }
    __syncthreads();
    if (tid < 32) {
        uint64_t m = 0ull;
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            const ulonglong2 kk = *(const ulonglong2 *) (s_key + 8 * tid + i);
            m = kk.x > m ? kk.x : m;
            m = kk.y > m ? kk.y : m;
        }
        s_gm[tid] = m;
    }
    __syncthreads();
    if (tid < 32) {  // dead groups (maximum 0) tie with each other and all write 0
        const uint64_t own = s_gm[tid];
        int r = 0;
#pragma unroll
        for (int g = 0; g < 32; g += 2) {
            const ulonglong2 kk = *(const ulonglong2 *) (s_gm + g);
            r += kk.x > own ? 1 : 0;
            r += kk.y > own ? 1 : 0;
        }
        if (r == k - 1) *s_t0 = own;
    }
    __syncthreads();
    const uint64_t t0 = *s_t0;
    // the candidates in expert order: one expert per thread, chunks of NT experts
    int C = 0;
    for (int e0 = 0; e0 < 256; e0 += NT) {
        const int e = e0 + tid;
        const uint64_t kt = e < 256 ? s_key[e] : 0ull;
        const bool cand = kt != 0ull && kt >= t0;
        const uint64_t b = __ballot(cand);
        if (lane == 0) s_cnt[wave] = __popcll(b);
        __syncthreads();
        int base = C;
        for (int w = 0; w < wave; ++w) base += s_cnt[w];
        if (cand) s_cand[base + __popcll(b & ((1ull << lane) - 1ull))] = kt;
        for (int w = 0; w < NT / kWave; ++w) C += s_cnt[w];
        __syncthreads();
    }
    const int part = tid % P;
    for (int c0 = 0; c0 < C; c0 += CPP) {
        const int c = c0 + tid / P;
        const uint64_t kc = c < C ? s_cand[c] : ~0ull;
        int rank = 0;
        for (int i = part; i < C; i += P) rank += s_cand[i] > kc ? 1 : 0;
        rank = lanes_sum_i<P>(rank);
        if (c < C && part == 0 && rank < k) {
            sel[rank] = (int) ~(uint32_t) kc;
            pv[rank] = __builtin_bit_cast(float, (uint32_t) (kc >> 32));
        }
    }
    __syncthreads();
}

// All-pairs form (n_expert <= 128 in route_topk_block): gating + top-k + renormalisation for one token by a whole
// workgroup of NT threads (n_expert <= 256). Wave 0
// computes the probabilities exactly as route_topk_wave (same fp32 operations, so the same bits) and stores for
// each expert the 64-bit key (bits(p) << 32) | ~e: p >= 0, so the keys order as (p descending, index ascending) and
// are all distinct. Then eight threads per expert each count the keys above the expert's own over one eighth of the
// experts; the expert with rank r < k goes to slot r - the same result as k rounds of argmax with ties to the lower
// index, without a dependent cross-lane chain. Must be called by every thread of the workgroup (it contains
// barriers). Results: sel[0..k) and their probabilities pv[0..k) in LDS, visible to the whole workgroup on return.
// gtid: the thread's index in its group of NT, as in route_topk_filter.
template <int NT>
__device__ __forceinline__ void route_topk_pairs(int gtid, const float *__restrict__ lg, int n_expert, int k,
                                                 int gating, uint64_t *s_key, int *sel, float *pv) {
    constexpr int P = 8;         // threads per expert
    constexpr int EPP = NT / P;  // experts per pass
    const int tid = gtid, lane = tid % kWave;
    if (NT >= 256 && gating != 0) {
        sigmoid_keys(tid, lg, n_expert, s_key);
    } else if (tid < kWave) {
        float p[4];
        if (gating == 0) {
            float v[4], m = -__builtin_inff();
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = lane + 64 * j;
                v[j] = e < n_expert ? lg[e] : -__builtin_inff();
                m = fmaxf(m, v[j]);
            }
            m = lanes_max<64>(m);
            float ev[4], s = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                ev[j] = lane + 64 * j < n_expert ? fns_expf(v[j] - m) : 0.0f;
                s = s + ev[j];
            }
            s = lanes_sum<64>(s);
            const float inv = 1.0f / s;
#pragma unroll
            for (int j = 0; j < 4; ++j) p[j] = ev[j] * inv;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = lane + 64 * j;
                p[j] = e < n_expert ? 1.0f / (1.0f + fns_expf(-lg[e])) : 0.0f;
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = lane + 64 * j;
            s_key[e] = e < n_expert ? ((uint64_t) __builtin_bit_cast(uint32_t, p[j]) << 32) | (uint32_t) ~e : 0ull;
        }
    }
    __syncthreads();
    const int part = tid % P;
    const int kpl = ((n_expert + 2 * P - 1) / (2 * P)) * 2;  // keys per thread, even (16-byte reads)
    for (int e0 = 0; e0 < n_expert; e0 += EPP) {
        const int e = e0 + tid / P;
        const uint64_t ke = s_key[e < 256 ? e : 255];
        int rank = 0;
        // the eight threads of an expert read 8 consecutive 16-byte pieces per step (no LDS bank conflicts between
        // them); together they cover keys [0, kpl * P)
#pragma unroll 4
        for (int i = 0; i < kpl; i += 2) {
            const ulonglong2 kk = *(const ulonglong2 *) (s_key + i * P + 2 * part);
            rank += kk.x > ke ? 1 : 0;
            rank += kk.y > ke ? 1 : 0;
        }
        rank = lanes_sum_i<P>(rank);
        if (e < n_expert && part == 0 && rank < k) {
            sel[rank] = e;
            pv[rank] = __builtin_bit_cast(float, (uint32_t) (ke >> 32));
        }
    }
    __syncthreads();
}

// Group form (n_expert <= 256, k <= 8, NT >= 256): gating and keys as route_topk_filter (wave 0, the same bits);
// then each expert's rank among the 16 experts of its group (16 consecutive experts), the group's top k stored as
// candidates (16 k of them, at group * k + rank), and the candidates ranked among themselves (eight threads per
// candidate). The overall top k are among the groups' top k, so the selection is route_topk_filter's (the same as
// k rounds of argmax with ties to the lower index), with three barriers and no single-wave phase after the keys.
// Candidate slots a group does not fill (fewer than k live experts in it) hold key 0 and rank below every live key.
// Scratch: keys [0, 256), candidates [256, 256 + 16 k).
template <int NT>
__device__ __forceinline__ void route_topk_groups(int gtid, const float *__restrict__ lg, int n_expert, int k,
                                                  int gating, uint64_t *scratch, int *sel, float *pv) {
    static_assert(NT >= 256 && NT % 64 == 0 && NT <= 1024, "one thread per expert");
    constexpr int P = 8, CPP = NT / P;
    uint64_t *s_key = scratch, *s_cand = scratch + 256;
    const int tid = gtid, lane = tid % kWave, nc = 16 * k;
    if (gating != 0) {
        sigmoid_keys(tid, lg, n_expert, s_key);
        for (int i = tid; i < nc; i += NT) s_cand[i] = 0ull;
    } else if (tid < kWave) {  // softmax: wave 0, the fixed reduction order
        float p[4];
        if (gating == 0) {
            float v[4], m = -__builtin_inff();
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = lane + 64 * j;
                v[j] = e < n_expert ? lg[e] : -__builtin_inff();
                m = fmaxf(m, v[j]);
            }
            m = lanes_max<64>(m);
            float ev[4], s = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                ev[j] = lane + 64 * j < n_expert ? fns_expf(v[j] - m) : 0.0f;
                s = s + ev[j];
            }
            s = lanes_sum<64>(s);
            const float inv = 1.0f / s;
#pragma unroll
            for (int j = 0; j < 4; ++j) p[j] = ev[j] * inv;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = lane + 64 * j;
                p[j] = e < n_expert ? 1.0f / (1.0f + fns_expf(-lg[e])) : 0.0f;
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = lane + 64 * j;
            s_key[e] = e < n_expert ? ((uint64_t) __builtin_bit_cast(uint32_t, p[j]) << 32) | (uint32_t) ~e : 0ull;
        }
    } else {
        for (int i = tid - kWave; i < nc; i += NT - kWave) s_cand[i] = 0ull;
    }
    __syncthreads();
    if (tid < 256) {
        const int g = tid >> 4;
        const uint64_t ke = s_key[tid];
        int r = 0;
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
            const ulonglong2 kk = *(const ulonglong2 *) (s_key + 16 * g + i);
            r += kk.x > ke ? 1 : 0;
            r += kk.y > ke ? 1 : 0;
        }
        if (r < k && ke != 0ull) s_cand[g * k + r] = ke;
    }
    __syncthreads();
    const int part = tid % P;
    for (int c0 = 0; c0 < nc; c0 += CPP) {
        const int c = c0 + tid / P;
        const uint64_t kc = c < nc ? s_cand[c] : 0ull;
        int rank = 0;
#pragma unroll
        for (int j = 0; j < 128 / P; ++j) {  // nc <= 128: every read issued before the compares
            const int i = part + P * j;
            rank += i < nc && s_cand[i < nc ? i : 0] > kc ? 1 : 0;
        }
        rank = lanes_sum_i<P>(rank);
        if (c < nc && part == 0 && rank < k && kc != 0ull) {
            sel[rank] = (int) ~(uint32_t) kc;
            pv[rank] = __builtin_bit_cast(float, (uint32_t) (kc >> 32));
        }
    }
    __syncthreads();
}

// Gating + top-k + renormalisation for one token by a whole workgroup (n_expert <= 256): the all-pairs rank up to
// 128 experts; beyond, the group form (k <= 8, workgroups of 256 threads or more) or the group-maximum filter (4x the
// pairs at 256 experts). All give the same selection.
// gtid: the thread's index in its group of NT (the workgroup, or one of its equal groups, each ranking its own token).
template <int NT>
__device__ __forceinline__ void route_topk_block(int gtid, const float *__restrict__ lg, int n_expert, int k,
                                                 int gating, uint64_t *scratch, int *sel, float *pv) {
    if (n_expert <= 128) route_topk_pairs<NT>(gtid, lg, n_expert, k, gating, scratch, sel, pv);
    else if (NT >= 256 && k <= 8)
        route_topk_groups<(NT >= 256 ? NT : 256)>(gtid, lg, n_expert, k, gating, scratch, sel, pv);
    else route_topk_filter<NT>(gtid, lg, n_expert, k, gating, scratch, sel, pv);
}

// Combine weight of slot j (0 <= j < k < 16) from the selected probabilities pv[0..k): renormalised by their sum in
// slot order (floored at 2^-14) when norm is set.
__device__ __forceinline__ float route_weight(const float *pv, int k, int norm, int j) {
    float sum = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) sum += r < k ? pv[r] : 0.0f;
    return norm ? pv[j] / fmaxf(sum, 6.103515625e-5f) : pv[j];
}

}  // namespace fns::dev
