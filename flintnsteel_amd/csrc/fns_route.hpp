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

// Gating + top-k + renormalisation for one token by a whole workgroup of NT threads (n_expert <= 256): wave 0
// computes the probabilities exactly as route_topk_wave (same fp32 operations, so the same bits) into s_p (256
// entries, -inf past n_expert), then four threads per expert each count, over a contiguous quarter of the experts
// (float4 LDS reads), how many rank above it (higher p, or equal p and lower index); the expert with rank r < k goes to
// slot r. Equivalent to k rounds of argmax with ties to the lower index, with no dependent cross-lane chain.
// Must be called by every thread of the workgroup (it contains barriers). Results: sel[0..k), w[0..k) in LDS.
template <int NT>
__device__ __forceinline__ void route_topk_block(const float *__restrict__ lg, int n_expert, int k, int gating, int norm,
                                                 float *s_p, int *sel, float *pv, float *w) {
    constexpr int P = 4;               // threads per expert
    constexpr int EPP = NT / P;        // experts per pass
    const int tid = threadIdx.x, lane = tid % kWave;
    if (tid < kWave) {
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
            for (int j = 0; j < 4; ++j) s_p[lane + 64 * j] = lane + 64 * j < n_expert ? ev[j] * inv : -__builtin_inff();
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = lane + 64 * j;
                s_p[e] = e < n_expert ? 1.0f / (1.0f + fns_expf(-lg[e])) : -__builtin_inff();
            }
        }
    }
    __syncthreads();
    const int quarter = ((n_expert + 4 * P - 1) / (4 * P)) * 4;  // experts per part, multiple of 4
    const int part = tid % P;
    for (int e0 = 0; e0 < n_expert; e0 += EPP) {
        const int e = e0 + tid / P;
        const float pe = e < n_expert ? s_p[e] : -__builtin_inff();
        int rank = 0;
        const int j0 = part * quarter;
        for (int jj = 0; jj < quarter; jj += 4) {
            const int j = j0 + jj;
            if (j < 256) {
                const float4 p4 = *(const float4 *) (s_p + j);
                rank += (p4.x > pe || (p4.x == pe && j < e)) ? 1 : 0;
                rank += (p4.y > pe || (p4.y == pe && j + 1 < e)) ? 1 : 0;
                rank += (p4.z > pe || (p4.z == pe && j + 2 < e)) ? 1 : 0;
                rank += (p4.w > pe || (p4.w == pe && j + 3 < e)) ? 1 : 0;
            }
        }
        rank = lanes_sum_i<P>(rank);
        if (e < n_expert && part == 0 && rank < k) {
            sel[rank] = e;
            pv[rank] = pe;
        }
    }
    __syncthreads();
    if (tid < k) {
        float sum = 0.0f;
        for (int r = 0; r < k; ++r) sum += pv[r];
        w[tid] = norm ? pv[tid] / fmaxf(sum, 6.103515625e-5f) : pv[tid];
    }
}

}  // namespace fns::dev
