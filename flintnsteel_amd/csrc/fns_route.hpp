// fns_route.hpp - gating + top-k + renormalisation for one token on one wave64 (device code shared by the
// standalone route_topk kernel and the fused decode layer).
// Reference: src/kernels.cu:484-514 (k_route_topk: warp argmax rounds, ties to the lower index,
// w = p / max(sum, 6.103515625e-5)); softmax gating per llama.cpp build_moe_ffn.
#pragma once

#include "fns_common.hpp"

namespace fns::dev {

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
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, kWave));
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            p[j] = lane + 64 * j < n_expert ? fns_expf(v[j] - m) : 0.0f;
            s = s + p[j];
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, kWave);
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
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(v, o, kWave);
            const int oi = __shfl_xor(idx, o, kWave);
            if (ov > v || (ov == v && oi < idx)) {
                v = ov;
                idx = oi;
            }
        }
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

}  // namespace fns::dev
