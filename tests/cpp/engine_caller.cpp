// engine_caller.cpp - a C++ caller of the drop-in headers include/fns/ggml_kernels.h and include/fns/kernels.h that
// calls every MoE entry point exactly as the reference engine does, checked against the CPU oracle
// (oracle/libfns_oracle.so, test infrastructure). Built by tests/cpp/Makefile with hipcc; run by
// tests/test_gpu_cpp_caller.py on the GPU. Prints "ENGINE_CALLER_OK" and exits 0 when every check passes.
//
//   decode / verify (W = 1, 2 columns): Engine::ffn_block, reference src/engine.cu:655-696 and the helpers it calls,
//       Engine::gemv and Engine::dense_glu (src/engine.cu:585-588, :644-653);
//   prefill (T tokens): Engine::prefill_chunk's FFN, reference src/engine.cu:330-357.
// The layer is shaped like the reference model's MoE blocks (sigmoid gating, bf16 router, top-6, a shared expert),
// at a reduced size so the oracle finishes in seconds.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "fns/ggml_kernels.h"
#include "fns/kernels.h"
#include "fns_oracle.h"

using namespace fns;

namespace {

constexpr int E = 1024, NE = 32, K = 6, F = 512, FS = 1024;  // hidden, experts, top-k, expert width, shared width
constexpr int NV = 150144;  // output-head rows (the reference model's vocabulary, src/model.cpp:168-169), Q8_0
constexpr float EPS = 1e-6f;
int g_fail = 0;

#define HIPCHK(x)                                                                                  \
    do {                                                                                           \
        hipError_t e_ = (x);                                                                       \
        if (e_ != hipSuccess) {                                                                    \
            std::fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
            std::exit(2);                                                                          \
        }                                                                                          \
    } while (0)

struct Rng {  // xorshift64* + Box-Muller: seeded synthetic inputs
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed * 2654435761u + 1) {}
    double u() {
        s ^= s >> 12, s ^= s << 25, s ^= s >> 27;
        return ((s * 2685821657736338717ull) >> 11) * (1.0 / 9007199254740992.0);
    }
    float n() { return (float) (std::sqrt(-2.0 * std::log(u() + 1e-300)) * std::cos(6.283185307179586 * u())); }
};

std::vector<float> gauss(size_t n, float std, uint64_t seed) {
    Rng r(seed);
    std::vector<float> v(n);
    for (auto &x : v) x = r.n() * std;
    return v;
}

template <class T> T *to_dev(const std::vector<T> &h) {
    T *d = nullptr;
    HIPCHK(hipMalloc(&d, h.size() * sizeof(T) + 4096));
    HIPCHK(hipMemset(d, 0, h.size() * sizeof(T) + 4096));
    HIPCHK(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    return d;
}
template <class T> T *dev_zero(size_t n) {
    T *d = nullptr;
    HIPCHK(hipMalloc(&d, n * sizeof(T) + 4096));
    HIPCHK(hipMemset(d, 0, n * sizeof(T) + 4096));
    return d;
}
template <class T> std::vector<T> to_host(const T *d, size_t n) {
    std::vector<T> h(n);
    HIPCHK(hipDeviceSynchronize());
    HIPCHK(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost));
    return h;
}

std::vector<uint8_t> quantize(int type, const std::vector<float> &w, int64_t nrows, int64_t ncols) {
    std::vector<uint8_t> q(or_row_bytes(type, ncols) * nrows);
    if (or_quantize(type, w.data(), q.data(), nrows, ncols, 8)) std::abort();
    return q;
}

void check(bool ok, const char *what) {
    std::printf("%-52s %s\n", what, ok ? "ok" : "FAILED");
    if (!ok) ++g_fail;
}
// max |y - ref| / max |ref| <= tol
void check_close(const std::vector<float> &y, const std::vector<double> &ref, double tol, const char *what) {
    double m = 0, r = 1e-30;
    for (size_t i = 0; i < ref.size(); ++i) {
        m = std::fmax(m, std::fabs(y[i] - ref[i]));
        r = std::fmax(r, std::fabs(ref[i]));
    }
    char buf[160];
    std::snprintf(buf, sizeof buf, "%s (err %.2e)", what, m / r);
    check(m / r <= tol, buf);
}

uint16_t f32_to_bf16(float f) {  // round to nearest even
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return (uint16_t) ((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
float bf16_to_f32(uint16_t b) {
    const uint32_t u = (uint32_t) b << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// The layer: experts [gate | up | down] in one slot each (the reference's exp_table contract, src/engine.cu:375-471),
// a bf16 router, RMSNorm weights and a shared expert.
struct Layer {
    int gu_type = 12, down_type = 14, sh_gu_type = 13, sh_down_type = 12;
    size_t gate_bytes, up_bytes, down_bytes, slot_bytes;
    std::vector<uint8_t> slots;                   // NE slots, host copy
    std::vector<uint8_t> sh_gate, sh_up, sh_down;  // shared expert
    std::vector<float> router_f32, norm_w;
    std::vector<uint8_t> head;                    // Q8_0 [NV][E]: the engine's dense / output-head type
    void *head_d;
    char *slots_d;
    const char **table_d;
    uint16_t *router_d;
    float *norm_d;
    void *sh_gate_d, *sh_up_d, *sh_down_d;

    void build() {
        gate_bytes = or_row_bytes(gu_type, E) * F;
        up_bytes = gate_bytes;
        down_bytes = or_row_bytes(down_type, F) * E;
        slot_bytes = (gate_bytes + up_bytes + down_bytes + 255) / 256 * 256;
        slots.assign(slot_bytes * NE, 0);
        for (int e = 0; e < NE; ++e) {
            const auto g = quantize(gu_type, gauss((size_t) F * E, 0.02f, 100 + e), F, E);
            const auto u = quantize(gu_type, gauss((size_t) F * E, 0.02f, 300 + e), F, E);
            const auto d = quantize(down_type, gauss((size_t) E * F, 0.02f, 500 + e), E, F);
            std::memcpy(&slots[e * slot_bytes], g.data(), g.size());
            std::memcpy(&slots[e * slot_bytes + gate_bytes], u.data(), u.size());
            std::memcpy(&slots[e * slot_bytes + gate_bytes + up_bytes], d.data(), d.size());
        }
        slots_d = (char *) to_dev(slots);
        std::vector<const char *> tab(NE);
        for (int e = 0; e < NE; ++e) tab[e] = slots_d + e * slot_bytes;
        table_d = to_dev(tab);
        const auto rw = gauss((size_t) NE * E, 0.02f, 7);
        std::vector<uint16_t> rb(rw.size());
        router_f32.resize(rw.size());
        for (size_t i = 0; i < rw.size(); ++i) {
            rb[i] = f32_to_bf16(rw[i]);
            router_f32[i] = bf16_to_f32(rb[i]);
        }
        router_d = to_dev(rb);
        norm_w = gauss(E, 0.1f, 8);
        for (auto &v : norm_w) v += 1.0f;
        norm_d = to_dev(norm_w);
        sh_gate = quantize(sh_gu_type, gauss((size_t) FS * E, 0.02f, 11), FS, E);
        sh_up = quantize(sh_gu_type, gauss((size_t) FS * E, 0.02f, 12), FS, E);
        sh_down = quantize(sh_down_type, gauss((size_t) E * FS, 0.02f, 13), E, FS);
        sh_gate_d = to_dev(sh_gate);
        sh_up_d = to_dev(sh_up);
        sh_down_d = to_dev(sh_down);
        head = quantize(8, gauss((size_t) NV * E, 0.02f, 14), NV, E);
        head_d = to_dev(head);
    }
    const uint8_t *mat(int e, int which) const {  // 0 gate, 1 up, 2 down
        return &slots[e * slot_bytes + (which == 0 ? 0 : which == 1 ? gate_bytes : gate_bytes + up_bytes)];
    }
};

// float64 W . deq(xq row) for one matrix.
std::vector<double> ref_mv(int type, const void *w, int64_t ncols, int64_t nrows, const uint8_t *xq_row) {
    std::vector<double> y(nrows);
    const void *tab[1] = {w};
    const int32_t id0 = 0;
    or_mmvq_experts(type, tab, ncols, nrows, xq_row, 1, 1, &id0, 1, y.data());
    return y;
}
std::vector<uint8_t> ref_q8_1(const float *x, int64_t ncols, int64_t nrows) {
    std::vector<uint8_t> q(or_q8_1_row_bytes(ncols) * nrows);
    or_quantize_q8_1(x, q.data(), ncols, nrows);
    return q;
}

// ---- decode / verify: Engine::ffn_block (src/engine.cu:655-696) ---------------------------------------------------
void run_decode(const Layer &L, int W) {
    std::printf("-- ffn_block, %d column(s)\n", W);
    hipStream_t st;
    HIPCHK(hipStreamCreate(&st));
    const auto x_h = gauss((size_t) W * E, 1.0f, 40 + W);
    float *x_ = to_dev(x_h), *h_ = dev_zero<float>((size_t) W * E), *router_ = dev_zero<float>((size_t) W * NE);
    const size_t xq_bytes = std::max((size_t) W * q8_1_row_bytes(E), (size_t) W * K * q8_1_row_bytes(FS));
    uint8_t *xq_ = dev_zero<uint8_t>(xq_bytes);
    int32_t *ids_ = dev_zero<int32_t>((size_t) W * K);
    float *wsel_ = dev_zero<float>((size_t) W * K), *act_ = dev_zero<float>((size_t) W * K * F);
    float *escale_ = dev_zero<float>((size_t) W * K), *dexp_ = dev_zero<float>((size_t) W * K * E);
    float *gate_ = dev_zero<float>((size_t) W * FS), *up_ = dev_zero<float>((size_t) W * FS);
    float *sh_ = dev_zero<float>((size_t) W * E);
    const auto ggml = [](int t) { return (ggml_type) t; };

    k::rms_norm_q8_1(x_, L.norm_d, h_, xq_, E, EPS, W, st);
    const auto h = to_host(h_, (size_t) W * E);
    const auto xq_h = to_host(xq_, (size_t) W * q8_1_row_bytes(E));
    // the output head (Engine::gemv on a Q8_0 matrix of NV rows): W columns in one call
    float *head_out = dev_zero<float>((size_t) W * NV);
    mmvq(GGML_TYPE_Q8_0, L.head_d, E, NV, xq_, head_out, W, st);
    const auto head_h = to_host(head_out, (size_t) W * NV);
    k::gemv_bf16(L.router_d, h_, router_, E, NE, W, st);
    if (W == 1) k::route_topk(router_, ids_, wsel_, NE, K, st);
    else k::route_topk_batch(router_, ids_, wsel_, NE, K, W, st);
    mmvq_experts_swiglu(ggml(L.gu_type), L.table_d, 0, L.gate_bytes, E, F, xq_, W, ids_, W * K, act_, st);
    // dense_glu (src/engine.cu:644-653): gate and up GEMVs, then the GLU
    mmvq(ggml(L.sh_gu_type), L.sh_gate_d, E, FS, xq_, gate_, W, st);
    mmvq(ggml(L.sh_gu_type), L.sh_up_d, E, FS, xq_, up_, W, st);
    k::glu_mmvq(gate_, up_, up_, W * FS, st);
    k::amax_guard_q8_1(act_, escale_, xq_, F, W * K, st);
    const auto aq_h = to_host(xq_, (size_t) W * K * q8_1_row_bytes(F));
    mmvq_experts(ggml(L.down_type), L.table_d, L.gate_bytes + L.up_bytes, F, E, xq_, W * K, ids_, W * K, dexp_, st);
    // gemv (src/engine.cu:585-588): Q8_1 of the input, then mmvq
    quantize_q8_1(up_, xq_, FS, W, st);
    mmvq(ggml(L.sh_down_type), L.sh_down_d, FS, E, xq_, sh_, W, st);
    const auto sh = to_host(sh_, (size_t) W * E);
    if (W == 1) k::moe_combine(dexp_, escale_, wsel_, sh_, x_, E, K, st);
    else k::moe_combine_batch(dexp_, escale_, wsel_, sh_, x_, E, K, W, st);
    HIPCHK(hipStreamSynchronize(st));

    // oracle checks, each stage fed with the GPU's previous stage
    std::vector<double> h_ref((size_t) W * E);
    for (int c = 0; c < W; ++c) {
        double s = 0;
        for (int i = 0; i < E; ++i) s += (double) x_h[c * E + i] * x_h[c * E + i];
        const double sc = 1.0 / std::sqrt(s / E + EPS);
        for (int i = 0; i < E; ++i) h_ref[c * E + i] = x_h[c * E + i] * sc * L.norm_w[i];
    }
    check_close(h, h_ref, 1e-5, "rms_norm_q8_1: h");
    for (int c = 0; c < W; ++c) {
        const auto ref = ref_mv(8, L.head.data(), E, NV, &xq_h[c * q8_1_row_bytes(E)]);
        check_close(std::vector<float>(head_h.begin() + (size_t) c * NV, head_h.begin() + (size_t) (c + 1) * NV), ref,
                    1e-4, "mmvq Q8_0: output head (150144 rows)");
    }
    check(ref_q8_1(h.data(), E, W) == xq_h, "rms_norm_q8_1: Q8_1 of h bit-exact");
    std::vector<float> lg_ref((size_t) W * NE);
    or_router_f32(L.router_f32.data(), h.data(), lg_ref.data(), E, NE, W);
    const auto lg = to_host(router_, (size_t) W * NE);
    check_close(lg, std::vector<double>(lg_ref.begin(), lg_ref.end()), 1e-5, "gemv_bf16: router logits");
    std::vector<int32_t> ids_ref((size_t) W * K);
    std::vector<float> w_ref((size_t) W * K), probs((size_t) W * NE), margin(W);
    or_route_topk(lg.data(), ids_ref.data(), w_ref.data(), probs.data(), margin.data(), NE, K, W, 1, 1);
    const auto ids = to_host(ids_, (size_t) W * K);
    const auto wsel = to_host(wsel_, (size_t) W * K);
    check(ids == ids_ref && std::memcmp(wsel.data(), w_ref.data(), w_ref.size() * 4) == 0,
          W == 1 ? "route_topk: ids and weights bit-exact" : "route_topk_batch: ids and weights bit-exact");
    const auto act = to_host(act_, (size_t) W * K * F);
    std::vector<double> act_ref((size_t) W * K * F);
    for (int c = 0; c < W; ++c)
        for (int j = 0; j < K; ++j) {
            const int e = ids[c * K + j];
            const auto g = ref_mv(L.gu_type, L.mat(e, 0), E, F, &xq_h[c * q8_1_row_bytes(E)]);
            const auto u = ref_mv(L.gu_type, L.mat(e, 1), E, F, &xq_h[c * q8_1_row_bytes(E)]);
            or_swiglu(g.data(), u.data(), &act_ref[(size_t) (c * K + j) * F], F);
        }
    check_close(act, act_ref, 1e-4, "mmvq_experts_swiglu: act");
    std::vector<float> esc((size_t) W * K);
    for (int r = 0; r < W * K; ++r) esc[r] = or_amax_guard_scale(&act[(size_t) r * F], F);
    std::vector<float> scaled(act.size());
    for (size_t i = 0; i < act.size(); ++i) scaled[i] = act[i] / esc[i / F];
    check(ref_q8_1(scaled.data(), F, W * K) == aq_h, "amax_guard_q8_1: Q8_1 of act bit-exact");
    check(to_host(escale_, (size_t) W * K) == esc, "amax_guard_q8_1: escale bit-exact");
    // shared expert, then the combine
    std::vector<double> sh_ref((size_t) W * E);
    for (int c = 0; c < W; ++c) {
        const auto g = ref_mv(L.sh_gu_type, L.sh_gate.data(), E, FS, &xq_h[c * q8_1_row_bytes(E)]);
        const auto u = ref_mv(L.sh_gu_type, L.sh_up.data(), E, FS, &xq_h[c * q8_1_row_bytes(E)]);
        std::vector<double> a(FS);
        or_swiglu(g.data(), u.data(), a.data(), FS);
        std::vector<float> af(a.begin(), a.end());
        const auto q = ref_q8_1(af.data(), FS, 1);
        const auto s = ref_mv(L.sh_down_type, L.sh_down.data(), FS, E, q.data());
        std::copy(s.begin(), s.end(), sh_ref.begin() + (size_t) c * E);
    }
    check_close(sh, sh_ref, 1e-3, "dense_glu + gemv: shared expert");
    std::vector<double> out_ref((size_t) W * E);
    for (int c = 0; c < W; ++c) {
        for (int i = 0; i < E; ++i) out_ref[c * E + i] = x_h[c * E + i] + sh[c * E + i];
        for (int j = 0; j < K; ++j) {
            const int r = c * K + j;
            const auto d = ref_mv(L.down_type, L.mat(ids[r], 2), F, E, &aq_h[r * q8_1_row_bytes(F)]);
            for (int i = 0; i < E; ++i) out_ref[c * E + i] += d[i] * esc[r] * wsel[r];
        }
    }
    check_close(to_host(x_, (size_t) W * E), out_ref, 1e-4, W == 1 ? "moe_combine: x" : "moe_combine_batch: x");
    HIPCHK(hipStreamDestroy(st));
}

// ---- prefill: Engine::prefill_chunk's FFN (src/engine.cu:330-357) ----------------------------------------------
void run_prefill(const Layer &L, int T) {
    std::printf("-- prefill_chunk FFN, %d tokens\n", T);
    hipStream_t st;
    HIPCHK(hipStreamCreate(&st));
    const auto ggml = [](int t) { return (ggml_type) t; };
    const auto h_h = gauss((size_t) T * E, 1.0f, 77);
    const auto x_h = gauss((size_t) T * E, 1.0f, 78);
    float *h = to_dev(h_h), *x = to_dev(x_h), *router = dev_zero<float>((size_t) T * NE);
    int32_t *ids = dev_zero<int32_t>((size_t) T * K);
    float *wsel = dev_zero<float>((size_t) T * K), *gate = dev_zero<float>((size_t) T * K * std::max(F, FS));
    float *up = dev_zero<float>((size_t) T * K * std::max(F, FS)), *act = dev_zero<float>((size_t) T * K * std::max(F, FS));
    float *escale = dev_zero<float>((size_t) T * K), *dexp = dev_zero<float>((size_t) T * K * E);
    float *sh = dev_zero<float>((size_t) T * E);
    void *xq = dev_zero<uint8_t>(mmq_q8_1_bytes(E, T));
    // MmqIdsScratch with the reference's sizes (src/engine.cu:228-231)
    MmqIdsScratch mm;
    mm.ids_src1 = dev_zero<int32_t>((size_t) T * K + 128);
    mm.ids_dst = dev_zero<int32_t>((size_t) T * K + 128);
    mm.expert_bounds = dev_zero<int32_t>(NE + 1);
    mm.xq = dev_zero<uint8_t>(mmq_q8_1_bytes(std::max(E, F), (int64_t) T * K));
    const size_t down_off = L.gate_bytes + L.up_bytes;

    k::gemm_bf16_batch(nullptr, L.router_d, h, nullptr, router, E, NE, T, st);
    k::route_topk_batch(router, ids, wsel, NE, K, T, st);
    mmq_experts(ggml(L.gu_type), L.table_d, 0, E, F, NE, h, 1, T, ids, K, mm, gate, st);
    mmq_experts(ggml(L.gu_type), L.table_d, L.gate_bytes, E, F, NE, h, 1, T, ids, K, mm, up, st);
    k::swiglu(gate, up, act, F, T * K, st);
    k::amax_guard(act, escale, F, T * K, st);
    const auto act_h = to_host(act, (size_t) T * K * F);
    mmq_experts(ggml(L.down_type), L.table_d, down_off, F, E, NE, act, K, T, ids, K, mm, dexp, st);
    const auto dexp_h = to_host(dexp, (size_t) T * K * E);
    mmq(ggml(L.sh_gu_type), L.sh_gate_d, E, FS, h, T, xq, gate, st);
    mmq(ggml(L.sh_gu_type), L.sh_up_d, E, FS, h, T, xq, up, st);
    k::swiglu(gate, up, act, FS, T, st);
    const auto sact_h = to_host(act, (size_t) T * FS);
    mmq(ggml(L.sh_down_type), L.sh_down_d, FS, E, act, T, xq, sh, st);
    const auto sh_h = to_host(sh, (size_t) T * E);
    k::moe_combine_batch(dexp, escale, wsel, sh, x, E, K, T, st);
    HIPCHK(hipStreamSynchronize(st));

    // gemm_bf16_batch multiplies bf16 x bf16 (the reference rounds x to bf16 for cuBLAS: src/prefill_kernels.cu:217-233)
    std::vector<float> hb(h_h.size()), lg_ref((size_t) T * NE);
    for (size_t i = 0; i < h_h.size(); ++i) hb[i] = bf16_to_f32(f32_to_bf16(h_h[i]));
    or_router_f32(L.router_f32.data(), hb.data(), lg_ref.data(), E, NE, T);
    const auto lg = to_host(router, (size_t) T * NE);
    check_close(lg, std::vector<double>(lg_ref.begin(), lg_ref.end()), 1e-5, "gemm_bf16_batch: router logits");
    std::vector<int32_t> ids_ref((size_t) T * K);
    std::vector<float> w_ref((size_t) T * K), probs((size_t) T * NE), margin(T);
    or_route_topk(lg.data(), ids_ref.data(), w_ref.data(), probs.data(), margin.data(), NE, K, T, 1, 1);
    const auto ids_h = to_host(ids, (size_t) T * K);
    const auto w_h = to_host(wsel, (size_t) T * K);
    check(ids_h == ids_ref && std::memcmp(w_h.data(), w_ref.data(), w_ref.size() * 4) == 0,
          "route_topk_batch: ids and weights bit-exact");
    const auto hq = ref_q8_1(h_h.data(), E, T);
    std::vector<double> act_ref((size_t) T * K * F);
    for (int t = 0; t < T; ++t)
        for (int j = 0; j < K; ++j) {
            const int e = ids_h[t * K + j];
            const auto g = ref_mv(L.gu_type, L.mat(e, 0), E, F, &hq[t * q8_1_row_bytes(E)]);
            const auto u = ref_mv(L.gu_type, L.mat(e, 1), E, F, &hq[t * q8_1_row_bytes(E)]);
            std::vector<double> a(F);
            or_swiglu(g.data(), u.data(), a.data(), F);
            const float es = or_amax_guard_scale(std::vector<float>(a.begin(), a.end()).data(), F);
            for (int i = 0; i < F; ++i) act_ref[(size_t) (t * K + j) * F + i] = a[i] / es;
        }
    check_close(act_h, act_ref, 1e-3, "mmq_experts gate/up + swiglu + amax_guard: act");
    const auto aq = ref_q8_1(act_h.data(), F, T * K);
    std::vector<double> dexp_ref((size_t) T * K * E);
    for (int r = 0; r < T * K; ++r) {
        const auto d = ref_mv(L.down_type, L.mat(ids_h[r], 2), F, E, &aq[r * q8_1_row_bytes(F)]);
        std::copy(d.begin(), d.end(), dexp_ref.begin() + (size_t) r * E);
    }
    check_close(dexp_h, dexp_ref, 1e-3, "mmq_experts down: dexp");
    std::vector<double> sh_ref((size_t) T * E);
    const auto saq = ref_q8_1(sact_h.data(), FS, T);
    for (int t = 0; t < T; ++t) {
        const auto s = ref_mv(L.sh_down_type, L.sh_down.data(), FS, E, &saq[t * q8_1_row_bytes(FS)]);
        std::copy(s.begin(), s.end(), sh_ref.begin() + (size_t) t * E);
    }
    check_close(sh_h, sh_ref, 1e-3, "mmq (shared expert down): sh");
    std::vector<float> out_ref((size_t) T * E);
    or_moe_combine(dexp_h.data(), to_host(escale, (size_t) T * K).data(), w_h.data(), sh_h.data(), x_h.data(),
                   out_ref.data(), E, K, T);
    check(to_host(x, (size_t) T * E) == out_ref, "moe_combine_batch: bit-exact");
    HIPCHK(hipStreamDestroy(st));
}

}  // namespace

int main() {
    Layer L;
    L.build();
    run_decode(L, 1);
    run_decode(L, 2);
    run_prefill(L, 40);
    if (g_fail) {
        std::printf("ENGINE_CALLER_FAILED: %d check(s)\n", g_fail);
        return 1;
    }
    std::printf("ENGINE_CALLER_OK\n");
    return 0;
}
