// moe_slots.cpp - one MoE layer of a GGUF checkpoint made fully resident in HBM: expert slots [gate | up | down],
// the device table of slot pointers, router, RMSNorm weights and shared expert; and a dense FFN layer's matrices
// (include/fns/gguf.h).
// Reference: /root/reference/src/engine.cu:375-471 (Engine::place_experts; here every expert is resident),
// src/model.cpp:120-129,159-178 (tensor names, shapes, types and the mmvq_supports check).
#include "fns/gguf.h"

#include <hip/hip_runtime.h>

#include <stdexcept>
#include <vector>

#include "fns_host.hpp"

namespace fns {

namespace {

constexpr size_t kAlign = 256, kPad = 4096;  // slot alignment and trailing zero bytes (reference src/engine.cu:381)

[[noreturn]] void fail(int il, const std::string &what, const char *kind = "MoE layer ") {
    throw std::runtime_error(kind + std::to_string(il) + ": " + what);
}
void hip_ok(hipError_t e, const char *what) {
    if (e != hipSuccess) throw std::runtime_error(std::string("MoE layer build: ") + what + ": " + hipGetErrorString(e));
}
void *upload(const void *src, size_t n) {
    void *d = nullptr;
    hip_ok(hipMalloc(&d, n), "hipMalloc");
    const hipError_t e = hipMemcpy(d, src, n, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void) hipFree(d);
        hip_ok(e, "hipMemcpy");
    }
    return d;
}
void check_shape(int il, const GgufTensor &t, std::initializer_list<int64_t> ne, const char *kind = "MoE layer ") {
    int d = 0;
    for (int64_t v : ne)
        if (t.ne[d++] != v) fail(il, "unexpected shape of " + t.name, kind);
    for (; d < 4; ++d)
        if (t.ne[d] != 1) fail(il, "unexpected shape of " + t.name, kind);
}

}  // namespace

ResidentMoeLayer::~ResidentMoeLayer() {
    for (void *p : {slots, (void *) table, router, (void *) router_bias, (void *) ffn_norm, shexp_gate, shexp_up,
                    shexp_down})
        if (p) (void) hipFree(p);
}

void build_resident_moe_layer(const Gguf &f, int il, ResidentMoeLayer &out) {
    const std::string arch = f.get_str("general.architecture");
    const std::string p = "blk." + std::to_string(il) + ".";
    const GgufTensor &g = f.get_tensor(p + "ffn_gate_exps.weight");
    const GgufTensor &u = f.get_tensor(p + "ffn_up_exps.weight");
    const GgufTensor &dn = f.get_tensor(p + "ffn_down_exps.weight");
    const GgufTensor &r = f.get_tensor(p + "ffn_gate_inp.weight");
    const int64_t H = g.ne[0], F = g.ne[1], NE = g.ne[2];
    check_shape(il, g, {H, F, NE});
    check_shape(il, u, {H, F, NE});
    check_shape(il, dn, {F, H, NE});
    check_shape(il, r, {H, NE});
    if (u.type != g.type) fail(il, "gate and up experts have different types");
    if (!host::is_supported(g.type) || !host::is_supported(dn.type))
        fail(il, "expert types " + std::to_string(g.type) + "/" + std::to_string(dn.type) +
                     " are not supported by the GEMV kernels (mmvq_supports)");
    if (r.type != 0 && r.type != 30) fail(il, "router must be F32 or BF16");
    const int64_t ne_meta = (int64_t) f.get_u32_or(arch + ".expert_count", (uint32_t) NE);
    if (ne_meta != NE) fail(il, "expert_count differs from the expert tensors");
    const int k = (int) f.get_u32(arch + ".expert_used_count");
    if (k < 1 || k > NE) fail(il, "bad expert_used_count");
    const uint32_t gf = f.get_u32_or(arch + ".expert_gating_func", arch == "flint" ? 2u : 1u);
    if (gf != 1 && gf != 2) fail(il, "expert_gating_func must be 1 (softmax) or 2 (sigmoid)");
    // the reference requires an expert weight scale of 1 (src/model.cpp:83,167): the combine applies none
    const float ews = f.get_f32_or(arch + ".expert_weights_scale", 1.0f);
    if (ews != 1.0f) fail(il, "expert_weights_scale " + std::to_string(ews) + " is not 1 (the combine applies no scale)");

    out.hidden = (int) H;
    out.inter = (int) F;
    out.n_expert = (int) NE;
    out.k = k;
    out.gu_type = g.type;
    out.down_type = dn.type;
    out.router_dtype = r.type;
    out.gating = gf == 2 ? 1 : 0;
    out.norm_w = f.get_bool_or(arch + ".expert_weights_norm", true) ? 1 : 0;
    out.norm_eps = f.get_f32_or(arch + ".attention.layer_norm_rms_epsilon", 1e-6f);
    out.gate_bytes = g.nbytes / (size_t) NE;
    out.up_bytes = u.nbytes / (size_t) NE;
    out.down_bytes = dn.nbytes / (size_t) NE;
    out.slot_bytes = (out.gate_bytes + out.up_bytes + out.down_bytes + kAlign - 1) / kAlign * kAlign;

    // slots: one allocation, expert e at e * slot_bytes, kPad zero bytes after the last one
    const size_t total = (size_t) NE * out.slot_bytes + kPad;
    hip_ok(hipMalloc(&out.slots, total), "hipMalloc(slots)");
    hip_ok(hipMemset(out.slots, 0, total), "hipMemset(slots)");
    std::vector<void *> table((size_t) NE);
    for (int64_t e = 0; e < NE; ++e) {
        uint8_t *s = (uint8_t *) out.slots + (size_t) e * out.slot_bytes;
        hip_ok(hipMemcpy(s, (const uint8_t *) g.data + (size_t) e * out.gate_bytes, out.gate_bytes,
                         hipMemcpyHostToDevice), "hipMemcpy(gate)");
        hip_ok(hipMemcpy(s + out.gate_bytes, (const uint8_t *) u.data + (size_t) e * out.up_bytes, out.up_bytes,
                         hipMemcpyHostToDevice), "hipMemcpy(up)");
        hip_ok(hipMemcpy(s + out.gate_bytes + out.up_bytes, (const uint8_t *) dn.data + (size_t) e * out.down_bytes,
                         out.down_bytes, hipMemcpyHostToDevice), "hipMemcpy(down)");
        table[(size_t) e] = s;
    }
    out.table = (void **) upload(table.data(), table.size() * sizeof(void *));
    out.router = upload(r.data, r.nbytes);
    if (const GgufTensor *b = f.find_tensor(p + "exp_probs_b.bias")) {
        check_shape(il, *b, {NE});
        if (b->type != 0) fail(il, "exp_probs_b.bias must be F32");
        out.router_bias = (float *) upload(b->data, b->nbytes);
    }
    if (const GgufTensor *n = f.find_tensor(p + "ffn_norm.weight")) {
        check_shape(il, *n, {H});
        if (n->type != 0) fail(il, "ffn_norm.weight must be F32");
        out.ffn_norm = (float *) upload(n->data, n->nbytes);
    }
    const GgufTensor *sg = f.find_tensor(p + "ffn_gate_shexp.weight");
    if (sg) {
        const GgufTensor &su = f.get_tensor(p + "ffn_up_shexp.weight");
        const GgufTensor &sd = f.get_tensor(p + "ffn_down_shexp.weight");
        const int64_t Fs = sg->ne[1];
        check_shape(il, *sg, {H, Fs});
        check_shape(il, su, {H, Fs});
        check_shape(il, sd, {Fs, H});
        if (su.type != sg->type) fail(il, "shared expert gate and up have different types");
        if (!host::is_supported(sg->type) || !host::is_supported(sd.type))
            fail(il, "shared expert types are not supported by the GEMV kernels");
        out.shexp_inter = (int) Fs;
        out.shexp_gu_type = sg->type;
        out.shexp_down_type = sd.type;
        out.shexp_gate = upload(sg->data, sg->nbytes);
        out.shexp_up = upload(su.data, su.nbytes);
        out.shexp_down = upload(sd.data, sd.nbytes);
    }
}

ResidentDenseFfn::~ResidentDenseFfn() {
    for (void *p : {gate, up, down, (void *) ffn_norm})
        if (p) (void) hipFree(p);
}

void build_resident_dense_ffn(const Gguf &f, int il, ResidentDenseFfn &out) {
    const std::string arch = f.get_str("general.architecture");
    const std::string p = "blk." + std::to_string(il) + ".";
    constexpr const char *kind = "dense FFN layer ";
    auto failf = [&](const std::string &what) { fail(il, what, kind); };
    const GgufTensor &g = f.get_tensor(p + "ffn_gate.weight");
    const GgufTensor &u = f.get_tensor(p + "ffn_up.weight");
    const GgufTensor &dn = f.get_tensor(p + "ffn_down.weight");
    const int64_t H = g.ne[0], F = g.ne[1];
    check_shape(il, g, {H, F}, kind);
    check_shape(il, u, {H, F}, kind);
    check_shape(il, dn, {F, H}, kind);
    if (H <= 0 || H % 256 || F <= 0 || F % 256 || H > 65536 || F > 65536)
        failf("hidden and inter must be multiples of 256 (<= 65536)");
    for (const GgufTensor *t : {&g, &u, &dn})
        if (!host::is_supported(t->type))
            failf("type " + std::to_string(t->type) + " of " + t->name + " is not supported by the GEMV kernels "
                  "(mmvq_supports)");
    const GgufTensor *n = f.find_tensor(p + "ffn_norm.weight");
    if (n) {
        check_shape(il, *n, {H}, kind);
        if (n->type != 0) failf("ffn_norm.weight must be F32");
    }
    out.hidden = (int) H;
    out.inter = (int) F;
    out.gate_type = g.type;
    out.up_type = u.type;
    out.down_type = dn.type;
    out.norm_eps = f.get_f32_or(arch + ".attention.layer_norm_rms_epsilon", 1e-6f);
    out.gate = upload(g.data, g.nbytes);
    out.up = upload(u.data, u.nbytes);
    out.down = upload(dn.data, dn.nbytes);
    if (n) out.ffn_norm = (float *) upload(n->data, n->nbytes);
}

}  // namespace fns
