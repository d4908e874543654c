// dense_ffn.cpp - the dense FFN layer (the reference model's leading dense blocks) composed from the library's
// kernels, in its two forms:
//   decode / verify (reference src/engine.cu:655-667 with dense_glu :644-653 and gemv :585-588): rms_norm_q8_1 of x,
//     mmvq_swiglu of gate and up at one token (two mmvq and glu_mmvq at more, or when gate and up differ in type:
//     the same bits), quantize_q8_1 of act, mmvq of down, out = x + ffn;
//   prefill (reference src/engine.cu:331-337): rms_norm (the f32 output of rms_norm_q8_1, the reference's
//     rms_norm_mul), mmq of gate and of up, swiglu, mmq of down, out = x + ffn. When gate and up share a type the
//     tiled GEMM takes, gate and up run as one GLU launch (SwiGLU and act's Q8_1 in the epilogue, as the MoE
//     path's shared expert) and down with its K range split in up to 4 parts summed with the residual add.
// The GEMMs are the dense forms of the MoE path's kernels (mmvq.hip, mmq.hip); the layer adds no kernel of its own
// beyond the residual add.
#include <cstdint>

#include "fns_host.hpp"
#include "fns_internal.hpp"

namespace fns::impl {

namespace {

constexpr int kMaxParts = 4;  // K-split parts of the prefill form's down GEMM

struct DenseWs {
    float *h, *gate, *act, *ffn, *parts;
    void *xq;
    size_t total;
};

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

DenseWs dense_layout(const FnsDenseFfn *D, int64_t n, uint8_t *base) {
    const int64_t H = D->hidden, F = D->inter;
    const size_t sh = align256((size_t) n * H * 4), sf = align256((size_t) n * F * 4);
    const int64_t wide = H > F ? H : F;
    size_t sq = (size_t) n * host::q8_1_row_bytes(wide);
    const size_t img = mmq_q8_1_bytes(wide, n);
    if (img > sq) sq = img;
    DenseWs w{};
    size_t off = 0;
    w.h = (float *) (base + off), off += sh;
    w.gate = (float *) (base + off), off += sf;
    w.act = (float *) (base + off), off += sf;
    w.ffn = (float *) (base + off), off += sh;
    w.xq = base + off, off += align256(sq);
    w.parts = (float *) (base + off), off += (size_t) kMaxParts * sh;
    w.total = off;
    return w;
}

int check_desc(const FnsDenseFfn *D, int64_t n_tok) {
    if (!D) return host::set_error(host::ERR_SHAPE, "dense_ffn: null layer");
    if (D->hidden <= 0 || D->hidden % 256 || D->inter <= 0 || D->inter % 256 || D->hidden > 65536 ||
        D->inter > 65536 || n_tok < 0 || n_tok > 65535)
        return host::set_error(host::ERR_SHAPE, "dense_ffn: hidden and inter must be positive multiples of 256 "
                                                "(<= 65536), n_tok <= 65535 (hidden %d inter %d n_tok %lld)",
                               D->hidden, D->inter, (long long) n_tok);
    if (!D->gate || !D->up || !D->down) return host::set_error(host::ERR_SHAPE, "dense_ffn: null matrix");
    return host::OK;
}

}  // namespace

int dense_ffn_workspace(const FnsDenseFfn *D, int64_t n_tok, size_t *total) {
    FNS_TRY(check_desc(D, n_tok));
    if (!total) return host::set_error(host::ERR_SHAPE, "dense_ffn_workspace: null output");
    *total = dense_layout(D, n_tok, nullptr).total;
    return host::OK;
}

int dense_ffn(const FnsDenseFfn *D, const float *x, float *out, int64_t n_tok, void *ws, size_t ws_bytes, bool prefill,
              hipStream_t st) {
    FNS_TRY(check_desc(D, n_tok));
    if (!x || !out || (n_tok > 0 && !ws)) return host::set_error(host::ERR_SHAPE, "dense_ffn: null argument");
    if (n_tok == 0) return host::OK;
    const DenseWs w = dense_layout(D, n_tok, (uint8_t *) ws);
    if (ws_bytes < w.total)
        return host::set_error(host::ERR_SHAPE, "dense_ffn: workspace of %zu bytes, %zu needed", ws_bytes, w.total);
    const int H = D->hidden, F = D->inter, n = (int) n_tok;
    const float *h = x;
    if (prefill && D->gate_type == D->up_type && mmq_tiled(D->gate_type, H, F) && mmq_tiled(D->down_type, F, H)) {
        // the tiled GEMMs on images built once: x image, gate + up in one launch (SwiGLU and the Q8_1 of act in its
        // epilogue, the act images land in the gate/act region), down with its K range split so that the launch
        // fills the GPU, then out = x + (sum of the parts)
        if (D->ffn_norm) {
            FNS_TRY(rms_norm_q8_1(x, D->ffn_norm, w.h, w.xq, H, D->norm_eps, n, st));
            h = w.h;
        }
        FNS_TRY(mmq_quant_image(h, H, n_tok, w.xq, st));
        void *act_img = w.gate;  // n x F image bytes (4.125 per value) fit the gate and act regions together
        FNS_TRY(mmq_dense_glu(D->gate_type, D->gate, D->up, H, F, w.xq, n_tok, act_img, st));
        const int64_t items = (n_tok + 63) / 64 * ((H + 255) / 256);
        int parts = 1;
        while (parts < kMaxParts && items * parts * 2 <= 512 && F / 256 >= parts * 2) parts *= 2;
        FNS_TRY(mmq_dense_parts(D->down_type, D->down, F, H, act_img, n_tok, w.parts, parts, st));
        return add_parts(x, w.parts, parts, out, (int64_t) n * H, st);
    }
    if (prefill) {
        if (D->ffn_norm) {
            FNS_TRY(rms_norm_q8_1(x, D->ffn_norm, w.h, w.xq, H, D->norm_eps, n, st));
            h = w.h;
        }
        FNS_TRY(mmq(D->gate_type, D->gate, H, F, h, n_tok, w.xq, w.gate, st));
        FNS_TRY(mmq(D->up_type, D->up, H, F, h, n_tok, w.xq, w.act, st));
        FNS_TRY(swiglu(w.gate, w.act, w.act, F, n, st));
        FNS_TRY(mmq(D->down_type, D->down, F, H, w.act, n_tok, w.xq, w.ffn, st));
    } else {
        if ((int64_t) n * F > INT32_MAX)
            return host::set_error(host::ERR_SHAPE, "dense_ffn: decode form limited to n_tok * inter < 2^31 values");
        if (!host::is_supported(D->gate_type) || !host::is_supported(D->up_type) || !host::is_supported(D->down_type))
            return host::set_error(host::ERR_TYPE, "dense_ffn: a matrix type the GEMV kernels do not support");
        if (D->ffn_norm) FNS_TRY(rms_norm_q8_1(x, D->ffn_norm, w.h, w.xq, H, D->norm_eps, n, st));
        else FNS_TRY(quantize_q8_1(x, w.xq, H, n_tok, st));
        if (n == 1 && D->gate_type == D->up_type) {
            FNS_TRY(mmvq_swiglu(D->gate_type, D->gate, D->up, H, F, w.xq, w.act, st));
        } else {
            FNS_TRY(mmvq(D->gate_type, D->gate, H, F, w.xq, w.gate, n_tok, st));
            FNS_TRY(mmvq(D->up_type, D->up, H, F, w.xq, w.act, n_tok, st));
            FNS_TRY(glu_mmvq(w.gate, w.act, w.act, n * F, st));
        }
        FNS_TRY(quantize_q8_1(w.act, w.xq, F, n_tok, st));
        FNS_TRY(mmvq(D->down_type, D->down, F, H, w.xq, w.ffn, n_tok, st));
    }
    return add(x, w.ffn, out, (int64_t) n * H, st);
}

}  // namespace fns::impl
