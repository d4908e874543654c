// gguf_capi.cpp - extern "C" entry points of the GGUF reader and the resident MoE and dense FFN layers (include/fns_hip.h): thin
// forwards to include/fns/gguf.h; exceptions become FNS_ERR_IO / FNS_ERR_SHAPE with their message kept for
// fns_hip_last_error().
#include <cstring>
#include <exception>
#include <stdexcept>
#include <string>

#include "fns/gguf.h"
#include "fns_hip.h"
#include "fns_host.hpp"

using namespace fns;

struct FnsGguf {
    Gguf file;
    explicit FnsGguf(const char *path) : file(path) {}
};
struct FnsMoeResident {
    ResidentMoeLayer layer;
};
struct FnsDenseResident {
    ResidentDenseFfn ffn;
};

namespace {
void fill(const GgufTensor &t, FnsGgufTensorInfo *info) {
    info->type = t.type;
    info->n_dims = t.n_dims;
    for (int d = 0; d < 4; ++d) info->ne[d] = t.ne[d];
    info->nbytes = t.nbytes;
    info->offset = t.offset;
    info->data = t.data;
}
template <class F> int guarded(int code, F &&f) {
    try {
        return f();
    } catch (const std::exception &e) {
        return host::set_error(code, "%s", e.what());
    }
}
}  // namespace

extern "C" {

int fns_hip_gguf_open(const char *path, FnsGguf **out) {
    if (!path || !out) return host::set_error(host::ERR_SHAPE, "gguf_open: null argument");
    *out = nullptr;
    return guarded(FNS_ERR_IO, [&] {
        *out = new FnsGguf(path);
        return host::OK;
    });
}

void fns_hip_gguf_close(FnsGguf *file) { delete file; }

int fns_hip_gguf_info(const FnsGguf *file, uint32_t *version, int64_t *n_tensors, int64_t *n_kv, size_t *data_offset) {
    if (!file) return host::set_error(host::ERR_SHAPE, "gguf_info: null file");
    if (version) *version = file->file.version();
    if (n_tensors) *n_tensors = file->file.n_tensors();
    if (n_kv) *n_kv = file->file.n_kv();
    if (data_offset) *data_offset = file->file.data_offset();
    return host::OK;
}

int fns_hip_gguf_tensor(const FnsGguf *file, const char *name, FnsGgufTensorInfo *info) {
    if (!file || !name || !info) return host::set_error(host::ERR_SHAPE, "gguf_tensor: null argument");
    const GgufTensor *t = file->file.find_tensor(name);
    if (!t) return host::set_error(host::ERR_SHAPE, "gguf_tensor: no tensor %s", name);
    fill(*t, info);
    return host::OK;
}

int fns_hip_gguf_tensor_at(const FnsGguf *file, int64_t index, FnsGgufTensorInfo *info, const char **name) {
    if (!file || !info) return host::set_error(host::ERR_SHAPE, "gguf_tensor_at: null argument");
    if (index < 0 || index >= file->file.n_tensors())
        return host::set_error(host::ERR_SHAPE, "gguf_tensor_at: index %lld out of range", (long long) index);
    const GgufTensor &t = file->file.tensor(index);
    fill(t, info);
    if (name) *name = t.name.c_str();
    return host::OK;
}

int fns_hip_gguf_get_u32(const FnsGguf *file, const char *key, uint32_t *value) {
    if (!file || !key || !value) return host::set_error(host::ERR_SHAPE, "gguf_get_u32: null argument");
    return guarded(host::ERR_SHAPE, [&] {
        *value = file->file.get_u32(key);
        return host::OK;
    });
}
int fns_hip_gguf_get_f32(const FnsGguf *file, const char *key, float *value) {
    if (!file || !key || !value) return host::set_error(host::ERR_SHAPE, "gguf_get_f32: null argument");
    return guarded(host::ERR_SHAPE, [&] {
        *value = file->file.get_f32(key);
        return host::OK;
    });
}
int fns_hip_gguf_get_bool(const FnsGguf *file, const char *key, int *value) {
    if (!file || !key || !value) return host::set_error(host::ERR_SHAPE, "gguf_get_bool: null argument");
    return guarded(host::ERR_SHAPE, [&] {
        *value = file->file.get_bool(key) ? 1 : 0;
        return host::OK;
    });
}
int fns_hip_gguf_get_str(const FnsGguf *file, const char *key, const char **value) {
    if (!file || !key || !value) return host::set_error(host::ERR_SHAPE, "gguf_get_str: null argument");
    const int64_t id = file->file.find_key(key);
    if (id < 0 || file->file.kv(id).type != GGUF_STRING)
        return host::set_error(host::ERR_SHAPE, "gguf_get_str: no string key %s", key);
    *value = file->file.kv(id).str.c_str();
    return host::OK;
}

int fns_hip_moe_layer_from_gguf(const FnsGguf *file, int layer, FnsMoeResident **resident, FnsMoeLayer *desc) {
    if (!file || !resident || !desc) return host::set_error(host::ERR_SHAPE, "moe_layer_from_gguf: null argument");
    *resident = nullptr;
    return guarded(FNS_ERR_IO, [&] {
        FnsMoeResident *r = new FnsMoeResident;
        try {
            build_resident_moe_layer(file->file, layer, r->layer);
        } catch (...) {
            delete r;
            throw;
        }
        const ResidentMoeLayer &L = r->layer;
        std::memset(desc, 0, sizeof *desc);
        desc->hidden = L.hidden;
        desc->inter = L.inter;
        desc->n_expert = L.n_expert;
        desc->k = L.k;
        desc->gating = L.gating;
        desc->norm_w = L.norm_w;
        desc->guard = file->file.get_str("general.architecture") == "flint" ? 1 : 0;
        desc->router_dtype = L.router_dtype;
        desc->router_w = L.router;
        desc->gu_type = L.gu_type;
        desc->down_type = L.down_type;
        desc->table = (const void *const *) L.table;
        desc->gate_off = 0;
        desc->up_off = L.gate_bytes;
        desc->down_off = L.gate_bytes + L.up_bytes;
        desc->router_bias = L.router_bias;
        desc->ffn_norm = L.ffn_norm;
        desc->norm_eps = L.norm_eps;
        desc->shexp_inter = L.shexp_inter;
        desc->shexp_gu_type = L.shexp_inter ? L.shexp_gu_type : 0;
        desc->shexp_down_type = L.shexp_inter ? L.shexp_down_type : 0;
        desc->shexp_gate = L.shexp_gate;
        desc->shexp_up = L.shexp_up;
        desc->shexp_down = L.shexp_down;
        *resident = r;
        return host::OK;
    });
}

void fns_hip_moe_resident_free(FnsMoeResident *resident) { delete resident; }

int fns_hip_dense_ffn_from_gguf(const FnsGguf *file, int layer, FnsDenseResident **resident, FnsDenseFfn *desc) {
    if (!file || !resident || !desc) return host::set_error(host::ERR_SHAPE, "dense_ffn_from_gguf: null argument");
    *resident = nullptr;
    return guarded(FNS_ERR_IO, [&] {
        FnsDenseResident *r = new FnsDenseResident;
        try {
            build_resident_dense_ffn(file->file, layer, r->ffn);
        } catch (...) {
            delete r;
            throw;
        }
        const ResidentDenseFfn &D = r->ffn;
        std::memset(desc, 0, sizeof *desc);
        desc->hidden = D.hidden;
        desc->inter = D.inter;
        desc->gate_type = D.gate_type;
        desc->up_type = D.up_type;
        desc->down_type = D.down_type;
        desc->gate = D.gate;
        desc->up = D.up;
        desc->down = D.down;
        desc->ffn_norm = D.ffn_norm;
        desc->norm_eps = D.norm_eps;
        *resident = r;
        return host::OK;
    });
}

void fns_hip_dense_resident_free(FnsDenseResident *resident) { delete resident; }

}  // extern "C"
