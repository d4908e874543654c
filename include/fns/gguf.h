// include/fns/gguf.h - GGUF (v2/v3) reader over a read-only memory mapping of the whole file, and the fully resident
// expert slots of one MoE layer built from it.
//
// Replaces the reference's loader: /root/reference/src/model.cpp:30-136 (metadata through the ggml-base gguf API,
// tensor data through a Win32 file mapping; include/fns/model.h:14-21 Tensor views) and the slot placement of
// /root/reference/src/engine.cu:375-471 (Engine::place_experts: expert e of a layer is one slot [gate | up | down],
// 256-byte aligned, 4096 zero bytes after the last slot, a device table of slot pointers; include/fns/engine.h:28-32).
// On MI355X every expert stays in HBM, so placement is the trivial all-resident case and there is no host copy.
//
// The file format is the public GGUF layout (llama.cpp gguf.cpp / docs/gguf.md at the pinned commit 19ab5a5e):
//   "GGUF" | u32 version | u64 n_tensors | u64 n_kv | n_kv x (string key, u32 type, value)
//   | n_tensors x (string name, u32 n_dims, u64 ne[n_dims], u32 ggml_type, u64 offset) | padding to `alignment`
//   | tensor data (each tensor at data_offset + offset).
// Strings are u64 length + bytes; arrays are u32 element type + u64 count + elements; general.alignment (u32,
// default 32) aligns the data section and every tensor.
//
// Errors: the constructor and the slot builder throw std::runtime_error with a message naming the file and what is
// wrong (the reference's Model throws runtime_error too: src/model.cpp:17). Nothing here launches a kernel.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace fns {

// GGUF value types (public gguf.h enum gguf_type).
enum GgufType : uint32_t {
    GGUF_U8 = 0, GGUF_I8 = 1, GGUF_U16 = 2, GGUF_I16 = 3, GGUF_U32 = 4, GGUF_I32 = 5, GGUF_F32 = 6, GGUF_BOOL = 7,
    GGUF_STRING = 8, GGUF_ARRAY = 9, GGUF_U64 = 10, GGUF_I64 = 11, GGUF_F64 = 12,
};

// A view of a tensor in the mapped file; `ne` in ggml order (ne[0] = contiguous dimension). Mirrors the reference's
// fns::Tensor (include/fns/model.h:14-21).
struct GgufTensor {
    std::string name;
    int type = -1;  // ggml_type value
    int64_t ne[4] = {1, 1, 1, 1};
    int n_dims = 0;
    const void *data = nullptr;  // points into the mapping
    size_t nbytes = 0;
    size_t offset = 0;  // from the start of the data section
};

// One key/value pair: scalars decoded into u64/i64/f64 (and the raw bytes for arrays), strings kept as text.
struct GgufKv {
    std::string key;
    uint32_t type = 0;      // GgufType
    uint32_t arr_type = 0;  // element type of an array
    uint64_t arr_n = 0;     // element count of an array
    const void *arr_data = nullptr;  // first element of a fixed-size array (in the mapping)
    std::vector<std::string> arr_str;  // elements of a string array
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0.0;
    std::string str;
};

// Bytes of one row of `ne0` values of a ggml type (0 when the type is not one this reader knows).
size_t ggml_row_bytes(int type, int64_t ne0);

class Gguf {
public:
    explicit Gguf(const std::string &path);  // throws std::runtime_error on a missing, short or malformed file
    ~Gguf();
    Gguf(const Gguf &) = delete;
    Gguf &operator=(const Gguf &) = delete;

    uint32_t version() const { return version_; }
    size_t alignment() const { return alignment_; }
    size_t data_offset() const { return data_off_; }
    size_t file_size() const { return size_; }

    // gguf_find_key / gguf_get_val_* of the reference's loader (src/model.cpp:19-26): -1 / throw when absent or of
    // another type.
    int64_t find_key(const std::string &key) const;
    const GgufKv &kv(int64_t id) const { return kvs_[(size_t) id]; }
    int64_t n_kv() const { return (int64_t) kvs_.size(); }
    uint32_t get_u32(const std::string &key) const;
    float get_f32(const std::string &key) const;
    bool get_bool(const std::string &key) const;
    std::string get_str(const std::string &key) const;
    // Optional forms: the default when the key is absent.
    uint32_t get_u32_or(const std::string &key, uint32_t dflt) const;
    float get_f32_or(const std::string &key, float dflt) const;
    bool get_bool_or(const std::string &key, bool dflt) const;

    int64_t n_tensors() const { return (int64_t) tensors_.size(); }
    const GgufTensor &tensor(int64_t i) const { return tensors_[(size_t) i]; }
    const GgufTensor *find_tensor(const std::string &name) const;  // nullptr when absent
    const GgufTensor &get_tensor(const std::string &name) const;   // throws when absent

private:
    std::string path_;
    int fd_ = -1;
    const uint8_t *base_ = nullptr;
    size_t size_ = 0;
    uint32_t version_ = 0;
    size_t alignment_ = 32;
    size_t data_off_ = 0;
    std::vector<GgufKv> kvs_;
    std::vector<GgufTensor> tensors_;
};

// The routed experts of one MoE layer copied into HBM as slots [gate | up | down] (reference src/engine.cu:375-471),
// with the device table of slot pointers, plus the layer's router (and bias), RMSNorm weights and shared expert when
// the file has them. Tensor names follow the reference model (src/model.cpp:120-129): blk.N.ffn_gate_inp.weight,
// ffn_{gate,up,down}_exps.weight, ffn_{gate,up,down}_shexp.weight, ffn_norm.weight; exp_probs_b.bias is the
// optional router bias. Device memory is owned by this object and freed by its destructor.
struct ResidentMoeLayer {
    int hidden = 0, inter = 0, n_expert = 0, k = 0;
    int gu_type = -1, down_type = -1;
    int router_dtype = -1;       // ggml type of the router (F32 or BF16)
    int gating = 1;              // 0 softmax, 1 sigmoid
    int norm_w = 1;              // renormalise the selected weights
    float norm_eps = 0.0f;
    size_t gate_bytes = 0, up_bytes = 0, down_bytes = 0, slot_bytes = 0;
    void *slots = nullptr;       // n_expert * slot_bytes + 4096 bytes (the last 4096 zero)
    void **table = nullptr;      // [n_expert] device slot pointers
    void *router = nullptr;      // [n_expert][hidden]
    float *router_bias = nullptr;  // [n_expert] or null
    float *ffn_norm = nullptr;   // [hidden] or null
    int shexp_inter = 0, shexp_gu_type = -1, shexp_down_type = -1;
    void *shexp_gate = nullptr, *shexp_up = nullptr, *shexp_down = nullptr;

    ResidentMoeLayer() = default;
    ResidentMoeLayer(const ResidentMoeLayer &) = delete;
    ResidentMoeLayer &operator=(const ResidentMoeLayer &) = delete;
    ~ResidentMoeLayer();
};

// Builds layer `il` of the file (architecture prefix from general.architecture): shapes and types are checked against
// each other and against the GEMV kernels (mmvq_supports); expert_used_count, expert_weights_norm,
// expert_gating_func (1 softmax, 2 sigmoid; default sigmoid for "flint", the reference's gating) and
// attention.layer_norm_rms_epsilon come from the metadata. Copies with hipMemcpy on the current device. Throws
// std::runtime_error on a missing tensor, a shape or type mismatch or a HIP failure.
void build_resident_moe_layer(const Gguf &file, int il, ResidentMoeLayer &out);

// A dense FFN block of the reference model (its leading dense layers, src/model.cpp:120-125): blk.N.ffn_gate.weight,
// ffn_up.weight ([inter][hidden] blocks), ffn_down.weight ([hidden][inter]) and ffn_norm.weight copied into HBM.
// Device memory is owned by this object and freed by its destructor.
struct ResidentDenseFfn {
    int hidden = 0, inter = 0;
    int gate_type = -1, up_type = -1, down_type = -1;
    float norm_eps = 0.0f;
    void *gate = nullptr, *up = nullptr, *down = nullptr;
    float *ffn_norm = nullptr;  // [hidden] or null

    ResidentDenseFfn() = default;
    ResidentDenseFfn(const ResidentDenseFfn &) = delete;
    ResidentDenseFfn &operator=(const ResidentDenseFfn &) = delete;
    ~ResidentDenseFfn();
};

// Builds dense layer `il`: shapes checked against each other (hidden and inter multiples of 256), types against the
// GEMV kernels (mmvq_supports, as the reference's check, src/model.cpp:193-196); the epsilon from
// <arch>.attention.layer_norm_rms_epsilon. Throws std::runtime_error on a missing tensor, a mismatch or a HIP failure;
// every check runs before the first device allocation.
void build_resident_dense_ffn(const Gguf &file, int il, ResidentDenseFfn &out);

}  // namespace fns
