// gguf.cpp - GGUF reader over a read-only mmap of the whole file, and the fully resident expert slots of one MoE
// layer (include/fns/gguf.h). Reference: /root/reference/src/model.cpp:30-136 (loader), src/engine.cu:375-471 (slots).
#include "fns/gguf.h"

#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <stdexcept>

namespace fns {

namespace {

// Block size (values) and bytes per block of the ggml types a MoE checkpoint can hold (public ggml type traits).
struct TypeSize {
    int blck;
    int bytes;
};
TypeSize type_size(int t) {
    switch (t) {
        case 0: return {1, 4};     // F32
        case 1: return {1, 2};     // F16
        case 2: return {32, 18};   // Q4_0
        case 3: return {32, 20};   // Q4_1
        case 6: return {32, 22};   // Q5_0
        case 7: return {32, 24};   // Q5_1
        case 8: return {32, 34};   // Q8_0
        case 9: return {32, 36};   // Q8_1
        case 10: return {256, 84};   // Q2_K
        case 11: return {256, 110};  // Q3_K
        case 12: return {256, 144};  // Q4_K
        case 13: return {256, 176};  // Q5_K
        case 14: return {256, 210};  // Q6_K
        case 15: return {256, 292};  // Q8_K
        case 18: return {256, 98};   // IQ3_XXS
        case 21: return {256, 110};  // IQ3_S
        case 22: return {256, 82};   // IQ2_S
        case 23: return {256, 136};  // IQ4_XS
        case 24: return {1, 1};      // I8
        case 25: return {1, 2};      // I16
        case 26: return {1, 4};      // I32
        case 27: return {1, 8};      // I64
        case 28: return {1, 8};      // F64
        case 30: return {1, 2};      // BF16
        default: return {0, 0};
    }
}

size_t scalar_bytes(uint32_t t) {
    switch (t) {
        case GGUF_U8: case GGUF_I8: case GGUF_BOOL: return 1;
        case GGUF_U16: case GGUF_I16: return 2;
        case GGUF_U32: case GGUF_I32: case GGUF_F32: return 4;
        case GGUF_U64: case GGUF_I64: case GGUF_F64: return 8;
        default: return 0;
    }
}

// Bounds-checked cursor over the mapping.
struct Cursor {
    const uint8_t *p;
    size_t n, at = 0;
    const std::string &path;
    [[noreturn]] void fail(const std::string &what) const {
        throw std::runtime_error("gguf " + path + ": " + what + " (at byte " + std::to_string(at) + ")");
    }
    const uint8_t *take(size_t k) {
        if (k > n - at) fail("truncated file");
        const uint8_t *r = p + at;
        at += k;
        return r;
    }
    template <class T> T get() {
        T v;
        std::memcpy(&v, take(sizeof v), sizeof v);
        return v;
    }
    std::string str() {
        const uint64_t len = get<uint64_t>();
        if (len > (1u << 24)) fail("string of " + std::to_string(len) + " bytes");
        const uint8_t *s = take((size_t) len);
        return std::string((const char *) s, (size_t) len);
    }
};

void read_scalar(Cursor &c, uint32_t t, GgufKv &kv) {
    switch (t) {
        case GGUF_U8: kv.u = c.get<uint8_t>(); kv.i = (int64_t) kv.u; kv.f = (double) kv.u; break;
        case GGUF_I8: kv.i = c.get<int8_t>(); kv.u = (uint64_t) kv.i; kv.f = (double) kv.i; break;
        case GGUF_U16: kv.u = c.get<uint16_t>(); kv.i = (int64_t) kv.u; kv.f = (double) kv.u; break;
        case GGUF_I16: kv.i = c.get<int16_t>(); kv.u = (uint64_t) kv.i; kv.f = (double) kv.i; break;
        case GGUF_U32: kv.u = c.get<uint32_t>(); kv.i = (int64_t) kv.u; kv.f = (double) kv.u; break;
        case GGUF_I32: kv.i = c.get<int32_t>(); kv.u = (uint64_t) kv.i; kv.f = (double) kv.i; break;
        case GGUF_F32: kv.f = c.get<float>(); break;
        case GGUF_BOOL: kv.u = c.get<uint8_t>() ? 1 : 0; kv.i = (int64_t) kv.u; break;
        case GGUF_U64: kv.u = c.get<uint64_t>(); kv.i = (int64_t) kv.u; kv.f = (double) kv.u; break;
        case GGUF_I64: kv.i = c.get<int64_t>(); kv.u = (uint64_t) kv.i; kv.f = (double) kv.i; break;
        case GGUF_F64: kv.f = c.get<double>(); break;
        case GGUF_STRING: kv.str = c.str(); break;
        default: c.fail("value type " + std::to_string(t));
    }
}

}  // namespace

size_t ggml_row_bytes(int type, int64_t ne0) {
    const TypeSize s = type_size(type);
    if (!s.blck || ne0 % s.blck) return 0;
    return (size_t) (ne0 / s.blck) * (size_t) s.bytes;
}

Gguf::Gguf(const std::string &path) : path_(path) {
    fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd_ < 0) throw std::runtime_error("gguf " + path + ": cannot open");
    struct stat st;
    if (::fstat(fd_, &st) != 0 || st.st_size < 24) {
        ::close(fd_);
        fd_ = -1;
        throw std::runtime_error("gguf " + path + ": not a GGUF file (too short)");
    }
    size_ = (size_t) st.st_size;
    void *m = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (m == MAP_FAILED) {
        ::close(fd_);
        fd_ = -1;
        throw std::runtime_error("gguf " + path + ": mmap failed");
    }
    base_ = (const uint8_t *) m;
    try {
        Cursor c{base_, size_, 0, path_};
        if (std::memcmp(c.take(4), "GGUF", 4) != 0) c.fail("bad magic (not a GGUF file)");
        version_ = c.get<uint32_t>();
        if (version_ != 2 && version_ != 3) c.fail("unsupported version " + std::to_string(version_));
        const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
        // each key takes at least 12 bytes and each tensor entry 32: larger counts cannot fit in the file
        if (n_kv > size_ / 12 || n_tensors > size_ / 32) c.fail("implausible tensor / key count");
        kvs_.resize((size_t) n_kv);
        for (GgufKv &kv : kvs_) {
            kv.key = c.str();
            kv.type = c.get<uint32_t>();
            if (kv.type == GGUF_ARRAY) {
                kv.arr_type = c.get<uint32_t>();
                kv.arr_n = c.get<uint64_t>();
                if (kv.arr_type == GGUF_STRING) {
                    if (kv.arr_n > (1u << 24)) c.fail("array of " + std::to_string(kv.arr_n) + " strings");
                    kv.arr_str.reserve((size_t) kv.arr_n);
                    for (uint64_t i = 0; i < kv.arr_n; ++i) kv.arr_str.push_back(c.str());
                } else {
                    const size_t eb = scalar_bytes(kv.arr_type);
                    if (!eb) c.fail("array element type " + std::to_string(kv.arr_type) + " of " + kv.key);
                    if (kv.arr_n > (uint64_t) (c.n - c.at) / eb) c.fail("array past the end of the file: " + kv.key);
                    kv.arr_data = c.take((size_t) kv.arr_n * eb);
                }
            } else {
                read_scalar(c, kv.type, kv);
            }
        }
        const int64_t aid = find_key("general.alignment");
        if (aid >= 0) {
            if (kvs_[(size_t) aid].type != GGUF_U32 || kvs_[(size_t) aid].u == 0 ||
                (kvs_[(size_t) aid].u & (kvs_[(size_t) aid].u - 1)))
                c.fail("general.alignment must be a power-of-two u32");
            alignment_ = (size_t) kvs_[(size_t) aid].u;
        }
        tensors_.resize((size_t) n_tensors);
        for (GgufTensor &t : tensors_) {
            t.name = c.str();
            const uint32_t nd = c.get<uint32_t>();
            if (nd < 1 || nd > 4) c.fail("tensor " + t.name + ": " + std::to_string(nd) + " dimensions");
            t.n_dims = (int) nd;
            for (uint32_t d = 0; d < nd; ++d) {
                const uint64_t v = c.get<uint64_t>();
                if (v == 0 || v > ((uint64_t) 1 << 40)) c.fail("tensor " + t.name + ": bad dimension");
                t.ne[d] = (int64_t) v;
            }
            t.type = (int) c.get<uint32_t>();
            t.offset = (size_t) c.get<uint64_t>();
            const size_t row = ggml_row_bytes(t.type, t.ne[0]);
            if (!row) c.fail("tensor " + t.name + ": type " + std::to_string(t.type) + " with ne0 " +
                             std::to_string(t.ne[0]) + " is not supported");
            // row * ne1 * ne2 * ne3, one factor at a time: any partial product beyond the file size is rejected
            // before the next multiplication, so nothing wraps (each factor is at most 2^40, the file below 2^64)
            uint64_t nb = (uint64_t) row;
            for (int d = 1; d < 4; ++d) {
                uint64_t next = 0;
                if (__builtin_mul_overflow(nb, (uint64_t) t.ne[d], &next) || next > (uint64_t) size_)
                    c.fail("tensor " + t.name + ": larger than the file");
                nb = next;
            }
            if (nb > (uint64_t) size_) c.fail("tensor " + t.name + ": larger than the file");
            t.nbytes = (size_t) nb;
            if (t.offset % alignment_) c.fail("tensor " + t.name + ": offset not aligned");
        }
        data_off_ = (c.at + alignment_ - 1) / alignment_ * alignment_;
        for (GgufTensor &t : tensors_) {
            if (data_off_ + t.offset > size_ || t.nbytes > size_ - data_off_ - t.offset)
                throw std::runtime_error("gguf " + path_ + ": tensor outside the file: " + t.name);
            t.data = base_ + data_off_ + t.offset;
        }
    } catch (...) {
        ::munmap((void *) base_, size_);
        ::close(fd_);
        base_ = nullptr;
        fd_ = -1;
        throw;
    }
}

Gguf::~Gguf() {
    if (base_) ::munmap((void *) base_, size_);
    if (fd_ >= 0) ::close(fd_);
}

int64_t Gguf::find_key(const std::string &key) const {
    for (size_t i = 0; i < kvs_.size(); ++i)
        if (kvs_[i].key == key) return (int64_t) i;
    return -1;
}

namespace {
[[noreturn]] void kv_fail(const std::string &path, const std::string &key, const char *what) {
    throw std::runtime_error("gguf " + path + ": key " + key + ": " + what);
}
bool is_int_type(uint32_t t) {
    return t == GGUF_U8 || t == GGUF_I8 || t == GGUF_U16 || t == GGUF_I16 || t == GGUF_U32 || t == GGUF_I32 ||
           t == GGUF_U64 || t == GGUF_I64;
}
}  // namespace

uint32_t Gguf::get_u32(const std::string &key) const {
    const int64_t id = find_key(key);
    if (id < 0) kv_fail(path_, key, "missing");
    const GgufKv &v = kvs_[(size_t) id];
    if (!is_int_type(v.type) || v.i < 0 || v.u > 0xffffffffull) kv_fail(path_, key, "not a u32");
    return (uint32_t) v.u;
}
float Gguf::get_f32(const std::string &key) const {
    const int64_t id = find_key(key);
    if (id < 0) kv_fail(path_, key, "missing");
    const GgufKv &v = kvs_[(size_t) id];
    if (v.type != GGUF_F32 && v.type != GGUF_F64) kv_fail(path_, key, "not a float");
    return (float) v.f;
}
bool Gguf::get_bool(const std::string &key) const {
    const int64_t id = find_key(key);
    if (id < 0) kv_fail(path_, key, "missing");
    const GgufKv &v = kvs_[(size_t) id];
    if (v.type != GGUF_BOOL) kv_fail(path_, key, "not a bool");
    return v.u != 0;
}
std::string Gguf::get_str(const std::string &key) const {
    const int64_t id = find_key(key);
    if (id < 0) kv_fail(path_, key, "missing");
    const GgufKv &v = kvs_[(size_t) id];
    if (v.type != GGUF_STRING) kv_fail(path_, key, "not a string");
    return v.str;
}
uint32_t Gguf::get_u32_or(const std::string &key, uint32_t dflt) const {
    return find_key(key) < 0 ? dflt : get_u32(key);
}
float Gguf::get_f32_or(const std::string &key, float dflt) const { return find_key(key) < 0 ? dflt : get_f32(key); }
bool Gguf::get_bool_or(const std::string &key, bool dflt) const { return find_key(key) < 0 ? dflt : get_bool(key); }

const GgufTensor *Gguf::find_tensor(const std::string &name) const {
    for (const GgufTensor &t : tensors_)
        if (t.name == name) return &t;
    return nullptr;
}
const GgufTensor &Gguf::get_tensor(const std::string &name) const {
    const GgufTensor *t = find_tensor(name);
    if (!t) throw std::runtime_error("gguf " + path_ + ": missing tensor: " + name);
    return *t;
}

}  // namespace fns
