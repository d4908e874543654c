// fns_host.hpp - host-side helpers shared by the HIP translation units: error reporting for the C ABI, the abort
// behaviour of the C++ API (the reference aborts on launch failures and unsupported types: src/kernels.cu:9-16,
// src/ggml/ggml_cuda_host.cu:14-17), and small shape utilities.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

namespace fns::host {

// Error codes of the C ABI (include/fns_hip.h).
enum Status : int {
    OK = 0,
    ERR_TYPE = -1,    // unsupported ggml type
    ERR_SHAPE = -2,   // shape / argument precondition violated
    ERR_LAUNCH = -3,  // HIP launch or runtime error
    ERR_NOMEM = -4,   // a caller-provided buffer is too small
};

// Records a message for fns_hip_last_error() (thread-local) and returns `code`.
int set_error(int code, const char *fmt, ...);
const char *last_error();

// After a launch: converts a pending HIP error into ERR_LAUNCH.
int check_launch(const char *what);

// C++ API behaviour: print the last error and abort when `rc` is not OK.
void abort_on_error(int rc, const char *what);

inline int64_t pad512(int64_t n) { return (n + 511) / 512 * 512; }
inline bool is_kquant(int t) { return t == 11 || t == 12 || t == 13 || t == 14; }
// IQ formats: IQ3_XXS (18), IQ3_S (21), IQ2_S (22), IQ4_XS (23); the first three decode through codebooks that the
// engine registers (fns_hip_set_iq_grids).
inline bool is_iq(int t) { return t == 18 || t == 21 || t == 22 || t == 23; }
inline bool iq_needs_grid(int t) { return t == 18 || t == 21 || t == 22; }
bool iq_grids_ready();
void set_iq_grids_ready();
// Types that only the quarter-block kernels decode (no K-quant sub-block machinery): Q8_0 and the IQ formats.
inline bool is_quarter_only(int t) { return t == 8 || is_iq(t); }
// Every weight type the GEMV paths accept (mmvq_supports).
inline bool is_supported(int t) {
    return is_kquant(t) || t == 8 || (is_iq(t) && (!iq_needs_grid(t) || iq_grids_ready()));
}
// Bytes of 256 consecutive values of a row (a K-quant or IQ block; 8 Q8_0 blocks).
inline int64_t kquant_block_bytes(int t) {
    return t == 11 ? 110 : t == 12 ? 144 : t == 13 ? 176 : t == 14 ? 210 : t == 8 ? 272 : t == 23 ? 136 : t == 18 ? 98
         : t == 21 ? 110 : t == 22 ? 82 : 0;
}
inline int64_t q8_1_row_bytes(int64_t ncols) { return pad512(ncols) / 32 * 36; }

// Lane-group shape for a row of `nslots` 16-byte slots: lanes per row (a power of two dividing the slot count, at
// most the 64-lane wave) and slots per lane (0: runtime loop for uncommon shapes).
struct Shape {
    int lpr, spl;
};
inline Shape pick_shape(int nslots) {
    if (nslots % 64 == 0 && nslots / 64 <= 3) return {64, nslots / 64};
    if (nslots == 32) return {32, 1};
    if (nslots == 16) return {16, 1};
    if (nslots == 24) return {8, 3};
    if (nslots == 12) return {4, 3};
    return {64, 0};
}
inline int slots_per_block(int t) { return t == 11 ? 4 : 8; }

}  // namespace fns::host

#define FNS_TRY(...)                       \
    do {                                   \
        const int rc_ = (__VA_ARGS__);     \
        if (rc_ != ::fns::host::OK) return rc_; \
    } while (0)
