// fns_host.cpp - error reporting shared by the C ABI and the C++ API.
#include "fns_host.hpp"

#include <atomic>
#include <cstdarg>
#include <cstring>

namespace fns::host {

namespace {
thread_local char g_msg[512] = "";
}

int set_error(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_msg, sizeof g_msg, fmt, ap);
    va_end(ap);
    return code;
}

const char *last_error() { return g_msg; }

namespace {
std::atomic<bool> g_iq_ready{false};
}
bool iq_grids_ready() { return g_iq_ready.load(std::memory_order_acquire); }
void set_iq_grids_ready() { g_iq_ready.store(true, std::memory_order_release); }

int check_launch(const char *what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(ERR_LAUNCH, "%s: HIP error %s", what, hipGetErrorString(e));
    return OK;
}

void abort_on_error(int rc, const char *what) {
    if (rc == OK) return;
    std::fprintf(stderr, "fns %s failed (%d): %s\n", what, rc, g_msg);
    std::abort();
}

}  // namespace fns::host
