// selftest.hip - device self-test of the cross-lane primitives (fns_lanes.hpp): every xor_lane<O> must equal the
// LDS-crossbar shuffle __shfl_xor(v, O) on every lane. Run by the GPU tests before the kernels that rely on it.
#include "fns_common.hpp"
#include "fns_host.hpp"
#include "fns_internal.hpp"
#include "fns_lanes.hpp"

namespace fns {

using namespace fns::dev;

namespace {

template <int O> __device__ int check(int v) { return xor_lane_i<O>(v) != __shfl_xor(v, O, 64) ? 1 : 0; }

__global__ void k_selftest_lanes(int *bad) {
    const int v = (int) (threadIdx.x * 2654435761u + 12345u);
    int b = 0;
    b |= check<1>(v) << 0;
    b |= check<2>(v) << 1;
    b |= check<4>(v) << 2;
    b |= check<8>(v) << 3;
    b |= check<16>(v) << 4;
    b |= check<32>(v) << 5;
    // butterfly sums equal the xor-shuffle butterflies bit for bit
    const float f = (float) ((threadIdx.x * 7919u) % 1000u) * 0.37f - 150.0f;
    float ref = f;
    for (int o = 16; o > 0; o >>= 1) ref += __shfl_xor(ref, o, 64);
    float ref64 = f;
    for (int o = 32; o > 0; o >>= 1) ref64 += __shfl_xor(ref64, o, 64);
    if (__builtin_bit_cast(int, lanes_sum<32>(f)) != __builtin_bit_cast(int, ref)) b |= 1 << 6;
    if (__builtin_bit_cast(int, lanes_sum<64>(f)) != __builtin_bit_cast(int, ref64)) b |= 1 << 7;
    atomicOr(bad, b);
}

}  // namespace

namespace impl {

int selftest_lanes(int *bad_mask_device, hipStream_t st) {
    if (!bad_mask_device) return host::set_error(host::ERR_SHAPE, "selftest_lanes: null buffer");
    hipLaunchKernelGGL(k_selftest_lanes, dim3(1), dim3(64), 0, st, bad_mask_device);
    return host::check_launch("selftest_lanes");
}

}  // namespace impl

}  // namespace fns
