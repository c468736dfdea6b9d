// Device check of the quantizers' short division sequences (csrc/common.hpp)
// against IEEE division, over every float of their ranges:
//   div127_rn(x) == x / 127.0f   for every x in [0, +inf] (and NaN stays NaN)
//   rcp_rn(x)    == 1.0f / x     for every x in [2^-110, 2^122], +inf, NaN
// Prints the mismatch counts; exit status 0 only when both are zero.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <vector>

#include "../../oko-xpu-kernels_amd/csrc/common.hpp"

using namespace xpuint8;

constexpr uint32_t kRcpLo = (127u - 110u) << 23;   // 2^-110
constexpr uint32_t kRcpHi = (127u + 122u) << 23;   // 2^122

__global__ void check(unsigned long long* out) {
    unsigned long long bad_div = 0, bad_rcp = 0, n_rcp = 0;
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t b = blockIdx.x * blockDim.x + threadIdx.x; b <= 0x7F800000u; b += stride) {
        const float x = __uint_as_float(b);
        bad_div += __float_as_uint(div127_rn(x)) != __float_as_uint(x / 127.0f);
        if ((b >= kRcpLo && b <= kRcpHi) || b == 0x7F800000u) {
            bad_rcp += __float_as_uint(rcp_rn(x)) != __float_as_uint(1.0f / x);
            ++n_rcp;
        }
    }
    // NaN inputs: NaN out of both
    const float nan = __uint_as_float(0x7FC00000u + (threadIdx.x & 7));
    bad_div += div127_rn(nan) == div127_rn(nan);
    bad_rcp += rcp_rn(nan) == rcp_rn(nan);
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    out[3 * t + 0] = bad_div;
    out[3 * t + 1] = bad_rcp;
    out[3 * t + 2] = n_rcp;
}

int main() {
    const int blocks = 1024, threads = 256, n = blocks * threads;
    unsigned long long* d = nullptr;
    if (hipMalloc(&d, sizeof(unsigned long long) * 3 * n) != hipSuccess) return 2;
    hipLaunchKernelGGL(check, dim3(blocks), dim3(threads), 0, 0, d);
    if (hipDeviceSynchronize() != hipSuccess) return 2;
    std::vector<unsigned long long> h(3 * size_t(n));
    if (hipMemcpy(h.data(), d, sizeof(unsigned long long) * 3 * n, hipMemcpyDeviceToHost) !=
        hipSuccess)
        return 2;
    unsigned long long s[3] = {0, 0, 0};
    for (int t = 0; t < n; ++t)
        for (int i = 0; i < 3; ++i) s[i] += h[3 * size_t(t) + i];
    printf("div127_rn mismatches: %llu of %llu\n", s[0], 0x7F800001ull);
    printf("rcp_rn mismatches: %llu of %llu\n", s[1], s[2]);
    if (hipFree(d) != hipSuccess) return 2;
    return (s[0] == 0 && s[1] == 0) ? 0 : 1;
}
