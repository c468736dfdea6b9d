// Host-side generation of the activation tables (activations.hpp).
//
// Each entry is the reference's fp32 formula (src/xpuint8.cpp cited per line)
// evaluated on one bf16 input, with every transcendental taken as its
// correctly rounded fp32 value (the double-precision libm result rounded once
// to float), then rounded to bf16.  Built with -ffp-contract=off so each fp32
// operation rounds on its own, as in the reference's vector code.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <vector>

#include "activations.hpp"
#include "kernels.hpp"

namespace xpuint8 {
namespace {

float f32(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
uint32_t u32(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }

uint16_t to_bf16(float f) {
    const uint32_t u = u32(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return uint16_t((u >> 16) | 0x40u);
    return uint16_t((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
float bf16r(float f) { return f32(uint32_t(to_bf16(f)) << 16); }

float erf_cr(float x) { return float(std::erf(double(x))); }
float tanh_cr(float x) { return float(std::tanh(double(x))); }
float exp_cr(float x) { return float(std::exp(double(x))); }
float expm1_cr(float x) { return float(std::expm1(double(x))); }

// src/xpuint8.cpp:175-177
float gelu_erf(float x) { return (0.5f * x) * (1.0f + erf_cr(x * 0.7071067811865476f)); }

// src/xpuint8.cpp:195-197
float gelu_tanh(float x) {
    const float x2 = x * x;
    const float inner = (0.7978845608028654f * x) * (1.0f + 0.044715f * x2);
    return (0.5f * x) * (1.0f + tanh_cr(inner));
}

// src/xpuint8.cpp:142-148: tanh(z) = expm1(2a) / (expm1(2a) + 2), a = min(|z|, 20)
float tanh_fast(float z) {
    const float a = std::fmin(std::fabs(z), 20.0f);
    const float m = expm1_cr(2.0f * a);
    const float r = m / (m + 2.0f);
    return f32(u32(r) | (u32(z) & 0x80000000u));
}

std::vector<uint16_t> g_tables;
std::once_flag g_once;

void build() {
    g_tables.resize(size_t(kNumTables) * kTabSize);
    for (uint32_t b = 0; b < uint32_t(kTabSize); ++b) {
        const float x = f32(b << 16);
        uint16_t* t = g_tables.data();
        t[kTabGeluErf * kTabSize + b] = to_bf16(gelu_erf(x));
        t[kTabGeluTanh * kTabSize + b] = to_bf16(gelu_tanh(x));
        t[kTabSilu * kTabSize + b] = to_bf16(x / (1.0f + exp_cr(-x)));          // 202
        t[kTabSituTanhG * kTabSize + b] = to_bf16(tanh_fast(bf16r(x / 4.0f)));  // 151-152
        t[kTabSigmoid * kTabSize + b] = to_bf16(1.0f / (1.0f + exp_cr(-x)));    // 153-154
        t[kTabSituTanhH * kTabSize + b] = to_bf16(tanh_fast(bf16r(x / 25.0f))); // 155-156
        t[kTabSituGate * kTabSize + b] =                                         // 151-154
            to_bf16(f32(uint32_t(t[kTabSituTanhG * kTabSize + b]) << 16) *
                    f32(uint32_t(t[kTabSigmoid * kTabSize + b]) << 16));
    }
}

}  // namespace

const uint16_t* host_activation_tables() {
    std::call_once(g_once, build);
    return g_tables.data();
}

}  // namespace xpuint8
