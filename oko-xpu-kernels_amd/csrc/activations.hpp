// Fused activations as exact bf16 -> bf16 lookups.
//
// Every activation the reference fuses (src/xpuint8.cpp:119-220) is a chain of
// fp32 operations on a bf16 input whose result is rounded to bf16 before it
// meets anything else; the only genuinely two-input steps are products of two
// bf16 values, which are exact in fp32 and rounded once.  So each one-input
// step is a function on the 65536 bf16 encodings, and is tabulated once on the
// host (tables.hip) from its fp32 formula with correctly rounded transcendental
// values; the kernels gather from the table and do the exact products
// themselves.  The results are bit-identical to that fp32 formula for every
// input, by construction.
#pragma once

#include "common.hpp"

namespace xpuint8 {

// Table ids, each 65536 bf16 entries, laid out back to back.
enum ActTable : int {
    kTabGeluErf = 0,    // bf16(0.5x * (1 + erf(x * 0.70710678f)))        (175-177)
    kTabGeluTanh = 1,   // bf16(0.5x * (1 + tanh(0.79788456x(1+0.044715x^2))))  (195-198)
    kTabSilu = 2,       // bf16(x / (1 + exp(-x)))                          (202)
    kTabSituTanhG = 3,  // bf16(tanh_fast(bf16(x / 4)))                     (151-152)
    kTabSigmoid = 4,    // bf16(1 / (1 + exp(-x)))                          (153-154)
    kTabSituTanhH = 5,  // bf16(tanh_fast(bf16(x / 25)))                    (155-156)
    kTabSituGate = 6,   // bf16(table 3 * table 4): situ's gate factor, a
                        // function of the gate alone (the product of two bf16
                        // values is exact in fp32, then rounded once)
    kNumTables = 7,
};
constexpr int kTabSize = 65536;

// Device copy of the tables (defined in capi.hip).
const uint16_t* activation_tables();

__host__ __device__ constexpr bool act_paired(int act) { return act == 2 || act == 3 || act == 4; }

__device__ __forceinline__ float tab_lookup(const uint16_t* tab, int id, float x) {
    return __uint_as_float(uint32_t(tab[id * kTabSize + (__float_as_uint(x) >> 16)]) << 16);
}

// The activation on bf16-valued inputs; the result is bf16-valued.
// Paired ids: a is the first half, b the second
//   swiglu (2): a = gate, b = up; situ (3) and geglu (4): a = hidden, b = gate.
template <int ACT>
__device__ __forceinline__ float activate(const uint16_t* tab, float a, float b) {
    if constexpr (ACT == 0) {
        return a;
    } else if constexpr (ACT == 1) {
        return tab_lookup(tab, kTabGeluTanh, a);
    } else if constexpr (ACT == 2) {
        return bf16_round(tab_lookup(tab, kTabSilu, a) * b);
    } else if constexpr (ACT == 3) {
        const float tg = tab_lookup(tab, kTabSituTanhG, b);
        const float sg = tab_lookup(tab, kTabSigmoid, b);
        const float th = tab_lookup(tab, kTabSituTanhH, a);
        const float p = bf16_round(tg * sg);
        return bf16_round(p * th);
    } else if constexpr (ACT == 4) {
        return bf16_round(a * tab_lookup(tab, kTabGeluErf, b));
    } else {
        return tab_lookup(tab, kTabGeluErf, a);
    }
}

// The activation before its last bf16 rounding: bf16(activate_pre(..)) is
// activate(..) bit for bit (rounding to nearest even is idempotent, and the
// tables hold quiet NaNs), so a caller that packs two results with one
// v_cvt_pk_bf16_f32 can skip the separate rounding of each.
template <int ACT>
__device__ __forceinline__ float activate_pre(const uint16_t* tab, float a, float b) {
    if constexpr (ACT == 2) {
        return tab_lookup(tab, kTabSilu, a) * b;
    } else if constexpr (ACT == 3) {
        const float tg = tab_lookup(tab, kTabSituTanhG, b);
        const float sg = tab_lookup(tab, kTabSigmoid, b);
        const float th = tab_lookup(tab, kTabSituTanhH, a);
        return bf16_round(tg * sg) * th;
    } else if constexpr (ACT == 4) {
        return a * tab_lookup(tab, kTabGeluErf, b);
    } else {
        return activate<ACT>(tab, a, b);
    }
}

// activate_pre<ACT> from table words already read (t[] in act_fetch order:
// the tab_lookup arguments of activate_pre, bf16 bits), with its arithmetic.
__device__ __forceinline__ float tab_float(uint32_t w) { return __uint_as_float(w << 16); }
template <int ACT>
__device__ __forceinline__ float act_combine(float a, float b, const uint32_t* t) {
    if constexpr (ACT == 0) {
        return a;
    } else if constexpr (ACT == 1 || ACT == 5) {
        return tab_float(t[0]);
    } else if constexpr (ACT == 2) {
        return tab_float(t[0]) * b;
    } else if constexpr (ACT == 3) {
        return bf16_round(tab_float(t[0]) * tab_float(t[1])) * tab_float(t[2]);
    } else {
        return a * tab_float(t[0]);
    }
}

// A window of one activation table in LDS: the entries of the bf16 inputs
// whose exponent field is in [115, 131) (|x| in [2^-12, 2^4)), where the
// FFN's activations lie: 2048 positive inputs, then the 2048 negative ones.
// Input bits b sit at position 2048 * (b >> 15) + (b & 0x7FFF) - (115 << 7);
// inputs outside read the table in global memory.  Used for the GELU (erf)
// of the FFN's up-projection epilogue (ids 4 and 5, one lookup per value).
constexpr int kWinLo = 115 << 7, kWinHalf = 16 * 128, kWinSize = 2 * kWinHalf;
template <int ACT>
__host__ __device__ constexpr int act_window_table() {
    return (ACT == 4 || ACT == 5) ? kTabGeluErf : -1;
}
// bf16 input bits of window position w
__device__ __forceinline__ uint32_t win_bits(int w) {
    return (uint32_t(w >> 11) << 15) | uint32_t(kWinLo + (w & (kWinHalf - 1)));
}

}  // namespace xpuint8
