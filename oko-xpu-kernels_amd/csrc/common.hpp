// Device-side building blocks shared by the ConvRot kernels (gfx950, wave64).
//
// Arithmetic contract.  Every routine here reproduces, bit for bit, the fp32
// operation order of the reference kernels in okolenmi/oko-xpu-kernels
// src/xpuint8.cpp (cited per routine).  Files that include this header are
// compiled with -ffp-contract=off, so no multiply-add is ever fused.
//
// The Hadamard is evaluated *unscaled*: each of the four radix-4 axes adds and
// subtracts without the reference's factor 0.5, and the product 1/16 of the
// four factors is applied once at the end (or folded into the quantizer's
// reciprocal).  Scaling by a power of two commutes with IEEE rounding whenever
// no intermediate is subnormal or overflows, so for every input whose nonzero
// magnitudes lie in [2^-110, 2^120] the result equals the reference's
// ((0.5*a + 0.5*b) + ...) chains exactly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace xpuint8 {

constexpr int kGroup = 256;     // ConvRot group size (src/xpuint8.cpp:71)
constexpr int kWave = 64;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// 16-byte loads.  (A non-temporal hint measured slower on MI355X for these
// read-once streams: 5.5 vs 6.3 TB/s.)
__device__ __forceinline__ u32x4 load16(const void* p) {
    return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ i32x4 load16_i(const void* p) {
    return *reinterpret_cast<const i32x4*>(p);
}

// ----------------------------------------------------------------- bf16 <-> f32
__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }

// fp32 -> bf16, round to nearest even, NaN kept quiet with its sign (torch's
// conversion: (u >> 16) | 0x40 for a NaN).  gfx950's v_cvt_pk_bf16_f32 gives
// exactly these bits for every one of the 2^32 fp32 inputs (denormals, infinities
// and NaNs included; checked exhaustively on the device against the integer
// formula), so one instruction converts two values.
typedef float xpu_v2f __attribute__((ext_vector_type(2)));
typedef __bf16 xpu_v2bf __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(xpu_v2f{lo, hi}, xpu_v2bf));
}
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    return pack_bf16x2(f, 0.f) & 0xFFFFu;
}
__device__ __forceinline__ float bf16_round(float f) {
    return __uint_as_float(pack_bf16x2(f, 0.f) << 16);
}

// ------------------------------------------------------------ lane exchange
// DPP controls used here, each a lane xor inside a row of 16 lanes:
// quad_perm [1,0,3,2] = 0xB1 (xor 1), quad_perm [2,3,0,1] = 0x4E (xor 2),
// row_half_mirror = 0x141 (lane i <- 7-i in each half row: xor 7),
// row_mirror = 0x140 (lane i <- 15-i: xor 15).
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppXor7 = 0x141, kDppXor15 = 0x140;
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}
// ds_swizzle bit-mask mode inside 32 lanes: lane' = lane ^ XOR.
template <int XOR>
__device__ __forceinline__ float swz_xor(float x) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x1F | (XOR << 10)));
}

// ------------------------------------------------------------------ Hadamard
// One 4-point chain of ``inreg`` on positions (p0,p1,p2,p3) of a register,
// unscaled: out[o] = ((s0*p0 + s1*p1) + s2*p2) + s3*p3 with s = H4[o]
// (src/xpuint8.cpp:75, 290-301).  H4 rows: [1,1,1,-1] [1,1,-1,1] [1,-1,1,1]
// [-1,1,1,1].  (-p0 + p1) is computed as (p1 - p0), which is the same IEEE
// result.
__device__ __forceinline__ void h4_chain(float& p0, float& p1, float& p2, float& p3) {
    const float a = p0 + p1;
    const float b = p0 - p1;
    const float o0 = (a + p2) - p3;
    const float o1 = (a - p2) + p3;
    const float o2 = (b + p2) + p3;
    const float o3 = (p2 - b) + p3;
    p0 = o0; p1 = o1; p2 = o2; p3 = o3;
}

// Axes 0 and 1 of the group transform on one lane's 16-element register
// (element q of the register is group element 16*w + q): axis 0 runs over
// q & 3, axis 1 over (q >> 2) & 3, in that order (src/xpuint8.cpp:292-299).
__device__ __forceinline__ void hadamard_inreg(float (&v)[16]) {
#pragma unroll
    for (int b = 0; b < 16; b += 4) h4_chain(v[b], v[b + 1], v[b + 2], v[b + 3]);
#pragma unroll
    for (int c = 0; c < 4; ++c) h4_chain(v[c], v[c + 4], v[c + 8], v[c + 12]);
}

// Lane -> register assignment.  The 16 lanes of a group hold its 16
// registers w = i2 + 4*i3 (register w = group elements [16w, 16w+16)); lane
// sl holds register lane_w(sl), chosen so that the four lanes differing only
// in digit i2 are {L, L^1, L^2, L^3} and the four differing only in digit i3
// are {L, L^7, L^15, L^8}.  Both butterflies then use single-instruction DPP
// lane xors (1, 2 and 7, 15), which fold into the adds, instead of LDS-pipe
// swizzles.  sl = i2 ^ 7*(i3&1) ^ 15*(i3>>1), inverted:
//   i3 = gray(sl >> 2), i2 = (sl & 3) ^ (3 if i3 is 1 or 2).
__device__ __forceinline__ int lane_w(int sl) {
    const int hi = sl >> 2;
    const int i3 = hi ^ (hi >> 1);
    const int i2 = (sl & 3) ^ ((hi & 1) ? 3 : 0);
    return i2 + 4 * i3;
}

// Axes 2 and 3.  The 4-point butterfly over lanes {L, L^m1, L^m2, L^m1^m2}
// as the reference's bfly_xor (src/xpuint8.cpp:441-448): A = v + v[L^m1];
// B = v - v[L^m1]; out = A + B[L^m2].  With the lane holding index
// j = c1 + 2*c2 of the 4-point set (c1, c2 its m1, m2 components) this is
// bit-identical to bfly4 (src/xpuint8.cpp:279-285) for any masks m1, m2:
// each output is the same two IEEE additions of the same operands, up to
// commutation and the exact negation x + (b - a) == x - (a - b).
__device__ __forceinline__ void hadamard_xlane(float (&v)[16]) {
#pragma unroll
    for (int t = 0; t < 16; ++t) {           // axis 2: lane xor 1, xor 2
        const float p = dpp<kDppXor1>(v[t]);
        const float A = v[t] + p;
        const float B = v[t] - p;
        v[t] = A + dpp<kDppXor2>(B);
    }
#pragma unroll
    for (int t = 0; t < 16; ++t) {           // axis 3: lane xor 7, xor 15
        const float p = dpp<kDppXor7>(v[t]);
        const float A = v[t] + p;
        const float B = v[t] - p;
        v[t] = A + dpp<kDppXor15>(B);
    }
}

// The full unscaled group transform: the true rotation is this times 1/16.
__device__ __forceinline__ void hadamard16_unscaled(float (&v)[16]) {
    hadamard_inreg(v);
    hadamard_xlane(v);
}

// --------------------------------------------------------------- reductions
__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, dpp<kDppXor1>(x));
    x = fmaxf(x, dpp<kDppXor2>(x));
    x = fmaxf(x, dpp<kDppXor7>(x));
    x = fmaxf(x, dpp<kDppXor15>(x));
    x = fmaxf(x, swz_xor<16>(x));
    x = fmaxf(x, __shfl_xor(x, 32));
    return x;
}

// Max over the 16 lanes of an aligned segment (lanes 16j..16j+15) of the
// bit patterns of non-negative floats (which order like their values); an
// integer max folds its DPP operand into one instruction per step.
template <int CTRL>
__device__ __forceinline__ uint32_t dppu(uint32_t x) {
    return uint32_t(__builtin_amdgcn_mov_dpp(int(x), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ uint32_t segment_max_bits(uint32_t x) {
    x = max(x, dppu<kDppXor1>(x));
    x = max(x, dppu<kDppXor2>(x));
    x = max(x, dppu<kDppXor7>(x));
    x = max(x, dppu<kDppXor15>(x));
    return x;
}

// Max over the 16 lanes of an aligned segment (lanes 16j..16j+15).
__device__ __forceinline__ float segment_max(float x) {
    x = fmaxf(x, dpp<kDppXor1>(x));
    x = fmaxf(x, dpp<kDppXor2>(x));
    x = fmaxf(x, dpp<kDppXor7>(x));
    x = fmaxf(x, dpp<kDppXor15>(x));
    return x;
}

// -------------------------------------------------------------- quantizers
// rint(t) for |t| < 2^22 through the fp32 adder's round-to-nearest-even: the
// low byte of (t + 1.5*2^23)'s bits is the two's-complement int8 of rint(t).
__device__ __forceinline__ uint32_t rint_bits(float t) {
    return __float_as_uint(t + 12582912.0f);
}
// Pack the low bytes of four such words into one dword (element 0 lowest).
__device__ __forceinline__ uint32_t pack4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint32_t ab = __builtin_amdgcn_perm(b, a, 0x0c0c0400u);
    const uint32_t cd = __builtin_amdgcn_perm(d, c, 0x0c0c0400u);
    return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
}

// rint(x / s) with x / s the correctly rounded IEEE quotient, for |x/s| <= 127.5:
// the reciprocal product decides unless it lies within 2^-14 of a half-integer
// (it differs from the IEEE quotient by at most a few ulp, i.e. < 2^-15 at
// this magnitude); those rare lanes take the IEEE division.
__device__ __forceinline__ float rint_div(float x, float s, float inv) {
    const float y = x * inv;
    const float r = rintf(y);
    const float d = fabsf(fabsf(y - r) - 0.5f);
    if (__builtin_expect(d < 6.103515625e-05f, 0)) return rintf(x / s);
    return r;
}

}  // namespace xpuint8
