// Device-side building blocks shared by the ConvRot kernels (gfx950, wave64).
//
// Arithmetic contract.  Every routine here reproduces, bit for bit, the fp32
// operation order of the reference kernels in okolenmi/oko-xpu-kernels
// src/xpuint8.cpp (cited per routine).  Files that include this header are
// compiled with -ffp-contract=off, so no multiply-add is ever fused.
//
// The Hadamard is evaluated *unscaled* on the fast path: each of the four
// radix-4 axes adds and subtracts without the reference's factor 0.5, and the
// product 1/16 of the four factors is applied once at the end (or folded into
// the quantizer's reciprocal).  Scaling by a power of two commutes with IEEE
// rounding unless a result overflows or rounds in the subnormal range.  The
// second cannot happen: the inputs are bf16 values (multiples of 2^-133), every
// intermediate of either order is a multiple of 2^-137, and a sum of such
// multiples that falls below 2^-126 is exact.  The first is excluded by the
// input range: with every |x| < 2^120 an unscaled intermediate is at most
// 256*max|x| < 2^128.  Groups with an input at or above 2^120 (or an inf) take
// hadamard16_scaled, which is the reference's own operation order, factors of
// 0.5 included, and so overflows exactly where the reference does.
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

// Axes 2 and 3.  The reference's 4-point butterfly over lanes {L, L^m1, L^m2,
// L^m1^m2} (bfly_xor, src/xpuint8.cpp:441-448) forms, for the lane holding
// index j of the 4-point set,
//   out_j = A_j + B_(j^2),   A_j = x_j + x_(j^1),   B_j = x_j - x_(j^1)
// (bit-identical to bfly4, src/xpuint8.cpp:279-285).  A_j = A_(j^1) and
// B_(j^1) = -B_j exactly, so four lanes need only four distinct sums, and each
// lane forms one of them and then one output, two instructions instead of
// three:
//   step 1 (partner j^1): even j keeps A_j = x_j + x_(j^1), odd j keeps
//          B_j = x_j - x_(j^1);
//   step 2 (partner j^3): even j outputs out_j = A_j - B_(j^3) (= A_j + B_(j^2));
//          odd j outputs out_(j^2) = B_j + A_(j^3) (= A_(j^2) + B_j).
// Each step is x + s * dpp(x) with a per-lane sign s = +-1 (step 2 takes -s
// through the source negation modifier): one v_fmac_f32_dpp, whose product is
// exact, so it rounds exactly as the add or
// subtract it replaces (signed zeros included).  The lane with an odd j then
// holds output j^2: after both axes lane sl holds register lane_w_rot(sl).
// Index j^1 / j^3 is lane xor 1 / xor 3 for axis 2 (digit i2) and lane xor 7 /
// xor 8 for axis 3 (digit i3), all single DPP controls (quad_perm, row_half_mirror,
// row_ror:8).
struct XlaneSigns {
    float a2, a3;     // step-1 signs of axes 2 and 3; step 2 uses their negation
};
// The step-1 sign is -1 where the lane's digit is odd (bit 0 of i2 is bit 0 of
// w = lane_w(sl), bit 0 of i3 is bit 2 of w).
__device__ __forceinline__ XlaneSigns xlane_signs(int sl) {
    const uint32_t w = uint32_t(lane_w(sl));
    return XlaneSigns{__uint_as_float((w << 31) | 0x3F800000u),
                      __uint_as_float(((w >> 2) << 31) | 0x3F800000u)};
}
// The register (group elements [16w, 16w+16)) that lane sl holds once the
// transform is done: each digit of lane_w(sl) that is odd has its bit 1
// flipped (d -> d ^ 2).
__device__ __forceinline__ int lane_w_rot(int sl) {
    const int w = lane_w(sl);
    return w ^ ((w & 5) << 1);
}

// One step over the 16 registers: v[t] += s * v[t] of the DPP partner.  One
// asm block, so the compiler places nothing between its instructions; it
// starts and ends with two wait states (s_nop 1), which a DPP read of a VGPR
// needs after the VALU write of it (the compiler cannot see the writes inside
// an asm block, nor can it see that the block's DPP reads need them).
#define XPU_FMAC_DPP(I, S, CTRL) \
    "v_fmac_f32_dpp %" #I ", %" #I ", " S " " CTRL " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
#define XPU_FMAC_DPP16(S, CTRL)                                                                    \
    XPU_FMAC_DPP(0, S, CTRL) XPU_FMAC_DPP(1, S, CTRL) XPU_FMAC_DPP(2, S, CTRL)                     \
    XPU_FMAC_DPP(3, S, CTRL) XPU_FMAC_DPP(4, S, CTRL) XPU_FMAC_DPP(5, S, CTRL)                     \
    XPU_FMAC_DPP(6, S, CTRL) XPU_FMAC_DPP(7, S, CTRL) XPU_FMAC_DPP(8, S, CTRL)                     \
    XPU_FMAC_DPP(9, S, CTRL) XPU_FMAC_DPP(10, S, CTRL) XPU_FMAC_DPP(11, S, CTRL)                   \
    XPU_FMAC_DPP(12, S, CTRL) XPU_FMAC_DPP(13, S, CTRL) XPU_FMAC_DPP(14, S, CTRL)                  \
    XPU_FMAC_DPP(15, S, CTRL)
#define XPU_V16_OPERANDS(v)                                                                        \
    "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]),           \
        "+v"(v[7]), "+v"(v[8]), "+v"(v[9]), "+v"(v[10]), "+v"(v[11]), "+v"(v[12]), "+v"(v[13]),   \
        "+v"(v[14]), "+v"(v[15])

// axis 2: partners lane xor 1 (quad_perm [1,0,3,2]) and xor 3 ([3,2,1,0])
__device__ __forceinline__ void hadamard_axis2(float (&v)[16], const XlaneSigns& s) {
    asm volatile("s_nop 1\n\t"
                 XPU_FMAC_DPP16("%16", "quad_perm:[1,0,3,2]")
                 XPU_FMAC_DPP16("-%16", "quad_perm:[3,2,1,0]")
                 "s_nop 1"
                 : XPU_V16_OPERANDS(v)
                 : "v"(s.a2));
}
// axis 3: partners lane xor 7 (row_half_mirror) and xor 8 (row_ror:8)
__device__ __forceinline__ void hadamard_axis3(float (&v)[16], const XlaneSigns& s) {
    asm volatile("s_nop 1\n\t"
                 XPU_FMAC_DPP16("%16", "row_half_mirror")
                 XPU_FMAC_DPP16("-%16", "row_ror:8")
                 "s_nop 1"
                 : XPU_V16_OPERANDS(v)
                 : "v"(s.a3));
}
__device__ __forceinline__ void hadamard_xlane(float (&v)[16], const XlaneSigns& s) {
    hadamard_axis2(v, s);
    hadamard_axis3(v, s);
}
#undef XPU_FMAC_DPP
#undef XPU_FMAC_DPP16
#undef XPU_V16_OPERANDS

// The full unscaled group transform: the true rotation is this times 1/16.
// Lane sl of a 16-lane segment enters with register lane_w(sl) and leaves
// with register lane_w_rot(sl); s = xlane_signs(sl).
__device__ __forceinline__ void hadamard16_unscaled(float (&v)[16], const XlaneSigns& s) {
    hadamard_inreg(v);
    hadamard_xlane(v, s);
}

__device__ __forceinline__ void halve16(float (&v)[16]) {
#pragma unroll
    for (int t = 0; t < 16; ++t) v[t] *= 0.5f;
}

// The same transform in the reference's scaled operation order, giving the
// true rotation (no final 1/16).  Axes 0 and 1 multiply their inputs by the
// coefficients +-0.5 and then chain (src/xpuint8.cpp:290-301): the product by
// 0.5 is exact and the sign is the chain's add or subtract, so it is halve16
// then h4_chain.  Axes 2 and 3 form (p + n) * 0.5 with p, n unscaled sums
// (bfly4, src/xpuint8.cpp:279-285): the butterfly, then halve16.  This is the
// path for groups the fast form could overflow on; see the header comment.
__device__ __forceinline__ void hadamard16_scaled(float (&v)[16], const XlaneSigns& s) {
    halve16(v);
#pragma unroll
    for (int b = 0; b < 16; b += 4) h4_chain(v[b], v[b + 1], v[b + 2], v[b + 3]);
    halve16(v);
#pragma unroll
    for (int c = 0; c < 4; ++c) h4_chain(v[c], v[c + 4], v[c + 8], v[c + 12]);
    hadamard_axis2(v, s);
    halve16(v);
    hadamard_axis3(v, s);
    halve16(v);
}

// Inputs at or above this magnitude (or an inf) send a group to the scaled
// transform: below it, 256 * max|x| < 2^128 bounds every unscaled intermediate.
constexpr float kUnscaledLimit = 0x1p120f;

// Max |x| over a lane's 16 inputs; NaN inputs are ignored (fmaxf), and a NaN
// propagates through either transform the same way.
__device__ __forceinline__ float inmax16(const float (&v)[16], float m) {
#pragma unroll
    for (int t = 0; t < 16; ++t) m = fmaxf(m, fabsf(v[t]));
    return m;
}

// Whether any lane of the wave holds a group that needs the scaled transform.
// The result is wave-uniform, so the branch on it keeps every lane of a
// segment (and the DPP partners of each lane) on the same path.
__device__ __forceinline__ bool wave_needs_scaled(float inmax) {
    return __builtin_amdgcn_ballot_w64(!(inmax < kUnscaledLimit)) != 0;
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
// rint_bits of eight values, their low bytes packed into two dwords (element 0
// lowest): each add writes its result's low byte straight into byte 0 or 1 of
// a 16-bit half (SDWA dst_sel BYTE_0 zero-padded, then BYTE_1 with the rest
// preserved) and a shift-or joins two halves: ten instructions for eight
// values instead of eight adds and six byte permutes.  On gfx940 and later a
// VALU result written with dst_sel other than DWORD must not be read by the
// next instruction (the forwarded value is the unformatted result), so the
// four halves are interleaved and every reader is at least two instructions
// behind its writer; the compiler cannot see inside the block to do that.
__device__ __forceinline__ uint2 rint_pack8(const float (&t)[8]) {
    const float magic = 12582912.0f;
    uint32_t h0, h1, h2, h3;
    uint2 r;
#define XPU_SDWA_ADD(D, S, SEL, UNUSED) \
    "v_add_f32_sdwa %" #D ", %" #S ", %14 dst_sel:" SEL " dst_unused:" UNUSED " src0_sel:DWORD src1_sel:DWORD\n\t"
    asm(XPU_SDWA_ADD(2, 6, "BYTE_0", "UNUSED_PAD")
        XPU_SDWA_ADD(3, 8, "BYTE_0", "UNUSED_PAD")
        XPU_SDWA_ADD(4, 10, "BYTE_0", "UNUSED_PAD")
        XPU_SDWA_ADD(5, 12, "BYTE_0", "UNUSED_PAD")
        XPU_SDWA_ADD(2, 7, "BYTE_1", "UNUSED_PRESERVE")
        XPU_SDWA_ADD(3, 9, "BYTE_1", "UNUSED_PRESERVE")
        XPU_SDWA_ADD(4, 11, "BYTE_1", "UNUSED_PRESERVE")
        XPU_SDWA_ADD(5, 13, "BYTE_1", "UNUSED_PRESERVE")
        "v_lshl_or_b32 %0, %3, 16, %2\n\t"
        "v_lshl_or_b32 %1, %5, 16, %4"
        : "=&v"(r.x), "=&v"(r.y), "=&v"(h0), "=&v"(h1), "=&v"(h2), "=&v"(h3)
        : "v"(t[0]), "v"(t[1]), "v"(t[2]), "v"(t[3]), "v"(t[4]), "v"(t[5]), "v"(t[6]),
          "v"(t[7]), "v"(magic));
#undef XPU_SDWA_ADD
    return r;
}
// Pack the low bytes of four such words into one dword (element 0 lowest).
__device__ __forceinline__ uint32_t pack4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint32_t ab = __builtin_amdgcn_perm(b, a, 0x0c0c0400u);
    const uint32_t cd = __builtin_amdgcn_perm(d, c, 0x0c0c0400u);
    return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
}

// The two divisions a quantizer makes per row, as short exact sequences in
// place of the general correctly rounded division (~10 VALU operations each):
//
// div127_rn(x) == x / 127.0f (IEEE) for every x >= 0, +inf included: the
// product by r = RN(1/127) is within an ulp of the quotient, so its remainder
// x - 127q is exact in one fma and one correction step with r rounds to the
// IEEE quotient (the method for a divisor known in advance; a quotient by 127
// is never within 2^-32 of a rounding boundary, far beyond the step's 2^-47).
// +inf takes the plain product (the remainder would be NaN).
//
// rcp_rn(x) == 1.0f / x (IEEE) for x in [2^-110, 2^122] and for +inf / NaN:
// one Newton step with fma on v_rcp_f32's approximation.  The range holds
// every row scale the quantizers form (>= bf16(1e-30) / 127 and <= FLT_MAX /
// 127); both identities are checked over every float of their range on the
// device (tests/c_abi/rounding_check.hip).
__device__ __forceinline__ float div127_rn(float x) {
    constexpr float r = 1.0f / 127.0f;
    const float q = x * r;
    const float e = __builtin_fmaf(-q, 127.0f, x);
    const float c = __builtin_fmaf(e, r, q);
    return x <= 3.40282347e38f ? c : q;
}
__device__ __forceinline__ float rcp_rn(float x) {
    const float y = __builtin_amdgcn_rcpf(x);
    const float e = __builtin_fmaf(-x, y, 1.0f);
    const float z = __builtin_fmaf(e, y, y);
    return x <= 3.40282347e38f ? z : y;
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
