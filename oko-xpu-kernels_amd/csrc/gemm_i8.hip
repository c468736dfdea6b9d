// int8 x int8 -> int32 GEMM on CDNA4 MFMA (v_mfma_i32_16x16x64_i8), with the
// accumulator consumed in registers by a fused epilogue: int32 store, or the
// ConvRot dequant  bf16(float(acc) * (ws[n] * xs[m]) + bias[n])
// (src/xpuint8.cpp:692-710) applied on the way out.
//
//   C[m, n] = sum_k X[m, k] * W[n, k]      X int8 [M, K], W int8 [N, K]
//
// the "NT" product torch._int_mm(x, w.t()) of the reference's linear
// (python/xpu_kernels/int8/ops.py:634).
//
// Layout.  Each MFMA computes a 16 x 16 block D = W_blk * X_blk^T with the
// weight rows as the MFMA "A" operand, so lane l ends up holding
// D[n0 + 4*(l/16) + i][m0 + l%16], i = 0..3: four consecutive output columns
// of one row -- one 8-byte bf16 store (or one 16-byte int32 store) per block.
// The operand layout is lane l -> row l%16, bytes [16*(l/16), +16) of the
// 64-byte K step, for both operands; any K permutation shared by the two
// operands gives the same integer dot products.
//
// Tiling.  A block of WGM x WGN waves owns a BM x BN output tile; a wave owns
// (BM/WGM) x (BN/WGN), TM x TN MFMA blocks.  The X and W K-slices (BK = 64
// bytes per row) stream into a ring of STAGES LDS buffers with direct
// global->LDS loads (global_load_lds_dwordx4, no VGPR staging), issued
// STAGES-1 steps ahead of the MFMAs; each step waits only for its own loads
// (an explicit vmcnt) and one s_barrier.  Tiles are ordered so that each of
// the 8 XCDs (blockIdx % 8) works on a compact rectangle of the output,
// keeping its X rows and W rows in its own L2.
#include <algorithm>
#include <type_traits>

#include "activations.hpp"
#include "common.hpp"
#include "kernels.hpp"

namespace xpuint8 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

// s_waitcnt immediate that waits for vmcnt <= n only (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14; expcnt 6:4 and lgkmcnt 11:8 left at their maxima).
__host__ __device__ constexpr int vmcnt_imm(int n) {
    return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8);
}

// Two fp32 -> packed bf16 (round to nearest even; v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v2f{lo, hi}, v2bf));
}

// ----------------------------------------------------------------- epilogues
// Called once per 16x16 block with the lane's four values: row m, columns
// n..n+3 (n % 4 == 0, the whole block lies inside [0, N)).
//
// kPaired epilogues consume two accumulators per output element: the product
// with weight row n (first half) and with row half + n (second half), e.g.
// the FFN's hidden and gate columns; the kernel then interleaves the two
// halves' weight rows block by block so both land in the same lane.
struct EpiI32 {
    static constexpr bool kStaged = false;
    static constexpr bool kPaired = false;
    int32_t* c;
    int64_t ldc;
    __device__ __forceinline__ void operator()(int m, int n, const v4i& v) const {
        *reinterpret_cast<v4i*>(c + int64_t(m) * ldc + n) = v;
    }
};

// The int32 partial products of one K slice of a split across blocks (the
// split-K kernel launched with gridDim.y slices, slice blockIdx.y): slice s's
// [M, N] sums at c + s * slice_stride.  Integer sums are exact, so adding the
// slices in any order gives the full product bit for bit.
struct EpiSliceI32 {
    static constexpr bool kStaged = false;
    static constexpr bool kPaired = false;
    static constexpr bool kSlice = true;
    int32_t* c;
    int64_t ldc;
    int64_t slice_stride;
    __device__ __forceinline__ void operator()(int m, int n, const v4i& v) const {
        *reinterpret_cast<v4i*>(c + int64_t(blockIdx.y) * slice_stride + int64_t(m) * ldc + n) = v;
    }
};
template <class E, class = void>
struct IsSliceEpi : std::false_type {};
template <class E>
struct IsSliceEpi<E, std::void_t<decltype(E::kSlice)>> : std::integral_constant<bool, E::kSlice> {};

// bf16(float(acc) * (ws[n] * xs[m]) + bias[n]); ws == nullptr is a unit column
// scale (1.0f * xs[m] == xs[m]), bias may be null.
struct EpiDequant {
    static constexpr bool kStaged = true;
    static constexpr bool kPaired = false;
    uint16_t* out;
    int64_t ldo;
    const float* xs;
    const float* ws;
    const float* bias;       // fp32 bias, or
    const uint16_t* bias16;  // bf16 bias (widened exactly), or neither
    // per-row and per-column operands, loaded before any conversion so that
    // their memory latency is paid once per tile
    struct Col { float4 w, b; };
    __device__ __forceinline__ float row(int m) const { return xs[m]; }
    __device__ __forceinline__ Col col(int n) const {
        Col c;
        c.w = ws ? *reinterpret_cast<const float4*>(ws + n) : make_float4(1.f, 1.f, 1.f, 1.f);
        if (bias) {
            c.b = *reinterpret_cast<const float4*>(bias + n);
        } else if (bias16) {
            const uint2 u = *reinterpret_cast<const uint2*>(bias16 + n);
            c.b = make_float4(bf16lo(u.x), bf16hi(u.x), bf16lo(u.y), bf16hi(u.y));
        } else {
            c.b = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        return c;
    }
    // The persistent kernel keeps a tile's operands in LDS: the row scales,
    // then kColVals fp32 values per output column (column scale, bias), each
    // `stride` apart.
    static constexpr int kColVals = 2;
    __device__ __forceinline__ float col_value(int which, int n) const {
        if (which == 0) return ws ? ws[n] : 1.f;
        if (bias) return bias[n];
        if (bias16) return __uint_as_float(uint32_t(bias16[n]) << 16);
        return 0.f;
    }
    __device__ __forceinline__ Col col_lds(const float* c, int stride, int nl, int) const {
        return Col{*reinterpret_cast<const float4*>(c + nl),
                   *reinterpret_cast<const float4*>(c + stride + nl)};
    }
    // the four bf16 results of one row, columns n..n+3, packed
    __device__ __forceinline__ uint2 convert(const v4i& v, float x, const Col& c) const {
        float r0 = float(v[0]) * (c.w.x * x), r1 = float(v[1]) * (c.w.y * x);
        float r2 = float(v[2]) * (c.w.z * x), r3 = float(v[3]) * (c.w.w * x);
        if (bias || bias16) {
            r0 = r0 + c.b.x; r1 = r1 + c.b.y; r2 = r2 + c.b.z; r3 = r3 + c.b.w;
        }
        uint2 o;
        o.x = cvt_pk_bf16(r0, r1);
        o.y = cvt_pk_bf16(r2, r3);
        return o;
    }
    // eight finished bf16 values, row m, columns n..n+7
    __device__ __forceinline__ void store16(int m, int n, const uint4& v) const {
        *reinterpret_cast<uint4*>(out + int64_t(m) * ldo + n) = v;
    }
    __device__ __forceinline__ void operator()(int m, int n, const v4i& v) const {
        const uint2 o = convert(v, row(m), col(n));
        *reinterpret_cast<uint2*>(out + int64_t(m) * ldo + n) = o;
    }
};

// The dequant epilogue followed by the residual update of the reference's
// linear(residual=, residual_scale=) (python/xpu_kernels/int8/ops.py:639-644):
//   d = bf16(float(acc) * (ws[n] * xs[m]) + bias[n])     (EpiDequant)
//   out[m, n] = bf16(float(res[m, n]) + float(d) * float(rscale[n]))
// which is torch.addcmul(res, d, rscale) on bf16 tensors: the product of two
// bf16 values is exact in fp32, so the fp32 sum is the only rounding before
// the bf16 one, with or without a fused multiply-add.  res is bf16 [M, N]
// (row stride ldr); rscale bf16 [N].
struct EpiDequantRes : EpiDequant {
    const uint16_t* res;
    int64_t ldr;
    const uint16_t* rscale;
    __device__ __forceinline__ static uint32_t upd2(uint32_t d, uint32_t r, uint32_t s) {
        const float lo = bf16lo(r) + bf16lo(d) * bf16lo(s);
        const float hi = bf16hi(r) + bf16hi(d) * bf16hi(s);
        return cvt_pk_bf16(lo, hi);
    }
    __device__ __forceinline__ void store16(int m, int n, const uint4& v) const {
        const uint4 r = *reinterpret_cast<const uint4*>(res + int64_t(m) * ldr + n);
        const uint4 sc = *reinterpret_cast<const uint4*>(rscale + n);
        *reinterpret_cast<uint4*>(out + int64_t(m) * ldo + n) =
            make_uint4(upd2(v.x, r.x, sc.x), upd2(v.y, r.y, sc.y), upd2(v.z, r.z, sc.z),
                       upd2(v.w, r.w, sc.w));
    }
    __device__ __forceinline__ void operator()(int m, int n, const v4i& v) const {
        const uint2 d = convert(v, row(m), col(n));
        const uint2 r = *reinterpret_cast<const uint2*>(res + int64_t(m) * ldr + n);
        const uint2 sc = *reinterpret_cast<const uint2*>(rscale + n);
        *reinterpret_cast<uint2*>(out + int64_t(m) * ldo + n) =
            make_uint2(upd2(d.x, r.x, sc.x), upd2(d.y, r.y, sc.y));
    }
};

// The FFN up-projection's epilogue: dequant, then the activation, written as
// bf16 (src/xpuint8.cpp:238-261, the load side of the reference's fused
// dequant+activation+quantize kernel, moved into the GEMM's store):
//   d = bf16(float(acc) * (ws[n] * xs[m]))   for each half
//   out[m, n] = act(d_first, d_second)         (activations.hpp)
// bit-identical to what the fused quantizer forms in registers, so quantizing
// `out` afterwards gives its exact codes.
template <int ACT>
struct EpiAct {
    static constexpr bool kStaged = true;
    static constexpr bool kPaired = act_paired(ACT);
    uint16_t* out;
    int64_t ldo;
    const float* xs;
    const float* ws;          // per weight row: [2 * half] paired, [N] otherwise
    int half;                 // row offset of the second half (paired)
    const uint16_t* tab;      // device activation tables
    uint32_t win = 0;         // LDS address of the table window (0: none)
    static constexpr int kWinTab = act_window_table<ACT>();
    struct Col { float4 w; };
    __device__ __forceinline__ float row(int m) const { return xs[m]; }
    __device__ __forceinline__ Col col(int n) const {
        return Col{*reinterpret_cast<const float4*>(ws + n)};
    }
    // LDS-held operands (as EpiDequant): the first half's column scales, then
    // (paired) the second half's
    static constexpr int kColVals = kPaired ? 2 : 1;
    __device__ __forceinline__ float col_value(int which, int n) const {
        return ws[which ? half + n : n];
    }
    __device__ __forceinline__ Col col_lds(const float* c, int stride, int nl, int second) const {
        return Col{*reinterpret_cast<const float4*>(c + (second ? stride : 0) + nl)};
    }
    __device__ __forceinline__ static float deq(int a, float w, float x) {
        return bf16_round(float(a) * (w * x));
    }
    // the activations' last bf16 rounding is the packing conversion itself
    __device__ __forceinline__ uint2 convert(const v4i& v, float x, const Col& c) const {
        const float r0 = activate_pre<ACT>(tab, deq(v[0], c.w.x, x), 0.f);
        const float r1 = activate_pre<ACT>(tab, deq(v[1], c.w.y, x), 0.f);
        const float r2 = activate_pre<ACT>(tab, deq(v[2], c.w.z, x), 0.f);
        const float r3 = activate_pre<ACT>(tab, deq(v[3], c.w.w, x), 0.f);
        return make_uint2(cvt_pk_bf16(r0, r1), cvt_pk_bf16(r2, r3));
    }
    __device__ __forceinline__ uint2 convert2(const v4i& a, const v4i& b, float x, const Col& ca,
                                              const Col& cb) const {
        const float r0 = activate_pre<ACT>(tab, deq(a[0], ca.w.x, x), deq(b[0], cb.w.x, x));
        const float r1 = activate_pre<ACT>(tab, deq(a[1], ca.w.y, x), deq(b[1], cb.w.y, x));
        const float r2 = activate_pre<ACT>(tab, deq(a[2], ca.w.z, x), deq(b[2], cb.w.z, x));
        const float r3 = activate_pre<ACT>(tab, deq(a[3], ca.w.w, x), deq(b[3], cb.w.w, x));
        return make_uint2(cvt_pk_bf16(r0, r1), cvt_pk_bf16(r2, r3));
    }
    // convert / convert2 with the table read from the LDS window (win != 0):
    // four 16-bit LDS reads, one wait, and the global table only for inputs
    // outside the window, behind a wave-uniform branch that is rarely taken.
    // Same table words, so the same results.
    //
    // The four dequantized keys (the table's inputs: the gate for GEGLU, the
    // value for GELU) are rounded to bf16 two at a time, as packed pairs
    // (v_cvt_pk_bf16_f32 rounds each half to nearest even, deq()'s rounding),
    // and a pair's two window positions come from packed 16-bit integer
    // arithmetic.  With t = key - kWinLo (16 bits, wrapping), a key lies in
    // the window iff bits 11-14 of t are clear; t's bit 15 is then its sign
    // and bits 0-10 its index, so its byte offset in the window (positive
    // half first, win_bits' order) is (t << 1 & 0xFFE) | (t >> 3 & 0x1000).
    // A key outside reads some entry inside (the offset is masked to the
    // window) and is replaced from the global table.
    typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
    __device__ __forceinline__ uint2 win_finish(const float (&key)[4], const float (&val)[4]) const {
        const uint32_t kp[2] = {cvt_pk_bf16(key[0], key[1]), cvt_pk_bf16(key[2], key[3])};
        uint32_t t[4], tor = 0;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const u16x2 tt = __builtin_bit_cast(u16x2, kp[j]) -
                             u16x2{uint16_t(kWinLo), uint16_t(kWinLo)};
            tor |= __builtin_bit_cast(uint32_t, tt);
            const uint32_t lo2 = __builtin_bit_cast(uint32_t, u16x2(tt << u16x2{1, 1}));
            const uint32_t hi3 = __builtin_bit_cast(uint32_t, u16x2(tt >> u16x2{3, 3}));
            const uint32_t off = (lo2 & 0x0FFE0FFEu) | (hi3 & 0x10001000u);
            // win + each 16-bit half of off, one SDWA add each (the compiler
            // would fuse the low half's mask into the or above and add apart)
            uint32_t a0, a1;
            asm("v_add_u32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_0 "
                "src1_sel:DWORD"
                : "=v"(a0) : "v"(off), "v"(win));
            asm("v_add_u32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_1 "
                "src1_sel:DWORD"
                : "=v"(a1) : "v"(off), "v"(win));
            asm volatile("ds_read_u16 %0, %1" : "=v"(t[2 * j]) : "v"(a0));
            asm volatile("ds_read_u16 %0, %1" : "=v"(t[2 * j + 1]) : "v"(a1));
        }
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(t[0]), "+v"(t[1]), "+v"(t[2]), "+v"(t[3]));
        if (__builtin_amdgcn_ballot_w64((tor & 0x78007800u) != 0)) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t k = (kp[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
                if (((k - uint32_t(kWinLo)) & 0x7800u) != 0)
                    t[i] = tab[kWinTab * kTabSize + k];
            }
        }
        if constexpr (ACT == 4) {
            // the hidden values, rounded to bf16 in pairs, times the table's
            // gelu(gate): each product exact in fp32, then the packing's
            // rounding
            const uint32_t vp0 = cvt_pk_bf16(val[0], val[1]), vp1 = cvt_pk_bf16(val[2], val[3]);
            const float r0 = __uint_as_float(vp0 << 16) * tab_float(t[0]);
            const float r1 = __uint_as_float(vp0 & 0xFFFF0000u) * tab_float(t[1]);
            const float r2 = __uint_as_float(vp1 << 16) * tab_float(t[2]);
            const float r3 = __uint_as_float(vp1 & 0xFFFF0000u) * tab_float(t[3]);
            return make_uint2(cvt_pk_bf16(r0, r1), cvt_pk_bf16(r2, r3));
        } else {
            // a single lookup: the table's bf16 results through the same
            // packing conversion as the unwindowed form (NaN words included)
            return make_uint2(cvt_pk_bf16(tab_float(t[0]), tab_float(t[1])),
                              cvt_pk_bf16(tab_float(t[2]), tab_float(t[3])));
        }
    }
    // the dequant product before its bf16 rounding
    __device__ __forceinline__ static float deq_raw(int a, float w, float x) {
        return float(a) * (w * x);
    }
    __device__ __forceinline__ uint2 convert_w(const v4i& v, float x, const Col& c) const {
        static_assert(ACT == 5, "the windowed single-block form is GELU's");
        const float k[4] = {deq_raw(v[0], c.w.x, x), deq_raw(v[1], c.w.y, x),
                            deq_raw(v[2], c.w.z, x), deq_raw(v[3], c.w.w, x)};
        return win_finish(k, k);
    }
    __device__ __forceinline__ uint2 convert2_w(const v4i& av, const v4i& bv, float x, const Col& ca,
                                                const Col& cb) const {
        static_assert(ACT == 4, "the windowed pair form is GEGLU's");
        const float a[4] = {deq_raw(av[0], ca.w.x, x), deq_raw(av[1], ca.w.y, x),
                            deq_raw(av[2], ca.w.z, x), deq_raw(av[3], ca.w.w, x)};
        const float b[4] = {deq_raw(bv[0], cb.w.x, x), deq_raw(bv[1], cb.w.y, x),
                            deq_raw(bv[2], cb.w.z, x), deq_raw(bv[3], cb.w.w, x)};
        return win_finish(b, a);
    }
    __device__ __forceinline__ void store16(int m, int n, const uint4& v) const {
        *reinterpret_cast<uint4*>(out + int64_t(m) * ldo + n) = v;
    }
    // unstaged forms: one block of four columns (small tiles, unpaired
    // activations), or the first and second halves' blocks of the same four
    // columns (the skinny kernel, paired activations)
    __device__ __forceinline__ void operator()(int m, int n, const v4i& v) const {
        *reinterpret_cast<uint2*>(out + int64_t(m) * ldo + n) = convert(v, row(m), col(n));
    }
    __device__ __forceinline__ void pair(int m, int n, const v4i& a, const v4i& b) const {
        *reinterpret_cast<uint2*>(out + int64_t(m) * ldo + n) =
            convert2(a, b, row(m), col(n), col(half + n));
    }
};

// Whether an epilogue reads an activation table through an LDS window
// (EpiAct of a single-lookup activation).
template <class Epi, class = void>
struct HasWindow : std::false_type {};
template <class Epi>
struct HasWindow<Epi, std::void_t<decltype(Epi::kWinTab)>>
    : std::integral_constant<bool, (Epi::kWinTab >= 0)> {};
template <class Epi>
__host__ __device__ constexpr bool has_window() { return HasWindow<Epi>::value; }

// An epilogue's conversion of one block (or pair of blocks), through the LDS
// window or not.
template <bool WIN, class Epi>
__device__ __forceinline__ uint2 convert_one(const Epi& e, const v4i& v, float x,
                                             const typename Epi::Col& c) {
    if constexpr (WIN) return e.convert_w(v, x, c);
    else return e.convert(v, x, c);
}
template <bool WIN, class Epi>
__device__ __forceinline__ uint2 convert_pair(const Epi& e, const v4i& a, const v4i& b, float x,
                                              const typename Epi::Col& ca,
                                              const typename Epi::Col& cb) {
    if constexpr (WIN) return e.convert2_w(a, b, x, ca, cb);
    else return e.convert2(a, b, x, ca, cb);
}

// Row offset of a paired epilogue's second half (0 for the others).
template <class Epi>
__device__ __forceinline__ int pair_offset(const Epi& e) {
    if constexpr (Epi::kPaired) return e.half;
    else return 0;
}

// ----------------------------------------------------------------- kernel
// 16 zero bytes: the DMA source of operand chunks beyond K (a load cannot be
// predicated into zeros, so it reads these instead).
__device__ __attribute__((aligned(16))) int8_t g_zero16[16];

// LDS layout of one stage: (BM + BN) / 16 blocks of 1 KB, X blocks first.  A
// block holds 16 rows x 64 bytes; the 16-byte chunk c of row r sits at
// position c ^ ((r >> 1) & 3), so that the 16 rows read together by one
// quarter-wave land on distinct banks.  One block is exactly what one
// global_load_lds_dwordx4 writes (lane l -> bytes [16l, 16l+16)).
__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r >> 1) & 3); }

// LDS reads of MFMA fragments, issued as inline assembly so the kernel can
// place them all at the start of a K step and wait for each one just before
// its MFMAs (lgkm_wait<N>: at most N of this wave's LDS reads outstanding).
// The loop issues no scalar memory reads, which share the counter.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p));
}
__device__ __forceinline__ v4i lds_read16(uint32_t addr) {
    v4i r;
    asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(addr));
    return r;
}
// A transposing read of 8-bit elements (gfx950): in each group of 16 lanes,
// output lane 8a + b receives byte b of the 8 bytes addressed by lanes a,
// a+2, .., a+14, in that order.
typedef int v2i __attribute__((ext_vector_type(2)));
__device__ __forceinline__ v2i lds_read8_tr(uint32_t addr) {
    v2i r;
    asm volatile("ds_read_b64_tr_b8 %0, %1" : "=v"(r) : "v"(addr));
    return r;
}
// the same with a constant byte offset in the instruction's offset field (one
// address register serves a row of fragments)
template <int OFF>
__device__ __forceinline__ v4i lds_read16_at(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
    v4i r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
    return r;
}
// fragments i = 0 .. COUNT-1 at addr + i * 1024
template <int COUNT, int I = 0, int NF>
__device__ __forceinline__ void lds_read_frags(v4i (&f)[NF], uint32_t addr) {
    if constexpr (I < COUNT) {
        f[I] = lds_read16_at<I * 1024>(addr);
        lds_read_frags<COUNT, I + 1>(f, addr);
    }
}
// Wait until at most N LDS reads are outstanding; v is tied to the wait so
// its uses cannot be scheduled above it.
template <int N>
__device__ __forceinline__ void lgkm_wait(v4i& v) {
    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(v) : "n"(N));
}

// Wait for every outstanding LDS read, tied to all of a step's fragments: the
// one s_waitcnt comes first, then an empty volatile asm per fragment that
// "redefines" it, so no use of any fragment (an MFMA) can be scheduled above
// the wait.  (The inline-asm reads complete asynchronously, which the compiler
// does not know: a plain s_waitcnt builtin lets it hoist MFMAs above the wait.)
template <int TN, int TM>
__device__ __forceinline__ void lgkm_wait_all(v4i (&wf)[TN], v4i (&xf)[TM]) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(wf[0]));
#pragma unroll
    for (int a = 1; a < TN; ++a) asm volatile("" : "+v"(wf[a]));
#pragma unroll
    for (int b = 0; b < TM; ++b) asm volatile("" : "+v"(xf[b]));
}

// Column b of the wave's MFMA blocks: wait for X fragment b (and, for b = 0,
// every W fragment, which were read first), then TN MFMAs, then the step's
// b-th global->LDS load for a later stage (after_column(b)), so the wave's
// loads leave spread over the step instead of as a burst ahead of its MFMAs.
template <int TN, int TM, int B = 0, class F>
__device__ __forceinline__ void mfma_columns(v4i (&acc)[TN][TM], v4i (&wf)[TN], v4i (&xf)[TM],
                                             const F& after_column) {
    if constexpr (B < TM) {
        if constexpr (B == 0) {
#pragma unroll
            for (int a = 0; a < TN; ++a) lgkm_wait<TM>(wf[a]);
        }
        lgkm_wait<TM - 1 - B>(xf[B]);
#pragma unroll
        for (int a = 0; a < TN; ++a)
            acc[a][B] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[a], xf[B], acc[a][B], 0, 0, 0);
        after_column(B);
        // keep the next column's wait (and load) below these MFMAs
        __builtin_amdgcn_sched_barrier(0);
        mfma_columns<TN, TM, B + 1>(acc, wf, xf, after_column);
    }
}

// One 16-byte global -> LDS DMA per lane (global_load_lds_dwordx4): lane l's
// bytes land at ldst + 16*l; ldst must be the same for the whole wave.
__device__ __forceinline__ void dma16(const int8_t* gsrc, int8_t* ldst) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_global_load_lds(gsrc, (__attribute__((address_space(3))) void*)ldst, 16, 0,
                                     0);
#endif
}

template <int BM, int BN, int WGM, int WGN, int STAGES, class Epi>
__global__ __launch_bounds__(WGM * WGN * 64) void gemm_i8_kernel(
    const int8_t* __restrict__ X, int64_t ldx, const int8_t* __restrict__ W, int64_t ldw, int M,
    int N, int K, int tiles_m, int tiles_n, Epi epi) {
    constexpr int BK = 64;
    constexpr int NWAVES = WGM * WGN;
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int TM = WM / 16, TN = WN / 16;
    static_assert(WM % 16 == 0 && WN % 16 == 0, "wave tile must be whole MFMA blocks");
    constexpr int XB = BM / 16, WB = BN / 16, NB = XB + WB;      // 1 KB blocks per stage
    constexpr int PER_WAVE = (NB + NWAVES - 1) / NWAVES;       // DMA instructions per wave
    constexpr int STAGE_BYTES = NB * 1024;
    __shared__ __attribute__((aligned(1024))) int8_t smem[STAGES * STAGE_BYTES];
    // K slice blockIdx.y of a split across blocks (EpiSliceI32): K is the
    // slice's length, the operands' rows keep their full strides
    if constexpr (IsSliceEpi<Epi>::value) {
        X += int64_t(blockIdx.y) * K;
        W += int64_t(blockIdx.y) * K;
    }

    const int tiles = tiles_m * tiles_n;
    int t = blockIdx.x;
    if (tiles % 8 == 0) t = (t % 8) * (tiles / 8) + t / 8;
    constexpr int GROUP = 8;
    const int band = t / (GROUP * tiles_n);
    const int first_m = band * GROUP;
    const int gm = min(tiles_m - first_m, GROUP);
    const int in_band = t - band * GROUP * tiles_n;
    const int tile_m = first_m + in_band % gm;
    const int tile_n = in_band / gm;
    const int m0 = tile_m * BM, n0 = tile_n * BN;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WGN, wn = wave % WGN;

    // This lane's DMA sources: block j of a stage covers rows 16*(j' ) .. of X
    // (j < XB) or of W; lane l brings row l/4, chunk swz(l/4, l%4) of it.
    const int lr = lane >> 2;
    const int lc = swz(lr, lane & 3) * 16;
    const int8_t* src[PER_WAVE];
    int nblk = 0;
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
        const int j = wave + i * NWAVES;
        if (j < NB) ++nblk;
        if (j < XB) {
            const int r = min(m0 + 16 * j + lr, M - 1);
            src[i] = X + int64_t(r) * ldx + lc;
        } else {
            const int r = min(n0 + 16 * (j - XB) + lr, N - 1);
            src[i] = W + int64_t(r) * ldw + lc;
        }
    }
    auto issue = [&](int stage_buf, int k0) {
#pragma unroll
        for (int i = 0; i < PER_WAVE; ++i) {
            const int j = wave + i * NWAVES;
            if (j < NB) {
                const int8_t* p = (k0 + lc < K) ? src[i] + k0 : g_zero16;
                dma16(p, smem + stage_buf * STAGE_BYTES + j * 1024);
            }
        }
    };

    v4i acc[TN][TM];
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
        for (int b = 0; b < TM; ++b) acc[a][b] = v4i{0, 0, 0, 0};

    // operand read offset inside a block: row l%16, chunk l/16
    const int frag = (lane & 15) * 64 + swz(lane & 15, lane >> 4) * 16;
    const int KT = (K + BK - 1) / BK;
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
        if (s < KT) issue(s, s * BK);

    for (int kt = 0; kt < KT; ++kt) {
        // this wave's loads of step kt are done once at most the later
        // (STAGES - 2) steps' loads are outstanding; then every wave's are
        const int later = min(KT - 1 - kt, STAGES - 2);
        if (nblk == PER_WAVE) {
            if (later >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * PER_WAVE));
            else if (later == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(PER_WAVE));
            else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        } else {
            if (later >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * (PER_WAVE - 1)));
            else if (later == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(PER_WAVE - 1));
            else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        }
        __builtin_amdgcn_s_barrier();
        // the buffer refilled now was consumed at step kt-1, before this barrier
        if (kt + STAGES - 1 < KT) issue((kt + STAGES - 1) % STAGES, (kt + STAGES - 1) * BK);
        const int8_t* sb = smem + (kt % STAGES) * STAGE_BYTES;
        v4i wf[TN];
#pragma unroll
        for (int a = 0; a < TN; ++a)
            wf[a] = *reinterpret_cast<const v4i*>(sb + (XB + wn * (WN / 16) + a) * 1024 + frag);
#pragma unroll
        for (int b = 0; b < TM; ++b) {
            const v4i xf = *reinterpret_cast<const v4i*>(sb + (wm * (WM / 16) + b) * 1024 + frag);
#pragma unroll
            for (int a = 0; a < TN; ++a)
                acc[a][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[a], xf, acc[a][b], 0, 0, 0);
        }
    }

    // lane l of block (a, b): row m0 + wm*WM + 16b + l%16, columns n .. n+3 with
    // n = n0 + wn*WN + 16a + 4*(l/16)
    const int mrow = m0 + wm * WM + (lane & 15);
    const int ncol = n0 + wn * WN + 4 * (lane >> 4);
#pragma unroll
    for (int b = 0; b < TM; ++b) {
        const int m = mrow + 16 * b;
        if (m >= M) continue;
#pragma unroll
        for (int a = 0; a < TN; ++a) {
            const int n = ncol + 16 * a;
            if (n < N) epi(m, n, acc[a][b]);
        }
    }
}

// The staged epilogue of one wave: its TM x TN blocks of results (output
// rows m0w.., columns n0w..), RB row blocks (16*RB rows) per pass through
// `stg` (RB * 4 KB of idle LDS): 256-byte rows of 16-byte chunks, chunk c of
// row r at c ^ (r & 15), each row leaving as contiguous 16-byte stores.  The
// column operands arrive in registers, the row operand of row block b as
// rowv(b).  Paired epilogues take the (first, second) accumulator pairs
// (2a, 2a+1).
template <int TM, int TN, int WN_OUT, class Epi, int RB, class RowF>
__device__ __forceinline__ void staged_store(const Epi& epi, v4i (&acc)[TN][TM], const RowF& rowv,
                                             const typename Epi::Col (&ccol)[TN], int8_t* stg,
                                             int m0w, int n0w, int M, int N, int lane) {
    constexpr bool PAIRED = Epi::kPaired;
    constexpr int OUT_TN = PAIRED ? TN / 2 : TN;
    constexpr int STG_ROWS = 16 * RB;
    constexpr int CH = WN_OUT / 8;                                 // live chunks per row
    constexpr int ITEMS = STG_ROWS * CH;
    static_assert(CH <= 16, "staging shape");
    static_assert(TM % RB == 0, "whole passes");
#pragma unroll
    for (int pass = 0; pass < TM / RB; ++pass) {
#pragma unroll
        for (int bb = 0; bb < RB; ++bb) {
            const int b = RB * pass + bb;
            const int r = 16 * bb + (lane & 15);
            const float x = rowv(b);
            auto row_of_blocks = [&](auto Wc) {
                constexpr bool WIN = decltype(Wc)::value;
#pragma unroll
                for (int a = 0; a < OUT_TN; ++a) {
                    const int c = 16 * a + 4 * (lane >> 4);
                    uint2 v;
                    if constexpr (PAIRED)
                        v = convert_pair<WIN>(epi, acc[2 * a][b], acc[2 * a + 1][b], x, ccol[2 * a],
                                              ccol[2 * a + 1]);
                    else
                        v = convert_one<WIN>(epi, acc[a][b], x, ccol[a]);
                    *reinterpret_cast<uint2*>(stg + r * 256 + (((c >> 3) ^ (r & 15)) << 4) +
                                              (c & 7) * 2) = v;
                }
            };
            if constexpr (has_window<Epi>()) {
                if (epi.win) row_of_blocks(std::true_type{});
                else row_of_blocks(std::false_type{});
            } else {
                row_of_blocks(std::false_type{});
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);                       // lgkmcnt(0)
#pragma unroll
        for (int i = 0; i < (ITEMS + 63) / 64; ++i) {
            const int flat = i * 64 + lane;
            const int r = flat / CH, c = flat % CH;
            if (ITEMS % 64 == 0 || flat < ITEMS) {
                const uint4 v = *reinterpret_cast<const uint4*>(stg + r * 256 + ((c ^ (r & 15)) << 4));
                const int m = m0w + STG_ROWS * pass + r, n = n0w + 8 * c;
                if (m < M && n < N) epi.store16(m, n, v);
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);                       // reads done before reuse
    }
}

// staged_store with the row and column operands read from global memory, all
// before any conversion so that their latency is paid once
template <int TM, int TN, int WN_OUT, class Epi, int RB = 2>
__device__ __forceinline__ void staged_epilogue(const Epi& epi, v4i (&acc)[TN][TM], int8_t* stg,
                                                int m0w, int n0w, int M, int N, int lane) {
    float xrow[TM];
    typename Epi::Col ccol[TN];
#pragma unroll
    for (int b = 0; b < TM; ++b) xrow[b] = epi.row(min(m0w + 16 * b + (lane & 15), M - 1));
#pragma unroll
    for (int a = 0; a < TN; ++a) {
        if constexpr (Epi::kPaired)
            ccol[a] = epi.col(min(n0w + 16 * (a >> 1) + 4 * (lane >> 4), N - 4) +
                              ((a & 1) ? pair_offset(epi) : 0));
        else
            ccol[a] = epi.col(min(n0w + 16 * a + 4 * (lane >> 4), N - 4));
    }
    staged_store<TM, TN, WN_OUT, Epi, RB>(epi, acc, [&](int b) { return xrow[b]; }, ccol, stg,
                                          m0w, n0w, M, N, lane);
}

// ------------------------------------------------------------ large tiles
// A BM x BN tile per block of 4 waves in a WGM x WGN grid, two blocks per CU
// (so one block's prologue and epilogue overlap the other's main loop); a
// wave owns (BM/WGM) x (BN/WGN) = TM x TN MFMA blocks.  K runs in 64-byte
// steps through a ring of STAGES LDS stages filled by direct global->LDS
// loads issued STAGES-1 steps ahead; a stage is exactly (BM + BN) / 16 KB, so
// three 26 KB stages of two 256x160 blocks fit in a CU's 160 KB.  A step reads
// the wave's TM + TN fragments right after its barrier and runs TM * TN MFMAs on
// them; the other block's waves keep the matrix core busy meanwhile.
//
// N is the number of output columns.  With a kPaired epilogue the tile's BN
// weight rows are BN/2 output columns' worth of pairs: W block 2p holds rows
// n0 + 16p .. of the first half, block 2p+1 the same rows of the second half
// (epi.half rows further), and each wave's TN blocks are whole pairs.
//
// DMA sources are a per-tile base pointer (wave-uniform) plus a 32-bit offset
// inside the tile's rows, so no operand size limit beyond K <= 2^23 / BM.
template <int BM, int BN, int WGM, int WGN, int STAGES, bool KTAIL, class Epi>
__global__ __launch_bounds__(WGM * WGN * 64, 8 / (WGM * WGN)) void gemm_i8_big_kernel(
    const int8_t* __restrict__ X, int64_t ldx, const int8_t* __restrict__ W, int64_t ldw, int M,
    int N, int K, int tiles_m, int tiles_n, Epi epi) {
    constexpr int NW = WGM * WGN;                               // 4 or 8 waves
    static_assert(NW == 4 || NW == 8, "four or eight waves");
    constexpr int BK = 64;
    constexpr int WM = BM / WGM, WN = BN / WGN, TM = WM / 16, TN = WN / 16;
    constexpr int XB = BM / 16, WB = BN / 16;
    constexpr int NB = XB + WB;                                 // 1 KB blocks per stage
    constexpr int PER_WAVE = (NB + NW - 1) / NW;                // DMA per wave per step (max)
    constexpr int REM = NB % NW;                                // waves < REM issue PER_WAVE
    constexpr int STAGE_BYTES = NB * 1024;                      // unpadded: 3 stages x 2 blocks fit
    constexpr int RING = STAGES * STAGE_BYTES;
    constexpr int STG_ROWS = 32;                                // epilogue rows per pass
    static_assert(!Epi::kStaged || NW * STG_ROWS * 256 <= RING, "staging fits in the ring");
    static_assert(TM % 2 == 0, "epilogue passes of 32 rows");
    constexpr bool PAIRED = Epi::kPaired;
    static_assert(!PAIRED || (Epi::kStaged && TN % 2 == 0), "pairs are whole per wave");
    constexpr int OUT_TN = PAIRED ? TN / 2 : TN;                // output blocks per wave
    constexpr int WN_OUT = 16 * OUT_TN, BN_OUT = WN_OUT * WGN;  // output columns
    __shared__ __attribute__((aligned(1024))) int8_t smem[RING];

    const int tiles = tiles_m * tiles_n;
    int t = blockIdx.x;
    if (tiles % 8 == 0) t = (t % 8) * (tiles / 8) + t / 8;
    constexpr int GROUP = 8;
    const int band = t / (GROUP * tiles_n);
    const int first_m = band * GROUP;
    const int gm = min(tiles_m - first_m, GROUP);
    const int in_band = t - band * GROUP * tiles_n;
    const int m0 = (first_m + in_band % gm) * BM, n0 = (in_band / gm) * BN_OUT;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WGN, wn = wave % WGN;

    // DMA: wave w brings blocks w, w+NW, ... < NB of every step (PER_WAVE or
    // PER_WAVE - 1 of them); blocks 0..XB-1 are X rows, XB..NB-1 W rows.
    // Lane l: row l/4, chunk swz(l/4, l%4).  Rows past M or N repeat the last
    // row (their results are never stored).
    const int lr = lane >> 2;
    const int lc = swz(lr, lane & 3) * 16;
    const int8_t* const xbase = X + int64_t(m0) * ldx;
    const int8_t* const wbase = W + int64_t(n0) * ldw;
    const int8_t* const gbase = W + (int64_t(pair_offset(epi)) + n0) * ldw;
    const int8_t* base[PER_WAVE];
    int off[PER_WAVE];
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
        const int j = min(wave + NW * i, NB - 1);
        if (j < XB) {
            base[i] = xbase;
            off[i] = (min(m0 + 16 * j + lr, M - 1) - m0) * int(ldx) + lc;
        } else if constexpr (PAIRED) {
            const int jw = j - XB;
            base[i] = (jw & 1) ? gbase : wbase;
            off[i] = (min(n0 + 16 * (jw >> 1) + lr, N - 1) - n0) * int(ldw) + lc;
        } else {
            base[i] = wbase;
            off[i] = (min(n0 + 16 * (j - XB) + lr, N - 1) - n0) * int(ldw) + lc;
        }
    }
    const bool full_share = REM == 0 || wave < REM;             // issues PER_WAVE per step
    auto issue_one = [&](int i, int buf, int k0) {
        if (i == PER_WAVE - 1 && !full_share) return;
        const int8_t* p = base[i] + (off[i] + k0);
        if (KTAIL && k0 + lc >= K) p = g_zero16;
        dma16(p, smem + buf * STAGE_BYTES + (wave + NW * i) * 1024);
    };
    auto issue = [&](int buf, int k0) {
#pragma unroll
        for (int i = 0; i < PER_WAVE; ++i) issue_one(i, buf, k0);
    };
    // this wave's loads of a step are complete once at most `later` steps'
    // worth of its own loads remain outstanding
    auto wait_loads = [&](int later) {
        if (full_share) {
            if (later >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * PER_WAVE));
            else if (later == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(PER_WAVE));
            else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        } else {
            if (later >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * (PER_WAVE - 1)));
            else if (later == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(PER_WAVE - 1));
            else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        }
    };

    const int frag = (lane & 15) * 64 + swz(lane & 15, lane >> 4) * 16;
    const int xoff = (wm * TM) * 1024 + frag;
    const int woff = (XB + wn * TN) * 1024 + frag;
    const uint32_t sbase = lds_addr(smem);

    v4i acc[TN][TM];
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
        for (int b = 0; b < TM; ++b) acc[a][b] = v4i{0, 0, 0, 0};

    const int KT = (K + BK - 1) / BK;
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
        if (s < KT) issue(s, s * BK);
#pragma clang loop unroll(disable)
    for (int kt = 0; kt < KT; ++kt) {
        // step kt's loads are done once only the later steps' may be pending
        wait_loads(min(KT - 1 - kt, STAGES - 2));
        __builtin_amdgcn_s_barrier();
        // the buffer refilled during this step was read at step kt-1, before
        // this barrier; its loads go out between the MFMA columns
        const bool refill = kt + STAGES - 1 < KT;
        const int rbuf = (kt + STAGES - 1) % STAGES, rk0 = (kt + STAGES - 1) * BK;
        // all TN + TM fragment reads go out at once; column b's MFMAs wait
        // only for the reads up to X fragment b
        const uint32_t sb = sbase + (kt % STAGES) * STAGE_BYTES;
        v4i wf[TN], xf[TM];
#pragma unroll
        for (int i = 0; i < TN; ++i) wf[i] = lds_read16(sb + woff + i * 1024);
#pragma unroll
        for (int i = 0; i < TM; ++i) xf[i] = lds_read16(sb + xoff + i * 1024);
        static_assert(TM <= 16, "lgkmcnt range");
        constexpr int LPC = (PER_WAVE + TM - 1) / TM;           // loads per column
        mfma_columns<TN, TM>(acc, wf, xf, [&](int b) {
            if (refill) {
#pragma unroll
                for (int i = b * LPC; i < (b + 1) * LPC; ++i)
                    if (i < PER_WAVE) issue_one(i, rbuf, rk0);
            }
        });
    }

    if constexpr (Epi::kStaged) {
        __builtin_amdgcn_s_barrier();                              // ring no longer read
        staged_epilogue<TM, TN, WN_OUT, Epi>(epi, acc, smem + wave * (32 * 256),
                                             m0 + wm * WM, n0 + wn * WN_OUT, M, N, lane);
    } else {
        const int mrow = m0 + wm * WM + (lane & 15);
        const int ncol = n0 + wn * WN + 4 * (lane >> 4);
#pragma unroll
        for (int b = 0; b < TM; ++b) {
            const int m = mrow + 16 * b;
            if (m >= M) continue;
#pragma unroll
            for (int a = 0; a < TN; ++a) {
                const int n = ncol + 16 * a;
                if (n < N) epi(m, n, acc[a][b]);
            }
        }
    }
}

template <int BM, int BN, int WGM, int WGN, int STAGES, class Epi>
hipError_t launch_cfg(hipStream_t st, const int8_t* X, int64_t ldx, const int8_t* W, int64_t ldw,
                      int M, int N, int K, const Epi& epi) {
    const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
    hipLaunchKernelGGL((gemm_i8_kernel<BM, BN, WGM, WGN, STAGES, Epi>), dim3(unsigned(tm * tn)),
                       dim3(WGM * WGN * 64), 0, st, X, ldx, W, ldw, M, N, K, tm, tn, epi);
    return hipGetLastError();
}

// ------------------------------------------------------------ ping-pong
// BM x BN tiles (256 x 320) for one persistent block of 8 waves per CU, in two
// groups of 4 (group = the tile's row half, 2 x 4 waves of 128 x 80, or 4 x 2
// of 64 x 160 for paired epilogues), a ring of S = 4 LDS slots of 64-byte K
// steps filled by direct global->LDS loads.  Block b takes tiles b, b + G,
// b + 2G, ... (G = gridDim.x, one block per CU).  Within a tile the groups
// alternate roles every half step, so that on each SIMD one wave feeds the
// matrix core while the other moves data:
//   phase A(k): group 0 runs step k's MFMAs;  group 1 reads step k's
//               fragments and issues its loads for step k + S - 1
//   phase B(k): group 1 runs step k's MFMAs;  group 0 reads step k + 1's
//               fragments and issues its loads for step k + S - 1
// with one s_barrier between phases.  Step j's loads are complete (each wave
// waits for its own, then the barrier) before phase B(j - 1), the first
// reader of step j; its slot is refilled (for step j + S) only from phase
// A(j + 1) on, after its last reader, A(j).  Step k lives in slot (k + 1) % S.
//
// Between tiles: once a tile's last MFMAs are issued (every fragment read is
// complete), each wave issues the next tile's steps 0-2 into slots 1-3 and
// the global loads of its row/column operands, and only then runs this tile's
// epilogue, staged through slot 0.  Those loads are older than the epilogue's
// stores, so they land while it runs; one vmcnt(0) afterwards (the stores
// included) and a barrier start the next tile.  The epilogue's per-row and
// per-column operands come from LDS (two buffers after the ring, filled one
// tile ahead), not from global memory at the end of the tile.
//
// XT: X comes in the MFMA block layout (tiled_offset, the quantizer's tiled
// output), so each X block of a step is one contiguous 1 KB load instead of
// 16 row segments of 64 bytes: 61.1 -> 58.2 us at C3 (cold, timing-only
// builds of the load pattern), the direct-to-LDS path being bound by the
// number of cache lines an instruction touches.  WT: the weight too
// (pack_weight's copy), 58.1 -> 53.0 us at C3.
template <int BM, int BN, int WGM, int WGN, int S, bool KTAIL, class Epi, bool XT = false,
          bool WT = false>
__global__ __launch_bounds__(512, 1) void gemm_i8_pp_kernel(
    const int8_t* __restrict__ X, int64_t ldx, const int8_t* __restrict__ W, int64_t ldw, int M,
    int N, int K, int tiles_m, int tiles_n, Epi epi) {
    constexpr int NW = 8;
    static_assert(WGM * WGN == NW && WGM % 2 == 0, "two groups of four waves (row halves)");
    constexpr int BK = 64;
    constexpr int WM = BM / WGM, WN = BN / WGN, TM = WM / 16, TN = WN / 16;
    constexpr int XB = BM / 16, WB = BN / 16, NB = XB + WB;
    constexpr int PER = (NB + NW - 1) / NW;                     // loads per wave per step (max)
    constexpr int REM = NB % NW;                                // waves < REM issue PER
    static_assert(REM == 0 || REM == 4, "group 0 issues PER, group 1 PER or PER - 1");
    constexpr int PER0 = PER, PER1 = REM == 0 ? PER : PER - 1;
    constexpr int STAGE_BYTES = NB * 1024;
    constexpr int RING = S * STAGE_BYTES;
    static_assert(S == 4, "a tile's last slot stages the epilogue while the next tile's steps 0-2 "
                          "fill the other three");
    constexpr bool STAGED = Epi::kStaged;
    static_assert(!STAGED || NW * 16 * 256 <= STAGE_BYTES, "epilogue staging fits in one slot");
    constexpr bool PAIRED = Epi::kPaired;
    static_assert(!PAIRED || (STAGED && TN % 2 == 0), "pairs are whole per wave");
    constexpr int OUT_TN = PAIRED ? TN / 2 : TN;
    constexpr int WN_OUT = 16 * OUT_TN, BN_OUT = WN_OUT * WGN;
    // a tile's epilogue operands in LDS: BM row scales, then NCV x BN_OUT
    // column values; two buffers (the next tile's are written after this
    // tile's epilogue has read its own)
    constexpr int NCV = [] { if constexpr (STAGED) return Epi::kColVals; else return 0; }();
    constexpr int NSCALE = STAGED ? BM + NCV * BN_OUT : 0;
    constexpr int SCALE_BYTES = NSCALE * 4;
    constexpr int SPT = (NSCALE + 511) / 512;                   // operand values per thread
    // the activation table's LDS window, for an epilogue that has one
    constexpr int WIN_BYTES = has_window<Epi>() ? 2 * kWinSize : 0;
    __shared__ __attribute__((aligned(1024))) int8_t smem[RING + 2 * SCALE_BYTES + WIN_BYTES + 16];
    static_assert(RING + 2 * SCALE_BYTES + WIN_BYTES + 16 <= 160 * 1024, "LDS");
    Epi epi_w = epi;                    // the epilogue, with the window's address once filled

    const int tiles = tiles_m * tiles_n;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    const int g = wm / (WGM / 2);                               // group: the row half

    // tile origin of sequence number i: each XCD (i % 8, as blockIdx % 8)
    // takes a contiguous eighth of the tiles, walked in column bands of 8 row
    // tiles
    auto tile_origin = [&](int i, int& m0, int& n0) {
        int t = i;
        if (tiles % 8 == 0) t = (t % 8) * (tiles / 8) + t / 8;
        constexpr int GROUP = 8;
        const int band = t / (GROUP * tiles_n);
        const int first_m = band * GROUP;
        const int gm = min(tiles_m - first_m, GROUP);
        const int in_band = t - band * GROUP * tiles_n;
        m0 = (first_m + in_band % gm) * BM;
        n0 = (in_band / gm) * BN_OUT;
    };

    const int KT = (K + BK - 1) / BK;
    // DMA: wave w brings blocks w, w + NW, ... of every step; lane l row l/4,
    // chunk swz(l/4, l%4).  Rows past M or N repeat the last row (their
    // results are never stored).  The 32-bit offsets keep the saddr form.
    const int8_t* base[PER];
    int off[PER];
    // K offset of this lane's 16-byte chunk, for the zero fill past K
    const int lc_tail = KTAIL ? swz(lane >> 2, lane & 3) * 16 : 0;
    auto setup = [&](int m0, int n0) {
        // the lane index is formed afresh here (an asm the compiler cannot
        // merge with the kernel's other lane values), so nothing per-lane has
        // to stay live across the K loops for the next tile's setup
        int ln;
        asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
        const int lr = ln >> 2;
        const int lc = swz(lr, ln & 3) * 16;
        const int8_t* const xbase = X + int64_t(m0) * ldx;
        const int8_t* const wbase = W + int64_t(n0) * ldw;
        const int8_t* const gbase = W + (int64_t(pair_offset(epi)) + n0) * ldw;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int j = min(wave + NW * i, NB - 1);
            if (j < XB) {
                if constexpr (XT) {
                    // block (m0 / 16 + j) of 16 rows (the last one for row
                    // groups past M); lane l takes its bytes 16l .. 16l + 15
                    const int rg = min(m0 / 16 + j, (M + 15) / 16 - 1);
                    base[i] = X + int64_t(rg) * KT * 1024;
                    off[i] = ln * 16;
                } else {
                    base[i] = xbase;
                    off[i] = (min(m0 + 16 * j + lr, M - 1) - m0) * int(ldx) + lc;
                }
            } else if constexpr (WT) {
                // a block of the packed weight: rows n0 + 16 jb.. (the last
                // block for blocks past N), or for pairs the value (even jw)
                // or gate (odd jw) rows of pair jw / 2
                const int jw = j - XB;
                const int jb = PAIRED ? jw >> 1 : jw;
                const int nb = min(n0 / 16 + jb, (N - 1) / 16);
                const int pb = (PAIRED && (jw & 1)) ? pair_offset(epi) / 16 : 0;
                base[i] = W + int64_t(pb + nb) * KT * 1024;
                off[i] = ln * 16;
            } else if constexpr (PAIRED) {
                const int jw = j - XB;
                base[i] = (jw & 1) ? gbase : wbase;
                off[i] = (min(n0 + 16 * (jw >> 1) + lr, N - 1) - n0) * int(ldw) + lc;
            } else {
                base[i] = wbase;
                off[i] = (min(n0 + 16 * (j - XB) + lr, N - 1) - n0) * int(ldw) + lc;
            }
        }
    };
    // The ring runs on across tiles: a block's steps are numbered on from
    // tile to tile, and step kk of the current tile (whose first step has
    // number kb) lives in slot (kb + kk + 1) % S; ring0 = kb % S.
    int ring0 = 0;
    auto slot = [&](int kk) { return ((ring0 + kk + 1) & (S - 1)) * STAGE_BYTES; };
    // this wave's loads for ring position kk (its share of the stage's
    // blocks), from K offset kstep * BK of the tile set up last
    auto issue_at = [&](int kk, int kstep) {
        const int k0 = kstep * BK;
        int8_t* const st = smem + slot(kk);
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            if (i == PER - 1 && REM != 0 && g != 0) continue;
            const int8_t* p;
            if ((XT && wave + NW * i < XB) || (WT && wave + NW * i >= XB)) {
                // a tiled block: K step kstep is the row group's kstep-th
                // KB; bytes past K in a tiled X block meet zeros of W (the
                // packed weight's are zeros)
                p = base[i] + uint64_t(uint32_t(off[i] + kstep * 1024));
            } else {
                p = base[i] + uint64_t(uint32_t(off[i] + k0));
                if (KTAIL && k0 + lc_tail >= K) p = g_zero16;
            }
            dma16(p, st + (wave + NW * i) * 1024);
        }
    };
    auto issue = [&](int kk) { issue_at(kk, kk); };
    // wait until this wave's loads of every step before `later` more of its
    // own load batches are complete
    auto wait_batches = [&](int later) {
        if (g == 0) {
            if (later >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * PER0));
            else if (later == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(PER0));
            else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        } else {
            if (later >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * PER1));
            else if (later == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(PER1));
            else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        }
    };

    // the epilogue operands of a tile: global loads into registers (issued
    // early), written to LDS buffer `buf` once they have landed
    float sv[SPT > 0 ? SPT : 1];
    auto fetch_scales = [&](int m0, int n0) {
        if constexpr (STAGED) {
#pragma unroll
            for (int i = 0; i < SPT; ++i) {
                const int idx = threadIdx.x + 512 * i;
                float v = 0.f;
                if (idx < BM) {
                    v = epi.row(min(m0 + idx, M - 1));
                } else if (idx < NSCALE) {
                    const int c = idx - BM, which = c / BN_OUT, nl = c - which * BN_OUT;
                    v = epi.col_value(which, min(n0 + nl, N - 1));
                }
                sv[i] = v;
            }
        }
    };
    auto put_scales = [&](int buf) {
        if constexpr (STAGED) {
            float* d = reinterpret_cast<float*>(smem + RING + buf * SCALE_BYTES);
#pragma unroll
            for (int i = 0; i < SPT; ++i) {
                const int idx = threadIdx.x + 512 * i;
                if (idx < NSCALE) d[idx] = sv[i];
            }
        }
    };

    const int frag = (lane & 15) * 64 + swz(lane & 15, lane >> 4) * 16;
    const int xoff = (wm * TM) * 1024 + frag;
    const int woff = (XB + wn * TN) * 1024 + frag;
    const uint32_t sbase = lds_addr(smem);

    v4i acc[TN][TM];
    v4i wf[TN], xf[TM];
    auto read_frags = [&](int kk) {
        const uint32_t sb = sbase + slot(kk);
        lds_read_frags<TN>(wf, sb + woff);
        lds_read_frags<TM>(xf, sb + xoff);
    };
    auto compute = [&]() {
        lgkm_wait_all(wf, xf);                                  // fragments in
#pragma unroll
        for (int b = 0; b < TM; ++b)
#pragma unroll
            for (int a = 0; a < TN; ++a)
                acc[a][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[a], xf[b], acc[a][b], 0, 0, 0);
    };
    auto barrier = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };
    auto epilogue = [&](int m0, int n0, int buf) {
        if constexpr (STAGED) {
            const float* sc = reinterpret_cast<const float*>(smem + RING + buf * SCALE_BYTES);
            const float* xr = sc + wm * WM + (lane & 15);
            typename Epi::Col ccol[TN];
#pragma unroll
            for (int a = 0; a < TN; ++a) {
                if constexpr (PAIRED)
                    ccol[a] = epi.col_lds(sc + BM, BN_OUT,
                                          wn * WN_OUT + 16 * (a >> 1) + 4 * (lane >> 4), a & 1);
                else
                    ccol[a] = epi.col_lds(sc + BM, BN_OUT, wn * WN_OUT + 16 * a + 4 * (lane >> 4), 0);
            }
            // staged through the slot of the tile's last step (the other
            // three hold the next tile's first steps)
            staged_store<TM, TN, WN_OUT, Epi, 1>(epi_w, acc, [&](int b) { return xr[16 * b]; }, ccol,
                                                 smem + slot(KT - 1) + wave * (16 * 256),
                                                 m0 + wm * WM, n0 + wn * WN_OUT, M, N, lane);
        } else {
            const int mrow = m0 + wm * WM + (lane & 15);
            const int ncol = n0 + wn * WN + 4 * (lane >> 4);
#pragma unroll
            for (int b = 0; b < TM; ++b) {
                const int m = mrow + 16 * b;
                if (m >= M) continue;
#pragma unroll
                for (int a = 0; a < TN; ++a) {
                    const int n = ncol + 16 * a;
                    if (n < N) epi(m, n, acc[a][b]);
                }
            }
        }
    };

    int ti = blockIdx.x;
    if (ti >= tiles) return;
    if constexpr (WIN_BYTES > 0) {
        // the window, read once per block (visible after the first barrier)
        uint16_t* w = reinterpret_cast<uint16_t*>(smem + RING + 2 * SCALE_BYTES);
        const uint16_t* t = epi.tab + size_t(Epi::kWinTab) * kTabSize;
        for (int i = threadIdx.x; i < kWinSize; i += 512) w[i] = t[win_bits(i)];
        epi_w.win = lds_addr(w);
    }
    int m0, n0;
    tile_origin(ti, m0, n0);
    setup(m0, n0);
    // first tile: its operands, steps 0 .. S-2 requested, step 0 complete
    fetch_scales(m0, n0);
    for (int kk = 0; kk < S - 1; ++kk)
        if (kk < KT) issue(kk);
    wait_batches(min(S - 2, KT - 1));
    put_scales(0);
    barrier();
    for (int it = 0;; ++it) {
#pragma unroll
        for (int a = 0; a < TN; ++a)
#pragma unroll
            for (int b = 0; b < TM; ++b) acc[a][b] = v4i{0, 0, 0, 0};
        const int tnext = ti + int(gridDim.x);
        const bool more = tnext < tiles;
        int m0n = 0, n0n = 0;
        if (more) tile_origin(tnext, m0n, n0n);
        // With a next tile (and K steps enough), the loads of its steps 0-2
        // go out in this tile's last three steps, in the ring positions where
        // steps KT..KT+2 would go: the loop's loads never stop at the tile
        // boundary.  Every wait then has the usual number of later batches.
        const bool cont = more && KT >= S - 1;
        // the loop runs in two parts: steps 0 .. KT-S (this tile's loads, as
        // long as there are any) and, with cont, steps KT-S+1 .. KT-1 (the next
        // tile's loads, after setup() has switched the load addresses), so no
        // branch on the tile boundary sits inside either loop
        const int kmain = cont ? KT - (S - 1) : KT;
        // group 0 reads step 0's fragments; each group then runs its own loop
        // of (first half, barrier, second half, barrier), group 0 a half step
        // ahead
        if (g == 0) {
            read_frags(0);
            barrier();
#pragma clang loop unroll(disable)
            for (int k = 0; k < kmain; ++k) {
                compute();                                      // A(k)
                if (k + 1 < KT) wait_batches(min(S - 3, KT - 2 - k));
                barrier();
                if (k + 1 < KT) read_frags(k + 1);              // B(k)
                if (k + S - 1 < KT) issue(k + S - 1);
                barrier();
            }
            if (cont) {
                setup(m0n, n0n);
#pragma clang loop unroll(disable)
                for (int k = kmain; k < KT; ++k) {
                    compute();                                  // A(k)
                    if (k + 1 < KT) wait_batches(S - 3);
                    barrier();
                    if (k + 1 < KT) read_frags(k + 1);          // B(k)
                    issue_at(k + S - 1, k + S - 1 - KT);
                    barrier();
                }
            }
        } else {
            barrier();
#pragma clang loop unroll(disable)
            for (int k = 0; k < kmain; ++k) {
                read_frags(k);                                  // A(k)
                if (k + S - 1 < KT) issue(k + S - 1);
                if (k + 1 < KT) wait_batches(min(S - 2, KT - 2 - k));
                barrier();
                compute();                                      // B(k)
                barrier();
            }
            if (cont) {
                setup(m0n, n0n);
#pragma clang loop unroll(disable)
                for (int k = kmain; k < KT; ++k) {
                    read_frags(k);                              // A(k)
                    issue_at(k + S - 1, k + S - 1 - KT);
                    if (k + 1 < KT) wait_batches(S - 2);
                    barrier();
                    compute();                                  // B(k)
                    barrier();
                }
            }
        }
        // every fragment read has completed: the next tile's operands (and,
        // with too few K steps for the loop to have issued them, its first
        // steps) go out ahead of this tile's stores
        if (more) {
            if (!cont) {
                setup(m0n, n0n);
                for (int kk = 0; kk < S - 1; ++kk)
                    if (kk < KT) issue_at(KT + kk, kk);
            }
            fetch_scales(m0n, n0n);
        }
        epilogue(m0, n0, it & 1);
        if (!more) break;
        __builtin_amdgcn_s_waitcnt(0);                          // stores, loads, LDS all done
        put_scales((it + 1) & 1);
        barrier();
        ring0 = (ring0 + KT) & (S - 1);
        ti = tnext;
        m0 = m0n;
        n0 = n0n;
    }
}

// ------------------------------------------------------------ split K
// Narrow outputs with a long K (the FFN's down-projection, dx: N = 1280,
// K = 5120) give too few large tiles to fill the chip.  Here a 128 x 160
// tile belongs to a block of 8 waves in two teams of 4 (team = wave / 4, 2 x 2
// waves of 64 x 80 each): team 0 owns the first half of the K steps and team
// 1 the second, each through its own ring of S LDS stages.  The teams
// alternate between MFMAs and data movement every half step, so that on each
// SIMD one wave feeds the matrix core while the other moves data:
//   A(s): team 0 runs its step s;  team 1 reads its step s's fragments and
//         issues its loads for step s + S - 1
//   B(s): team 1 runs its step s;  team 0 reads its step s + 1's fragments
//         and issues its loads for step s + S - 1
// with one s_barrier between phases.  A team's step is complete (each wave
// waits for its own loads, then the barrier) before the phase that reads it;
// its stage is refilled only after the phase that consumed it.  The teams'
// partial sums then meet in LDS (exact int32 sums): with a dequant epilogue
// each team finishes half of the tile's rows and both run the epilogue; K
// slices hand team 1's sums to team 0, which stores the int32 slice.
template <int S, bool KTAIL, bool WNN, class Epi, bool XT = false, bool WT = false>
__global__ __launch_bounds__(512, 1) void gemm_i8_splitk_kernel(
    const int8_t* __restrict__ X, int64_t ldx, const int8_t* __restrict__ W, int64_t ldw, int M,
    int N, int K, int tiles_m, int tiles_n, Epi epi) {
    constexpr int BM = 128, BN = 160, BK = 64;
    constexpr int TM = 4, TN = 5, WM = 64, WN = 80;
    constexpr int XB = BM / 16, WB = BN / 16, NB = XB + WB;     // 18 blocks of 1 KB per stage
    constexpr int PER = (NB + 3) / 4, REM = NB % 4;
    constexpr int STAGE_BYTES = NB * 1024, RING = S * STAGE_BYTES;
    constexpr bool SLICE = IsSliceEpi<Epi>::value;
    static_assert(!Epi::kPaired && (Epi::kStaged || SLICE), "dequant or slice epilogues only");
    static_assert(!SLICE || !XT, "K slices of a row-major X");
    static_assert(!WT || !SLICE, "the packed weights: whole-K products");
    static_assert(2 * RING >= 4 * TN * (TM / 2) * 1024, "half of a team's accumulators fit");
    // K slice blockIdx.y of a split across blocks: K is the slice's length and
    // the operands' rows keep their full strides
    if constexpr (SLICE) {
        X += int64_t(blockIdx.y) * K;
        W += WNN ? int64_t(blockIdx.y) * K * ldw : int64_t(blockIdx.y) * K;
    }
    static_assert(S >= 3 && S <= 4, "three or four stages");
    __shared__ __attribute__((aligned(1024))) int8_t smem[2 * RING];

    // Blocks are dispatched to the 8 XCDs round robin (block b on b % 8),
    // each with its own L2: give every XCD a gx x (8 / gx) block of the tile
    // grid, with gx chosen so that it reads the fewest operand rows (at the
    // FFN's down-projection, 32 x 8 tiles: 8 x 4 tiles per XCD, X and W read
    // 4 and 2 times over instead of X 8 times).
    int tmi = blockIdx.x % tiles_m, tni = blockIdx.x / tiles_m;
    {
        int best = 0, cost = 0;
        for (int gx = 1; gx <= 8; gx *= 2) {
            const int gy = 8 / gx;
            if (tiles_m % gx || tiles_n % gy) continue;
            const int c = (tiles_m / gx) * BM + (tiles_n / gy) * BN;
            if (!best || c < cost) best = gx, cost = c;
        }
        if (best) {
            const int x = blockIdx.x % 8, j = blockIdx.x / 8;
            const int lm = tiles_m / best;                      // row tiles per XCD
            const int ln = tiles_n / (8 / best);
            tmi = (x % best) * lm + j % lm;
            tni = (x / best) * ln + j / lm;
        }
    }
    const int m0 = tmi * BM, n0 = tni * BN;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int team = wave >> 2, wt = wave & 3;
    const int wm = wt >> 1, wn = wt & 1;
    int8_t* ring = smem + team * RING;

    const int KT = (K + BK - 1) / BK, KH = (KT + 1) / 2;      // team 0 takes the first KH
    const int kt0 = team * KH, nst = min(KT, kt0 + KH) - kt0; // this team's steps

    const int lr = lane >> 2;
    const int lc = swz(lr, lane & 3) * 16;
    const int8_t* const xbase = X + int64_t(m0) * ldx;
    // The weight is W[n, k] (NT: row n, K-contiguous) or, with WNN, W[k, n]
    // (row k of the contraction, n contiguous: the NN product's right operand
    // as stored).  An NN stage holds the step's 64 contraction rows x 160
    // columns as 10 blocks of 32 rows x 32 bytes, block 5*rb + cg for rows
    // 32rb.. and columns 32cg..; row r of a block is 32 bytes at 32r, its two
    // 16-byte halves swapped when r & 16 (so that the transposing fragment
    // reads of rows r and r + 16 fall on different banks).  DMA lane l fills
    // row l/2, stored half l%2.  With WT the weight comes packed in that
    // stage order (pack_weight_nn: block (s, n/32, rb) the 1 KB at
    // ((s * N/32 + n/32) * 2 + rb) * 1024, zeros past K), one contiguous load
    // per block instead of 32 quarter lines; N % 32 == 0.
    const int8_t* const wbase = WNN ? W + n0 : W + int64_t(n0) * ldw;
    const int8_t* base[PER];
    int off[PER];
    int krow[PER];                     // WNN: the lane's contraction row within a step
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int j = min(wt + 4 * i, NB - 1);
        krow[i] = 0;
        if (j < XB && XT) {
            // X in the MFMA block layout: row block m0/16 + j (the last one
            // for blocks past M), one contiguous 1 KB per step
            const int mb = min(m0 / 16 + j, (M + 15) / 16 - 1);
            base[i] = X + int64_t(mb) * ((K + BK - 1) / BK) * 1024;
            off[i] = 16 * lane;
        } else if (j < XB) {
            base[i] = xbase;
            off[i] = (min(m0 + 16 * j + lr, M - 1) - m0) * int(ldx) + lc;
        } else if constexpr (WNN) {
            const int jj = j - XB, rb = jj / 5, cg = jj - 5 * rb;
            const int kr = lane >> 1, half = (lane & 1) ^ ((kr >> 4) & 1);
            krow[i] = 32 * rb + kr;
            if constexpr (WT) {
                base[i] = W + int64_t(min(n0 / 32 + cg, N / 32 - 1) * 2 + rb) * 1024;
                off[i] = 16 * lane;
            } else {
                base[i] = wbase;
                off[i] = krow[i] * int(ldw) + min(32 * cg + 16 * half, N - n0 - 16);
            }
        } else if constexpr (WT) {
            // the packed weight's block n0/16 + (j - XB) (the last one for
            // blocks past N), one contiguous 1 KB per step
            base[i] = W + int64_t(min(n0 / 16 + (j - XB), (N - 1) / 16)) * KT * 1024;
            off[i] = 16 * lane;
        } else {
            base[i] = wbase;
            off[i] = (min(n0 + 16 * (j - XB) + lr, N - 1) - n0) * int(ldw) + lc;
        }
    }
    const bool full_share = REM == 0 || wt < REM;
    // this wave's loads for the team's step s
    auto issue = [&](int s) {
        const int k0 = (kt0 + s) * BK;
        int8_t* const st = ring + (s % S) * STAGE_BYTES;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            if (i == PER - 1 && !full_share) break;
            const int j = wt + 4 * i;
            const int8_t* p;
            if (WNN && WT && j >= XB) {
                // a packed step is N / 32 x 2 blocks (N * 64 bytes)
                p = base[i] + uint64_t(off[i]) + uint64_t(kt0 + s) * uint64_t(N) * 64;
            } else if (WNN && j >= XB) {
                p = base[i] + uint64_t(uint32_t(off[i]) + uint32_t(k0) * uint32_t(ldw));
                if (KTAIL && k0 + krow[i] >= K) p = g_zero16;
            } else if ((XT && j < XB) || (WT && j >= XB)) {
                // bytes past K in the last step are multiplied by W's zeros
                p = base[i] + uint64_t(off[i]) + uint64_t(kt0 + s) * 1024;
            } else {
                p = base[i] + uint64_t(uint32_t(off[i] + k0));
                if (KTAIL && k0 + lc >= K) p = g_zero16;
            }
            dma16(p, st + j * 1024);
        }
    };
    auto wait_batches = [&](int later) {
        if (full_share) {
            if (later >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * PER));
            else if (later == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(PER));
            else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        } else {
            if (later >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * (PER - 1)));
            else if (later == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(PER - 1));
            else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        }
    };
    const int frag = (lane & 15) * 64 + swz(lane & 15, lane >> 4) * 16;
    const int xoff = (wm * TM) * 1024 + frag;
    const int woff = (XB + wn * TN) * 1024 + frag;
    const uint32_t rbase = lds_addr(ring);
    // WNN fragments: a lane of group g = l/16 needs the 16 contraction bytes
    // 16g.. of its column (l%16 of the 16-column block), which two transposing
    // reads (ds_read_b64_tr_b8) deliver: in each 16-lane group, output lane
    // 8a + b receives byte b of the 8 bytes addressed by lanes a, a+2, ..,
    // a+14, in that order; so source lane j points at row 16(g&1) + 8h + j/2
    // of its row block, bytes 8(j&1).. of the block's column pair half.  The
    // swap of halves at r & 16 is (g & 1) here.
    uint32_t wnn_off[TN][2];
    if constexpr (WNN) {
        const int g = lane >> 4, j = lane & 15;
#pragma unroll
        for (int a = 0; a < TN; ++a) {
            const int blk = wn * TN + a, cg = blk >> 1;
            const int half = (blk & 1) ^ (g & 1);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int kr = 16 * (g & 1) + 8 * h + (j >> 1);
                wnn_off[a][h] = uint32_t((XB + 5 * (g >> 1) + cg) * 1024 + kr * 32 + half * 16 +
                                         8 * (j & 1));
            }
        }
    }

    v4i acc[TN][TM];
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
        for (int b = 0; b < TM; ++b) acc[a][b] = v4i{0, 0, 0, 0};
    v4i wf[TN], xf[TM];
    auto read_frags = [&](int s) {
        const uint32_t sb = rbase + (s % S) * STAGE_BYTES;
        if constexpr (WNN) {
#pragma unroll
            for (int i = 0; i < TN; ++i) {
                const v2i lo = lds_read8_tr(sb + wnn_off[i][0]);
                const v2i hi = lds_read8_tr(sb + wnn_off[i][1]);
                wf[i] = v4i{lo.x, lo.y, hi.x, hi.y};
            }
        } else {
#pragma unroll
            for (int i = 0; i < TN; ++i) wf[i] = lds_read16(sb + woff + i * 1024);
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) xf[i] = lds_read16(sb + xoff + i * 1024);
    };
    auto compute = [&]() {
        lgkm_wait_all(wf, xf);                                  // fragments in
#pragma unroll
        for (int b = 0; b < TM; ++b)
#pragma unroll
            for (int a = 0; a < TN; ++a)
                acc[a][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[a], xf[b], acc[a][b], 0, 0, 0);
    };
    auto barrier = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };

    // The epilogue's row and column operands (this team's half of the wave's
    // rows, all of its columns), loaded before the operands so that their
    // latency is paid under the main loop.
    constexpr int H = TM / 2;
    float xrow[H];
    typename std::conditional_t<SLICE, EpiDequant, Epi>::Col ccol[TN];
    if constexpr (!SLICE) {
        const int mh = m0 + wm * WM + (team == 0 ? 0 : 16 * H);
#pragma unroll
        for (int b = 0; b < H; ++b) xrow[b] = epi.row(min(mh + 16 * b + (lane & 15), M - 1));
#pragma unroll
        for (int a = 0; a < TN; ++a)
            ccol[a] = epi.col(min(n0 + wn * WN + 16 * a + 4 * (lane >> 4), N - 4));
    }

    for (int s = 0; s < S - 1; ++s)
        if (s < nst) issue(s);
    if (nst > 0) wait_batches(min(S - 2, nst - 1));
    barrier();
    if (team == 0) {
        if (nst > 0) read_frags(0);
        barrier();
#pragma clang loop unroll(disable)
        for (int s = 0; s < KH; ++s) {
            if (s < nst) compute();                             // A(s)
            if (s + 1 < nst) wait_batches(min(S - 3, nst - 2 - s));
            barrier();
            if (s + 1 < nst) read_frags(s + 1);                 // B(s)
            if (s + S - 1 < nst) issue(s + S - 1);
            barrier();
        }
    } else {
        barrier();
#pragma clang loop unroll(disable)
        for (int s = 0; s < KH; ++s) {
            if (s < nst) read_frags(s);                         // A(s)
            if (s + S - 1 < nst) issue(s + S - 1);
            barrier();
            if (s < nst) compute();                             // B(s)
            if (s + 1 < nst) wait_batches(min(S - 2, nst - 2 - s));
            barrier();
        }
    }

    v4i* xchg = reinterpret_cast<v4i*>(smem);
    if constexpr (!SLICE) {
        // The two teams' partial sums meet in LDS, and each team finishes half
        // of the tile: team 0 the wave's row blocks [0, H), team 1 [H, TM).
        // Each wave hands the other half to its partner (same wt, other team)
        // and adds the partner's half of its own; then all 8 waves run the
        // epilogue (staging areas past the hand-over area).
        static_assert(8 * TN * H * 1024 + 8 * 32 * 256 <= 2 * RING, "hand-over and staging fit");
        __syncthreads();                                    // the ring's last reads are done
        v4i mine[TN][H];
        if (team == 0) {
#pragma unroll
            for (int a = 0; a < TN; ++a)
#pragma unroll
                for (int bb = 0; bb < H; ++bb) {
                    xchg[((wave * TN + a) * H + bb) * 64 + lane] = acc[a][H + bb];
                    mine[a][bb] = acc[a][bb];
                }
        } else {
#pragma unroll
            for (int a = 0; a < TN; ++a)
#pragma unroll
                for (int bb = 0; bb < H; ++bb) {
                    xchg[((wave * TN + a) * H + bb) * 64 + lane] = acc[a][bb];
                    mine[a][bb] = acc[a][H + bb];
                }
        }
        __syncthreads();
        const int pw = wave ^ 4;
#pragma unroll
        for (int a = 0; a < TN; ++a)
#pragma unroll
            for (int bb = 0; bb < H; ++bb) mine[a][bb] += xchg[((pw * TN + a) * H + bb) * 64 + lane];
        staged_store<H, TN, WN, Epi, 2>(epi, mine, [&](int b) { return xrow[b]; }, ccol,
                                        smem + 8 * TN * H * 1024 + wave * (32 * 256),
                                        m0 + wm * WM + (team == 0 ? 0 : 16 * H), n0 + wn * WN, M,
                                        N, lane);
        return;
    }
    // K slices: team 1 -> team 0 through LDS, TM/2 rows of blocks at a time
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        __syncthreads();
        if (team == 1) {
#pragma unroll
            for (int a = 0; a < TN; ++a)
#pragma unroll
                for (int bb = 0; bb < TM / 2; ++bb)
                    xchg[((wt * TN + a) * (TM / 2) + bb) * 64 + lane] = acc[a][h * (TM / 2) + bb];
        }
        __syncthreads();
        if (team == 0) {
#pragma unroll
            for (int a = 0; a < TN; ++a)
#pragma unroll
                for (int bb = 0; bb < TM / 2; ++bb)
                    acc[a][h * (TM / 2) + bb] += xchg[((wt * TN + a) * (TM / 2) + bb) * 64 + lane];
        }
    }
    __syncthreads();
    if constexpr (SLICE) {
        // lane l of block (a, b): row m0 + wm*WM + 16b + l%16, columns n .. n+3
        // with n = n0 + wn*WN + 16a + 4*(l/16)
        if (team == 0) {
#pragma unroll
            for (int b = 0; b < TM; ++b) {
                const int m = m0 + wm * WM + 16 * b + (lane & 15);
#pragma unroll
                for (int a = 0; a < TN; ++a) {
                    const int n = n0 + wn * WN + 16 * a + 4 * (lane >> 4);
                    if (m < M && n < N) epi(m, n, acc[a][b]);
                }
            }
        }
    }
}

template <bool WNN = false, class Epi, bool XT = false, bool WT = false>
hipError_t launch_splitk(hipStream_t st, const int8_t* X, int64_t ldx, const int8_t* W,
                         int64_t ldw, int M, int N, int K, const Epi& epi) {
    constexpr int S = 4;                        // 2 x 4 x 18 KB of LDS
    const int tm = (M + 127) / 128, tn = (N + 159) / 160;
    if (K % 64 == 0)
        hipLaunchKernelGGL((gemm_i8_splitk_kernel<S, false, WNN, Epi, XT, WT>),
                           dim3(unsigned(tm * tn)), dim3(512), 0, st, X, ldx, W, ldw, M, N, K, tm,
                           tn, epi);
    else
        hipLaunchKernelGGL((gemm_i8_splitk_kernel<S, true, WNN, Epi, XT, WT>),
                           dim3(unsigned(tm * tn)), dim3(512), 0, st, X, ldx, W, ldw, M, N, K, tm,
                           tn, epi);
    return hipGetLastError();
}


// ------------------------------------------------------------ skinny M
// M <= 64: the product streams the weight once, so it is bound by HBM
// bandwidth, and tiles of 128+ rows would leave most CUs idle.  A block owns 16
// weight rows (one MFMA row block) and all MB 16-row blocks of X; its NW waves
// take every NW-th 64-byte K step and keep their operands in registers, loaded
// straight from global memory in the MFMA layout (lane l: row l%16, bytes
// 16*(l/16) of the step) D steps ahead.  With NW = 16 a block requests its
// whole 64 KB weight slice (K = 4096) at once, one block per CU: the weight is
// streamed at the HBM rate instead of at the latency of a few steps in flight
// per wave.  The NW partial accumulators meet in LDS; the epilogue is the
// per-block form of the same Epi.  NW follows the number of K steps (about
// four per wave): at M=16, N=4096 and K=4096 sixteen waves cut the cold call
// from 8.7 to 7.2 us, while at K=1280 four waves stay fastest (6.8 us against
// 7.7 with eight and 8.6 with sixteen).  A paired epilogue (the FFN's
// up-projection) takes the same kernel with the rows n and half + n of each
// output column block in the block, so that both operands of its activation
// meet in one lane: two column blocks (four weight blocks) per block, which
// at ffn = 5120, K = 1280 took 6.0 / 9.4 / 13.5 us cold at M = 1 / 64 / 128
// against 6.3 / 11.2 / 16.5 with one (every block reads all of X, so fewer,
// wider blocks read less of it).
// WT: the weight packed (pack_weight), each lane's 16 bytes of a step read
// from its block's contiguous 1 KB (chunk c of row r at (c ^ ((r >> 1) & 3)) *
// 16), so one load instruction covers whole cache lines: 7.3 -> 6.2 us cold at
// M = 16, N = K = 4096 (timing-only build of the pattern).  XT: X in the MFMA
// block layout (tiled_offset) the same way.
template <int MB, int NW, int NB, class Epi, bool WT = false, bool XT = false>
__global__ __launch_bounds__(NW * 64) void gemm_i8_skinny_kernel(
    const int8_t* __restrict__ X, int64_t ldx, const int8_t* __restrict__ W, int64_t ldw, int M,
    int N, int K, Epi epi) {
    // NB weight blocks of 16 rows per block: rows n0 + 16p, or, for a paired
    // epilogue (an FFN's up-projection), NB / 2 column blocks of both halves:
    // rows n0 + 16c (p = c) and half + n0 + 16c (p = NB/2 + c), the operands of
    // the activation at output columns n0 + 16c
    constexpr bool PAIRED = Epi::kPaired;
    constexpr int NC = PAIRED ? NB / 2 : NB;                 // output column blocks
    static_assert(!PAIRED || NB % 2 == 0, "a paired epilogue takes both halves of each block");
    static_assert(NW * NB * MB <= 160, "the partial sums fit in the CU's 160 KB of LDS");
    static_assert(!WT || !IsSliceEpi<Epi>::value, "the packed weight: whole-K products");
    static_assert(!XT || !IsSliceEpi<Epi>::value, "x in the block layout: whole-K products");
    constexpr int D = NW >= 16 ? 4 : (MB * NB <= 2 ? 8 : (MB * NB <= 8 ? 4 : 2));  // steps in flight
    __shared__ v4i part[NW][NB * MB][64];
    // K slice blockIdx.y of a split across blocks (EpiSliceI32): K is the
    // slice's length, the operands' rows keep their full strides.  Otherwise
    // blockIdx.y is a chunk of 16 * MB rows (batches above 128 rows)
    int m_base = 0;
    if constexpr (IsSliceEpi<Epi>::value) {
        X += int64_t(blockIdx.y) * K;
        W += int64_t(blockIdx.y) * K;
    } else {
        m_base = int(blockIdx.y) * 16 * MB;
        if constexpr (!XT) X += int64_t(m_base) * ldx;
        M -= m_base;
    }
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n0 = blockIdx.x * 16 * NC;
    const int kb = 16 * (lane >> 4);                         // lane's bytes within a step
    const int8_t* wrow[NB];
#pragma unroll
    for (int p = 0; p < NB; ++p) {
        if constexpr (WT) {
            // block n/16 of the packed weight (the last one past N), or the
            // gate half's pair_offset/16 further; this lane's chunk in it
            const int nb = min(n0 / 16 + (p % NC), (N - 1) / 16) +
                           (p >= NC ? pair_offset(epi) / 16 : 0);
            const int r = lane & 15;
            wrow[p] = W + int64_t(nb) * ((K + 63) / 64) * 1024 + r * 64 +
                      ((((lane >> 4) ^ (r >> 1)) & 3) << 4);
        } else {
            const int r = min(n0 + 16 * (p % NC) + (lane & 15), N - 1) +
                          (p >= NC ? pair_offset(epi) : 0);
            wrow[p] = W + int64_t(r) * ldw + kb;
        }
    }
    const int8_t* xrow[MB];
#pragma unroll
    for (int b = 0; b < MB; ++b) {
        if constexpr (XT) {
            // the block of rows m_base + 16b (the last one past M): its rows
            // past M hold whatever the quantizer left, read into outputs the
            // epilogue never stores
            const int r = lane & 15;
            xrow[b] = X + (int64_t(m_base / 16 + min(b, (M - 1) / 16)) * ((K + 63) / 64)) * 1024 +
                      r * 64 + ((((lane >> 4) ^ (r >> 1)) & 3) << 4);
        } else {
            xrow[b] = X + int64_t(min(16 * b + (lane & 15), M - 1)) * ldx + kb;
        }
    }
    const int S = (K + 63) / 64;                             // K steps
    // the wave's t-th step (pairing consecutive steps in one wave, so it reads
    // both halves of a 128-byte row segment back to back, measured slower)
    auto stepidx = [&](int t) { return wave + NW * t; };
    v4i wbuf[D][NB], xbuf[D][MB];
    auto load = [&](int slot, int step) {
        const int k = step * 64;
        if (step < S && k + kb < K) {
#pragma unroll
            for (int p = 0; p < NB; ++p)
                wbuf[slot][p] = *reinterpret_cast<const v4i*>(wrow[p] + (WT ? int64_t(step) * 1024 : k));
#pragma unroll
            for (int b = 0; b < MB; ++b)
                xbuf[slot][b] = *reinterpret_cast<const v4i*>(xrow[b] + (XT ? int64_t(step) * 1024 : k));
        } else {
#pragma unroll
            for (int p = 0; p < NB; ++p) wbuf[slot][p] = v4i{0, 0, 0, 0};
#pragma unroll
            for (int b = 0; b < MB; ++b) xbuf[slot][b] = v4i{0, 0, 0, 0};
        }
    };
    v4i acc[NB][MB];
#pragma unroll
    for (int p = 0; p < NB; ++p)
#pragma unroll
        for (int b = 0; b < MB; ++b) acc[p][b] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < D; ++j) load(j, stepidx(j));
    for (int s0 = 0; stepidx(s0) < S; s0 += D) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
#pragma unroll
            for (int p = 0; p < NB; ++p)
#pragma unroll
                for (int b = 0; b < MB; ++b)
                    acc[p][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wbuf[j][p], xbuf[j][b],
                                                                      acc[p][b], 0, 0, 0);
            load(j, stepidx(s0 + j + D));
        }
    }
#pragma unroll
    for (int p = 0; p < NB; ++p)
#pragma unroll
        for (int b = 0; b < MB; ++b) part[wave][p * MB + b][lane] = acc[p][b];
    __syncthreads();
    // lane l holds rows 4*(l/16)+i of a weight block (n) for x row l%16 (m)
    if constexpr (PAIRED) {
        // wave w finishes (column block, m-block) pairs w, w+NW, ...: both
        // halves in one lane
        for (int t = wave; t < NC * MB; t += NW) {
            v4i v = part[0][t][lane], v2 = part[0][NC * MB + t][lane];
#pragma unroll
            for (int w = 1; w < NW; ++w) {
                v += part[w][t][lane];
                v2 += part[w][NC * MB + t][lane];
            }
            const int m = 16 * (t % MB) + (lane & 15);
            const int n = n0 + 16 * (t / MB) + 4 * (lane >> 4);
            if (m < M && n < N) epi.pair(m_base + m, n, v, v2);
        }
    } else {
        // wave w finishes (weight block, m-block) pairs w, w+NW, ...
        for (int t = wave; t < NB * MB; t += NW) {
            v4i v = part[0][t][lane];
#pragma unroll
            for (int w = 1; w < NW; ++w) v += part[w][t][lane];
            const int m = 16 * (t % MB) + (lane & 15);
            const int n = n0 + 16 * (t / MB) + 4 * (lane >> 4);
            if (m < M && n < N) epi(m_base + m, n, v);
        }
    }
}

// The skinny kernel over a (ceil(N / 16NB), nsl) grid (nsl > 1: K slices of
// an EpiSliceI32, K being the slice's length) with NW waves by the number of
// K steps.  M <= 64 for any epilogue; up to 128 (8 m-blocks) for a paired or
// slice epilogue; a paired epilogue above 128 rows over a (ceil(N / 8NB),
// ceil(M / 128)) grid of 128-row chunks.
template <int NB, class Epi, bool WT = false, bool XT = false>
hipError_t launch_skinny(hipStream_t st, const int8_t* X, int64_t ldx, const int8_t* W,
                         int64_t ldw, int M, int N, int K, const Epi& epi, int nsl = 1) {
    constexpr bool kWide = Epi::kPaired || IsSliceEpi<Epi>::value;
    const int cols = Epi::kPaired ? 8 * NB : 16 * NB;
    const int chunks = Epi::kPaired && M > 128 ? (M + 127) / 128 : 1;
    const dim3 grid(unsigned((N + cols - 1) / cols), unsigned(chunks > 1 ? chunks : nsl));
    const int mrows = chunks > 1 ? 128 : M;     // rows per block (the last chunk ragged)
    const int S = (K + 63) / 64;
    auto go = [&](auto NWc) {
        constexpr int NWV = decltype(NWc)::value;
        const dim3 block(NWV * 64);
#define XPU_SKINNY(MBV)                                                                         \
    hipLaunchKernelGGL((gemm_i8_skinny_kernel<MBV, NWV, NB, Epi, WT, XT>), grid, block, 0, st, X, \
                       ldx, W, ldw, M, N, K, epi)
        switch ((mrows + 15) / 16) {
            case 1: XPU_SKINNY(1); break;
            case 2: XPU_SKINNY(2); break;
            case 3: XPU_SKINNY(3); break;
            case 4: XPU_SKINNY(4); break;
            default:
                if constexpr (kWide) {
                    switch ((mrows + 15) / 16) {
                        case 5: XPU_SKINNY(5); break;
                        case 6: XPU_SKINNY(6); break;
                        case 7: XPU_SKINNY(7); break;
                        default: XPU_SKINNY(8); break;
                    }
                } else {
                    XPU_SKINNY(4);
                }
                break;
        }
#undef XPU_SKINNY
    };
    // LDS for the partial sums is NW x NB*MB x 1 KB: 16 waves for one weight
    // block and M <= 64, 8 for two weight blocks, 4 for four
    if constexpr (NB == 1 && !kWide) {
        if (S >= 64) {
            go(std::integral_constant<int, 16>{});
            return hipGetLastError();
        }
    }
    if constexpr (NB <= 2) {
        if (S >= 32) {
            go(std::integral_constant<int, 8>{});
            return hipGetLastError();
        }
    }
    go(std::integral_constant<int, 4>{});
    return hipGetLastError();
}

// Tile choice: the 256 x 320 ping-pong tile when it gives at least one tile
// per CU (8-12% faster than the two-block 256 x 160 kernel at M=4096, K=1280
// and 2560, N=5120 and 10240, interleaved A/B timing); else the large tile
// (256 x 160, 4 waves of 128 x 80, two blocks per CU, two LDS stages) when it
// gives at least 192 tiles; otherwise the small one (128 x 128, 4 waves of
// 64 x 64, four stages); M <= 64 takes the weight-streaming skinny kernel;
// a narrow output with K >= 2048 (too few large tiles) the split-K kernel.
// Paired epilogues take the skinny kernel at M <= 256 (in 128-row chunks
// above 128: at ffn = 5120, K = 1280, cold, 23.5 -> 14.4 us at M = 129 and
// 25.4 -> 22.7 us at M = 256, though 1.7 us slower warm there), else the
// ping-pong tile (as 4 x 2 waves) or the large one.
constexpr int kSkinnyPairedM = 256;

// The persistent ping-pong kernel over 256 x 320 tiles, one block per CU (X
// row-major with row stride ldx, or XT: in the MFMA block layout).
template <bool XT, bool WT = false, class Epi>
hipError_t launch_pp(hipStream_t st, const int8_t* X, int64_t ldx, const int8_t* W, int64_t ldw,
                     int M, int N, int K, const Epi& epi) {
    constexpr int WGM = Epi::kPaired ? 4 : 2, WGN = 8 / WGM;
    const int tm = (M + 255) / 256, tn = Epi::kPaired ? (N + 159) / 160 : (N + 319) / 320;
    const dim3 grid(unsigned(std::min<int64_t>(int64_t(tm) * tn, device_cus())));
    if (K % 64 == 0)
        hipLaunchKernelGGL((gemm_i8_pp_kernel<256, 320, WGM, WGN, 4, false, Epi, XT, WT>), grid,
                           dim3(512), 0, st, X, ldx, W, ldw, M, N, K, tm, tn, epi);
    else
        hipLaunchKernelGGL((gemm_i8_pp_kernel<256, 320, WGM, WGN, 4, true, Epi, XT, WT>), grid,
                           dim3(512), 0, st, X, ldx, W, ldw, M, N, K, tm, tn, epi);
    return hipGetLastError();
}

template <class Epi>
hipError_t launch_gemm(hipStream_t st, const int8_t* X, int64_t ldx, const int8_t* W, int64_t ldw,
                       int M, int N, int K, const Epi& epi, const int8_t* Wp = nullptr) {
    constexpr int BM = 256, BN = 160, STAGES = 2;
    // Wp (optional): pack_weight's copy of W, which the skinny kernel reads
    // instead of W (the other kernels here read W)
    constexpr bool kPackable = !IsSliceEpi<Epi>::value;
    if constexpr (Epi::kPaired) {
        if (M <= kSkinnyPairedM) {
            if constexpr (kPackable) {
                if (Wp) return launch_skinny<4, Epi, true>(st, X, ldx, Wp, 0, M, N, K, epi);
            }
            return launch_skinny<4>(st, X, ldx, W, ldw, M, N, K, epi);
        }
        // the ping-pong tile, 4 x 2 waves of 64 x 160 (five whole pairs each),
        // when it gives one tile per CU (5% faster at the FFN up-projection)
        const int tm = (M + BM - 1) / BM, tn_pp = (N + 159) / 160;
        if (int64_t(tm) * tn_pp >= device_cus()) {
            return launch_pp<false>(st, X, ldx, W, ldw, M, N, K, epi);
        }
        // 4 x 1 waves of 64 x 160: each wave holds five (first, second) pairs
        const int tn = (N + BN / 2 - 1) / (BN / 2);
        if (K % 64 == 0)
            hipLaunchKernelGGL((gemm_i8_big_kernel<BM, BN, 4, 1, STAGES, false, Epi>),
                               dim3(unsigned(tm * tn)), dim3(256), 0, st, X, ldx, W, ldw, M, N, K,
                               tm, tn, epi);
        else
            hipLaunchKernelGGL((gemm_i8_big_kernel<BM, BN, 4, 1, STAGES, true, Epi>),
                               dim3(unsigned(tm * tn)), dim3(256), 0, st, X, ldx, W, ldw, M, N, K,
                               tm, tn, epi);
        return hipGetLastError();
    } else {
        if (M <= 64) {
            if constexpr (kPackable) {
                if (Wp) return launch_skinny<1, Epi, true>(st, X, ldx, Wp, 0, M, N, K, epi);
            }
            return launch_skinny<1>(st, X, ldx, W, ldw, M, N, K, epi);
        }
        const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
        if constexpr (Epi::kStaged) {
            // narrow output, long K: split K inside 128 x 160 tiles instead
            if (splitk_applies(M, N, K)) return launch_splitk(st, X, ldx, W, ldw, M, N, K, epi);
        }
        // one 256 x 320 ping-pong tile per CU when they fill every CU
        const int tn_pp = (N + 319) / 320;
        if (int64_t(tm) * tn_pp >= device_cus()) {
            return launch_pp<false>(st, X, ldx, W, ldw, M, N, K, epi);
        }
        if (int64_t(tm) * tn >= 192) {
            if (K % 64 == 0)
                hipLaunchKernelGGL((gemm_i8_big_kernel<BM, BN, 2, 2, STAGES, false, Epi>),
                                   dim3(unsigned(tm * tn)), dim3(256), 0, st, X, ldx, W, ldw, M, N,
                                   K, tm, tn, epi);
            else
                hipLaunchKernelGGL((gemm_i8_big_kernel<BM, BN, 2, 2, STAGES, true, Epi>),
                                   dim3(unsigned(tm * tn)), dim3(256), 0, st, X, ldx, W, ldw, M, N,
                                   K, tm, tn, epi);
            return hipGetLastError();
        }
        return launch_cfg<128, 128, 2, 2, 4>(st, X, ldx, W, ldw, M, N, K, epi);
    }
}

// ------------------------------------------------------- standalone dequant
// A block of T threads converts 4TU columns of one row: lane t takes four
// columns at 4t + 4Tu (u < U), so each wave-wide 16-byte load covers 1 KB of
// the accumulator row without gaps and each 8-byte store 512 bytes of the
// output row.  The (row, column block) pair of a block is one scalar division
// per block; blocks stride over the M * ceil(N / 4TU) pairs.  T = 256 and
// U = DQ_U (DQ_COLS columns) by default.
// (Measured at M = 4096, cold: 2 slots per block were fastest or within 2% at
// N = 1280, 5120 and 10240; 1 slot was 5-18% slower there, up to 4 slots 16%
// slower at N = 5120; 1 slot was 1 us faster at N = 3072.)
// With nsl > 1 the accumulator is the sum of nsl int32 slices sl_stride
// apart (the partial products of a K split across blocks): integer sums, so
// the dequant sees the exact full product.  The bias is fp32 (bias), bf16
// (bias16, widened exactly) or absent.
constexpr int DQ_U = 2, DQ_COLS = 256 * 4 * DQ_U;

// Few rows (fewer than two default blocks per CU: the sum of K slices of a
// small batch) take T = 64, U = 1, 256 columns a block, so that more blocks
// share the slices' loads (M=200, N=1280, 8 slices: 21.2 -> 19.1 us for the
// whole linear).
template <int T, int U>
__global__ __launch_bounds__(T) void dequant_kernel(const int32_t* __restrict__ acc,
                                                   int64_t acc_ld, uint16_t* __restrict__ out,
                                                   const float* __restrict__ xs,
                                                   const float* __restrict__ ws,
                                                   const float* __restrict__ bias,
                                                   const uint16_t* __restrict__ bias16, int64_t M,
                                                   int64_t N, int nsl, int64_t sl_stride) {
    constexpr int COLS = 4 * T * U, STEP = 4 * T;
    const int64_t chunks = (N + COLS - 1) / COLS, tasks = M * chunks;
    for (int64_t bt = blockIdx.x; bt < tasks; bt += gridDim.x) {
        const int64_t m = bt / chunks;
        const int64_t c0 = (bt - m * chunks) * COLS + 4 * int64_t(threadIdx.x);
        const int32_t* pa = acc + m * acc_ld;
        uint16_t* po = out + m * N;
        const float x = xs[m];
        i32x4 a[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (c0 + STEP * u < N) a[u] = load16_i(pa + c0 + STEP * u);
#pragma unroll 2
        for (int sl = 1; sl < nsl; ++sl) {
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (c0 + STEP * u < N) a[u] += load16_i(pa + sl * sl_stride + c0 + STEP * u);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t c = c0 + STEP * u;
            if (c >= N) break;
            const float4 w = ws ? *reinterpret_cast<const float4*>(ws + c)
                                : make_float4(1.f, 1.f, 1.f, 1.f);
            float r0 = float(a[u].x) * (w.x * x), r1 = float(a[u].y) * (w.y * x);
            float r2 = float(a[u].z) * (w.z * x), r3 = float(a[u].w) * (w.w * x);
            if (bias) {
                const float4 b = *reinterpret_cast<const float4*>(bias + c);
                r0 = r0 + b.x; r1 = r1 + b.y; r2 = r2 + b.z; r3 = r3 + b.w;
            } else if (bias16) {
                const uint2 u2 = *reinterpret_cast<const uint2*>(bias16 + c);
                r0 = r0 + bf16lo(u2.x); r1 = r1 + bf16hi(u2.x);
                r2 = r2 + bf16lo(u2.y); r3 = r3 + bf16hi(u2.y);
            }
            *reinterpret_cast<uint2*>(po + c) = make_uint2(cvt_pk_bf16(r0, r1), cvt_pk_bf16(r2, r3));
        }
    }
}

// ------------------------------------------------------------ int8 transpose
// out[c, r] = in[r, c] (R, C multiples of 16), through a 128 x 128 byte LDS
// tile per block of 256 threads:
//  * in: each thread loads four 16-byte chunks (rows t/8 + 32i, chunk t%8), so
//    8 lanes cover a whole 128-byte row segment;
//  * LDS: row r's 16-byte chunk k sits at slot k ^ ((r / 16) % 8);
//  * out: thread t owns input rows 16*(t%8) .. +15 of input columns
//    4*(t/8) .. +3: sixteen dword reads, a 4 x 4 byte register transpose per
//    four rows, and four 16-byte stores, 8 lanes per 128-byte output segment.
// Tiles past R or C are masked per 16-byte chunk.
__device__ __forceinline__ void transpose4x4(const uint32_t (&w)[4], uint32_t (&o)[4]) {
    // w[i] = bytes (row i, columns 0..3); o[j] = bytes (column j, rows 0..3)
    const uint32_t lo01 = __builtin_amdgcn_perm(w[1], w[0], 0x05010400u);
    const uint32_t hi01 = __builtin_amdgcn_perm(w[1], w[0], 0x07030602u);
    const uint32_t lo23 = __builtin_amdgcn_perm(w[3], w[2], 0x05010400u);
    const uint32_t hi23 = __builtin_amdgcn_perm(w[3], w[2], 0x07030602u);
    o[0] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
    o[1] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
    o[2] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
    o[3] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
}

__global__ __launch_bounds__(256) void transpose_i8_kernel(const int8_t* __restrict__ in,
                                                          int8_t* __restrict__ out, int64_t R,
                                                          int64_t C) {
    __shared__ __attribute__((aligned(16))) uint8_t tile[128 * 128];
    const int t = threadIdx.x;
    const int64_t r0 = int64_t(blockIdx.y) * 128, c0 = int64_t(blockIdx.x) * 128;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = 32 * i + (t >> 3), k = t & 7;
        const int64_t r = r0 + row, c = c0 + 16 * k;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (r < R && c < C) v = *reinterpret_cast<const uint4*>(in + r * C + c);
        *reinterpret_cast<uint4*>(tile + row * 128 + ((k ^ ((row >> 4) & 7)) << 4)) = v;
    }
    __syncthreads();
    const int rg = t & 7, cg = t >> 3;                 // rows 16rg.., columns 4cg..
    uint32_t col[4][4];                                // [output column j][row quad q]
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 16 * rg + 4 * q + i;
            const int k = cg >> 2;                      // 16-byte chunk of column 4cg
            w[i] = *reinterpret_cast<const uint32_t*>(tile + row * 128 + ((k ^ rg) << 4) +
                                                      (cg & 3) * 4);
        }
        uint32_t o[4];
        transpose4x4(w, o);
#pragma unroll
        for (int j = 0; j < 4; ++j) col[j][q] = o[j];
    }
    const int64_t r = r0 + 16 * rg;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t c = c0 + 4 * cg + j;
        if (c < C && r < R)
            *reinterpret_cast<uint4*>(out + c * R + r) =
                make_uint4(col[j][0], col[j][1], col[j][2], col[j][3]);
    }
}

}  // namespace

// Whether launch_gemm takes the persistent ping-pong kernel for a staged
// epilogue: 256 x 320 tiles (paired: 256 x 160 output columns) filling every
// CU at least once, where no skinny or split-K kernel comes first.
bool pp_applies(int M, int N, int K, bool paired) {
    const int64_t tm = (M + 255) / 256;
    if (paired) return M > kSkinnyPairedM && tm * ((N + 159) / 160) >= device_cus();
    return M > 64 && !splitk_applies(M, N, K) && tm * ((N + 319) / 320) >= device_cus();
}


// Whether launch_gemm takes the split-K kernel for a staged epilogue.
bool splitk_applies(int M, int N, int K) {
    if (M <= 64) return false;
    const int64_t tm = (M + 255) / 256, tn = (N + 159) / 160;
    const int64_t tiles_split = int64_t((M + 127) / 128) * ((N + 159) / 160);
    return tm * tn < 192 && K >= 1024 && tiles_split >= 128;
}

// Rows few enough (two 128-row tiles at most) that the slices take the
// 128 x 128 kernel, whose narrower tiles give more blocks per slice
static bool slices_small_tiles(int M) { return M <= 256; }

// K slices on the skinny kernel (two weight blocks per block, slices of at
// least 1024) for batches of 33-128 rows: above 64 rows in place of the
// 128 x 128 kernel, at 33-64 rows only where the unsplit skinny kernel has
// fewer than 128 blocks (N < 2048).  Measured cold, with the dequant pass
// that adds the slices included: M=64, N=1280, K=5120 16.5 -> 12.5 us; M=100
// 19.4 -> 14.5; M=128, N=4096, K=4096 22.8 -> 19.9; but M=1 7.8 -> 8.9 and
// M=16 9.5 -> 9.9 (N=1280, K=5120), M=48, N=3072, K=3072 10.7 -> 11.7.
// Slices of 512 were 1.5-2.5 us slower than slices of 1024 at M=64-128, and
// one weight block per block 0.5-20 us slower.
constexpr int kSkinnySliceNB = 2, kSkinnySliceMin = 1024;
// The skinny kernel's slice count: the fewest (power of two) that give at
// least 256 blocks; 0 when it does not apply or no split fits.
static int skinny_slices(int M, int N, int K) {
    if (M <= 32 || M > 128 || (M <= 64 && N >= 2048) || K % 64 != 0) return 0;
    const int64_t blocks = (N + 16 * kSkinnySliceNB - 1) / (16 * kSkinnySliceNB);
    int s = 1;
    while (blocks * s < 256 && (K / 64) % (2 * s) == 0 && K / (2 * s) >= kSkinnySliceMin) s *= 2;
    return s > 1 ? s : 0;
}

// K slices for a split of the product across blocks: the skinny kernel's
// (above) where they apply; else, when the output has fewer 128 x 160 tiles
// than the split-K kernel takes (128) and M > 64, the fewest power-of-two
// slices that give at least 192 blocks, each slice at least 1024 long (512 on
// the 128 x 128 kernel, M <= 256) and a whole number of 64-byte steps; 0 when
// no split applies (128 tiles or more, or K too short).  (With 128-191 tiles the split-K kernel
// alone measured faster: 28.8 against 41.2 us at M=2100, N=1296, K=2304, and
// 1 us at M=2048 and 4096 with 128 tiles.)
int gemm_slices(int M, int N, int K) {
    if (K % 64 != 0) return 0;
    if (const int s = skinny_slices(M, N, K)) return s;
    if (M <= 64) return 0;
    const int64_t tiles = int64_t((M + 127) / 128) * ((N + 159) / 160);
    if (tiles >= 128) return 0;
    if (slices_small_tiles(M)) {
        // the 128 x 128 kernel: its tiles, slices down to 512 long
        const int64_t t128 = int64_t((M + 127) / 128) * ((N + 127) / 128);
        int s = 1;
        while (t128 * s < 192 && (K / 64) % (2 * s) == 0 && K / (2 * s) >= 512) s *= 2;
        return s > 1 ? s : 0;
    }
    int s = 1;
    while (tiles * s < 192 && (K / 64) % (2 * s) == 0 && K / (2 * s) >= 1024) s *= 2;
    return s > 1 ? s : 0;
}

// The int32 partial products of nsl = gemm_slices(M, N, K) K slices, slice s
// at part + s * M * N (row stride N): the skinny, 128 x 128 or split-K kernel
// over a (tiles, nsl) grid, as gemm_slices chose.
hipError_t gemm_i32_slices(hipStream_t st, const int8_t* X, int64_t ldx, const int8_t* W,
                           int64_t ldw, int32_t* part, int M, int N, int K, int nsl) {
    const EpiSliceI32 epi{part, int64_t(N), int64_t(M) * N};
    if (skinny_slices(M, N, K) == nsl)
        return launch_skinny<kSkinnySliceNB>(st, X, ldx, W, ldw, M, N, K / nsl, epi, nsl);
    if (slices_small_tiles(M)) {
        const int tm = (M + 127) / 128, tn = (N + 127) / 128;
        hipLaunchKernelGGL((gemm_i8_kernel<128, 128, 2, 2, 4, EpiSliceI32>),
                           dim3(unsigned(tm * tn), unsigned(nsl)), dim3(256), 0, st, X, ldx, W,
                           ldw, M, N, K / nsl, tm, tn, epi);
        return hipGetLastError();
    }
    const int tm = (M + 127) / 128, tn = (N + 159) / 160;
    hipLaunchKernelGGL((gemm_i8_splitk_kernel<4, false, false, EpiSliceI32, false>),
                       dim3(unsigned(tm * tn), unsigned(nsl)), dim3(512), 0, st, X, ldx, W, ldw,
                       M, N, K / nsl, tm, tn, EpiSliceI32{part, int64_t(N), int64_t(M) * N});
    return hipGetLastError();
}

// The same with B stored [K, N] (the NN product, the split-K kernel's
// transposing weight reads): for M > 256 only (the 128 x 128 kernel has no NN
// form; callers transpose B for M <= 256)
hipError_t gemm_i32_slices_nn(hipStream_t st, const int8_t* X, int64_t ldx, const int8_t* Bkn,
                              int64_t ldb, int32_t* part, int M, int N, int K, int nsl) {
    if (slices_small_tiles(M)) return hipErrorInvalidValue;
    const int tm = (M + 127) / 128, tn = (N + 159) / 160;
    hipLaunchKernelGGL((gemm_i8_splitk_kernel<4, false, true, EpiSliceI32, false>),
                       dim3(unsigned(tm * tn), unsigned(nsl)), dim3(512), 0, st, X, ldx, Bkn, ldb,
                       M, N, K / nsl, tm, tn, EpiSliceI32{part, int64_t(N), int64_t(M) * N});
    return hipGetLastError();
}
bool slices_need_nt(int M) { return slices_small_tiles(M); }

// B[k, n] as stored (the NN product); the 32-bit DMA offsets of the weight
// need K * ldb below 2^32
bool splitk_nn_applies(int M, int N, int K, int64_t ldb) {
    return splitk_applies(M, N, K) && N % 16 == 0 && int64_t(K + 64) * ldb < (int64_t(1) << 32);
}

hipError_t gemm_i32(hipStream_t st, const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb,
                    int32_t* C, int64_t ldc, int M, int N, int K) {
    return launch_gemm(st, A, lda, B, ldb, M, N, K, EpiI32{C, ldc});
}

hipError_t gemm_dequant(hipStream_t st, const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb,
                        void* out, int64_t ldo, const float* xs, const float* ws, const float* bias,
                        const uint16_t* bias16, int M, int N, int K, const int8_t* Bp) {
    return launch_gemm(st, A, lda, B, ldb, M, N, K,
                       EpiDequant{static_cast<uint16_t*>(out), ldo, xs, ws, bias, bias16}, Bp);
}

hipError_t gemm_dequant_nn(hipStream_t st, const int8_t* A, int64_t lda, const int8_t* Bkn,
                           int64_t ldb, void* out, int64_t ldo, const float* xs, int M, int N,
                           int K, bool* done) {
    *done = splitk_nn_applies(M, N, K, ldb);
    if (!*done) return hipSuccess;
    return launch_splitk<true>(st, A, lda, Bkn, ldb, M, N, K,
                               EpiDequant{static_cast<uint16_t*>(out), ldo, xs, nullptr, nullptr,
                                          nullptr});
}

hipError_t gemm_dequant_xt(hipStream_t st, const int8_t* At, const int8_t* B, int64_t ldb,
                           void* out, int64_t ldo, const float* xs, const float* ws,
                           const float* bias, const uint16_t* bias16, int M, int N, int K,
                           bool packed) {
    const EpiDequant epi{static_cast<uint16_t*>(out), ldo, xs, ws, bias, bias16};
    if (packed) return launch_splitk<false, EpiDequant, true, true>(st, At, 0, B, 0, M, N, K, epi);
    return launch_splitk<false, EpiDequant, true>(st, At, 0, B, ldb, M, N, K, epi);
}

hipError_t gemm_dequant_pp_xt(hipStream_t st, const int8_t* At, const int8_t* B, int64_t ldb,
                              void* out, int64_t ldo, const float* xs, const float* ws,
                              const float* bias, const uint16_t* bias16, int M, int N, int K,
                              bool packed) {
    const EpiDequant epi{static_cast<uint16_t*>(out), ldo, xs, ws, bias, bias16};
    if (packed) return launch_pp<true, true>(st, At, 0, B, 0, M, N, K, epi);
    return launch_pp<true>(st, At, 0, B, ldb, M, N, K, epi);
}

template <int ACT>
static hipError_t act_pp_xt(hipStream_t st, const int8_t* At, const int8_t* B, int64_t ldb,
                            const EpiAct<ACT>& epi, int M, int N, int K, bool packed) {
    if (packed) return launch_pp<true, true>(st, At, 0, B, 0, M, N, K, epi);
    return launch_pp<true>(st, At, 0, B, ldb, M, N, K, epi);
}

hipError_t gemm_act_pp_xt(hipStream_t st, const int8_t* At, const int8_t* B, int64_t ldb,
                          void* out, int64_t ldo, const float* xs, const float* ws, int M, int N,
                          int K, int act, bool packed) {
    uint16_t* o = static_cast<uint16_t*>(out);
    const uint16_t* tab = activation_tables();
    switch (act) {
        case 3: return act_pp_xt(st, At, B, ldb, EpiAct<3>{o, ldo, xs, ws, N, tab}, M, N, K, packed);
        case 4: return act_pp_xt(st, At, B, ldb, EpiAct<4>{o, ldo, xs, ws, N, tab}, M, N, K, packed);
        case 5: return act_pp_xt(st, At, B, ldb, EpiAct<5>{o, ldo, xs, ws, N, tab}, M, N, K, packed);
        default: return hipErrorInvalidValue;
    }
}

bool skinny_applies(int M, bool paired) { return M <= (paired ? kSkinnyPairedM : 64); }

hipError_t gemm_dequant_skinny_xt(hipStream_t st, const int8_t* At, const int8_t* Bp, void* out,
                                  int64_t ldo, const float* xs, const float* ws, const float* bias,
                                  const uint16_t* bias16, int M, int N, int K) {
    const EpiDequant epi{static_cast<uint16_t*>(out), ldo, xs, ws, bias, bias16};
    return launch_skinny<1, EpiDequant, true, true>(st, At, 0, Bp, 0, M, N, K, epi);
}

hipError_t gemm_act_skinny_xt(hipStream_t st, const int8_t* At, const int8_t* Bp, void* out,
                              int64_t ldo, const float* xs, const float* ws, int M, int N, int K,
                              int act) {
    uint16_t* o = static_cast<uint16_t*>(out);
    const uint16_t* tab = activation_tables();
    switch (act) {
        case 3: return launch_skinny<4, EpiAct<3>, true, true>(st, At, 0, Bp, 0, M, N, K,
                                                              EpiAct<3>{o, ldo, xs, ws, N, tab});
        case 4: return launch_skinny<4, EpiAct<4>, true, true>(st, At, 0, Bp, 0, M, N, K,
                                                              EpiAct<4>{o, ldo, xs, ws, N, tab});
        case 5: return launch_skinny<1, EpiAct<5>, true, true>(st, At, 0, Bp, 0, M, N, K,
                                                              EpiAct<5>{o, ldo, xs, ws, N, tab});
        default: return hipErrorInvalidValue;
    }
}

hipError_t gemm_dequant_nn_xt(hipStream_t st, const int8_t* At, const int8_t* Bkn, int64_t ldb,
                              void* out, int64_t ldo, const float* xs, int M, int N, int K,
                              bool packed) {
    const EpiDequant epi{static_cast<uint16_t*>(out), ldo, xs, nullptr, nullptr, nullptr};
    if (packed) return launch_splitk<true, EpiDequant, true, true>(st, At, 0, Bkn, 0, M, N, K, epi);
    return launch_splitk<true, EpiDequant, true>(st, At, 0, Bkn, ldb, M, N, K, epi);
}

hipError_t gemm_dequant_residual(hipStream_t st, const int8_t* A, int64_t lda, const int8_t* B,
                                 int64_t ldb, void* out, int64_t ldo, const float* xs,
                                 const float* ws, const float* bias, const uint16_t* bias16,
                                 const void* res, int64_t ldr, const void* rscale, int M, int N,
                                 int K) {
    EpiDequantRes e;
    static_cast<EpiDequant&>(e) =
        EpiDequant{static_cast<uint16_t*>(out), ldo, xs, ws, bias, bias16};
    e.res = static_cast<const uint16_t*>(res);
    e.ldr = ldr;
    e.rscale = static_cast<const uint16_t*>(rscale);
    return launch_gemm(st, A, lda, B, ldb, M, N, K, e);
}

hipError_t gemm_dequant_residual_xt(hipStream_t st, const int8_t* At, const int8_t* B,
                                    int64_t ldb, void* out, int64_t ldo, const float* xs,
                                    const float* ws, const float* bias, const uint16_t* bias16,
                                    const void* res, int64_t ldr, const void* rscale, int M, int N,
                                    int K, bool packed) {
    EpiDequantRes e;
    static_cast<EpiDequant&>(e) =
        EpiDequant{static_cast<uint16_t*>(out), ldo, xs, ws, bias, bias16};
    e.res = static_cast<const uint16_t*>(res);
    e.ldr = ldr;
    e.rscale = static_cast<const uint16_t*>(rscale);
    if (pp_applies(M, N, K, false)) {
        if (packed) return launch_pp<true, true>(st, At, 0, B, 0, M, N, K, e);
        return launch_pp<true>(st, At, 0, B, ldb, M, N, K, e);
    }
    if (splitk_applies(M, N, K)) {
        if (packed) return launch_splitk<false, EpiDequantRes, true, true>(st, At, 0, B, 0, M, N, K, e);
        return launch_splitk<false, EpiDequantRes, true>(st, At, 0, B, ldb, M, N, K, e);
    }
    return hipErrorInvalidValue;
}

hipError_t gemm_i32_pp_xt(hipStream_t st, const int8_t* At, const int8_t* B, int64_t ldb,
                          int32_t* C, int64_t ldc, int M, int N, int K, bool packed) {
    const EpiI32 epi{C, ldc};
    if (packed) return launch_pp<true, true>(st, At, 0, B, 0, M, N, K, epi);
    return launch_pp<true>(st, At, 0, B, ldb, M, N, K, epi);
}

hipError_t gemm_act(hipStream_t st, const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb,
                    void* out, int64_t ldo, const float* xs, const float* ws, int M, int N, int K,
                    int act, const int8_t* Bp) {
    uint16_t* o = static_cast<uint16_t*>(out);
    const uint16_t* tab = activation_tables();
    switch (act) {
        case 3: return launch_gemm(st, A, lda, B, ldb, M, N, K, EpiAct<3>{o, ldo, xs, ws, N, tab}, Bp);
        case 4: return launch_gemm(st, A, lda, B, ldb, M, N, K, EpiAct<4>{o, ldo, xs, ws, N, tab}, Bp);
        case 5: return launch_gemm(st, A, lda, B, ldb, M, N, K, EpiAct<5>{o, ldo, xs, ws, N, tab}, Bp);
        default: return hipErrorInvalidValue;
    }
}

hipError_t dequant_epilogue(hipStream_t st, const int32_t* acc, int64_t acc_ld, void* out,
                            const float* xs, const float* ws, const float* bias, int64_t M,
                            int64_t N) {
    return dequant_slices(st, acc, acc_ld, 1, 0, out, xs, ws, bias, nullptr, M, N);
}

hipError_t dequant_slices(hipStream_t st, const int32_t* acc, int64_t acc_ld, int nsl,
                          int64_t sl_stride, void* out, const float* xs, const float* ws,
                          const float* bias, const uint16_t* bias16, int64_t M, int64_t N) {
    int64_t blocks = M * ((N + DQ_COLS - 1) / DQ_COLS);
    if (blocks == 0) return hipSuccess;
    uint16_t* o = static_cast<uint16_t*>(out);
    if (blocks < 2 * device_cus()) {
        hipLaunchKernelGGL((dequant_kernel<64, 1>), dim3(unsigned(M * ((N + 255) / 256))), dim3(64),
                           0, st, acc, acc_ld, o, xs, ws, bias, bias16, M, N, nsl, sl_stride);
        return hipGetLastError();
    }
    if (blocks > (int64_t(1) << 20)) blocks = int64_t(1) << 20;
    hipLaunchKernelGGL((dequant_kernel<256, DQ_U>), dim3(unsigned(blocks)), dim3(256), 0, st, acc,
                       acc_ld, o, xs, ws, bias, bias16, M, N, nsl, sl_stride);
    return hipGetLastError();
}

hipError_t transpose_i8(hipStream_t st, const int8_t* in, int8_t* out, int64_t R, int64_t C) {
    const dim3 grid(unsigned((C + 127) / 128), unsigned((R + 127) / 128));
    hipLaunchKernelGGL(transpose_i8_kernel, grid, dim3(256), 0, st, in, out, R, C);
    return hipGetLastError();
}

// ------------------------------------------------------------ packed weight
// w [N, K] (row-major, K % 16 == 0) in the MFMA block layout (tiled_offset),
// zeros past K and past N: thread t writes the layout's 16-byte chunk t,
// position p of row r of its block, which holds the row's chunk p ^ ((r >> 1) & 3)
__global__ __launch_bounds__(256) void pack_weight_kernel(const int8_t* __restrict__ w,
                                                          int8_t* __restrict__ out, int64_t N,
                                                          int K, int KB, int64_t chunks) {
    const int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (t >= chunks) return;
    const int64_t blk = t >> 6;
    const int l = int(t & 63), r = l >> 2, c = (l & 3) ^ ((r >> 1) & 3);
    const int64_t nb = blk / KB;
    const int k = int(blk - nb * KB) * 64 + 16 * c;
    const int64_t n = 16 * nb + r;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (n < N && k < K) v = *reinterpret_cast<const uint4*>(w + n * K + k);
    reinterpret_cast<uint4*>(out)[t] = v;
}

hipError_t pack_weight(hipStream_t st, const int8_t* w, int8_t* out, int64_t N, int K) {
    const int KB = (K + 63) / 64;
    const int64_t chunks = tiled_bytes(N, K) / 16;
    hipLaunchKernelGGL(pack_weight_kernel, dim3(unsigned((chunks + 255) / 256)), dim3(256), 0, st,
                       w, out, N, K, KB, chunks);
    return hipGetLastError();
}

// w [R, C] (row-major: R contraction rows, C = the product's columns, C % 32
// == 0) in the NN stage order of the split-K kernel: per 64-row step s, per
// 32-column group cb, per 32-row half rb the 1 KB block ((s * C/32 + cb) * 2 +
// rb) * 1024, in which 16-byte chunk l holds row l/2 of the half, column half
// (l & 1) ^ ((l >> 5) & 1) of the group; zeros past R
__global__ __launch_bounds__(256) void pack_weight_nn_kernel(const int8_t* __restrict__ w,
                                                             int8_t* __restrict__ out, int64_t R,
                                                             int C, int64_t chunks) {
    const int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (t >= chunks) return;
    const int64_t blk = t >> 6;
    const int l = int(t & 63), kr = l >> 1, h = (l & 1) ^ ((kr >> 4) & 1);
    const int groups = C / 32;
    const int rb = int(blk & 1);
    const int64_t sg = blk >> 1;
    const int64_t step = sg / groups;
    const int cb = int(sg - step * groups);
    const int64_t r = 64 * step + 32 * rb + kr;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (r < R) v = *reinterpret_cast<const uint4*>(w + r * C + 32 * cb + 16 * h);
    reinterpret_cast<uint4*>(out)[t] = v;
}

int64_t packed_nn_bytes(int64_t R, int64_t C) { return ((R + 63) / 64) * 64 * C; }

hipError_t pack_weight_nn(hipStream_t st, const int8_t* w, int8_t* out, int64_t R, int C) {
    const int64_t chunks = packed_nn_bytes(R, C) / 16;
    hipLaunchKernelGGL(pack_weight_nn_kernel, dim3(unsigned((chunks + 255) / 256)), dim3(256), 0,
                       st, w, out, R, C, chunks);
    return hipGetLastError();
}

}  // namespace xpuint8
