// Row-wise ConvRot kernels: rotate+quantize (with optional fused activation or
// fused dequant+activation), rotate only, the gradient row quantizer, the
// weight preparation and the weight dequantization.
//
// Lane assignment (all kernels): a 256-point ConvRot group is held by 16
// lanes, each holding one 16-element register of it (elements [16w, 16w+16)
// in lane L for w = lane_w(L), a permutation of the reference sub-group
// kernel's w = L, src/xpuint8.cpp:406-438, that keeps every cross-lane
// butterfly on DPP; after the transform the lane holds register
// lane_w_rot(L), which is where its results are stored).  Row kernels
// keep the whole row in registers across as many 16-lane segments as it needs
// (rowquant_seg_kernel); rows too long for that use the two-pass variant, one
// wave per row, which re-reads the row (from L2) to quantize it.
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"
#include "activations.hpp"

namespace xpuint8 {
namespace {

constexpr int kRowsPerBlock = 4;     // 4 waves = 4 rows per 256-thread block

// Element (r, col) of a row-major array whose base is already advanced to a
// block's first row: the offset is formed in 32 bits (r and col are small,
// r*ld + col < 2^32), so the address is a wave-uniform base plus one 32-bit
// lane offset.
// (r < 64 and ld < 2^24: a 24-bit multiply.)
template <class T>
__device__ __forceinline__ T* at32(T* base, int r, int64_t ld, int col) {
    using B = typename std::conditional<std::is_const<T>::value, const char, char>::type;
    const uint32_t off = (__umul24(uint32_t(r), uint32_t(ld)) + uint32_t(col)) * uint32_t(sizeof(T));
    return reinterpret_cast<T*>(reinterpret_cast<B*>(base) + uint64_t(off));
}

// ------------------------------------------------------- table windows in LDS
// The activations read their tables through LDS copies of a window of each
// table: the entries of the bf16 inputs with |x| in [2^-20, 2^8) (exponent
// field in [107, 135)), 3584 positive then 3584 negative, 14 KB per table,
// filled once per block.  Inputs outside a window (zeros, |x| < 2^-20,
// |x| >= 256, infinities, NaNs) take the tables in global memory behind a
// wave-uniform branch; the same table words either way.  (The window is wider
// than the GEMM epilogue's, whose LDS is scarcer: with [2^-12, 16), roughly
// one wave in five of normal-distributed inputs had an input below it, and
// nearly every wave of rows with 1% outlier channels x30 one above it.)
// One window for the one-lookup activations (gelu_tanh, swiglu's SiLU, the erf
// GELU of GEGLU and GELU), two for situ: its gate factor bf16(tanh(g/4) *
// sigmoid(g)), a function of the gate alone, and tanh(h/25) of the hidden value.
constexpr int kRowWinLo = 107 << 7, kRowWinHalf = 28 * 128, kRowWinSize = 2 * kRowWinHalf;
constexpr int kRowWinUnits = kRowWinSize / 8;       // 16-byte units per window
static_assert(kRowWinHalf % (8 * 64) == 0, "a DMA chunk (64 units) stays in one sign half");

template <int ACT>
__host__ __device__ constexpr int win_count() {
    return ACT == 3 ? 2 : (ACT == 1 || ACT == 2 || ACT == 4 || ACT == 5) ? 1 : 0;
}
template <int ACT>
__host__ __device__ constexpr int win_table(int j) {
    return ACT == 1 ? kTabGeluTanh
         : ACT == 2 ? kTabSilu
         : (ACT == 4 || ACT == 5) ? kTabGeluErf
         : j == 0 ? kTabSituGate : kTabSituTanhH;
}

// Loaders that read through windows declare kWins > 0, win_tab(j) and expand_w().
template <class L, class = void>
struct LoaderWins : std::integral_constant<int, 0> {};
template <class L>
struct LoaderWins<L, std::void_t<decltype(L::kWins)>> : std::integral_constant<int, L::kWins> {};
// Loaders whose expand() (the global-table form) should run right after each
// fetch when several groups are fetched: they declare kExpandAtFetch.
template <class L, class = void>
struct LoaderEarly : std::false_type {};
template <class L>
struct LoaderEarly<L, std::void_t<decltype(L::kExpandAtFetch)>>
    : std::integral_constant<bool, L::kExpandAtFetch> {};

// 16-byte unit i < kRowWinUnits of table T's window: the first half of the
// units are table words kRowWinLo + 8i (positive inputs), the second half the
// same for the negative ones
__device__ __forceinline__ const uint4* win_unit(const uint16_t* tab, int T, int i) {
    constexpr int H = kRowWinUnits / 2;
    const uint32_t word = (i >= H ? 0x8000u : 0u) + uint32_t(kRowWinLo) + 8u * uint32_t(i >= H ? i - H : i);
    return reinterpret_cast<const uint4*>(tab + size_t(T) * kTabSize + word);
}

// Whether bf16 bits k lie outside the windows
__device__ __forceinline__ bool win_outside(uint32_t k) {
    return (k & 0x7FFFu) - uint32_t(kRowWinLo) >= uint32_t(kRowWinHalf);
}
// The window word of bf16 bits k (clamped into the window when outside)
__device__ __forceinline__ uint32_t win_word(const uint16_t* win, uint32_t k) {
    const uint32_t rel = (k & 0x7FFFu) - uint32_t(kRowWinLo);
    return win[((k & 0x8000u) ? uint32_t(kRowWinHalf) : 0u) + min(rel, uint32_t(kRowWinHalf - 1))];
}

// activate<ACT>(a, b) for 16 inputs given by their bf16 bits (ka: the first
// input, kb: the second; unused for the one-input activations), the tables
// read through the windows at win (win_count<ACT>() of them, back to back),
// with a wave-uniform branch, rarely taken, for lookup operands outside the
// windows.  One-lookup activations read all 16 words, then patch the missing
// ones from the table in global memory.  Situ (two lookups) instead
// recomputes a missing output from the global tables, so that only inputs and
// outputs are live across the branch: patching its words kept every word and
// key live and cost the kernel half its occupancy (47 against 106-124 VGPRs;
// 32.5 against 51 us for quantize_act at 4096 x 5120, then with three
// tables), while for the one-lookup activations patching measured faster
// (dequant_act_quantize GELU at 4096 x 5120: 26.9 against 30.4 us).
template <int ACT>
__device__ __forceinline__ void act_windowed(const uint16_t* win, const uint16_t* tab,
                                             const uint32_t (&ka)[16], const uint32_t (&kb)[16],
                                             float (&v)[16]) {
    if constexpr (ACT == 3) {
        bool miss = false;
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            // bf16(bf16(tg * sg) * th) with the gate factor read whole
            const float p = tab_float(win_word(win, kb[t]));
            const float th = tab_float(win_word(win + kRowWinSize, ka[t]));
            miss = miss || win_outside(ka[t]) || win_outside(kb[t]);
            v[t] = bf16_round(p * th);
        }
        if (__builtin_amdgcn_ballot_w64(miss)) {
#pragma unroll
            for (int t = 0; t < 16; ++t)
                if (win_outside(ka[t]) || win_outside(kb[t]))
                    v[t] = activate<3>(tab, __uint_as_float(ka[t] << 16),
                                       __uint_as_float(kb[t] << 16));
        }
    } else {
        constexpr int T = win_table<ACT>(0);
        const uint32_t* k = ACT == 4 ? kb : ka;
        uint32_t w[16];
        bool miss = false;
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            miss = miss || win_outside(k[t]);
            w[t] = win_word(win, k[t]);
        }
        if (__builtin_amdgcn_ballot_w64(miss)) {
#pragma unroll
            for (int t = 0; t < 16; ++t)
                if (win_outside(k[t])) w[t] = tab[T * kTabSize + k[t]];
        }
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            if constexpr (ACT == 1 || ACT == 5) {
                v[t] = tab_float(w[t]);
            } else {
                const float a = __uint_as_float(ka[t] << 16), b = __uint_as_float(kb[t] << 16);
                v[t] = bf16_round(act_combine<ACT>(a, b, &w[t]));
            }
        }
    }
}

// ------------------------------------------------------------------ loaders
// A loader produces the pre-rotation values of elements [col, col+16) of a
// row, as bf16-valued floats, in two steps: fetch() issues the memory reads
// and returns them raw, expand() turns them into floats.  Kernels that
// pipeline rows call fetch() for the next row before working on the current
// one, so the reads stay in flight during the arithmetic.

struct LoadBF16 {
    const uint16_t* x;
    int64_t ld;
    struct Raw { u32x4 a, b; };
    __device__ __forceinline__ Raw fetch(int64_t row, int col) const {
        const uint16_t* p = x + row * ld + col;
        return Raw{load16(p), load16(p + 8)};
    }
    // the same loader with row 0 at row0, and fetch() from it with 32-bit
    // offsets (r < rows per block)
    __device__ __forceinline__ LoadBF16 rebase(int64_t row0) const { return {x + row0 * ld, ld}; }
    __device__ __forceinline__ Raw fetch_r(int r, int col) const {
        const uint16_t* p = at32(x, r, ld, col);
        return Raw{load16(p), load16(p + 8)};
    }
    __device__ __forceinline__ void expand(const Raw& r, float (&v)[16]) const {
        const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) { v[2 * j] = bf16lo(w[j]); v[2 * j + 1] = bf16hi(w[j]); }
    }
    __device__ __forceinline__ void operator()(int64_t row, int col, float (&v)[16]) const {
        expand(fetch(row, col), v);
    }
};

// An activation on bf16 input(s) (src/xpuint8.cpp:190-220).  Paired ids read
// the first half at col and the second half at col + half.
template <int ACT>
struct LoadAct {
    const uint16_t* x;
    int64_t ld;
    int64_t half;
    const uint16_t* tab;   // activation tables (activations.hpp)
    struct Raw { LoadBF16::Raw a, b; };
    __device__ __forceinline__ Raw fetch(int64_t row, int col) const {
        Raw r;
        r.a = LoadBF16{x, ld}.fetch(row, col);
        if constexpr (act_paired(ACT)) r.b = LoadBF16{x + half, ld}.fetch(row, col);
        return r;
    }
    __device__ __forceinline__ LoadAct rebase(int64_t row0) const {
        return {x + row0 * ld, ld, half, tab};
    }
    __device__ __forceinline__ Raw fetch_r(int rr, int col) const {
        Raw r;
        r.a = LoadBF16{x, ld}.fetch_r(rr, col);
        if constexpr (act_paired(ACT)) r.b = LoadBF16{x + half, ld}.fetch_r(rr, col);
        return r;
    }
    __device__ __forceinline__ void expand(const Raw& r, float (&v)[16]) const {
        float a[16];
        LoadBF16{x, ld}.expand(r.a, a);
        if constexpr (act_paired(ACT)) {
            float b[16];
            LoadBF16{x, ld}.expand(r.b, b);
#pragma unroll
            for (int t = 0; t < 16; ++t) v[t] = activate<ACT>(tab, a[t], b[t]);
        } else {
#pragma unroll
            for (int t = 0; t < 16; ++t) v[t] = activate<ACT>(tab, a[t], 0.f);
        }
    }
    static constexpr int kWins = win_count<ACT>();
    __host__ __device__ static constexpr int win_tab(int j) { return win_table<ACT>(j); }
    __device__ __forceinline__ void expand_w(const Raw& r, float (&v)[16],
                                             const uint16_t* win) const {
        uint32_t ka[16], kb[16];
        const uint32_t wa[8] = {r.a.a.x, r.a.a.y, r.a.a.z, r.a.a.w, r.a.b.x, r.a.b.y, r.a.b.z, r.a.b.w};
        const uint32_t wb[8] = {r.b.a.x, r.b.a.y, r.b.a.z, r.b.a.w, r.b.b.x, r.b.b.y, r.b.b.z, r.b.b.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            ka[2 * j] = wa[j] & 0xFFFFu;
            ka[2 * j + 1] = wa[j] >> 16;
            kb[2 * j] = act_paired(ACT) ? wb[j] & 0xFFFFu : 0u;
            kb[2 * j + 1] = act_paired(ACT) ? wb[j] >> 16 : 0u;
        }
        act_windowed<ACT>(win, tab, ka, kb, v);
    }
    __device__ __forceinline__ void operator()(int64_t row, int col, float (&v)[16]) const {
        expand(fetch(row, col), v);
    }
};

// Dequantize the up-projection accumulator, then the activation
// (src/xpuint8.cpp:238-261): h = bf16(float(acc) * (ws[n] * xs[m])).
template <int ACT>
struct LoadDequantAct {
    const int32_t* acc;
    int64_t ld;            // accumulator row stride
    int64_t half;          // column offset of the gate half (paired only)
    const float* xs;
    const float* ws;
    const uint16_t* tab;
    __device__ __forceinline__ void deq(int64_t row, int64_t c0, float xsr, float (&o)[16]) const {
        const int32_t* p = acc + row * ld + c0;
        const float4* q = reinterpret_cast<const float4*>(ws + c0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const i32x4 a = load16_i(p + 4 * j);
            const float4 w = q[j];
            o[4 * j + 0] = bf16_round(float(a.x) * (w.x * xsr));
            o[4 * j + 1] = bf16_round(float(a.y) * (w.y * xsr));
            o[4 * j + 2] = bf16_round(float(a.z) * (w.z * xsr));
            o[4 * j + 3] = bf16_round(float(a.w) * (w.w * xsr));
        }
    }
    // Raw: the dequantized bf16 values, two to a word: the first half in the
    // low 16 bits, the gate half (paired) in the high ones
    struct Raw { uint32_t w[16]; };
    __device__ __forceinline__ Raw fetch(int64_t row, int col) const {
        Raw r;
        const float xsr = xs[row];
        float h[16], g[16];
        deq(row, col, xsr, h);
        if constexpr (act_paired(ACT)) deq(row, col + half, xsr, g);
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            r.w[t] = __float_as_uint(h[t]) >> 16;
            if constexpr (act_paired(ACT)) r.w[t] |= __float_as_uint(g[t]) & 0xFFFF0000u;
        }
        return r;
    }
    __device__ __forceinline__ LoadDequantAct rebase(int64_t row0) const {
        return {acc + row0 * ld, ld, half, xs + row0, ws, tab};
    }
    __device__ __forceinline__ Raw fetch_r(int r, int col) const { return fetch(r, col); }
    __device__ __forceinline__ void expand(const Raw& r, float (&v)[16]) const {
#pragma unroll
        for (int t = 0; t < 16; ++t)
            v[t] = activate<ACT>(tab, __uint_as_float(r.w[t] << 16),
                                 __uint_as_float(r.w[t] & 0xFFFF0000u));
    }
    static constexpr int kWins = win_count<ACT>();
    // without windows (two groups per lane), expand each group as soon as it
    // is fetched: one group's table reads in flight at a time keeps the
    // kernel within its registers
    static constexpr bool kExpandAtFetch = true;
    __host__ __device__ static constexpr int win_tab(int j) { return win_table<ACT>(j); }
    __device__ __forceinline__ void expand_w(const Raw& r, float (&v)[16],
                                             const uint16_t* win) const {
        uint32_t ka[16], kb[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            ka[t] = r.w[t] & 0xFFFFu;
            kb[t] = r.w[t] >> 16;
        }
        act_windowed<ACT>(win, tab, ka, kb, v);
    }
    __device__ __forceinline__ void operator()(int64_t row, int col, float (&v)[16]) const {
        expand(fetch(row, col), v);
    }
};

// bf16(bf16(dy) * bf16(ws[n])): the column-scaled gradient of linear_dx_int8
// (python/xpu_kernels/int8/ops.py:366).  The product of two bf16 values is
// exact in fp32, so this is one rounding.
struct LoadColScaled {
    const uint16_t* x;
    int64_t ld;
    const float* colscale;   // may be null: plain bf16 rows
    struct Raw { LoadBF16::Raw x; float4 c[4]; };
    __device__ __forceinline__ LoadColScaled rebase(int64_t row0) const {
        return {x + row0 * ld, ld, colscale};
    }
    __device__ __forceinline__ Raw fetch_r(int rr, int col) const {
        Raw r;
        r.x = LoadBF16{x, ld}.fetch_r(rr, col);
        if (colscale) {
            const float4* q = reinterpret_cast<const float4*>(colscale + col);
#pragma unroll
            for (int j = 0; j < 4; ++j) r.c[j] = q[j];
        }
        return r;
    }
    __device__ __forceinline__ Raw fetch(int64_t row, int col) const {
        Raw r;
        r.x = LoadBF16{x, ld}.fetch(row, col);
        if (colscale) {
            const float4* q = reinterpret_cast<const float4*>(colscale + col);
#pragma unroll
            for (int j = 0; j < 4; ++j) r.c[j] = q[j];
        }
        return r;
    }
    __device__ __forceinline__ void expand(const Raw& r, float (&v)[16]) const {
        LoadBF16{x, ld}.expand(r.x, v);
        if (colscale) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 w = r.c[j];
                v[4 * j + 0] = bf16_round(v[4 * j + 0] * bf16_round(w.x));
                v[4 * j + 1] = bf16_round(v[4 * j + 1] * bf16_round(w.y));
                v[4 * j + 2] = bf16_round(v[4 * j + 2] * bf16_round(w.z));
                v[4 * j + 3] = bf16_round(v[4 * j + 3] * bf16_round(w.w));
            }
        }
    }
    __device__ __forceinline__ void operator()(int64_t row, int col, float (&v)[16]) const {
        expand(fetch(row, col), v);
    }
};

// int8 weight times its row scale, rounded to bf16 (src/xpuint8.cpp:98-107).
struct LoadDequantWeight {
    const int8_t* w8;
    int64_t ld;
    const float* scale;
    struct Raw { int4 a; float s; };
    __device__ __forceinline__ Raw fetch(int64_t row, int col) const {
        return Raw{*reinterpret_cast<const int4*>(w8 + row * ld + col), scale[row]};
    }
    __device__ __forceinline__ LoadDequantWeight rebase(int64_t row0) const {
        return {w8 + row0 * ld, ld, scale + row0};
    }
    __device__ __forceinline__ Raw fetch_r(int r, int col) const {
        return Raw{*reinterpret_cast<const int4*>(at32(w8, r, ld, col)), scale[r]};
    }
    __device__ __forceinline__ void expand(const Raw& r, float (&v)[16]) const {
        const uint32_t w[4] = {uint32_t(r.a.x), uint32_t(r.a.y), uint32_t(r.a.z), uint32_t(r.a.w)};
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int8_t b = int8_t((w[j >> 2] >> (8 * (j & 3))) & 0xFF);
            v[j] = bf16_round(float(b) * r.s);
        }
    }
    __device__ __forceinline__ void operator()(int64_t row, int col, float (&v)[16]) const {
        expand(fetch(row, col), v);
    }
};

// --------------------------------------------------------------- quantizers
enum QMode : int {
    kRecip = 0,     // ConvRot quantizer: rint(v * (1/s)), s = max(rowmax/127, 1e-30)
                    //   (src/xpuint8.cpp:264-276, 494-498)
    kDivide = 1,    // torch chain: rint(v / s) with IEEE division (ops.py:320-330)
    kPrepare = 2,   // prepare_weight: v rounded to bf16 first, the floor is
                    //   bf16(1e-30), rint(v / s) (ops.py:93-99)
};

__device__ __forceinline__ float row_scale(int mode, float rowmax) {
    if (mode == kPrepare) {
        // bf16(1e-30f) = 0x0DA2 << 16
        return div127_rn(fmaxf(rowmax, __uint_as_float(0x0DA20000u)));
    }
    return fmaxf(div127_rn(rowmax), 1e-30f);
}

// Quantize 16 values: the values themselves unless ROT, in which case the
// rotation is u * dom (dom = 1/16 for the unscaled transform's sums, 1 for the
// scaled one's).
template <bool ROT, int MODE>
__device__ __forceinline__ uint4 quant16(const float (&u)[16], float s, float inv, float dom) {
    if constexpr (MODE == kRecip) {
        // rint(fl(u/16) * inv) == rint(u * fl(inv/16)): both products are exact
        // power-of-two rescalings of the same rounded product.
        const float k = ROT ? inv * dom : inv;
        float a[8], b[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            a[t] = u[t] * k;
            b[t] = u[t + 8] * k;
        }
        const uint2 lo = rint_pack8(a), hi = rint_pack8(b);
        return make_uint4(lo.x, lo.y, hi.x, hi.y);
    } else {
        uint32_t b[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            float x = ROT ? u[t] * dom : u[t];
            if (MODE == kPrepare) x = bf16_round(x);
            b[t] = rint_bits(rint_div(x, s, inv));
        }
        uint4 r;
        r.x = pack4(b[0], b[1], b[2], b[3]);
        r.y = pack4(b[4], b[5], b[6], b[7]);
        r.z = pack4(b[8], b[9], b[10], b[11]);
        r.w = pack4(b[12], b[13], b[14], b[15]);
        return r;
    }
}

// Running max of |u| over 16 raw values.
__device__ __forceinline__ float absmax16(const float (&u)[16], float m) {
#pragma unroll
    for (int t = 0; t < 16; ++t) m = fmaxf(m, fabsf(u[t]));
    return m;
}

// Rotate one lane's register of each of its P groups in place, choosing the
// transform for the whole wave: the unscaled one unless some input of the
// wave is at or above kUnscaledLimit (common.hpp), then the reference's scaled
// one.  Returns dom, the factor from the values left in v to the rotation
// (1/16 or 1), which the callers apply to the row max and in the quantizer;
// both products are exact (a power of two on a value that neither overflows
// nor rounds in the subnormal range).
template <int P>
__device__ __forceinline__ float rotate_groups(float (&v)[P][16], const XlaneSigns& sgn) {
    float mi = 0.f;
#pragma unroll
    for (int p = 0; p < P; ++p) mi = inmax16(v[p], mi);
    if (__builtin_expect(wave_needs_scaled(mi), 0)) {
#pragma unroll
        for (int p = 0; p < P; ++p) hadamard16_scaled(v[p], sgn);
        return 1.0f;
    }
#pragma unroll
    for (int p = 0; p < P; ++p) hadamard16_unscaled(v[p], sgn);
    return 0.0625f;
}

// The row max of the values the quantizer sees, from the max of the rotated
// (or, without ROT, raw) ones: bf16 rounding (kPrepare) is monotone
// non-decreasing, so f(max|u|) == max f(|u|) and one application suffices.
template <int MODE>
__device__ __forceinline__ float finish_max(float x) {
    if (MODE == kPrepare) x = bf16_round(x);
    return x;
}

// Segmented row kernel.  A segment is 16 lanes holding P (1 or 2) whole
// 256-groups of one row (lane L of the segment loads register lane_w(L) of
// each of its groups and stores register lane_w_rot(L)); a row is S = G/P consecutive segments and a block is
// R whole rows, so R*S*16 threads (rounded up to whole waves with idle
// padding segments).  The row is register-resident (16P floats per lane):
// the group maxima are reduced inside the segment with DPP, combined across
// the row's segments with one LDS atomic max per segment, and the row is
// then quantized from registers and stored with one 16-byte store per group.
//
// Lanes with no row of their own (padding segments, rows past M) load a valid
// row anyway (row M-1), so the loads need no branch; they publish nothing and
// store nothing.  When FULL (K % 256 == 0, every rotating kernel) no column
// is masked either; otherwise columns past K read as zeros.
constexpr int kMaxSegments = 64;     // 1024 threads

// s_barrier after this wave's LDS operations have completed, without waiting
// for its outstanding global loads (which __syncthreads() would).  The
// "memory" clobber keeps the compiler from moving memory operations across.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int P, bool ROT, int MODE, bool FULL, class Loader, bool TILED = false>
__global__ __launch_bounds__(1024) void rowquant_seg_kernel(Loader load, int8_t* __restrict__ q,
                                                           float* __restrict__ scale, int64_t M,
                                                           int K, int S, int R, int s_mul) {
    __shared__ uint32_t row_max[kMaxSegments];
    // (one group per lane only: with two, the paired dequant loaders would
    // exceed the register budget)
    constexpr int NW = P == 1 ? LoaderWins<Loader>::value : 0;
    __shared__ __align__(16) uint16_t win[NW > 0 ? NW * kRowWinSize : 8];
    // each window is CH chunks of 64 16-byte units; a wave copies a chunk with
    // one global -> LDS DMA (no registers staged), the block's waves taking
    // the NW * CH chunks in turn, before the row is read
#if defined(__HIP_DEVICE_COMPILE__)
    if constexpr (NW > 0) {
        constexpr int CH = kRowWinUnits / 64;
        const int lane = threadIdx.x & 63;
        for (int c = threadIdx.x >> 6; c < NW * CH; c += blockDim.x >> 6) {
            const int w = c / CH, u = 64 * (c - w * CH);
            __builtin_amdgcn_global_load_lds(
                win_unit(load.tab, Loader::win_tab(w), u + lane),
                (__attribute__((address_space(3))) void*)(win + w * kRowWinSize + 8 * u), 16, 0, 0);
        }
    }
#endif
    const int seg = threadIdx.x >> 4;
    const int sl = threadIdx.x & 15;
    const int r = int(__umul24(seg, s_mul)) >> 12;   // seg / S (exact for seg, S <= 64)
    const int sg = seg - int(__umul24(r, S));        // segment within the row
    // addresses: the block's first row is wave-uniform, a lane's own row
    // offset r (clamped to the last row) is small
    const int64_t row0 = int64_t(blockIdx.x) * R;
    const bool live = r < R && row0 + r < M;
    const int r_ld = min(r, int(min(M - 1 - row0, int64_t(R - 1))));
    const Loader lb = load.rebase(row0);
    int col[P];
    typename Loader::Raw raw[P];
    float v[P][16];
    constexpr bool EARLY = NW == 0 && LoaderEarly<Loader>::value;
    const XlaneSigns sgn = xlane_signs(sl);
#pragma unroll
    for (int p = 0; p < P; ++p) {
        col[p] = (sg * P + p) * kGroup + lane_w(sl) * 16;
        if constexpr (FULL) {
            raw[p] = lb.fetch_r(r_ld, col[p]);
        } else {
            raw[p] = typename Loader::Raw{};
            if (col[p] < K) raw[p] = lb.fetch_r(r_ld, col[p]);
        }
        if constexpr (EARLY) lb.expand(raw[p], v[p]);
    }
    if (threadIdx.x < R) row_max[threadIdx.x] = 0u;
    // every wave's window DMAs have landed before the barrier (this waits for
    // the row's reads too, which the next step needs anyway)
    if constexpr (NW > 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();                               // the zeros (and windows) land before any use
#pragma unroll
    for (int p = 0; p < P; ++p) {
        if constexpr (NW > 0) lb.expand_w(raw[p], v[p], win);
        else if constexpr (!EARLY) lb.expand(raw[p], v[p]);
    }
    float dom = 1.0f;
    if constexpr (ROT) dom = rotate_groups<P>(v, sgn);
    float m = 0.f;
#pragma unroll
    for (int p = 0; p < P; ++p) m = absmax16(v[p], m);
    if constexpr (ROT) m *= dom;
    // m >= 0 (never NaN), so its bit pattern orders like its value
    const uint32_t mb = segment_max_bits(__float_as_uint(m));
    if (live && sl == 0) atomicMax(&row_max[r], mb);
    lds_barrier();
    if (!live) return;
    const float rowmax = __uint_as_float(row_max[r]);
    const float sc = row_scale(MODE, finish_max<MODE>(rowmax));
    const float inv = rcp_rn(sc);
    if (sg == 0 && sl == 0) scale[row0 + r] = sc;
    int8_t* const qrow = q + row0 * K;
    // the transform leaves register lane_w_rot(sl) of the group in the lane
    const int dcol = ROT ? (lane_w_rot(sl) - lane_w(sl)) * 16 : 0;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint4 w = quant16<ROT, MODE>(v[p], sc, inv, dom);
        if (FULL || col[p] < K) {
            if constexpr (TILED)
                *reinterpret_cast<uint4*>(q + tiled_offset(row0 + r, col[p] + dcol, (K + 63) / 64)) = w;
            else
                *reinterpret_cast<uint4*>(at32(qrow, r, K, col[p] + dcol)) = w;
        }
    }
}

// Column-scaled rows (quantize_row with a column scale, e.g. linear_dx_int8's
// dy): each lane owns 16 consecutive columns and a block takes RL rows
// through the same lanes, so a lane loads its 16 fp32 column scales -- twice
// the bytes of the bf16 row piece they scale -- and rounds them to bf16 once
// for RL rows instead of once per row.  The arithmetic is LoadColScaled's and
// the kDivide quantizer's: bf16(x * bf16(w)), the row max of |.| (one LDS slot
// per row, one atomic max per 16 lanes), then rint(v / s).  Lanes past N load
// column 0 and store nothing; rows past M load row M - 1 and store nothing.
template <int RL, bool TILED>
__global__ __launch_bounds__(1024) void rowquant_cs_kernel(const uint16_t* __restrict__ x,
                                                          const float* __restrict__ colscale,
                                                          int8_t* __restrict__ q,
                                                          float* __restrict__ scale, int64_t M,
                                                          int N) {
    __shared__ uint32_t row_max[RL];
    const int lc = int(threadIdx.x) * 16;
    const bool has = lc < N;
    const int col = has ? lc : 0;
    const int64_t row0 = int64_t(blockIdx.x) * RL;
    // the scales first, then every row: a row's values wait only for it
    const float4* cp = reinterpret_cast<const float4*>(colscale + col);
    const float4 c0 = cp[0], c1 = cp[1], c2 = cp[2], c3 = cp[3];
    LoadBF16::Raw raw[RL];
#pragma unroll
    for (int r = 0; r < RL; ++r)
        raw[r] = LoadBF16{x, N}.fetch(min(row0 + r, M - 1), col);
    if (threadIdx.x < RL) row_max[threadIdx.x] = 0u;
    // bf16(w), each packing conversion rounding two scales
    const uint32_t wp[8] = {pack_bf16x2(c0.x, c0.y), pack_bf16x2(c0.z, c0.w),
                            pack_bf16x2(c1.x, c1.y), pack_bf16x2(c1.z, c1.w),
                            pack_bf16x2(c2.x, c2.y), pack_bf16x2(c2.z, c2.w),
                            pack_bf16x2(c3.x, c3.y), pack_bf16x2(c3.z, c3.w)};
    lds_barrier();                               // the zeroed maxima land before any atomic
    uint32_t vp[RL][8];                          // bf16(x * bf16(w)), packed pairs
#pragma unroll
    for (int r = 0; r < RL; ++r) {
        float v[16];
        LoadBF16{x, N}.expand(raw[r], v);
        float m = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t p = pack_bf16x2(v[2 * j] * __uint_as_float(wp[j] << 16),
                                           v[2 * j + 1] * __uint_as_float(wp[j] & 0xFFFF0000u));
            vp[r][j] = p;
            m = fmaxf(m, fabsf(__uint_as_float(p << 16)));
            m = fmaxf(m, fabsf(__uint_as_float(p & 0xFFFF0000u)));
        }
        if (!has) m = 0.f;
        // m >= 0 (never NaN), so its bit pattern orders like its value
        const uint32_t mb = segment_max_bits(__float_as_uint(m));
        if ((threadIdx.x & 15) == 0) atomicMax(&row_max[r], mb);
    }
    lds_barrier();
    const int KB = (N + 63) / 64;
#pragma unroll
    for (int r = 0; r < RL; ++r) {
        const int64_t row = row0 + r;
        if (row >= M) break;
        const float sc = row_scale(kDivide, __uint_as_float(row_max[r]));
        const float inv = rcp_rn(sc);
        if (threadIdx.x == 0) scale[row] = sc;
        float v[16];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            v[2 * j] = __uint_as_float(vp[r][j] << 16);
            v[2 * j + 1] = __uint_as_float(vp[r][j] & 0xFFFF0000u);
        }
        const uint4 w = quant16<false, kDivide>(v, sc, inv, 1.0f);
        if (has) {
            if constexpr (TILED)
                *reinterpret_cast<uint4*>(q + tiled_offset(row, col, KB)) = w;
            else
                *reinterpret_cast<uint4*>(q + row * N + col) = w;
        }
    }
}

// The column-scaled kernel's rows per block, and whether it takes a shape:
// whole 16-column pieces, one lane each, at most one block's 1024 lanes.
constexpr int kColScaledRows = 2;
inline bool colscaled_rows_applies(int N) { return N % 16 == 0 && N > 0 && N <= 16 * 1024; }

template <bool TILED>
hipError_t launch_colscaled(hipStream_t st, const uint16_t* x, const float* colscale, int8_t* q,
                            float* scale, int64_t M, int N) {
    const int threads = ((N / 16 + 63) / 64) * 64;
    const dim3 grid(unsigned((M + kColScaledRows - 1) / kColScaledRows));
    const dim3 block{unsigned(threads)};
    hipLaunchKernelGGL((rowquant_cs_kernel<kColScaledRows, TILED>), grid, block, 0, st, x,
                       colscale, q, scale, M, N);
    return hipGetLastError();
}

// Rows too long for registers: pass 1 finds the row max, pass 2 recomputes
// each slot (the re-read comes from L2) and stores it.
template <bool ROT, int MODE, class Loader>
__global__ __launch_bounds__(256) void rowquant_2pass_kernel(Loader load, int8_t* __restrict__ q,
                                                            float* __restrict__ scale,
                                                            int64_t M, int K) {
    const int lane = threadIdx.x & 63;
    const int64_t row = int64_t(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= M) return;
    const int slots = (K + 1023) / 1024;
    const XlaneSigns sgn = xlane_signs(lane & 15);
    const int w_in = lane_w(lane & 15), w_st = ROT ? lane_w_rot(lane & 15) : w_in;
    float m = 0.f;
    for (int s = 0; s < slots; ++s) {
        float v[1][16];
        const int col = s * 1024 + (lane >> 4) * kGroup + w_in * 16;
        if (col < K) load(row, col, v[0]);
        else {
#pragma unroll
            for (int t = 0; t < 16; ++t) v[0][t] = 0.f;
        }
        if constexpr (ROT) {
            const float dom = rotate_groups<1>(v, sgn);
            m = fmaxf(m, absmax16(v[0], 0.f) * dom);
        } else {
            m = absmax16(v[0], m);
        }
    }
    const float rowmax = finish_max<MODE>(wave_max(m));
    const float sc = row_scale(MODE, rowmax);
    const float inv = rcp_rn(sc);
    if (lane == 0) scale[row] = sc;
    for (int s = 0; s < slots; ++s) {
        float v[1][16];
        const int col = s * 1024 + (lane >> 4) * kGroup + w_in * 16;
        if (col < K) load(row, col, v[0]);
        else {
#pragma unroll
            for (int t = 0; t < 16; ++t) v[0][t] = 0.f;
        }
        float dom = 1.0f;
        if constexpr (ROT) dom = rotate_groups<1>(v, sgn);
        const uint4 r = quant16<ROT, MODE>(v[0], sc, inv, dom);
        const int cst = col + (w_st - w_in) * 16;   // same 256-group as col
        if (cst < K) *reinterpret_cast<uint4*>(q + row * K + cst) = r;
    }
}

// Launch shape of the segmented kernel for a row of G groups: P = 1 (one
// group per lane; measured fastest on MI355X at K = 5120, ahead of P = 2 and
// of several rows per block) unless G > kMaxSegments, then P = 2 for even G;
// S = G/P; then R rows per block with R*S a multiple of 4 (whole waves) near
// 16 segments (256 threads) or, when that would exceed kMaxSegments, one row
// padded to whole waves.  nseg is the block's segment count.  Returns false
// when no P fits (rows longer than 128 groups, or odd and longer than 64).
inline bool seg_shape(int G, int& P, int& S, int& R, int& nseg) {
    P = (G > kMaxSegments && G % 2 == 0) ? 2 : 1;
    S = G / P;
    if (S > kMaxSegments) return false;
    int rmin = 4;
    while (rmin > 1 && (S * (rmin / 2)) % 4 == 0) rmin /= 2;
    if (rmin * S <= kMaxSegments) {
        R = rmin;
        while (R * 2 * S <= 16) R *= 2;
        nseg = R * S;
    } else {
        R = 1;
        nseg = (S + 3) & ~3;
    }
    return true;
}

template <int P, bool ROT, int MODE, bool FULL, class Loader, bool TILED = false>
void launch_seg(hipStream_t st, const Loader& ld, int8_t* q, float* scale, int64_t M, int K,
                int S, int R, int nseg) {
    const dim3 grid(unsigned((M + R - 1) / R)), block(unsigned(nseg * 16));
    const int s_mul = (4096 + S - 1) / S;
    hipLaunchKernelGGL((rowquant_seg_kernel<P, ROT, MODE, FULL, Loader, TILED>), grid, block, 0,
                       st, ld, q, scale, M, K, S, R, s_mul);
}

// TILED: q in the MFMA block layout (tiled_offset); only for rows that the
// segmented kernel takes (rowquant_can_tile)
template <bool ROT, int MODE, class Loader, bool TILED = false>
hipError_t launch_rowquant(hipStream_t st, const Loader& ld, int8_t* q, float* scale, int64_t M,
                           int K) {
    const int G = (K + kGroup - 1) / kGroup;
    int P, S, R, nseg;
    if (seg_shape(G, P, S, R, nseg)) {
        if constexpr (ROT) {     // rotating entry points guarantee K % 256 == 0
            if (P == 2) launch_seg<2, ROT, MODE, true, Loader, TILED>(st, ld, q, scale, M, K, S, R, nseg);
            else        launch_seg<1, ROT, MODE, true, Loader, TILED>(st, ld, q, scale, M, K, S, R, nseg);
        } else {
            const bool full = K % kGroup == 0;
            if (P == 2) {
                if (full) launch_seg<2, ROT, MODE, true, Loader, TILED>(st, ld, q, scale, M, K, S, R, nseg);
                else      launch_seg<2, ROT, MODE, false, Loader, TILED>(st, ld, q, scale, M, K, S, R, nseg);
            } else {
                if (full) launch_seg<1, ROT, MODE, true, Loader, TILED>(st, ld, q, scale, M, K, S, R, nseg);
                else      launch_seg<1, ROT, MODE, false, Loader, TILED>(st, ld, q, scale, M, K, S, R, nseg);
            }
        }
    } else if constexpr (TILED) {
        return hipErrorInvalidValue;    // callers check rowquant_can_tile
    } else {
        const dim3 grid(unsigned((M + kRowsPerBlock - 1) / kRowsPerBlock)), block(256);
        hipLaunchKernelGGL((rowquant_2pass_kernel<ROT, MODE, Loader>), grid, block, 0, st, ld, q,
                           scale, M, K);
    }
    return hipGetLastError();
}

// ------------------------------------------------------------ rotate only
// Every 256-group is independent, so the tensor is a flat list of M*K/256
// groups (K % 256 == 0); a 16-lane segment rotates one group at a time, a
// block's 16 segments take 16 consecutive groups per grid-stride step.
template <class Loader>
__global__ __launch_bounds__(256) void rotate_kernel(Loader load, uint16_t* __restrict__ out,
                                                     int64_t M, int K) {
    const int sl = threadIdx.x & 15;
    const XlaneSigns sgn = xlane_signs(sl);
    const int w_out = lane_w_rot(sl);
    const int64_t G = K / kGroup;
    const int64_t total = M * G;
    for (int64_t g = int64_t(blockIdx.x) * 16 + (threadIdx.x >> 4); g < total;
         g += int64_t(gridDim.x) * 16) {
        const int64_t row = g / G;
        const int gcol = int(g - row * G) * kGroup;
        float v[1][16];
        load(row, gcol + lane_w(sl) * 16, v[0]);
        const float dom = rotate_groups<1>(v, sgn);
        const float* u = v[0];
        const int col = gcol + w_out * 16;
        uint4 a, b;
        a.x = pack_bf16x2(u[0] * dom, u[1] * dom);
        a.y = pack_bf16x2(u[2] * dom, u[3] * dom);
        a.z = pack_bf16x2(u[4] * dom, u[5] * dom);
        a.w = pack_bf16x2(u[6] * dom, u[7] * dom);
        b.x = pack_bf16x2(u[8] * dom, u[9] * dom);
        b.y = pack_bf16x2(u[10] * dom, u[11] * dom);
        b.z = pack_bf16x2(u[12] * dom, u[13] * dom);
        b.w = pack_bf16x2(u[14] * dom, u[15] * dom);
        uint4* p = reinterpret_cast<uint4*>(out + row * K + col);
        p[0] = a;
        p[1] = b;
    }
}

// The loop exit can differ between the segments of a wave on the last step;
// that is safe because the butterfly only exchanges lanes inside a segment
// (DPP lane xors 1, 3, 7 and 8), whose 16 lanes always share g, and the
// choice of transform is a ballot over the lanes still in the loop.
template <class Loader>
hipError_t launch_rotate(hipStream_t st, const Loader& ld, uint16_t* out, int64_t M, int K) {
    const int64_t groups = M * (K / kGroup);
    int64_t blocks = (groups + 15) / 16;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL((rotate_kernel<Loader>), dim3(unsigned(blocks)), dim3(256), 0, st, ld,
                       out, M, K);
    return hipGetLastError();
}


// ------------------------------------------------------------ column sums
// out[n] = bf16(sum over m of x[m, n]) for bf16 x [M, N] (N % 8 == 0), the
// bias gradient dy.sum(dim=0) of the reference's backward
// (python/xpu_kernels/int8/ops.py:276), in a fixed order: fp32 sums of
// kColChunk consecutive rows, each in row order (colsum_part_kernel: a lane
// takes 8 columns, 16-byte loads, one chunk of rows), then the chunk sums
// (colsum_final_kernel): eight interleaved running sums, sum w over chunks w,
// w + 8, w + 16, ... in order, added in the order w = 0..7; one rounding to
// bf16.  HBM-bound: one
// read of x plus 4 bytes per column per chunk of partials.
constexpr int kColChunk = 32, kColCols = 2048;

// Chunk c of rows for every block row c = blockIdx.y, blockIdx.y + gridDim.y, ...
// (the grid's y extent is capped at 65535).
__global__ __launch_bounds__(256) void colsum_part_kernel(const uint16_t* __restrict__ x,
                                                          float* __restrict__ part, int64_t M,
                                                          int N, int chunks) {
    const int n = blockIdx.x * kColCols + threadIdx.x * 8;
    if (n >= N) return;
    for (int c = blockIdx.y; c < chunks; c += gridDim.y) {
        const int64_t m0 = int64_t(c) * kColChunk;
        const int rows = int(min(int64_t(kColChunk), M - m0));
        const uint16_t* p = x + m0 * N + n;
        float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        // eight rows' loads in flight, summed in row order
        for (int r0 = 0; r0 < rows; r0 += 8) {
            uint4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (r0 + u < rows) v[u] = *reinterpret_cast<const uint4*>(p + int64_t(r0 + u) * N);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (r0 + u < rows) {
                    a[0] += bf16lo(v[u].x); a[1] += bf16hi(v[u].x);
                    a[2] += bf16lo(v[u].y); a[3] += bf16hi(v[u].y);
                    a[4] += bf16lo(v[u].z); a[5] += bf16hi(v[u].z);
                    a[6] += bf16lo(v[u].w); a[7] += bf16hi(v[u].w);
                }
            }
        }
        float* o = part + int64_t(c) * N + n;
        *reinterpret_cast<float4*>(o) = make_float4(a[0], a[1], a[2], a[3]);
        *reinterpret_cast<float4*>(o + 4) = make_float4(a[4], a[5], a[6], a[7]);
    }
}

// The chunk sums of 64 columns per block of 8 waves: wave w adds chunks w,
// w + 8, w + 16, ... in that order (all its loads issued first), then the
// eight wave sums are added in wave order.
// out_f32: the bf16-rounded sum written as the fp32 it widens to (exact), for a
// gradient whose parameter is fp32
__global__ __launch_bounds__(512) void colsum_final_kernel(const float* __restrict__ part,
                                                           void* __restrict__ out, int chunks,
                                                           int N, int out_f32) {
    __shared__ float t[8][64];
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int n = blockIdx.x * 64 + l;
    const int nc = min(n, N - 1);
    float a = 0.f;
    for (int c0 = w; c0 < chunks; c0 += 8 * 16) {
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int c = c0 + 8 * i;
            v[i] = c < chunks ? part[int64_t(c) * N + nc] : 0.f;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (c0 + 8 * i < chunks) a += v[i];
    }
    t[w][l] = a;
    __syncthreads();
    if (w == 0 && n < N) {
        float s = t[0][l];
#pragma unroll
        for (int i = 1; i < 8; ++i) s += t[i][l];
        const uint32_t b = f32_to_bf16_bits(s);
        if (out_f32) static_cast<uint32_t*>(out)[n] = b << 16;
        else static_cast<uint16_t*>(out)[n] = uint16_t(b);
    }
}

}  // namespace

// ------------------------------------------------------------------- entry
hipError_t convrot_quantize(hipStream_t st, const void* x, int8_t* q, float* scale, int64_t M,
                            int K, int act) {
    const uint16_t* xb = static_cast<const uint16_t*>(x);
    const uint16_t* tab = activation_tables();
    const int64_t in_ld = act_paired(act) ? 2 * int64_t(K) : K;
    switch (act) {
        case 0: return launch_rowquant<true, kRecip>(st, LoadBF16{xb, K}, q, scale, M, K);
        case 1: return launch_rowquant<true, kRecip>(st, LoadAct<1>{xb, in_ld, K, tab}, q, scale, M, K);
        case 2: return launch_rowquant<true, kRecip>(st, LoadAct<2>{xb, in_ld, K, tab}, q, scale, M, K);
        case 3: return launch_rowquant<true, kRecip>(st, LoadAct<3>{xb, in_ld, K, tab}, q, scale, M, K);
        case 4: return launch_rowquant<true, kRecip>(st, LoadAct<4>{xb, in_ld, K, tab}, q, scale, M, K);
        case 5: return launch_rowquant<true, kRecip>(st, LoadAct<5>{xb, in_ld, K, tab}, q, scale, M, K);
        default: return hipErrorInvalidValue;
    }
}

hipError_t dequant_act_quantize(hipStream_t st, const int32_t* acc, int64_t acc_ld, int8_t* q,
                                float* scale, const float* xs, const float* ws, int64_t M, int K,
                                int act) {
    const uint16_t* tab = activation_tables();
    switch (act) {
        case 3: return launch_rowquant<true, kRecip>(st, LoadDequantAct<3>{acc, acc_ld, K, xs, ws, tab}, q, scale, M, K);
        case 4: return launch_rowquant<true, kRecip>(st, LoadDequantAct<4>{acc, acc_ld, K, xs, ws, tab}, q, scale, M, K);
        case 5: return launch_rowquant<true, kRecip>(st, LoadDequantAct<5>{acc, acc_ld, K, xs, ws, tab}, q, scale, M, K);
        default: return hipErrorInvalidValue;
    }
}

hipError_t rotate_bf16(hipStream_t st, const void* x, void* out, int64_t M, int K) {
    return launch_rotate(st, LoadBF16{static_cast<const uint16_t*>(x), K},
                         static_cast<uint16_t*>(out), M, K);
}

hipError_t dequant_weight(hipStream_t st, const int8_t* w8, const float* scale, void* out,
                          int64_t N, int K) {
    return launch_rotate(st, LoadDequantWeight{w8, K, scale}, static_cast<uint16_t*>(out), N, K);
}

hipError_t prepare_weight(hipStream_t st, const void* w, int8_t* q, float* scale, int64_t N,
                          int K) {
    return launch_rowquant<true, kPrepare>(st, LoadBF16{static_cast<const uint16_t*>(w), K}, q,
                                           scale, N, K);
}

hipError_t quantize_row(hipStream_t st, const void* x, const float* colscale, int8_t* q,
                        float* scale, int64_t M, int N, bool tiled) {
    if (colscale && colscaled_rows_applies(N)) {
        const uint16_t* xb = static_cast<const uint16_t*>(x);
        if (tiled) return launch_colscaled<true>(st, xb, colscale, q, scale, M, N);
        return launch_colscaled<false>(st, xb, colscale, q, scale, M, N);
    }
    const LoadColScaled ld{static_cast<const uint16_t*>(x), N, colscale};
    if (tiled) return launch_rowquant<false, kDivide, LoadColScaled, true>(st, ld, q, scale, M, N);
    return launch_rowquant<false, kDivide>(st, ld, q, scale, M, N);
}

bool rowquant_can_tile(int K) {
    int P, S, R, nseg;
    return seg_shape((K + kGroup - 1) / kGroup, P, S, R, nseg);
}

hipError_t convrot_quantize_tiled(hipStream_t st, const void* x, int8_t* q, float* scale,
                                  int64_t M, int K) {
    return launch_rowquant<true, kRecip, LoadBF16, true>(
        st, LoadBF16{static_cast<const uint16_t*>(x), K}, q, scale, M, K);
}

int64_t colsum_work_bytes(int64_t M, int64_t N) {
    return ((M + kColChunk - 1) / kColChunk) * N * 4;
}

hipError_t column_sum_bf16(hipStream_t st, const void* x, void* out, int64_t M, int N,
                           float* part, bool out_f32) {
    const int chunks = int((M + kColChunk - 1) / kColChunk);
    hipLaunchKernelGGL(colsum_part_kernel, dim3(unsigned((N + kColCols - 1) / kColCols),
                                                unsigned(min(chunks, 65535))),
                       dim3(256), 0, st, static_cast<const uint16_t*>(x), part, M, N, chunks);
    if (const hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    hipLaunchKernelGGL(colsum_final_kernel, dim3(unsigned((N + 63) / 64)), dim3(512), 0, st, part,
                       out, chunks, N, out_f32 ? 1 : 0);
    return hipGetLastError();
}

}  // namespace xpuint8
