// Row-wise ConvRot kernels: rotate+quantize (with optional fused activation or
// fused dequant+activation), rotate only, the gradient row quantizer, the
// weight preparation and the weight dequantization.
//
// Work decomposition (all kernels): a wave64 owns one row.  A "slot" is 1024
// consecutive elements of the row: 64 lanes x 16 elements, i.e. four 256-point
// ConvRot groups with 16 lanes per group, lane L of a group holding elements
// [16L, 16L+16) -- the register/lane assignment of the reference's sub-group
// kernel (src/xpuint8.cpp:406-438).  The whole row stays in registers (SLOTS x
// 16 floats per lane), the row absmax is a wave reduction (no LDS, no
// barrier), then the row is quantized and stored with one 16-byte store per
// slot.  Rows longer than kMaxSlots*1024 use the two-pass variant, which
// re-reads the row (from L2) to quantize it.
#include "common.hpp"
#include "kernels.hpp"
#include "activations.hpp"

namespace xpuint8 {
namespace {

constexpr int kRowsPerBlock = 4;     // 4 waves = 4 rows per 256-thread block

// ------------------------------------------------------------------ loaders
// A loader fills v[16] with the pre-rotation values of elements
// [col, col+16) of a row, as bf16-valued floats.

struct LoadBF16 {
    const uint16_t* x;
    int64_t ld;
    __device__ __forceinline__ void operator()(int64_t row, int col, float (&v)[16]) const {
        const uint16_t* p = x + row * ld + col;
        const u32x4 a = load16_nt(p);
        const u32x4 b = load16_nt(p + 8);
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) { v[2 * j] = bf16lo(w[j]); v[2 * j + 1] = bf16hi(w[j]); }
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
    __device__ __forceinline__ void operator()(int64_t row, int col, float (&v)[16]) const {
        float a[16];
        LoadBF16{x, ld}(row, col, a);
        if constexpr (act_paired(ACT)) {
            float b[16];
            LoadBF16{x + half, ld}(row, col, b);
#pragma unroll
            for (int t = 0; t < 16; ++t) v[t] = activate<ACT>(tab, a[t], b[t]);
        } else {
#pragma unroll
            for (int t = 0; t < 16; ++t) v[t] = activate<ACT>(tab, a[t], 0.f);
        }
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
            const i32x4 a = load16_nt_i(p + 4 * j);
            const float4 w = q[j];
            o[4 * j + 0] = bf16_round(float(a.x) * (w.x * xsr));
            o[4 * j + 1] = bf16_round(float(a.y) * (w.y * xsr));
            o[4 * j + 2] = bf16_round(float(a.z) * (w.z * xsr));
            o[4 * j + 3] = bf16_round(float(a.w) * (w.w * xsr));
        }
    }
    __device__ __forceinline__ void operator()(int64_t row, int col, float (&v)[16]) const {
        const float xsr = xs[row];
        float h[16];
        deq(row, col, xsr, h);
        if constexpr (act_paired(ACT)) {
            float g[16];
            deq(row, col + half, xsr, g);
#pragma unroll
            for (int t = 0; t < 16; ++t) v[t] = activate<ACT>(tab, h[t], g[t]);
        } else {
#pragma unroll
            for (int t = 0; t < 16; ++t) v[t] = activate<ACT>(tab, h[t], 0.f);
        }
    }
};

// bf16(bf16(dy) * bf16(ws[n])): the column-scaled gradient of linear_dx_int8
// (python/xpu_kernels/int8/ops.py:366).  The product of two bf16 values is
// exact in fp32, so this is one rounding.
struct LoadColScaled {
    const uint16_t* x;
    int64_t ld;
    const float* colscale;   // may be null: plain bf16 rows
    __device__ __forceinline__ void operator()(int64_t row, int col, float (&v)[16]) const {
        LoadBF16{x, ld}(row, col, v);
        if (colscale) {
            const float4* q = reinterpret_cast<const float4*>(colscale + col);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 w = q[j];
                v[4 * j + 0] = bf16_round(v[4 * j + 0] * bf16_round(w.x));
                v[4 * j + 1] = bf16_round(v[4 * j + 1] * bf16_round(w.y));
                v[4 * j + 2] = bf16_round(v[4 * j + 2] * bf16_round(w.z));
                v[4 * j + 3] = bf16_round(v[4 * j + 3] * bf16_round(w.w));
            }
        }
    }
};

// int8 weight times its row scale, rounded to bf16 (src/xpuint8.cpp:98-107).
struct LoadDequantWeight {
    const int8_t* w8;
    int64_t ld;
    const float* scale;
    __device__ __forceinline__ void operator()(int64_t row, int col, float (&v)[16]) const {
        const int4 a = *reinterpret_cast<const int4*>(w8 + row * ld + col);
        const float s = scale[row];
        const uint32_t w[4] = {uint32_t(a.x), uint32_t(a.y), uint32_t(a.z), uint32_t(a.w)};
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int8_t b = int8_t((w[j >> 2] >> (8 * (j & 3))) & 0xFF);
            v[j] = bf16_round(float(b) * s);
        }
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
        return fmaxf(rowmax, __uint_as_float(0x0DA20000u)) / 127.0f;
    }
    return fmaxf(rowmax / 127.0f, 1e-30f);
}

// Quantize 16 values (already in their final scaled form unless ROT, in which
// case they are the unscaled Hadamard sums: the rotation is u/16).
template <bool ROT, int MODE>
__device__ __forceinline__ uint4 quant16(const float (&u)[16], float s, float inv) {
    uint32_t b[16];
    if constexpr (MODE == kRecip) {
        // rint(fl(u/16) * inv) == rint(u * fl(inv/16)): both products are exact
        // power-of-two rescalings of the same rounded product.
        const float k = ROT ? inv * 0.0625f : inv;
#pragma unroll
        for (int t = 0; t < 16; ++t) b[t] = rint_bits(u[t] * k);
    } else {
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            float x = ROT ? u[t] * 0.0625f : u[t];
            if (MODE == kPrepare) x = bf16_round(x);
            b[t] = rint_bits(rint_div(x, s, inv));
        }
    }
    uint4 r;
    r.x = pack4(b[0], b[1], b[2], b[3]);
    r.y = pack4(b[4], b[5], b[6], b[7]);
    r.z = pack4(b[8], b[9], b[10], b[11]);
    r.w = pack4(b[12], b[13], b[14], b[15]);
    return r;
}

template <bool ROT, int MODE>
__device__ __forceinline__ float absmax16(const float (&u)[16], float m) {
#pragma unroll
    for (int t = 0; t < 16; ++t) {
        float x = ROT ? u[t] * 0.0625f : u[t];
        if (MODE == kPrepare) x = bf16_round(x);
        m = fmaxf(m, fabsf(x));
    }
    return m;
}

// One wave per row, the whole row in registers.
template <int SLOTS, bool ROT, int MODE, class Loader>
__global__ __launch_bounds__(256) void rowquant_kernel(Loader load, int8_t* __restrict__ q,
                                                      float* __restrict__ scale, int64_t M,
                                                      int K) {
    const int lane = threadIdx.x & 63;
    const int64_t row = int64_t(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= M) return;                       // whole wave leaves together
    float v[SLOTS][16];
    float m = 0.f;
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        const int col = s * 1024 + lane * 16;
        if (col < K) {
            load(row, col, v[s]);
        } else {
#pragma unroll
            for (int t = 0; t < 16; ++t) v[s][t] = 0.f;
        }
        if constexpr (ROT) hadamard16_unscaled(v[s]);   // every lane takes part
        m = absmax16<ROT, MODE>(v[s], m);
    }
    const float rowmax = wave_max(m);
    const float sc = row_scale(MODE, rowmax);
    const float inv = 1.0f / sc;
    if (lane == 0) scale[row] = sc;
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        const int col = s * 1024 + lane * 16;
        const uint4 r = quant16<ROT, MODE>(v[s], sc, inv);
        if (col < K) *reinterpret_cast<uint4*>(q + row * K + col) = r;
    }
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
    float m = 0.f;
    for (int s = 0; s < slots; ++s) {
        float v[16];
        const int col = s * 1024 + lane * 16;
        if (col < K) load(row, col, v);
        else {
#pragma unroll
            for (int t = 0; t < 16; ++t) v[t] = 0.f;
        }
        if constexpr (ROT) hadamard16_unscaled(v);
        m = absmax16<ROT, MODE>(v, m);
    }
    const float rowmax = wave_max(m);
    const float sc = row_scale(MODE, rowmax);
    const float inv = 1.0f / sc;
    if (lane == 0) scale[row] = sc;
    for (int s = 0; s < slots; ++s) {
        float v[16];
        const int col = s * 1024 + lane * 16;
        if (col < K) load(row, col, v);
        else {
#pragma unroll
            for (int t = 0; t < 16; ++t) v[t] = 0.f;
        }
        if constexpr (ROT) hadamard16_unscaled(v);
        const uint4 r = quant16<ROT, MODE>(v, sc, inv);
        if (col < K) *reinterpret_cast<uint4*>(q + row * K + col) = r;
    }
}

template <bool ROT, int MODE, class Loader>
hipError_t launch_rowquant(hipStream_t st, const Loader& ld, int8_t* q, float* scale, int64_t M,
                           int K) {
    const dim3 grid(unsigned((M + kRowsPerBlock - 1) / kRowsPerBlock)), block(256);
    const int slots = (K + 1023) / 1024;
    switch (slots) {
#define XPU_SLOT(n)                                                                     \
    case n:                                                                             \
        hipLaunchKernelGGL((rowquant_kernel<n, ROT, MODE, Loader>), grid, block, 0, st, \
                           ld, q, scale, M, K);                                         \
        break;
        XPU_SLOT(1) XPU_SLOT(2) XPU_SLOT(3) XPU_SLOT(4) XPU_SLOT(5) XPU_SLOT(6) XPU_SLOT(7)
        XPU_SLOT(8)
#undef XPU_SLOT
        default:
            hipLaunchKernelGGL((rowquant_2pass_kernel<ROT, MODE, Loader>), grid, block, 0, st,
                               ld, q, scale, M, K);
    }
    return hipGetLastError();
}

// ------------------------------------------------------------ rotate only
// Every 256-group is independent, so the tensor is a flat list of groups;
// a wave takes four groups (one slot) at a time.
template <class Loader>
__global__ __launch_bounds__(256) void rotate_kernel(Loader load, uint16_t* __restrict__ out,
                                                     int64_t M, int K) {
    const int lane = threadIdx.x & 63;
    const int64_t slots_per_row = (K + 1023) / 1024;
    const int64_t total = M * slots_per_row;
    const int64_t wave = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int64_t nwaves = int64_t(gridDim.x) * 4;
    for (int64_t w = wave; w < total; w += nwaves) {
        const int64_t row = w / slots_per_row;
        const int col = int(w - row * slots_per_row) * 1024 + lane * 16;
        float v[16];
        if (col < K) load(row, col, v);
        else {
#pragma unroll
            for (int t = 0; t < 16; ++t) v[t] = 0.f;
        }
        hadamard16_unscaled(v);
        if (col < K) {
            uint4 a, b;
            a.x = pack_bf16x2(v[0] * 0.0625f, v[1] * 0.0625f);
            a.y = pack_bf16x2(v[2] * 0.0625f, v[3] * 0.0625f);
            a.z = pack_bf16x2(v[4] * 0.0625f, v[5] * 0.0625f);
            a.w = pack_bf16x2(v[6] * 0.0625f, v[7] * 0.0625f);
            b.x = pack_bf16x2(v[8] * 0.0625f, v[9] * 0.0625f);
            b.y = pack_bf16x2(v[10] * 0.0625f, v[11] * 0.0625f);
            b.z = pack_bf16x2(v[12] * 0.0625f, v[13] * 0.0625f);
            b.w = pack_bf16x2(v[14] * 0.0625f, v[15] * 0.0625f);
            uint4* p = reinterpret_cast<uint4*>(out + row * K + col);
            p[0] = a;
            p[1] = b;
        }
    }
}

template <class Loader>
hipError_t launch_rotate(hipStream_t st, const Loader& ld, uint16_t* out, int64_t M, int K) {
    const int64_t waves = M * ((K + 1023) / 1024);
    int64_t blocks = (waves + 3) / 4;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL((rotate_kernel<Loader>), dim3(unsigned(blocks)), dim3(256), 0, st, ld,
                       out, M, K);
    return hipGetLastError();
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
                        float* scale, int64_t M, int N) {
    return launch_rowquant<false, kDivide>(
        st, LoadColScaled{static_cast<const uint16_t*>(x), N, colscale}, q, scale, M, N);
}

}  // namespace xpuint8
