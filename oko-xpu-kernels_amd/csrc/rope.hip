// RMSNorm + rotary embedding reading the int8 GEMM's int32 accumulator: the
// fused q/k consumer of a quantized qkv projection
// (python/xpu_kernels/triton/rope.py:149-222, _rms_rope_rows_dq_kernel).
//
// For each (batch b, position s, head h) row of D = head_dim values:
//   x[d]   = bf16(float(acc[d]) * (w_scale[h*D + d] * x_scale[b, s]))   (the
//            dequant epilogue's expression and rounding)
//   inv    = 1 / sqrt(sum_d x[d]^2 / D + eps)
//   y[d]   = bf16(x[d] * inv * scale[d])
//   pair (d0, d1) = (p, p + D/2) (split half) or (2p, 2p + 1) (interleaved):
//   out[d0] = bf16(F00[p] * y[d0] + F01[p] * y[d1])
//   out[d1] = bf16(F10[p] * y[d0] + F11[p] * y[d1])
// with F the [2, 2] rotation of pair p in freqs_cis [FB, FS, 1, D/2, 2, 2]
// (FB, FS broadcast when 1).  The reference's own check of this kernel
// against its torch chain is a tolerance (reduction order of the row sum and
// its rsqrt), so the sum here is the wave's butterfly order and inv uses the
// correctly rounded sqrt and division.
#include "common.hpp"
#include "kernels.hpp"

namespace xpuint8 {
namespace {

struct RopeArgs {
    const int32_t* acc;
    int64_t a_sb, a_ss, a_sh;            // element strides; the head dim is contiguous
    const float* xs;
    int64_t xs_sb, xs_ss;
    const float* ws;                     // [H * D]
    const float* freqs;
    int64_t f_sb, f_ss, f_sdim, f_srot, f_spair;
    int64_t f_batch, f_seq;              // 1 = broadcast
    const float* scale;                  // [D]
    uint16_t* out;                       // [B, S, H, D] contiguous
    int64_t B, S;
    int H, D;
    float eps;
    int split_half;
};

// Sum over the 64 lanes of a wave: DPP inside rows of 16, then the two
// cross-row steps (each step adds two disjoint lane groups that hold equal
// partial sums, so every lane ends with the same total).
__device__ __forceinline__ float wave_sum(float x) {
    x += dpp<kDppXor1>(x);
    x += dpp<kDppXor2>(x);
    x += dpp<kDppXor7>(x);
    x += dpp<kDppXor15>(x);
    x += swz_xor<16>(x);
    x += __shfl_xor(x, 32);
    return x;
}

// One block of four waves per (b, s) position; wave w takes heads w, w + 4,
// ...  A lane handles pairs l and l + 64 of a head row (D <= 256).  The
// position's rotation and the norm weight are loaded once per wave, and the
// next head's accumulator and column scales are requested before the current
// head's row sum, so each wave keeps one head's loads in flight.
__global__ __launch_bounds__(256) void rms_rope_dq_kernel(RopeArgs a) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    if (wave >= a.H) return;
    const uint32_t bs = blockIdx.x;
    const uint32_t b32 = bs / uint32_t(a.S);
    const int64_t b = b32, s = bs - b32 * uint32_t(a.S);
    const float xsr = a.xs[b * a.xs_sb + s * a.xs_ss];
    const int32_t* accp = a.acc + b * a.a_sb + s * a.a_ss;
    const float* f = a.freqs + (a.f_batch == 1 ? 0 : b) * a.f_sb + (a.f_seq == 1 ? 0 : s) * a.f_ss;
    uint16_t* outp = a.out + int64_t(bs) * a.H * a.D;
    const int np = a.D / 2;

    // per lane: its pairs' dims, rotation and norm weight (idle lanes repeat
    // the last pair so that every load stays in bounds)
    int d0[2], d1[2];
    float s0[2], s1[2], f00[2], f01[2], f10[2], f11[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int p = min(lane + 64 * j, np - 1);
        d0[j] = a.split_half ? p : 2 * p;
        d1[j] = a.split_half ? p + np : 2 * p + 1;
        s0[j] = a.scale[d0[j]]; s1[j] = a.scale[d1[j]];
        const float* fp = f + p * a.f_sdim;
        f00[j] = fp[0]; f01[j] = fp[a.f_spair];
        f10[j] = fp[a.f_srot]; f11[j] = fp[a.f_srot + a.f_spair];
    }
    auto fetch = [&](int h, int32_t (&a0)[2], int32_t (&a1)[2], float (&w0)[2], float (&w1)[2]) {
        const int32_t* acc = accp + int64_t(h) * a.a_sh;
        const float* w = a.ws + h * a.D;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            a0[j] = acc[d0[j]]; a1[j] = acc[d1[j]];
            w0[j] = w[d0[j]]; w1[j] = w[d1[j]];
        }
    };
    int32_t a0[2], a1[2];
    float w0[2], w1[2];
    fetch(wave, a0, a1, w0, w1);
    for (int h = wave; h < a.H; h += 4) {
        float x0[2], x1[2];
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            x0[j] = bf16_round(float(a0[j]) * (w0[j] * xsr));
            x1[j] = bf16_round(float(a1[j]) * (w1[j] * xsr));
            if (lane + 64 * j < np) {
                ss = ss + x0[j] * x0[j];
                ss = ss + x1[j] * x1[j];
            }
        }
        if (h + 4 < a.H) fetch(h + 4, a0, a1, w0, w1);
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss / float(a.D) + a.eps);
        uint16_t* o = outp + h * a.D;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            if (lane + 64 * j < np) {
                const float y0 = bf16_round(x0[j] * inv * s0[j]);
                const float y1 = bf16_round(x1[j] * inv * s1[j]);
                o[d0[j]] = uint16_t(f32_to_bf16_bits(f00[j] * y0 + f01[j] * y1));
                o[d1[j]] = uint16_t(f32_to_bf16_bits(f10[j] * y0 + f11[j] * y1));
            }
        }
    }
}

}  // namespace

hipError_t rms_rope_dequant(hipStream_t st, const int32_t* acc, int64_t a_sb, int64_t a_ss,
                            int64_t a_sh, const float* xs, int64_t xs_sb, int64_t xs_ss,
                            const float* ws, const float* freqs, int64_t f_sb, int64_t f_ss,
                            int64_t f_sdim, int64_t f_srot, int64_t f_spair, int64_t f_batch,
                            int64_t f_seq, const float* scale, void* out, int64_t B, int64_t S,
                            int H, int D, float eps, int split_half) {
    RopeArgs a{acc, a_sb, a_ss, a_sh, xs, xs_sb, xs_ss, ws, freqs, f_sb, f_ss, f_sdim, f_srot,
               f_spair, f_batch, f_seq, scale, static_cast<uint16_t*>(out), B, S, H, D, eps,
               split_half};
    hipLaunchKernelGGL(rms_rope_dq_kernel, dim3(unsigned(B * S)), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace xpuint8
