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
    int f_vec;                           // rotations contiguous and 16-byte aligned
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

// The same for D = 64 or 128 with a head row on L = D / 8 lanes: lane q of a
// head handles pairs 4q .. 4q+3, i.e. 16-byte loads of the accumulator and of
// the column scales (two per pair half: dims 4q.. and D/2 + 4q.. when split,
// 8q .. 8q+7 when interleaved) and 8- or 16-byte stores.  A wave holds 64 / L
// heads side by side and a block ceil(H / (64 / L)) waves, one pass each, so
// a position's whole accumulator slice is requested at once.  The row sum is
// the lane's eight squares in order, then the L-lane butterfly (DPP).
template <int D, bool SPLIT>
__global__ __launch_bounds__(1024) void rms_rope_dq_vec_kernel(RopeArgs a) {
    constexpr int L = D / 8, HPW = 64 / L, NP = D / 2;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int q = lane % L;
    const int h_raw = wave * HPW + lane / L;
    const bool live = h_raw < a.H;
    const int h = live ? h_raw : a.H - 1;           // idle lanes read a valid row
    const uint32_t bs = blockIdx.x;
    const uint32_t b32 = bs / uint32_t(a.S);
    const int64_t b = b32, s = bs - b32 * uint32_t(a.S);
    const float xsr = a.xs[b * a.xs_sb + s * a.xs_ss];
    const int32_t* acc = a.acc + b * a.a_sb + s * a.a_ss + int64_t(h) * a.a_sh;
    const float* w = a.ws + h * D;
    const float* f = a.freqs + (a.f_batch == 1 ? 0 : b) * a.f_sb + (a.f_seq == 1 ? 0 : s) * a.f_ss;
    // dims of the lane's four pairs: first members at e0 .. e0+3 (split) or
    // 8q, 8q+2, .. (interleaved); second members D/2 further or one further
    const int e0 = SPLIT ? 4 * q : 8 * q;
    int4 r0, r1;
    float4 w0, w1, c0, c1;
    if constexpr (SPLIT) {
        r0 = *reinterpret_cast<const int4*>(acc + e0);
        r1 = *reinterpret_cast<const int4*>(acc + NP + e0);
        w0 = *reinterpret_cast<const float4*>(w + e0);
        w1 = *reinterpret_cast<const float4*>(w + NP + e0);
        c0 = *reinterpret_cast<const float4*>(a.scale + e0);
        c1 = *reinterpret_cast<const float4*>(a.scale + NP + e0);
    } else {
        const int4 ra = *reinterpret_cast<const int4*>(acc + e0);
        const int4 rb = *reinterpret_cast<const int4*>(acc + e0 + 4);
        r0 = make_int4(ra.x, ra.z, rb.x, rb.z);
        r1 = make_int4(ra.y, ra.w, rb.y, rb.w);
        const float4 wa = *reinterpret_cast<const float4*>(w + e0);
        const float4 wb = *reinterpret_cast<const float4*>(w + e0 + 4);
        w0 = make_float4(wa.x, wa.z, wb.x, wb.z);
        w1 = make_float4(wa.y, wa.w, wb.y, wb.w);
        const float4 ca = *reinterpret_cast<const float4*>(a.scale + e0);
        const float4 cb = *reinterpret_cast<const float4*>(a.scale + e0 + 4);
        c0 = make_float4(ca.x, ca.z, cb.x, cb.z);
        c1 = make_float4(ca.y, ca.w, cb.y, cb.w);
    }
    // the four pairs' rotations, requested with the rest (one 16-byte load a
    // pair in the usual contiguous [.., D/2, 2, 2] layout)
    float F[4][4];
    const int p0 = SPLIT ? e0 : e0 / 2;
    if (a.f_vec) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float4 v = *reinterpret_cast<const float4*>(f + (p0 + t) * 4);
            F[t][0] = v.x; F[t][1] = v.y; F[t][2] = v.z; F[t][3] = v.w;
        }
    } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float* fp = f + (p0 + t) * a.f_sdim;
            F[t][0] = fp[0]; F[t][1] = fp[a.f_spair];
            F[t][2] = fp[a.f_srot]; F[t][3] = fp[a.f_srot + a.f_spair];
        }
    }
    const int a0[4] = {r0.x, r0.y, r0.z, r0.w}, a1[4] = {r1.x, r1.y, r1.z, r1.w};
    const float ws0[4] = {w0.x, w0.y, w0.z, w0.w}, ws1[4] = {w1.x, w1.y, w1.z, w1.w};
    const float sc0[4] = {c0.x, c0.y, c0.z, c0.w}, sc1[4] = {c1.x, c1.y, c1.z, c1.w};
    float x0[4], x1[4], ss = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        x0[t] = bf16_round(float(a0[t]) * (ws0[t] * xsr));
        x1[t] = bf16_round(float(a1[t]) * (ws1[t] * xsr));
        ss = ss + x0[t] * x0[t];
        ss = ss + x1[t] * x1[t];
    }
    ss += dpp<kDppXor1>(ss);
    ss += dpp<kDppXor2>(ss);
    ss += dpp<kDppXor7>(ss);
    if constexpr (L == 16) ss += dpp<kDppXor15>(ss);
    const float inv = 1.0f / sqrtf(ss / float(D) + a.eps);
    uint32_t o0[2], o1[2];
#pragma unroll
    for (int t = 0; t < 4; t += 2) {
        float r[2][2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const float y0 = bf16_round(x0[t + u] * inv * sc0[t + u]);
            const float y1 = bf16_round(x1[t + u] * inv * sc1[t + u]);
            r[u][0] = F[t + u][0] * y0 + F[t + u][1] * y1;
            r[u][1] = F[t + u][2] * y0 + F[t + u][3] * y1;
        }
        if constexpr (SPLIT) {
            o0[t / 2] = pack_bf16x2(r[0][0], r[1][0]);
            o1[t / 2] = pack_bf16x2(r[0][1], r[1][1]);
        } else {
            o0[t / 2] = pack_bf16x2(r[0][0], r[0][1]);
            o1[t / 2] = pack_bf16x2(r[1][0], r[1][1]);
        }
    }
    if (!live) return;
    uint16_t* o = a.out + (int64_t(bs) * a.H + h) * D;
    if constexpr (SPLIT) {
        *reinterpret_cast<uint2*>(o + e0) = make_uint2(o0[0], o0[1]);
        *reinterpret_cast<uint2*>(o + NP + e0) = make_uint2(o1[0], o1[1]);
    } else {
        *reinterpret_cast<uint4*>(o + e0) = make_uint4(o0[0], o1[0], o0[1], o1[1]);
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
               split_half, 0};
    // the vector kernel when a head row is 64 or 128 dims, a block of whole
    // waves holds every head of a position, and the accumulator, column scales,
    // norm weight and output allow 16-byte accesses
    const auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    const int hpw = D == 128 ? 4 : 8;
    const int waves = (H + hpw - 1) / hpw;
    if ((D == 64 || D == 128) && waves <= 16 && al16(acc) && al16(ws) && al16(scale) &&
        al16(out) && a_sb % 4 == 0 && a_ss % 4 == 0 && a_sh % 4 == 0) {
        a.f_vec = f_sdim == 4 && f_srot == 2 && f_spair == 1 && al16(freqs) && f_sb % 4 == 0 &&
                  f_ss % 4 == 0;
        const dim3 grid(unsigned(B * S)), block(unsigned(64 * waves));
        if (D == 128) {
            if (split_half) hipLaunchKernelGGL((rms_rope_dq_vec_kernel<128, true>), grid, block, 0, st, a);
            else            hipLaunchKernelGGL((rms_rope_dq_vec_kernel<128, false>), grid, block, 0, st, a);
        } else {
            if (split_half) hipLaunchKernelGGL((rms_rope_dq_vec_kernel<64, true>), grid, block, 0, st, a);
            else            hipLaunchKernelGGL((rms_rope_dq_vec_kernel<64, false>), grid, block, 0, st, a);
        }
        return hipGetLastError();
    }
    hipLaunchKernelGGL(rms_rope_dq_kernel, dim3(unsigned(B * S)), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace xpuint8
