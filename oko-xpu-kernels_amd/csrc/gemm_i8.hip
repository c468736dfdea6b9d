// int8 x int8 -> int32 GEMM on CDNA4 MFMA (v_mfma_i32_32x32x32_i8), with the
// accumulator consumed in-register by an epilogue: int32 store, or the
// ConvRot dequant  bf16(float(acc) * (ws[n] * xs[m]) + bias[n])
// (src/xpuint8.cpp:692-710) fused into the store.
//
// C[m, n] = sum_k A[m, k] * B[n, k]   (A int8 [M, K], B int8 [N, K], both
// K-contiguous: the "NT" form of torch._int_mm(a, b.t()) that the reference's
// linear calls, python/xpu_kernels/int8/ops.py:634).
//
// Block tile BM x BN, K step BK, 256 threads = 4 waves in a 2 x 2 grid; a wave
// owns a (BM/2) x (BN/2) tile of 32 x 32 MFMA blocks.  A and B tiles are staged
// through LDS (row pitch BK+16 bytes, conflict-free 16-byte reads), double
// buffered with register prefetch of the next K step.
#include "common.hpp"
#include "kernels.hpp"

namespace xpuint8 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

struct EpiI32 {
    int32_t* c;
    int64_t ldc;
    __device__ __forceinline__ void operator()(int i, int j, int v) const { c[int64_t(i) * ldc + j] = v; }
};

// The dequant epilogue; ws == nullptr means a unit column scale (1.0f * xs is xs).
struct EpiDequant {
    uint16_t* out;
    int64_t ldo;
    const float* xs;
    const float* ws;
    const float* bias;
    __device__ __forceinline__ void operator()(int i, int j, int v) const {
        const float w = ws ? ws[j] : 1.0f;
        float r = float(v) * (w * xs[i]);
        if (bias) r = r + bias[j];
        out[int64_t(i) * ldo + j] = uint16_t(f32_to_bf16_bits(r));
    }
};

template <int BM, int BN, int BK, class Epi>
__global__ __launch_bounds__(256) void gemm_i8_kernel(const int8_t* __restrict__ A, int64_t lda,
                                                     const int8_t* __restrict__ B, int64_t ldb,
                                                     int M, int N, int K, Epi epi) {
    constexpr int PITCH = BK + 16;
    constexpr int WTM = BM / 2, WTN = BN / 2;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    constexpr int CPR = BK / 16;                 // 16-byte chunks per tile row
    constexpr int A_CH = BM * CPR / 256, B_CH = BN * CPR / 256;
    static_assert(A_CH * 256 == BM * CPR && B_CH * 256 == BN * CPR, "tile/thread mismatch");
    __shared__ __attribute__((aligned(16))) int8_t sA[2][BM * PITCH];
    __shared__ __attribute__((aligned(16))) int8_t sB[2][BN * PITCH];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

    int4 ra[A_CH], rb[B_CH];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < A_CH; ++i) {
            const int c = tid + i * 256, r = c / CPR, kc = (c % CPR) * 16;
            const int gm = m0 + r;
            ra[i] = (gm < M && k0 + kc < K)
                        ? *reinterpret_cast<const int4*>(A + int64_t(gm) * lda + k0 + kc)
                        : make_int4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < B_CH; ++i) {
            const int c = tid + i * 256, r = c / CPR, kc = (c % CPR) * 16;
            const int gn = n0 + r;
            rb[i] = (gn < N && k0 + kc < K)
                        ? *reinterpret_cast<const int4*>(B + int64_t(gn) * ldb + k0 + kc)
                        : make_int4(0, 0, 0, 0);
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_CH; ++i) {
            const int c = tid + i * 256, r = c / CPR, kc = (c % CPR) * 16;
            *reinterpret_cast<int4*>(&sA[buf][r * PITCH + kc]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < B_CH; ++i) {
            const int c = tid + i * 256, r = c / CPR, kc = (c % CPR) * 16;
            *reinterpret_cast<int4*>(&sB[buf][r * PITCH + kc]) = rb[i];
        }
    };

    v16i acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = v16i{0};

    const int KT = (K + BK - 1) / BK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < KT) gload((kt + 1) * BK);
#pragma unroll
        for (int kk = 0; kk < BK / 32; ++kk) {
            v4i af[TM], bf[TN];
            const int koff = kk * 32 + (lane >> 5) * 16;
#pragma unroll
            for (int a = 0; a < TM; ++a)
                af[a] = *reinterpret_cast<const v4i*>(
                    &sA[cur][(wm * WTM + a * 32 + (lane & 31)) * PITCH + koff]);
#pragma unroll
            for (int b = 0; b < TN; ++b)
                bf[b] = *reinterpret_cast<const v4i*>(
                    &sB[cur][(wn * WTN + b * 32 + (lane & 31)) * PITCH + koff]);
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int b = 0; b < TN; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[a], bf[b], acc[a][b], 0, 0, 0);
        }
        if (kt + 1 < KT) sstore(cur ^ 1);
        __syncthreads();
    }

    // 32x32 accumulator layout: register r of lane l holds
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int i = m0 + wm * WTM + a * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const int j = n0 + wn * WTN + b * 32 + (lane & 31);
                if (i < M && j < N) epi(i, j, acc[a][b][r]);
            }
}

template <class Epi>
hipError_t launch_gemm(hipStream_t st, const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb,
                       int M, int N, int K, const Epi& epi) {
    constexpr int BM = 128, BN = 128, BK = 64;
    const dim3 grid(unsigned((N + BN - 1) / BN), unsigned((M + BM - 1) / BM));
    hipLaunchKernelGGL((gemm_i8_kernel<BM, BN, BK, Epi>), grid, dim3(256), 0, st, A, lda, B, ldb,
                       M, N, K, epi);
    return hipGetLastError();
}

// ------------------------------------------------------- standalone dequant
// One thread per 16 output columns (N % 16 == 0), grid-stride.
__global__ __launch_bounds__(256) void dequant_kernel(const int32_t* __restrict__ acc,
                                                     int64_t acc_ld, uint16_t* __restrict__ out,
                                                     const float* __restrict__ xs,
                                                     const float* __restrict__ ws,
                                                     const float* __restrict__ bias, int64_t M,
                                                     int64_t N) {
    const int64_t nvec = N / 16, total = M * nvec;
    for (int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
         t += int64_t(gridDim.x) * blockDim.x) {
        const int64_t m = t / nvec, c = (t - m * nvec) * 16;
        const int32_t* pa = acc + m * acc_ld + c;
        const float4* pw = reinterpret_cast<const float4*>(ws + c);
        const float4* pb = reinterpret_cast<const float4*>(bias + c);
        const float x = xs[m];
        uint32_t o[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const i32x4 a = load16_nt_i(pa + 4 * j);
            const float4 w = pw[j];
            float r0 = float(a.x) * (w.x * x), r1 = float(a.y) * (w.y * x);
            float r2 = float(a.z) * (w.z * x), r3 = float(a.w) * (w.w * x);
            if (bias) {
                const float4 b = pb[j];
                r0 = r0 + b.x; r1 = r1 + b.y; r2 = r2 + b.z; r3 = r3 + b.w;
            }
            o[2 * j] = pack_bf16x2(r0, r1);
            o[2 * j + 1] = pack_bf16x2(r2, r3);
        }
        uint4* po = reinterpret_cast<uint4*>(out + m * N + c);
        po[0] = make_uint4(o[0], o[1], o[2], o[3]);
        po[1] = make_uint4(o[4], o[5], o[6], o[7]);
    }
}

// ------------------------------------------------------------ int8 transpose
// out[c, r] = in[r, c]; 64 x 64 tiles through LDS.
__global__ __launch_bounds__(256) void transpose_i8_kernel(const int8_t* __restrict__ in,
                                                          int8_t* __restrict__ out, int64_t R,
                                                          int64_t C) {
    __shared__ int8_t tile[64][65];
    const int64_t r0 = int64_t(blockIdx.y) * 64, c0 = int64_t(blockIdx.x) * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int i = ty; i < 64; i += 4) {
        const int64_t r = r0 + i, c = c0 + tx;
        tile[i][tx] = (r < R && c < C) ? in[r * C + c] : int8_t(0);
    }
    __syncthreads();
    for (int i = ty; i < 64; i += 4) {
        const int64_t c = c0 + i, r = r0 + tx;
        if (c < C && r < R) out[c * R + r] = tile[tx][i];
    }
}

}  // namespace

hipError_t gemm_i32(hipStream_t st, const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb,
                    int32_t* C, int64_t ldc, int M, int N, int K) {
    return launch_gemm(st, A, lda, B, ldb, M, N, K, EpiI32{C, ldc});
}

hipError_t gemm_dequant(hipStream_t st, const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb,
                        void* out, int64_t ldo, const float* xs, const float* ws, const float* bias,
                        int M, int N, int K) {
    return launch_gemm(st, A, lda, B, ldb, M, N, K,
                       EpiDequant{static_cast<uint16_t*>(out), ldo, xs, ws, bias});
}

hipError_t dequant_epilogue(hipStream_t st, const int32_t* acc, int64_t acc_ld, void* out,
                            const float* xs, const float* ws, const float* bias, int64_t M,
                            int64_t N) {
    const int64_t total = M * (N / 16);
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(dequant_kernel, dim3(unsigned(blocks)), dim3(256), 0, st, acc, acc_ld,
                       static_cast<uint16_t*>(out), xs, ws, bias, M, N);
    return hipGetLastError();
}

hipError_t transpose_i8(hipStream_t st, const int8_t* in, int8_t* out, int64_t R, int64_t C) {
    const dim3 grid(unsigned((C + 63) / 64), unsigned((R + 63) / 64));
    hipLaunchKernelGGL(transpose_i8_kernel, grid, dim3(256), 0, st, in, out, R, C);
    return hipGetLastError();
}

}  // namespace xpuint8
