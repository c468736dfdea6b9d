// Internal launchers (one per kernel family).  All are asynchronous on the
// given stream, validate nothing (the C ABI in capi.hip does), and return the
// launch status.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace xpuint8 {

// The MFMA block layout of an int8 GEMM operand [M, K]: the GEMM kernels' LDS
// stage layout, laid out in memory, so that one 16-row block of a 64-byte K
// step is one contiguous 1 KB direct-to-LDS load.  Block (m/16, k/64) sits at
// ((m/16) * KB + k/64) * 1024 (KB = ceil(K/64)); in it, row r = m%16 at 64r and
// its 16-byte chunk c = (k%64)/16 at position c ^ ((r >> 1) & 3).  Rows past
// M in the last block and bytes past K in the last column of blocks are
// unspecified (the GEMM multiplies them by zeros or never stores them).
__host__ __device__ inline int64_t tiled_bytes(int64_t M, int64_t K) {
    return ((M + 15) / 16) * ((K + 63) / 64) * 1024;
}
__host__ __device__ inline int64_t tiled_offset(int64_t m, int k, int KB) {
    const int r = int(m & 15), c = (k >> 4) & 3;
    return (((m >> 4) * KB + (k >> 6)) << 10) + (r << 6) + ((c ^ ((r >> 1) & 3)) << 4);
}

// rowquant.hip
hipError_t convrot_quantize(hipStream_t st, const void* x, int8_t* q, float* scale, int64_t M,
                            int K, int act);
hipError_t dequant_act_quantize(hipStream_t st, const int32_t* acc, int64_t acc_ld, int8_t* q,
                                float* scale, const float* xs, const float* ws, int64_t M, int K,
                                int act);
hipError_t rotate_bf16(hipStream_t st, const void* x, void* out, int64_t M, int K);
hipError_t dequant_weight(hipStream_t st, const int8_t* w8, const float* scale, void* out,
                          int64_t N, int K);
hipError_t prepare_weight(hipStream_t st, const void* w, int8_t* q, float* scale, int64_t N,
                          int K);
hipError_t quantize_row(hipStream_t st, const void* x, const float* colscale, int8_t* q,
                        float* scale, int64_t M, int N, bool tiled = false);
// the quantizers above (rotating with act 0, and quantize_row) can write q in
// the MFMA block layout (tiled = true) for rows of this length
bool rowquant_can_tile(int K);
hipError_t convrot_quantize_tiled(hipStream_t st, const void* x, int8_t* q, float* scale,
                                  int64_t M, int K);

// bf16 column sums out[n] = bf16(sum_m x[m, n]) (N % 8 == 0) through fp32
// partials in part (colsum_work_bytes(M, N) bytes); out_f32 writes each
// bf16-rounded sum as the fp32 it widens to
int64_t colsum_work_bytes(int64_t M, int64_t N);
hipError_t column_sum_bf16(hipStream_t st, const void* x, void* out, int64_t M, int N,
                           float* part, bool out_f32 = false);

// gemm_i8.hip
hipError_t gemm_i32(hipStream_t st, const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb,
                    int32_t* C, int64_t ldc, int M, int N, int K);
// Bp (here and in gemm_act; optional): pack_weight's copy of B, which the
// skinny kernel reads instead of B
hipError_t gemm_dequant(hipStream_t st, const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb,
                        void* out, int64_t ldo, const float* xs, const float* ws, const float* bias,
                        const uint16_t* bias16, int M, int N, int K, const int8_t* Bp = nullptr);
// the dequant GEMM with B stored [K, N] (the NN product, no column scale), when
// the split-K kernel takes the shape; *done = false (nothing launched) otherwise
hipError_t gemm_dequant_nn(hipStream_t st, const int8_t* A, int64_t lda, const int8_t* Bkn,
                           int64_t ldb, void* out, int64_t ldo, const float* xs, int M, int N,
                           int K, bool* done);
// whether the split-K kernel takes the dequant GEMM of this shape, and its NN
// form (gemm_dequant_nn) with B stored [K, N] at row stride ldb
bool splitk_applies(int M, int N, int K);
bool splitk_nn_applies(int M, int N, int K, int64_t ldb);
// the split-K dequant GEMMs with A in the MFMA block layout (tiled_offset);
// callers check splitk_applies first.  packed: B is pack_weight's copy of the
// weight (the block layout too; ldb unused)
hipError_t gemm_dequant_xt(hipStream_t st, const int8_t* At, const int8_t* B, int64_t ldb,
                           void* out, int64_t ldo, const float* xs, const float* ws,
                           const float* bias, const uint16_t* bias16, int M, int N, int K,
                           bool packed = false);
hipError_t gemm_dequant_nn_xt(hipStream_t st, const int8_t* At, const int8_t* Bkn, int64_t ldb,
                              void* out, int64_t ldo, const float* xs, int M, int N, int K,
                              bool packed = false);
// whether the persistent ping-pong kernel takes the dequant GEMM (paired:
// the FFN's up-projection) of this shape, and those GEMMs with A in the MFMA
// block layout on that kernel
bool pp_applies(int M, int N, int K, bool paired);
hipError_t gemm_dequant_pp_xt(hipStream_t st, const int8_t* At, const int8_t* B, int64_t ldb,
                              void* out, int64_t ldo, const float* xs, const float* ws,
                              const float* bias, const uint16_t* bias16, int M, int N, int K,
                              bool packed = false);
hipError_t gemm_act_pp_xt(hipStream_t st, const int8_t* At, const int8_t* B, int64_t ldb,
                          void* out, int64_t ldo, const float* xs, const float* ws, int M, int N,
                          int K, int act, bool packed = false);
// w [N, K] int8 (row-major, K % 16 == 0) in the MFMA block layout, the bytes
// past K zero: the packed weight the GEMMs above read with packed = true
// (tiled_bytes(N, K) bytes at out)
hipError_t pack_weight(hipStream_t st, const int8_t* w, int8_t* out, int64_t N, int K);
// w [R, C] int8 (row-major, C % 32 == 0) in the split-K kernel's NN stage
// order, the rows past R zero (packed_nn_bytes(R, C) bytes): the NN products'
// packed right operand (gemm_dequant_nn_xt with packed = true)
int64_t packed_nn_bytes(int64_t R, int64_t C);
hipError_t pack_weight_nn(hipStream_t st, const int8_t* w, int8_t* out, int64_t R, int C);
// the same with the residual update out = bf16(res + d * rscale[n]) (bf16 res, rscale)
hipError_t gemm_dequant_residual(hipStream_t st, const int8_t* A, int64_t lda, const int8_t* B,
                                 int64_t ldb, void* out, int64_t ldo, const float* xs,
                                 const float* ws, const float* bias, const uint16_t* bias16,
                                 const void* res, int64_t ldr, const void* rscale, int M, int N,
                                 int K);
// the same two GEMMs with A in the MFMA block layout (packed: B is pack_weight's
// copy): the residual epilogue on the persistent or the split-K kernel (callers
// check pp_applies / splitk_applies; other shapes are refused), and the int32
// product on the persistent kernel (callers check pp_applies)
hipError_t gemm_dequant_residual_xt(hipStream_t st, const int8_t* At, const int8_t* B,
                                    int64_t ldb, void* out, int64_t ldo, const float* xs,
                                    const float* ws, const float* bias, const uint16_t* bias16,
                                    const void* res, int64_t ldr, const void* rscale, int M, int N,
                                    int K, bool packed);
hipError_t gemm_i32_pp_xt(hipStream_t st, const int8_t* At, const int8_t* B, int64_t ldb,
                          int32_t* C, int64_t ldc, int M, int N, int K, bool packed);
// out[m, n] = act(bf16(acc(n) * ws[n] * xs[m]), bf16(acc(N + n) * ws[N + n] * xs[m])) for the
// paired activations 3 (situ) and 4 (GEGLU), whose B has 2N rows; act 5 (GELU) takes N rows
hipError_t gemm_act(hipStream_t st, const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb,
                    void* out, int64_t ldo, const float* xs, const float* ws, int M, int N, int K,
                    int act, const int8_t* Bp = nullptr);
// The skinny kernel with x in the MFMA block layout (At) and the packed weight
// (Bp), for the batches launch_gemm gives it (skinny_applies: M <= 64; paired
// activations 3 and 4, M <= 256); a linear's callers check gemm_slices first
bool skinny_applies(int M, bool paired);
hipError_t gemm_dequant_skinny_xt(hipStream_t st, const int8_t* At, const int8_t* Bp, void* out,
                                  int64_t ldo, const float* xs, const float* ws, const float* bias,
                                  const uint16_t* bias16, int M, int N, int K);
hipError_t gemm_act_skinny_xt(hipStream_t st, const int8_t* At, const int8_t* Bp, void* out,
                              int64_t ldo, const float* xs, const float* ws, int M, int N, int K,
                              int act);
hipError_t dequant_epilogue(hipStream_t st, const int32_t* acc, int64_t acc_ld, void* out,
                            const float* xs, const float* ws, const float* bias, int64_t M,
                            int64_t N);
// the same on the sum of nsl int32 slices sl_stride apart, with an fp32 (bias)
// or bf16 (bias16) bias or neither; ws == nullptr is a unit column scale
hipError_t dequant_slices(hipStream_t st, const int32_t* acc, int64_t acc_ld, int nsl,
                          int64_t sl_stride, void* out, const float* xs, const float* ws,
                          const float* bias, const uint16_t* bias16, int64_t M, int64_t N);
// K slices of a split of the product across blocks (0: none applies), and the
// slices' int32 partial products, slice s at part + s * M * N (row stride N)
int gemm_slices(int M, int N, int K);
hipError_t gemm_i32_slices(hipStream_t st, const int8_t* X, int64_t ldx, const int8_t* W,
                           int64_t ldw, int32_t* part, int M, int N, int K, int nsl);
// the same with B stored [K, N]; only where !slices_need_nt(M) (others
// transpose B and call gemm_i32_slices); ldb * (K + 64) below 2^32
hipError_t gemm_i32_slices_nn(hipStream_t st, const int8_t* X, int64_t ldx, const int8_t* Bkn,
                              int64_t ldb, int32_t* part, int M, int N, int K, int nsl);
bool slices_need_nt(int M);
hipError_t transpose_i8(hipStream_t st, const int8_t* in, int8_t* out, int64_t R, int64_t C);

// gemm_bf16.hip: the dense dx with its contraction split across blocks
// (bf16_nn_slices slices, 0 when none applies): the slices' fp32 partials in
// part (nsl * M * K floats), then their sum rounded to bf16 into out
int bf16_nn_slices(int M, int N, int K);
hipError_t gemm_bf16_nn_slices(hipStream_t st, const void* dy, int64_t ldy, const void* w,
                               int64_t ldw, void* out, int64_t ldo, int M, int N, int K,
                               float* part, int nsl);
// gemm_bf16.hip: dw[n, k] = sum_m dy[m, n] * x[m, k] (bf16, fp32 accumulate)
hipError_t gemm_bf16_tn(hipStream_t st, const void* dy, int64_t ldy, const void* x, int64_t ldx,
                        void* dw, int64_t ldo, int R, int N, int K);
// gemm_bf16.hip: out[m, k] = sum_n dy[m, n] * w[n, k] (bf16, fp32 accumulate)
hipError_t gemm_bf16_nn(hipStream_t st, const void* dy, int64_t ldy, const void* w, int64_t ldw,
                        void* out, int64_t ldo, int M, int N, int K);

// rope.hip: RMSNorm + rotary embedding of an int32 accumulator slice
hipError_t rms_rope_dequant(hipStream_t st, const int32_t* acc, int64_t a_sb, int64_t a_ss,
                            int64_t a_sh, const float* xs, int64_t xs_sb, int64_t xs_ss,
                            const float* ws, const float* freqs, int64_t f_sb, int64_t f_ss,
                            int64_t f_sdim, int64_t f_srot, int64_t f_spair, int64_t f_batch,
                            int64_t f_seq, const float* scale, void* out, int64_t B, int64_t S,
                            int H, int D, float eps, int split_half);

// capi.hip: compute units of the current device (persistent grids)
int device_cus();

// tables.hip: the host copy of the activation tables (activations.hpp)
const uint16_t* host_activation_tables();

}  // namespace xpuint8
