/* libxpuint8 for MI355X (gfx950): the ConvRot INT8 linear as a C ABI.
 *
 * Drop-in for the C ABI of okolenmi/oko-xpu-kernels'
 * include/xpu_kernels/convrot.h (lines cited per function), which
 * python/xpu_kernels/int8/_lib.py binds through ctypes.  Differences:
 *
 *  - the `_stream` variants take a HIP stream (`hipStream_t`, passed as
 *    `const void *`; NULL is the default stream) where the reference takes a
 *    `sycl::queue *`.  They enqueue asynchronously and never wait.  The
 *    non-stream variants run on the default stream and synchronize it.
 *  - the entry points the reference left to torch (`torch._int_mm`, the
 *    prepare_weight / quantize_row / linear_dw chains) are here too, so the
 *    whole path runs in this library: see the second half of this file.
 *
 * Conventions.  Every pointer is a device pointer to a contiguous row-major
 * buffer owned by the caller; the library allocates no device memory.  bf16
 * tensors are passed as `void *` (16-bit storage).  Sizes are int64_t.  Every
 * function returns 0 on success or an error code, with a message available
 * from xpuint8_last_error() (thread-local):
 *   1 no usable device (or init failed)      4 unsupported size
 *   2 bad dimensions (<= 0, N % 16, stride)  5 HIP launch / runtime error
 *   3 K not a multiple of 256                6 bad argument (null pointer,
 *                                              unknown activation)
 * Arguments are validated before any device call, so argument errors are
 * reported identically with or without a GPU.
 */
#ifndef XPUINT8_H
#define XPUINT8_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- library ----------------------------------------------------------- */

/* Select the current HIP device, check it is gfx950 and upload the
 * activation tables.  Replaces convrot.h:31-32. */
int xpuint8_init(void);

/* Device name ("AMD Instinct MI355X ..."), or NULL if no device.
 * Replaces convrot.h:34-35. */
const char *xpuint8_device_name(void);

/* The ConvRot group size, 256.  Replaces convrot.h:37-39. */
int xpuint8_convrot_groupsize(void);

/* Message of the last error on this thread.  Replaces convrot.h:115. */
const char *xpuint8_last_error(void);

/* ---- the reference's own entry points ---------------------------------- */

/* Rotate + quantize: bf16 x[M,K] -> int8 q[M,K] + fp32 scale[M].
 * K % 256 == 0.  Replaces convrot.h:41-49. */
int xpuint8_convrot_quantize(const void *x, int8_t *q, float *scale, int64_t M, int64_t K);
int xpuint8_convrot_quantize_stream(const void *stream, const void *x, int8_t *q, float *scale,
                                    int64_t M, int64_t K);

/* The same with an activation fused into the load (ids as convrot.h:51-59:
 * 1 gelu_tanh [M,K], 2 swiglu [M,2K] = [gate|up], 3 situ [M,2K] =
 * [hidden|gate], 4 geglu_erf [M,2K] = [hidden|gate], 5 gelu_erf [M,K]).
 * K is the output width.  Replaces convrot.h:60-64. */
int xpuint8_convrot_quantize_act(const void *x, int8_t *q, float *scale, int64_t M, int64_t K,
                                 int32_t activation);
int xpuint8_convrot_quantize_act_stream(const void *stream, const void *x, int8_t *q,
                                        float *scale, int64_t M, int64_t K, int32_t activation);

/* int8 w8[N,K] * fp32 w_scale[N] -> bf16 out[N,K] with the rotation undone
 * (the inverse of prepare_weight).  Replaces convrot.h:66-72. */
int xpuint8_dequant_weight(const void *w8, const float *w_scale, void *out, int64_t N,
                           int64_t K);
int xpuint8_dequant_weight_stream(const void *stream, const void *w8, const float *w_scale,
                                  void *out, int64_t N, int64_t K);

/* Rotation only, bf16 x[M,K] -> bf16 xr[M,K].  Replaces convrot.h:74-76. */
int xpuint8_convrot_rotate_bf16(const void *x, void *xr, int64_t M, int64_t K);
int xpuint8_convrot_rotate_bf16_stream(const void *stream, const void *x, void *xr, int64_t M,
                                       int64_t K);

/* out[m,n] = bf16(float(acc[m,n]) * (w_scale[n] * x_scale[m]) + bias[n]);
 * bias may be NULL; N % 16 == 0.  Replaces convrot.h:78-86. */
int xpuint8_dequant_epilogue(const int32_t *acc, void *out, const float *x_scale,
                             const float *w_scale, const float *bias, int64_t M, int64_t N);
int xpuint8_dequant_epilogue_stream(const void *stream, const int32_t *acc, void *out,
                                    const float *x_scale, const float *w_scale,
                                    const float *bias, int64_t M, int64_t N);

/* The same on a [M,N] column slice of a [M, acc_row_stride] accumulator.
 * Replaces convrot.h:87-97. */
int xpuint8_dequant_epilogue_slice(const int32_t *acc, void *out, const float *x_scale,
                                   const float *w_scale, const float *bias, int64_t M,
                                   int64_t N, int64_t acc_row_stride);
int xpuint8_dequant_epilogue_slice_stream(const void *stream, const int32_t *acc, void *out,
                                          const float *x_scale, const float *w_scale,
                                          const float *bias, int64_t M, int64_t N,
                                          int64_t acc_row_stride);

/* Dequant + activation (3 situ, 4 geglu_erf: acc [M,2K] = [hidden|gate];
 * 5 gelu_erf: acc [M,K]) + rotate + quantize -> int8 q[M,K] + scale[M].
 * w_scale has 2K (paired) or K entries.  Replaces convrot.h:98-113. */
int xpuint8_dequant_act_quantize(const void *acc, int8_t *q, float *scale, const float *x_scale,
                                 const float *w_scale, int64_t M, int64_t K, int32_t activation);
int xpuint8_dequant_act_quantize_stream(const void *stream, const void *acc, int8_t *q,
                                        float *scale, const float *x_scale,
                                        const float *w_scale, int64_t M, int64_t K,
                                        int32_t activation);

/* ---- what the reference delegated to torch ----------------------------- */

/* c[M,N] = a[M,K] @ b[N,K]^T, int8 x int8 -> int32, exact.  K % 16 == 0,
 * K <= 131072 (no int32 overflow).  Replaces torch._int_mm(a, b.t()) at
 * python/xpu_kernels/int8/ops.py:587 and :634. */
int xpuint8_int8_gemm_stream(const void *stream, const int8_t *a, const int8_t *b, int32_t *c,
                             int64_t M, int64_t N, int64_t K);

/* c[M,N] = a[M,K] @ b[K,N] (both row-major: the contraction runs down b's
 * rows).  `work` is a caller-owned int8 buffer of N*K bytes that receives b^T.
 * Replaces torch._int_mm(q, w8) at python/xpu_kernels/int8/ops.py:371. */
int xpuint8_int8_gemm_nn_stream(const void *stream, const int8_t *a, const int8_t *b, int32_t *c,
                                int64_t M, int64_t N, int64_t K, int8_t *work);

/* The linear's GEMM with the dequant epilogue fused into its store:
 * out[m,n] = bf16(float(sum_k xq[m,k] w8[n,k]) * (w_scale[n] * x_scale[m]) + bias[n]),
 * bit-identical to xpuint8_int8_gemm_stream followed by
 * xpuint8_dequant_epilogue_stream.  bias may be NULL; it is fp32[N] when
 * bias_bf16 == 0 and bf16[N] when bias_bf16 == 1 (widened exactly, as the
 * reference's bias.float()).  N % 16 == 0.
 * Replaces torch._int_mm + dequant at python/xpu_kernels/int8/ops.py:634-638. */
int xpuint8_linear_gemm_stream(const void *stream, const int8_t *xq, const float *x_scale,
                               const int8_t *w8, const float *w_scale, const void *bias,
                               int32_t bias_bf16, void *out, int64_t M, int64_t N, int64_t K);

/* x quantized as by xpuint8_convrot_quantize_stream, with q written in the
 * MFMA block layout that the GEMM of xpuint8_linear_stream reads: block
 * (m/16, k/64) of 16 rows x 64 bytes is the 1 KB at
 * ((m/16) * ceil(K/64) + k/64) * 1024, row r = m%16 at 64r in it and the
 * row's 16-byte chunk c = (k%64)/16 at 16 * (c ^ ((r >> 1) & 3)).  q holds
 * ceil(M/16) * ceil(K/64) * 1024 bytes; rows past M in the last block are
 * left unwritten.  K % 256 == 0, K <= 16384 (or K / 256 even, up to 32768).
 * No counterpart in the
 * reference: it exposes the intermediate the one-call linear keeps
 * internally, so that the GEMM can be run (and timed) on its own. */
int xpuint8_convrot_quantize_tiled_stream(const void *stream, const void *x, int8_t *q,
                                          float *scale, int64_t M, int64_t K);

/* xpuint8_linear_gemm_stream with xq in that block layout, bit for bit the
 * same result.  Only for the shapes whose GEMM reads it (the persistent
 * kernel: M > 64 with ceil(M/256) * ceil(N/320) tiles >= the CU count; the
 * split-K kernel: narrow outputs with K >= 1024); other shapes return an
 * error.  No counterpart in the reference (see above). */
int xpuint8_linear_gemm_tiled_stream(const void *stream, const int8_t *xq, const float *x_scale,
                                     const int8_t *w8, const float *w_scale, const void *bias,
                                     int32_t bias_bf16, void *out, int64_t M, int64_t N,
                                     int64_t K);

/* The whole INT8 linear in one call: out = xpuint8_linear_gemm_stream of
 * xpuint8_convrot_quantize_stream(x), bit for bit, with x bf16 [M,K], the
 * quantized activation and its row scales kept in `work` (a device buffer of
 * at least xpuint8_linear_workspace_size(M, N, K) bytes, 16-byte aligned; it
 * needs no clearing).  Inside it q is laid out for the GEMM that reads it (the
 * MFMA block layout when the split-K kernel takes the shape: narrow outputs
 * with a long K, as the FFN's down-projection), which is why the
 * intermediate is not exposed.  An output too small to fill the GPU (fewer
 * than 128 tiles of 128 x 160, with K long enough to split: K >= 2048, or
 * K >= 1024 for M <= 256; for 33 <= M <= 128, fewer than 256 blocks of 32
 * columns with K >= 2048) has its product split in K across blocks; the
 * workspace then also holds the slices' int32 partial products, whose sum
 * is exact.  K % 256 == 0, N % 16 == 0; bias as in
 * xpuint8_linear_gemm_stream.  Replaces quantize + torch._int_mm + dequant at
 * python/xpu_kernels/int8/ops.py:622-638 and the down-projection of ffn
 * (ops.py:716-719). */
int xpuint8_linear_stream(const void *stream, const void *x, const int8_t *w8,
                          const float *w_scale, const void *bias, int32_t bias_bf16, void *out,
                          int64_t M, int64_t N, int64_t K, void *work, int64_t work_bytes);

/* The workspace xpuint8_linear_stream needs, in bytes, or -1 when the shape is
 * not supported.  No device needed.  A helper of the entry point above, with
 * no counterpart in the reference. */
int64_t xpuint8_linear_workspace_size(int64_t M, int64_t N, int64_t K);

/* xpuint8_linear_gemm_stream followed by the residual update of
 * linear(residual=, residual_scale=), fused into the same store:
 *   d[m,n]   = the linear_gemm result (bf16),
 *   out[m,n] = bf16(float(residual[m,n]) + float(d[m,n]) * float(residual_scale[n]))
 * with residual bf16 [M,N] and residual_scale bf16 [N]: torch.addcmul(residual,
 * d, residual_scale) on bf16 tensors, bit for bit (the bf16 product is exact
 * in fp32).  out may be residual itself (each element is read before it is
 * written, by the same thread).  Replaces the dequant + addcmul of
 * python/xpu_kernels/int8/ops.py:634-644. */
int xpuint8_linear_gemm_residual_stream(const void *stream, const int8_t *xq,
                                        const float *x_scale, const int8_t *w8,
                                        const float *w_scale, const void *bias, int32_t bias_bf16,
                                        const void *residual, const void *residual_scale,
                                        void *out, int64_t M, int64_t N, int64_t K);

/* The FFN's up-projection with the dequant and the activation fused into the
 * GEMM's store:
 *   d_j[m,n] = bf16(float(sum_k xq[m,k] w8[j*N+n,k]) * (w_scale[j*N+n] * x_scale[m]))
 *   out[m,n] = act(d_0, d_1)      bf16 [M,N]
 * for the paired activations 3 (situ: hidden, gate) and 4 (GEGLU: hidden,
 * gate), whose w8 is [2N, K] = [first half | second half]; for 5 (GELU-erf)
 * w8 is [N, K] and out = gelu(d_0).  `out` quantized by
 * xpuint8_convrot_quantize_stream equals xpuint8_dequant_act_quantize_stream
 * of the int32 accumulator, bit for bit, without the accumulator round trip.
 * N % 16 == 0, K % 16 == 0.  Replaces torch._int_mm + the load side of
 * dequant_act_quantize in ffn (python/xpu_kernels/int8/ops.py:714-715). */
int xpuint8_ffn_up_stream(const void *stream, const int8_t *xq, const float *x_scale,
                          const int8_t *w8, const float *w_scale, void *out, int64_t M, int64_t N,
                          int64_t K, int32_t activation);

/* The whole FFN in one call:
 *   (xq, xs) = xpuint8_convrot_quantize_stream(x)            x bf16 [M,K]
 *   v        = xpuint8_ffn_up_stream(xq, xs, up_w8, up_scale) bf16 [M,inner]
 *   out      = xpuint8_linear_stream(v, down_w8, down_scale, bias)  bf16 [M,K]
 * bit for bit, with up_w8 [2*inner, K] for activations 3 and 4 and
 * [inner, K] for 5, up_scale fp32 per up row, down_w8 int8 [K, inner],
 * down_scale fp32 [K], bias as in xpuint8_linear_gemm_stream (the
 * up-projection is unbiased).  The intermediates live in `work`, a device
 * buffer of at least xpuint8_ffn_workspace_size(M, inner, K, activation)
 * bytes, 16-byte aligned; it needs no clearing.  K % 256 == 0,
 * inner % 256 == 0.  Replaces ffn (python/xpu_kernels/int8/ops.py:649-719):
 * its quantize, torch._int_mm, dequant_act_quantize, torch._int_mm and
 * dequant, in four kernels (five when the down-projection is split in K). */
int xpuint8_ffn_stream(const void *stream, const void *x, const int8_t *up_w8,
                       const float *up_scale, const int8_t *down_w8, const float *down_scale,
                       const void *bias, int32_t bias_bf16, void *out, int64_t M, int64_t inner,
                       int64_t K, int32_t activation, void *work, int64_t work_bytes);

/* The workspace xpuint8_ffn_stream needs, in bytes, or -1 when the shape or
 * the activation is not supported.  No device needed.  A helper of the entry
 * point above, with no counterpart in the reference. */
int64_t xpuint8_ffn_workspace_size(int64_t M, int64_t inner, int64_t K, int32_t activation);

/* ---- the packed weight (no counterpart in the reference) ----
 * A prepared weight w8 int8 [N,K] (row-major, as prepare_weight returns it)
 * copied into the MFMA block layout of xpuint8_convrot_quantize_tiled_stream
 * (16-row x 64-byte blocks, each one contiguous 1 KB), the bytes past K zero.
 * The GEMMs that stream the weight through LDS then load whole cache lines
 * (one 1 KB block per load) instead of 16 half lines; the results are the
 * same bits.  The packed copy is derived data: a caller that changes w8
 * packs it again.  N % 16 == 0, K % 16 == 0. */

/* The bytes of the packed copy of an [N,K] weight (N * K rounded up to whole
 * blocks), or -1 for an unsupported shape.  No device needed. */
int64_t xpuint8_packed_weight_bytes(int64_t N, int64_t K);

/* packed = w8 [N,K] in the MFMA block layout (xpuint8_packed_weight_bytes(N, K)
 * bytes, 16-byte aligned; w8 16-byte aligned). */
int xpuint8_pack_weight_stream(const void *stream, const int8_t *w8, int8_t *packed, int64_t N,
                               int64_t K);

/* xpuint8_linear_stream, bit for bit, reading w8_packed (w8 packed by
 * xpuint8_pack_weight_stream) in the GEMMs that take the block layout and w8
 * in the others; w8_packed may be null (then it is xpuint8_linear_stream).
 * The workspace is xpuint8_linear_workspace_size(M, N, K). */
int xpuint8_linear_packed_stream(const void *stream, const void *x, const int8_t *w8,
                                 const int8_t *w8_packed, const float *w_scale, const void *bias,
                                 int32_t bias_bf16, void *out, int64_t M, int64_t N, int64_t K,
                                 void *work, int64_t work_bytes);

/* The whole of linear(x, w8, ws, bias, residual=, residual_scale=) in one call:
 * xpuint8_convrot_quantize_stream(x) then xpuint8_linear_gemm_residual_stream,
 * bit for bit, with the quantized activation in `work`
 * (xpuint8_linear_workspace_size(M, N, K) bytes) laid out for the GEMM that
 * reads it (the MFMA block layout where the persistent or the split-K kernel
 * takes the shape), and w8_packed (optional) read there in place of w8.
 * Replaces quantize + torch._int_mm + dequant + addcmul at
 * python/xpu_kernels/int8/ops.py:631-644; no counterpart as one call. */
int xpuint8_linear_residual_packed_stream(const void *stream, const void *x, const int8_t *w8,
                                          const int8_t *w8_packed, const float *w_scale,
                                          const void *bias, int32_t bias_bf16,
                                          const void *residual, const void *residual_scale,
                                          void *out, int64_t M, int64_t N, int64_t K, void *work,
                                          int64_t work_bytes);

/* linear_acc in one call: (q, x_scale) = xpuint8_convrot_quantize_stream(x),
 * acc[M,N] = q @ w8^T (int32, exact), bit for bit, the codes in `work`
 * (xpuint8_linear_workspace_size(M, N, K) bytes suffice) laid out for the
 * GEMM (the MFMA block layout where the persistent kernel takes the shape),
 * and w8_packed (optional) read there in place of w8.  x_scale fp32 [M] is
 * an output.  Replaces quantize + torch._int_mm at
 * python/xpu_kernels/int8/ops.py:571-588; no counterpart as one call. */
int xpuint8_linear_acc_packed_stream(const void *stream, const void *x, const int8_t *w8,
                                     const int8_t *w8_packed, int32_t *acc, float *x_scale,
                                     int64_t M, int64_t N, int64_t K, void *work,
                                     int64_t work_bytes);

/* xpuint8_linear_gemm_tiled_stream, bit for bit, with the weight given only
 * packed; its shapes and those of the skinny kernel (M <= 64 with no split
 * in K: N >= 2048, or M <= 32) -- others return an error. */
int xpuint8_linear_gemm_packed_stream(const void *stream, const int8_t *xq, const float *x_scale,
                                      const int8_t *w8_packed, const float *w_scale,
                                      const void *bias, int32_t bias_bf16, void *out, int64_t M,
                                      int64_t N, int64_t K);

/* xpuint8_ffn_stream, bit for bit, with either weight's packed copy (or null)
 * read where its GEMM takes the block layout.  The workspace is
 * xpuint8_ffn_workspace_size(M, inner, K, activation). */
int xpuint8_ffn_packed_stream(const void *stream, const void *x, const int8_t *up_w8,
                              const int8_t *up_packed, const float *up_scale,
                              const int8_t *down_w8, const int8_t *down_packed,
                              const float *down_scale, const void *bias, int32_t bias_bf16,
                              void *out, int64_t M, int64_t inner, int64_t K, int32_t activation,
                              void *work, int64_t work_bytes);

/* The weight's second packed form, for linear_dx_int8's product q @ w8 (the
 * contraction over w8's rows): w8 [N,K] in the NN stage order of that GEMM,
 * per 64 rows and 32 columns two 1 KB blocks of 32 rows x 32 bytes (block
 * ((s * K/32 + c) * 2 + h) * 1024 for rows 64s + 32h.. and columns 32c..; in
 * it, 16-byte chunk l holds row l/2, column half (l & 1) ^ ((l >> 5) & 1)),
 * zeros past N.  xpuint8_packed_weight_nn_bytes(N, K) = ceil(N/64) * 64 * K,
 * or -1 (N % 16 == 0, K % 32 == 0 required).  No device needed for the size. */
int64_t xpuint8_packed_weight_nn_bytes(int64_t N, int64_t K);
int xpuint8_pack_weight_nn_stream(const void *stream, const int8_t *w8, int8_t *packed, int64_t N,
                                  int64_t K);

/* The backward of int8_linear(mode="int8") in one call: dbias = the column
 * sums of dy (xpuint8_column_sum_stream, bit for bit; bf16, or with
 * dbias_fp32 = 1 the fp32 each bf16 sum widens to, which is what the bias
 * of an fp32 parameter receives; dbias may be null) and dx =
 * xpuint8_linear_dx_int8_stream(dy, w_scale, w8), bit for bit, reading
 * w8_packed_nn (optional) as xpuint8_linear_dx_int8_packed_stream does.
 * `work` holds xpuint8_linear_backward_int8_workspace_size(M, N, K) bytes.
 * Replaces the bias-gradient sum and linear_dx_int8 of
 * python/xpu_kernels/int8/ops.py:270-289; no counterpart as one call. */
int64_t xpuint8_linear_backward_int8_workspace_size(int64_t M, int64_t N, int64_t K);
int xpuint8_linear_backward_int8_stream(const void *stream, const void *dy, const float *w_scale,
                                        const int8_t *w8, const int8_t *w8_packed_nn, void *dx,
                                        void *dbias, int32_t dbias_fp32, int64_t M, int64_t N,
                                        int64_t K, void *work, int64_t work_bytes);

/* The backward of int8_linear(mode="dense") in one call: dbias as in
 * xpuint8_linear_backward_int8_stream, and dx = dy @ dequant_weight(w8,
 * w_scale) (xpuint8_dequant_weight_stream then xpuint8_linear_dx_stream, bit
 * for bit), the dequantized weight in `work`
 * (xpuint8_linear_backward_dense_workspace_size(M, N, K) bytes: 2*N*K for it,
 * the column sums' partials, and a small batch's split contraction).  K % 256
 * == 0, N % 16 == 0.  Replaces the bias-gradient sum, dequant_weight and
 * linear_dx of python/xpu_kernels/int8/ops.py:270-289; no counterpart as one
 * call. */
int64_t xpuint8_linear_backward_dense_workspace_size(int64_t M, int64_t N, int64_t K);
int xpuint8_linear_backward_dense_stream(const void *stream, const void *dy, const int8_t *w8,
                                         const float *w_scale, void *dx, void *dbias,
                                         int32_t dbias_fp32, int64_t M, int64_t N, int64_t K,
                                         void *work, int64_t work_bytes);

/* xpuint8_linear_dx_int8_stream, bit for bit, reading w8_packed_nn (w8 packed
 * by xpuint8_pack_weight_nn_stream; null reads w8) where the split-K GEMM
 * takes the product. */
int xpuint8_linear_dx_int8_packed_stream(const void *stream, const void *dy, const float *w_scale,
                                         const int8_t *w8, const int8_t *w8_packed_nn, void *dx,
                                         int64_t M, int64_t N, int64_t K, void *work,
                                         int64_t work_bytes);

/* linear_dx_int8's GEMM: dx[m,k] = bf16(float(sum_n q[m,n] w8[n,k]) * a[m]),
 * the NN product with the row-scale epilogue.  `work` holds w8^T (K*N bytes).
 * Replaces torch._int_mm(q, w8) + dequant(acc, a, ones) at
 * python/xpu_kernels/int8/ops.py:371-376. */
int xpuint8_dx_gemm_stream(const void *stream, const int8_t *q, const float *a,
                           const int8_t *w8, void *dx, int64_t M, int64_t N, int64_t K,
                           int8_t *work);

/* linear_dx_int8 in one call: dL/dx of the INT8 linear against the weight
 * still in int8,
 *   d = bf16(dy * bf16(w_scale[n])),  (q, a) = quantize_row(d),
 *   dx = rotate_bf16(bf16(float(sum_n q[m,n] w8[n,k]) * a[m]))
 * with dy bf16 [M,N], w8 int8 [N,K] (prepared: rotated rows), w_scale fp32
 * [N], dx bf16 [M,K].  K % 256 == 0, N % 16 == 0.  `work` is a device buffer
 * of at least xpuint8_linear_dx_int8_workspace_size(M, N, K) bytes (the
 * quantized gradient, its scales, the transposed weight and the product before
 * the inverse rotation; for small batches, whose [M,K] output has too few
 * tiles to fill the GPU, also the int32 partial products of the contraction
 * split across blocks), 16-byte aligned; it is fully written before it is
 * read, so it needs no clearing.  Replaces linear_dx_int8
 * (python/xpu_kernels/int8/ops.py:353-377): its torch multiply, the Triton
 * quantize_row, torch._int_mm, dequant and rotate. */
int xpuint8_linear_dx_int8_stream(const void *stream, const void *dy, const float *w_scale,
                                  const int8_t *w8, void *dx, int64_t M, int64_t N, int64_t K,
                                  void *work, int64_t work_bytes);

/* The workspace xpuint8_linear_dx_int8_stream needs, in bytes, or -1 when the
 * shape is not supported.  No device needed.  A helper of the entry point
 * above, with no counterpart in the reference. */
int64_t xpuint8_linear_dx_int8_workspace_size(int64_t M, int64_t N, int64_t K);

/* xpuint8_linear_dx_int8_stream without the workspace argument and without
 * allocating anything: for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  The workspace is the
 * library's own fixed array of 64 MiB per device (67108864 bytes, reserved
 * when the library is loaded and kept until the process ends); a shape whose
 * xpuint8_linear_dx_int8_workspace_size exceeds it is rejected with code 4
 * (config 5, M=4096 N=5120 K=1280, needs 38 MB).  Every call on a device
 * shares that array: calls that overlap on one device (two streams, two
 * threads) race and must be serialised by the caller.  The result equals
 * xpuint8_linear_dx_int8_stream's bit for bit.  Under stream capture: the
 * library's set-up of a device (a synchronous upload of the activation
 * tables and the lookup of this array's address, on the first call on that
 * device) cannot be captured, so run it before the capture begins --
 * xpuint8_init() with the device current, or any uncaptured call on it. */
int xpuint8_linear_dx_int8_noalloc_stream(const void *stream, const void *dy, const float *w_scale,
                                          const int8_t *w8, void *dx, int64_t M, int64_t N,
                                          int64_t K);

/* prepare_weight in one kernel, bit-identical to the torch chain of
 * python/xpu_kernels/int8/ops.py:93-99: bf16 w[N,K] -> int8 q[N,K] + fp32
 * scale[N].  (xpuint8_convrot_quantize is prepare_weight_fused.) */
int xpuint8_prepare_weight_stream(const void *stream, const void *w, int8_t *q, float *scale,
                                  int64_t N, int64_t K);

/* Per-row int8 quantization without rotation (the gradient row quantizer):
 * x bf16 [M,N] -> q int8 [M,N] + scale fp32 [M], bit-identical to
 * quantize_row_torch (python/xpu_kernels/int8/ops.py:320-330).  With a
 * non-NULL col_scale[N] the row is first bf16(x * bf16(col_scale)), the
 * dy * w_scale product of ops.py:366.  N % 16 == 0.  Replaces the Triton
 * quantize_row (python/xpu_kernels/triton/quantize.py:63-126). */
int xpuint8_quantize_row_stream(const void *stream, const void *x, const float *col_scale,
                                int8_t *q, float *scale, int64_t M, int64_t N);

/* Column sums of a bf16 matrix, out[n] = bf16(sum_m x[m,n]): x bf16 [M,N],
 * out bf16 [N], N % 16 == 0.  The bias gradient dy.sum(dim=0) of the
 * reference's backward (python/xpu_kernels/int8/ops.py:276, 821), which torch
 * reduces in an order of its own; here the order is fixed: fp32 sums of 32
 * consecutive rows, each in row order, then those sums in order, rounded to
 * bf16 (to nearest even) once.  work: xpuint8_column_sum_workspace_size(M, N)
 * bytes (the fp32 partial sums), 16-byte aligned. */
int xpuint8_column_sum_stream(const void *stream, const void *x, void *out, int64_t M, int64_t N,
                              void *work, int64_t work_bytes);

/* The workspace xpuint8_column_sum_stream needs, in bytes, or -1 when the
 * shape is not supported.  No device needed.  No counterpart in the
 * reference. */
int64_t xpuint8_column_sum_workspace_size(int64_t M, int64_t N);

/* The weight gradient of a linear: dw[n,k] = sum_m dy[m,n] * x[m,k], dy bf16
 * [M,N], x bf16 [M,K], dw bf16 [N,K]; fp32 accumulation, one RNE rounding.
 * N % 16 == 0, K % 16 == 0.  Replaces the torch matmul dy^T @ x of linear_dw
 * (python/xpu_kernels/int8/ops.py:207-238). */
int xpuint8_linear_dw_stream(const void *stream, const void *dy, const void *x, void *dw,
                             int64_t M, int64_t N, int64_t K);

/* The activation gradient of a linear with a bf16 weight (the dense-mode
 * backward): dx[m,k] = sum_n dy[m,n] * w[n,k], dy bf16 [M,N], w bf16 [N,K]
 * (the unrotated weight, e.g. from xpuint8_dequant_weight_stream), dx bf16
 * [M,K]; fp32 accumulation, one RNE rounding.  N % 16 == 0, K % 16 == 0.
 * `work` may be NULL.  A small batch, whose [M,K] output has too few tiles to
 * fill the GPU, with a `work` of xpuint8_linear_dx_workspace_size(M, N, K)
 * bytes (16-byte aligned; no clearing needed) has the contraction split
 * across blocks: their fp32 partial sums are added in a fixed order, then
 * rounded once, so the result is as above up to the order of the fp32 sum.
 * Replaces the torch matmul dy @ w of linear_dx
 * (python/xpu_kernels/int8/ops.py:194-204). */
int xpuint8_linear_dx_stream(const void *stream, const void *dy, const void *w, void *dx,
                             int64_t M, int64_t N, int64_t K, void *work, int64_t work_bytes);

/* The workspace xpuint8_linear_dx_stream uses for this shape, in bytes: 0
 * when the contraction is not split, -1 when the shape is not supported.  No
 * device needed.  A helper of the entry point above (no reference
 * counterpart). */
int64_t xpuint8_linear_dx_workspace_size(int64_t M, int64_t N, int64_t K);

/* RMSNorm + rotary embedding of q or k read straight from the int32
 * accumulator of a quantized qkv projection (one [B,S,H,D] slice of it):
 *   x = bf16(float(acc) * (w_scale[h*D+d] * x_scale[b,s])),
 *   y = bf16(x * rsqrt(mean_d(x^2) + epsilon) * scale[d]),
 *   out = the pairwise rotation of y by freqs_cis (fp32 [FB,FS,1,D/2,2,2],
 *         FB in {1,B}, FS in {1,S}), pairs (p, p+D/2) when split_half else
 *         (2p, 2p+1); out bf16 [B,S,H,D] contiguous.
 * acc's head dim is contiguous (element strides given for b, s, h); x_scale is
 * [B,S] with the given strides; w_scale fp32 [H*D]; scale fp32 [D]; D even,
 * 2 <= D <= 256.  Replaces the Triton _rms_rope_rows_dq_kernel behind
 * rms_rope_split_half_dequant (python/xpu_kernels/triton/rope.py:149-222,
 * 378-405, 643-652). */
int xpuint8_rms_rope_dequant_stream(const void *stream, const int32_t *acc, int64_t acc_stride_b,
                                    int64_t acc_stride_s, int64_t acc_stride_h,
                                    const float *x_scale, int64_t xs_stride_b,
                                    int64_t xs_stride_s, const float *w_scale, const float *freqs,
                                    int64_t f_stride_b, int64_t f_stride_s, int64_t f_stride_dim,
                                    int64_t f_stride_rot, int64_t f_stride_pair, int64_t f_batch,
                                    int64_t f_seq, const float *scale, void *out, int64_t B,
                                    int64_t S, int64_t H, int64_t D, float epsilon,
                                    int32_t split_half);

/* Host copy of an activation table (65536 bf16 entries indexed by the bf16
 * bit pattern of the input): 0 gelu_erf, 1 gelu_tanh, 2 silu, 3 situ's
 * tanh(bf16(x/4)), 4 sigmoid, 5 situ's tanh(bf16(x/25)), 6 situ's gate
 * factor bf16(table 3 * table 4).  No device needed.
 * No counterpart in the reference: it exposes the exact functions the fused
 * activations apply, for verification. */
int xpuint8_activation_table(int32_t id, uint16_t *out);

#ifdef __cplusplus
}
#endif
#endif /* XPUINT8_H */
