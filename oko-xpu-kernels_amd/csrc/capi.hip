// The C ABI (include/xpuint8.h): argument validation, error reporting, device
// initialisation and dispatch to the launchers in kernels.hpp.
//
// Validation runs before any HIP call, so an argument error is reported the
// same way on a machine without a GPU.  Errors are thread-local strings
// (the reference keeps one process-global string, src/xpuint8.cpp:36-50).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "activations.hpp"
#include "kernels.hpp"
#include "../../include/xpuint8.h"

namespace xpuint8 {

// Device copy of the activation tables.  Host code reaches it only through
// the address hipGetSymbolAddress returns for the current device.
__device__ uint16_t g_act_tables[kNumTables * kTabSize];

// The workspace of the no-allocation entry point
// (xpuint8_linear_dx_int8_noalloc_stream): one 64 MiB array on every device
// the library runs on, held until the process ends.  In host code `scratch`
// names a host-side stand-in, not device memory: its device address is taken
// once per device at set-up (ensure_device, g_scratch) and only that address
// is ever passed to a kernel.  Every call on a device shares its array, so
// calls that overlap on one device race.
constexpr size_t kScratchBytes = size_t(64) << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

namespace {

thread_local std::string t_error;

int fail(int code, const std::string& msg) {
    t_error = msg;
    return code;
}

constexpr int kMaxDevices = 64;
std::mutex g_mutex;
std::string g_device_name[kMaxDevices];
const uint16_t* g_tab_dev[kMaxDevices] = {};
char* g_scratch[kMaxDevices] = {};        // device address of `scratch`, per device
int g_cus[kMaxDevices] = {};
std::atomic<bool> g_ready[kMaxDevices] = {};

// Per-device set-up: architecture check and table upload.  Returns 0 or an
// error code (message set).
int ensure_device() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(1, "no HIP device available");
    if (dev < 0 || dev >= kMaxDevices) return fail(1, "device index out of range");
    if (g_ready[dev].load(std::memory_order_acquire)) return 0;
    std::lock_guard<std::mutex> lock(g_mutex);
    if (g_ready[dev].load(std::memory_order_relaxed)) return 0;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess)
        return fail(1, "hipGetDeviceProperties failed");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(1, std::string("libxpuint8 is built for gfx950 only; device ") +
                           std::to_string(dev) + " is " + prop.gcnArchName);
    void* sym = nullptr;
    hipError_t e = hipGetSymbolAddress(&sym, HIP_SYMBOL(g_act_tables));
    if (e != hipSuccess || sym == nullptr)
        return fail(5, std::string("hipGetSymbolAddress(activation tables): ") + hipGetErrorString(e));
    e = hipMemcpy(sym, host_activation_tables(), sizeof(uint16_t) * kNumTables * kTabSize,
                  hipMemcpyHostToDevice);
    if (e != hipSuccess)
        return fail(5, std::string("uploading the activation tables: ") + hipGetErrorString(e));
    g_tab_dev[dev] = static_cast<const uint16_t*>(sym);
    void* sp = nullptr;
    e = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch));
    if (e != hipSuccess || sp == nullptr)
        return fail(5, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch[dev] = static_cast<char*>(sp);
    g_cus[dev] = prop.multiProcessorCount;
    g_device_name[dev] = prop.name;
    g_ready[dev].store(true, std::memory_order_release);
    return 0;
}

int launched(hipError_t e, const char* what) {
    if (e != hipSuccess) return fail(5, std::string(what) + ": " + hipGetErrorString(e));
    return 0;
}

// Synchronous wrappers: run on the default stream and wait for it.
int finish(int rc, const char* what) {
    if (rc != 0) return rc;
    const hipError_t e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) return fail(5, std::string(what) + ": " + hipGetErrorString(e));
    return 0;
}

hipStream_t as_stream(const void* s) { return static_cast<hipStream_t>(const_cast<void*>(s)); }

constexpr int64_t kMaxK = 131072;          // 127*127*K < 2^31
constexpr int64_t kMaxDim = (int64_t(1) << 31) - 1;
constexpr int64_t kMaxGemmM = int64_t(65535) * 128;   // grid.y limit of the GEMM launch

int check_rows(int64_t M, int64_t K) {
    if (M <= 0 || K <= 0) return fail(2, "M and K must be positive");
    if (K % 256 != 0) return fail(3, "K must be divisible by the ConvRot group size (256)");
    if (K > kMaxK || M > kMaxDim) return fail(4, "K must be <= 131072 and M < 2^31");
    return 0;
}

int check_epilogue(int64_t M, int64_t N) {
    if (M <= 0 || N <= 0 || N % 16 != 0)
        return fail(2, "M, N must be positive and N must be a multiple of 16");
    if (M > kMaxDim || N > kMaxDim) return fail(4, "M and N must be < 2^31");
    return 0;
}

int check_gemm(int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || N <= 0 || K <= 0) return fail(2, "M, N and K must be positive");
    if (K % 16 != 0 || N % 16 != 0) return fail(2, "K and N must be multiples of 16");
    if (K > kMaxK) return fail(4, "K must be <= 131072 (int32 accumulator range)");
    if (M > kMaxGemmM || N > kMaxDim) return fail(4, "M must be <= 8388480 and N < 2^31");
    return 0;
}

// Every buffer is read and written with 16-byte vector accesses.
#define XPU_NONNULL(p)                                          \
    if (!(p)) return fail(6, #p " must not be null");           \
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0)               \
    return fail(6, #p " must be 16-byte aligned")
#define XPU_ALIGNED_OPT(p)                                      \
    if ((p) && reinterpret_cast<uintptr_t>(p) % 16 != 0)        \
    return fail(6, #p " must be 16-byte aligned")
#define XPU_TRY(expr)              \
    do {                           \
        const int rc_ = (expr);    \
        if (rc_ != 0) return rc_;  \
    } while (0)

// The workspace of linear_dx_int8: the row-quantized column-scaled gradient
// q [M,N] int8 (row-major, or in the MFMA block layout when the split-K
// kernel reads it) and its row scales a [M] fp32, the transposed weight w8^T
// [K,N] int8 (the GEMM's K-contiguous operand, for shapes the split-K kernel
// does not take), and the product before the inverse rotation, bf16 [M,K];
// for a product split in K across blocks (gemm_slices of the [M,K] output
// over the contraction N), then the slices' int32 [M,K] partial products.
// Each piece starts on a 256-byte boundary.
struct DxWork {
    size_t q, a, wt, pre, part, total;
};
DxWork dx_work_layout(int64_t M, int64_t N, int64_t K) {
    auto up = [](int64_t b) { return (size_t(b) + 255) & ~size_t(255); };
    DxWork w;
    w.q = 0;
    w.a = w.q + up(std::max(M * N, tiled_bytes(M, N)));
    w.wt = w.a + up(4 * M);
    w.pre = w.wt + up(N * K);
    w.part = w.pre + up(2 * M * K);
    const int nsl = gemm_slices(int(M), int(K), int(N));
    w.total = w.part + (nsl > 0 ? size_t(nsl) * size_t(M) * size_t(K) * 4 : 0);
    return w;
}

int check_dx(int64_t M, int64_t N, int64_t K) {
    XPU_TRY(check_rows(M, K));               // the inverse rotation: K % 256
    XPU_TRY(check_epilogue(M, N));           // the row quantizer: N % 16
    return check_gemm(M, K, N);              // q [M,N] @ w8 [N,K], contraction over N
}

// quantize_row (column-scaled) -> w8^T -> GEMM with the row-scale epilogue ->
// inverse rotation, all on one stream, through the workspace at `work`.
// wnn (optional): pack_weight_nn's copy of w8, read by the split-K GEMM.
int dx_chain(hipStream_t st, const void* dy, const float* w_scale, const int8_t* w8, void* dx,
             int64_t M, int64_t N, int64_t K, char* work, const int8_t* wnn = nullptr) {
    const DxWork L = dx_work_layout(M, N, K);
    int8_t* q = reinterpret_cast<int8_t*>(work + L.q);
    float* a = reinterpret_cast<float*>(work + L.a);
    int8_t* wt = reinterpret_cast<int8_t*>(work + L.wt);
    void* pre = work + L.pre;
    // the split-K kernel reads w8 [N, K] as it is stored (transposing LDS
    // reads) and q in the MFMA block layout, written so by the quantizer;
    // other shapes take a row-major q, the transposed copy and the NT kernels
    if (splitk_nn_applies(int(M), int(K), int(N), K) && rowquant_can_tile(int(N))) {
        XPU_TRY(launched(quantize_row(st, dy, w_scale, q, a, M, int(N), true),
                         "linear_dx_int8 (quantize_row)"));
        XPU_TRY(launched(gemm_dequant_nn_xt(st, q, wnn ? wnn : w8, K, pre, K, a, int(M), int(K),
                                            int(N), wnn != nullptr),
                         "linear_dx_int8 (gemm)"));
        return launched(rotate_bf16(st, pre, dx, M, int(K)), "linear_dx_int8 (rotate)");
    }
    // too few output tiles for the chip: the contraction split across blocks,
    // the slices' int32 partial sums added by the dequant pass (unit column
    // scale, row scale a)
    if (const int nsl = gemm_slices(int(M), int(K), int(N))) {
        int32_t* part = reinterpret_cast<int32_t*>(work + L.part);
        XPU_TRY(launched(quantize_row(st, dy, w_scale, q, a, M, int(N)),
                         "linear_dx_int8 (quantize_row)"));
        if (slices_need_nt(int(M))) {
            XPU_TRY(launched(transpose_i8(st, w8, wt, N, K), "linear_dx_int8 (transpose)"));
            XPU_TRY(launched(gemm_i32_slices(st, q, N, wt, N, part, int(M), int(K), int(N), nsl),
                             "linear_dx_int8 (gemm)"));
        } else {
            XPU_TRY(launched(gemm_i32_slices_nn(st, q, N, w8, K, part, int(M), int(K), int(N),
                                                nsl),
                             "linear_dx_int8 (gemm)"));
        }
        XPU_TRY(launched(dequant_slices(st, part, K, nsl, M * K, pre, a, nullptr, nullptr,
                                        nullptr, M, K),
                         "linear_dx_int8 (dequant)"));
        return launched(rotate_bf16(st, pre, dx, M, int(K)), "linear_dx_int8 (rotate)");
    }
    XPU_TRY(launched(quantize_row(st, dy, w_scale, q, a, M, int(N)), "linear_dx_int8 (quantize_row)"));
    bool nn = false;
    XPU_TRY(launched(gemm_dequant_nn(st, q, N, w8, K, pre, K, a, int(M), int(K), int(N), &nn),
                     "linear_dx_int8 (gemm)"));
    if (!nn) {
        XPU_TRY(launched(transpose_i8(st, w8, wt, N, K), "linear_dx_int8 (transpose)"));
        XPU_TRY(launched(gemm_dequant(st, q, N, wt, N, pre, K, a, nullptr, nullptr, nullptr,
                                      int(M), int(K), int(N)),
                         "linear_dx_int8 (gemm)"));
    }
    return launched(rotate_bf16(st, pre, dx, M, int(K)), "linear_dx_int8 (rotate)");
}

// The workspace of xpuint8_linear_stream: x quantized, q int8 (row-major, or
// in the MFMA block layout when the split-K kernel reads it), then its row
// scales fp32 [M], on a 256-byte boundary; for a product split across blocks
// in K (gemm_slices), then the slices' int32 partial products, also on a
// 256-byte boundary.
size_t linear_work_q_bytes(int64_t M, int64_t K) {
    return (size_t(std::max(M * K, tiled_bytes(M, K))) + 255) & ~size_t(255);
}
size_t linear_work_part_offset(int64_t M, int64_t K) {
    return (linear_work_q_bytes(M, K) + 4 * size_t(M) + 255) & ~size_t(255);
}
size_t linear_work_bytes(int64_t M, int64_t N, int64_t K) {
    const int nsl = gemm_slices(int(M), int(N), int(K));
    if (nsl > 0) return linear_work_part_offset(M, K) + size_t(nsl) * size_t(M) * size_t(N) * 4;
    return linear_work_q_bytes(M, K) + 4 * size_t(M);
}

// quantize + GEMM + dequant of xpuint8_linear_stream on checked arguments.
// wp (optional): pack_weight's copy of w8, read instead of w8 by the kernels
// that take the block layout (the split-K, persistent and skinny ones).
int linear_run(hipStream_t st, const void* x, const int8_t* w8, const float* w_scale,
               const void* bias, int32_t bias_bf16, void* out, int64_t M, int64_t N, int64_t K,
               void* work, const int8_t* wp = nullptr) {
    const int8_t* wb = wp ? wp : w8;
    int8_t* q = static_cast<int8_t*>(work);
    float* xs = reinterpret_cast<float*>(static_cast<char*>(work) + linear_work_q_bytes(M, K));
    const float* b32 = bias_bf16 ? nullptr : static_cast<const float*>(bias);
    const uint16_t* b16 = bias_bf16 ? static_cast<const uint16_t*>(bias) : nullptr;
    // too few output tiles for the chip: the product split in K across
    // blocks, each slice's int32 partial sums in the workspace, then one pass
    // that adds them and applies the dequant
    if (const int nsl = gemm_slices(int(M), int(N), int(K))) {
        int32_t* part = reinterpret_cast<int32_t*>(static_cast<char*>(work) +
                                                   linear_work_part_offset(M, K));
        XPU_TRY(launched(convrot_quantize(st, x, q, xs, M, int(K), 0), "linear (quantize)"));
        XPU_TRY(launched(gemm_i32_slices(st, q, K, w8, K, part, int(M), int(N), int(K), nsl),
                         "linear (gemm)"));
        return launched(dequant_slices(st, part, N, nsl, M * N, out, xs, w_scale, b32, b16, M, N),
                        "linear (dequant)");
    }
    // narrow outputs with a long K take the split-K kernel, which reads q in
    // the MFMA block layout; the other shapes a row-major q
    if (splitk_applies(int(M), int(N), int(K)) && rowquant_can_tile(int(K))) {
        XPU_TRY(launched(convrot_quantize_tiled(st, x, q, xs, M, int(K)), "linear (quantize)"));
        return launched(gemm_dequant_xt(st, q, wb, K, out, N, xs, w_scale, b32, b16, int(M),
                                        int(N), int(K), wp != nullptr),
                        "linear (gemm)");
    }
    // the persistent kernel reads q in the MFMA block layout too
    if (pp_applies(int(M), int(N), int(K), false) && rowquant_can_tile(int(K))) {
        XPU_TRY(launched(convrot_quantize_tiled(st, x, q, xs, M, int(K)), "linear (quantize)"));
        return launched(gemm_dequant_pp_xt(st, q, wb, K, out, N, xs, w_scale, b32, b16, int(M),
                                           int(N), int(K), wp != nullptr),
                        "linear (gemm)");
    }
    // and the skinny one, given the packed weight
    if (wp && skinny_applies(int(M), false) && rowquant_can_tile(int(K))) {
        XPU_TRY(launched(convrot_quantize_tiled(st, x, q, xs, M, int(K)), "linear (quantize)"));
        return launched(gemm_dequant_skinny_xt(st, q, wp, out, N, xs, w_scale, b32, b16, int(M),
                                               int(N), int(K)),
                        "linear (gemm)");
    }
    XPU_TRY(launched(convrot_quantize(st, x, q, xs, M, int(K), 0), "linear (quantize)"));
    return launched(gemm_dequant(st, q, K, w8, K, out, N, xs, w_scale, b32, b16, int(M), int(N),
                                 int(K), wp),
                    "linear (gemm)");
}

// The four launches of the FFN after its up-projection's quantize: the
// up-projection GEMM with the activation in its store, then the linear of
// the activation.  Workspace: the activation bf16 [M, inner], then one
// region that first holds x quantized (row-major q, then its row scales on a
// 256-byte boundary) and then, once the up-projection has read it, the
// down-projection's linear workspace.
size_t ffn_work_region_offset(int64_t M, int64_t inner) {
    return (size_t(M) * size_t(inner) * 2 + 255) & ~size_t(255);
}
size_t ffn_work_bytes(int64_t M, int64_t inner, int64_t K) {
    const size_t up = linear_work_q_bytes(M, K) + 4 * size_t(M);
    return ffn_work_region_offset(M, inner) + std::max(up, linear_work_bytes(M, K, inner));
}

int ffn_check(int64_t M, int64_t inner, int64_t K, int32_t activation) {
    if (activation != 3 && activation != 4 && activation != 5)
        return fail(6, "ffn supports activation 3 (situ), 4 (GEGLU) or 5 (GELU-erf)");
    XPU_TRY(check_rows(M, K));           // x rotated: K % 256
    XPU_TRY(check_rows(M, inner));       // the activation rotated: inner % 256
    XPU_TRY(check_epilogue(M, inner));
    XPU_TRY(check_epilogue(M, K));
    XPU_TRY(check_gemm(M, act_paired(activation) ? 2 * inner : inner, K));
    return check_gemm(M, K, inner);
}

// The FFN of xpuint8_ffn_stream on checked arguments; up_wp / down_wp
// (optional) are pack_weight's copies of the two weights.
int ffn_run(hipStream_t st, const void* x, const int8_t* up_w8, const int8_t* up_wp,
            const float* up_scale, const int8_t* down_w8, const int8_t* down_wp,
            const float* down_scale, const void* bias, int32_t bias_bf16, void* out, int64_t M,
            int64_t inner, int64_t K, int32_t activation, void* work) {
    char* v = static_cast<char*>(work);
    char* region = v + ffn_work_region_offset(M, inner);
    int8_t* xq = reinterpret_cast<int8_t*>(region);
    float* xs = reinterpret_cast<float*>(region + linear_work_q_bytes(M, K));
    // the persistent up-projection reads xq in the MFMA block layout
    if (pp_applies(int(M), int(inner), int(K), act_paired(activation)) &&
        rowquant_can_tile(int(K))) {
        XPU_TRY(launched(convrot_quantize_tiled(st, x, xq, xs, M, int(K)), "ffn (quantize)"));
        XPU_TRY(launched(gemm_act_pp_xt(st, xq, up_wp ? up_wp : up_w8, K, v, inner, xs, up_scale,
                                        int(M), int(inner), int(K), activation, up_wp != nullptr),
                         "ffn (up projection)"));
    } else if (up_wp && skinny_applies(int(M), act_paired(activation)) &&
               rowquant_can_tile(int(K))) {
        // so does the skinny one, given the packed weight
        XPU_TRY(launched(convrot_quantize_tiled(st, x, xq, xs, M, int(K)), "ffn (quantize)"));
        XPU_TRY(launched(gemm_act_skinny_xt(st, xq, up_wp, v, inner, xs, up_scale, int(M),
                                            int(inner), int(K), activation),
                         "ffn (up projection)"));
    } else {
        XPU_TRY(launched(convrot_quantize(st, x, xq, xs, M, int(K), 0), "ffn (quantize)"));
        XPU_TRY(launched(gemm_act(st, xq, K, up_w8, K, v, inner, xs, up_scale, int(M),
                                  int(inner), int(K), activation, up_wp),
                         "ffn (up projection)"));
    }
    return linear_run(st, v, down_w8, down_scale, bias, bias_bf16, out, M, K, inner, region,
                      down_wp);
}

// The checks shared by the one-call linear entry points.
int linear_check(const void* x, const int8_t* w8, const float* w_scale, const void* bias,
                 int32_t bias_bf16, const void* out, int64_t M, int64_t N, int64_t K,
                 const void* work, int64_t work_bytes) {
    XPU_TRY(check_rows(M, K));
    XPU_TRY(check_epilogue(M, N));
    XPU_TRY(check_gemm(M, N, K));
    XPU_NONNULL(x); XPU_NONNULL(w8); XPU_NONNULL(w_scale); XPU_NONNULL(out); XPU_NONNULL(work);
    XPU_ALIGNED_OPT(bias);
    if (bias_bf16 != 0 && bias_bf16 != 1) return fail(2, "bias_bf16 must be 0 or 1");
    if (work_bytes < int64_t(linear_work_bytes(M, N, K)))
        return fail(2, "work must hold xpuint8_linear_workspace_size(M, N, K) bytes");
    return 0;
}

int ffn_args_check(const void* x, const int8_t* up_w8, const float* up_scale,
                   const int8_t* down_w8, const float* down_scale, const void* bias,
                   int32_t bias_bf16, const void* out, int64_t M, int64_t inner, int64_t K,
                   int32_t activation, const void* work, int64_t work_bytes) {
    XPU_TRY(ffn_check(M, inner, K, activation));
    XPU_NONNULL(x); XPU_NONNULL(up_w8); XPU_NONNULL(up_scale); XPU_NONNULL(down_w8);
    XPU_NONNULL(down_scale); XPU_NONNULL(out); XPU_NONNULL(work);
    XPU_ALIGNED_OPT(bias);
    if (bias_bf16 != 0 && bias_bf16 != 1) return fail(2, "bias_bf16 must be 0 or 1");
    if (work_bytes < int64_t(ffn_work_bytes(M, inner, K)))
        return fail(2, "work must hold xpuint8_ffn_workspace_size(M, inner, K, activation) bytes");
    return 0;
}

int act_ok(int32_t act) {
    if (act < 1 || act > 5)
        return fail(6, "activation must be 1 (GELU-tanh), 2 (SwiGLU), 3 (situ), 4 (GEGLU) "
                       "or 5 (GELU-erf)");
    return 0;
}

}  // namespace

int device_cus() {
    int dev = 0;
    (void)hipGetDevice(&dev);
    const int n = (dev >= 0 && dev < kMaxDevices) ? g_cus[dev] : 0;
    return n > 0 ? n : 256;
}

const uint16_t* activation_tables() {
    int dev = 0;
    (void)hipGetDevice(&dev);
    return (dev >= 0 && dev < kMaxDevices) ? g_tab_dev[dev] : nullptr;
}

}  // namespace xpuint8

using namespace xpuint8;

extern "C" {

int xpuint8_init(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return fail(1, "no HIP device available");
    return ensure_device();
}

const char* xpuint8_device_name(void) {
    if (ensure_device() != 0) return nullptr;
    int dev = 0;
    (void)hipGetDevice(&dev);
    return g_device_name[dev].c_str();
}

int xpuint8_convrot_groupsize(void) { return 256; }

const char* xpuint8_last_error(void) { return t_error.c_str(); }

// ---------------------------------------------------------------- quantize
int xpuint8_convrot_quantize_stream(const void* stream, const void* x, int8_t* q, float* scale,
                                    int64_t M, int64_t K) {
    XPU_TRY(check_rows(M, K));
    XPU_NONNULL(x); XPU_NONNULL(q); XPU_NONNULL(scale);
    XPU_TRY(ensure_device());
    return launched(convrot_quantize(as_stream(stream), x, q, scale, M, int(K), 0),
                    "convrot_quantize");
}

int xpuint8_convrot_quantize_tiled_stream(const void* stream, const void* x, int8_t* q,
                                          float* scale, int64_t M, int64_t K) {
    XPU_TRY(check_rows(M, K));
    XPU_NONNULL(x); XPU_NONNULL(q); XPU_NONNULL(scale);
    if (!rowquant_can_tile(int(K))) return fail(2, "convrot_quantize_tiled: K too long");
    XPU_TRY(ensure_device());
    return launched(convrot_quantize_tiled(as_stream(stream), x, q, scale, M, int(K)),
                    "convrot_quantize_tiled");
}

int xpuint8_convrot_quantize(const void* x, int8_t* q, float* scale, int64_t M, int64_t K) {
    return finish(xpuint8_convrot_quantize_stream(nullptr, x, q, scale, M, K), "convrot_quantize");
}

int xpuint8_convrot_quantize_act_stream(const void* stream, const void* x, int8_t* q,
                                        float* scale, int64_t M, int64_t K, int32_t activation) {
    XPU_TRY(act_ok(activation));
    XPU_TRY(check_rows(M, K));
    XPU_NONNULL(x); XPU_NONNULL(q); XPU_NONNULL(scale);
    XPU_TRY(ensure_device());
    return launched(convrot_quantize(as_stream(stream), x, q, scale, M, int(K), activation),
                    "convrot_quantize_act");
}

int xpuint8_convrot_quantize_act(const void* x, int8_t* q, float* scale, int64_t M, int64_t K,
                                 int32_t activation) {
    return finish(xpuint8_convrot_quantize_act_stream(nullptr, x, q, scale, M, K, activation),
                  "convrot_quantize_act");
}

// ------------------------------------------------------------------ rotate
int xpuint8_convrot_rotate_bf16_stream(const void* stream, const void* x, void* xr, int64_t M,
                                       int64_t K) {
    XPU_TRY(check_rows(M, K));
    XPU_NONNULL(x); XPU_NONNULL(xr);
    XPU_TRY(ensure_device());
    return launched(rotate_bf16(as_stream(stream), x, xr, M, int(K)), "convrot_rotate_bf16");
}

int xpuint8_convrot_rotate_bf16(const void* x, void* xr, int64_t M, int64_t K) {
    return finish(xpuint8_convrot_rotate_bf16_stream(nullptr, x, xr, M, K), "convrot_rotate_bf16");
}

// ---------------------------------------------------------- dequant weight
int xpuint8_dequant_weight_stream(const void* stream, const void* w8, const float* w_scale,
                                  void* out, int64_t N, int64_t K) {
    if (N <= 0 || K <= 0) return fail(2, "N and K must be positive");
    XPU_TRY(check_rows(N, K));
    XPU_NONNULL(w8); XPU_NONNULL(w_scale); XPU_NONNULL(out);
    XPU_TRY(ensure_device());
    return launched(dequant_weight(as_stream(stream), static_cast<const int8_t*>(w8), w_scale, out,
                                   N, int(K)),
                    "dequant_weight");
}

int xpuint8_dequant_weight(const void* w8, const float* w_scale, void* out, int64_t N, int64_t K) {
    return finish(xpuint8_dequant_weight_stream(nullptr, w8, w_scale, out, N, K), "dequant_weight");
}

// ---------------------------------------------------------------- dequant
int xpuint8_dequant_epilogue_slice_stream(const void* stream, const int32_t* acc, void* out,
                                          const float* x_scale, const float* w_scale,
                                          const float* bias, int64_t M, int64_t N,
                                          int64_t acc_row_stride) {
    if (M <= 0 || N <= 0 || N % 16 != 0 || acc_row_stride < N)
        return fail(2, "M, N must be positive, N a multiple of 16, acc_row_stride >= N");
    XPU_TRY(check_epilogue(M, N));
    if (acc_row_stride % 4 != 0)
        return fail(2, "acc_row_stride must be a multiple of 4 (16-byte rows)");
    XPU_NONNULL(acc); XPU_NONNULL(out); XPU_NONNULL(x_scale); XPU_NONNULL(w_scale);
    XPU_ALIGNED_OPT(bias);
    XPU_TRY(ensure_device());
    return launched(dequant_epilogue(as_stream(stream), acc, acc_row_stride, out, x_scale, w_scale,
                                     bias, M, N),
                    "dequant_epilogue");
}

int xpuint8_dequant_epilogue_stream(const void* stream, const int32_t* acc, void* out,
                                    const float* x_scale, const float* w_scale, const float* bias,
                                    int64_t M, int64_t N) {
    XPU_TRY(check_epilogue(M, N));
    return xpuint8_dequant_epilogue_slice_stream(stream, acc, out, x_scale, w_scale, bias, M, N, N);
}

int xpuint8_dequant_epilogue(const int32_t* acc, void* out, const float* x_scale,
                             const float* w_scale, const float* bias, int64_t M, int64_t N) {
    return finish(xpuint8_dequant_epilogue_stream(nullptr, acc, out, x_scale, w_scale, bias, M, N),
                  "dequant_epilogue");
}

int xpuint8_dequant_epilogue_slice(const int32_t* acc, void* out, const float* x_scale,
                                   const float* w_scale, const float* bias, int64_t M, int64_t N,
                                   int64_t acc_row_stride) {
    return finish(xpuint8_dequant_epilogue_slice_stream(nullptr, acc, out, x_scale, w_scale, bias,
                                                        M, N, acc_row_stride),
                  "dequant_epilogue_slice");
}

// -------------------------------------------------- dequant+act+quantize
int xpuint8_dequant_act_quantize_stream(const void* stream, const void* acc, int8_t* q,
                                        float* scale, const float* x_scale, const float* w_scale,
                                        int64_t M, int64_t K, int32_t activation) {
    if (activation != 3 && activation != 4 && activation != 5)
        return fail(6, "dequant_act_quantize supports activation 3 (situ), 4 (GEGLU) or "
                       "5 (GELU-erf)");
    XPU_TRY(check_rows(M, K));
    XPU_NONNULL(acc); XPU_NONNULL(q); XPU_NONNULL(scale); XPU_NONNULL(x_scale);
    XPU_NONNULL(w_scale);
    XPU_TRY(ensure_device());
    const int64_t ld = act_paired(activation) ? 2 * K : K;
    return launched(dequant_act_quantize(as_stream(stream), static_cast<const int32_t*>(acc), ld,
                                         q, scale, x_scale, w_scale, M, int(K), activation),
                    "dequant_act_quantize");
}

int xpuint8_dequant_act_quantize(const void* acc, int8_t* q, float* scale, const float* x_scale,
                                 const float* w_scale, int64_t M, int64_t K, int32_t activation) {
    return finish(xpuint8_dequant_act_quantize_stream(nullptr, acc, q, scale, x_scale, w_scale, M,
                                                      K, activation),
                  "dequant_act_quantize");
}

// ------------------------------------------------------------------- GEMMs
int xpuint8_int8_gemm_stream(const void* stream, const int8_t* a, const int8_t* b, int32_t* c,
                             int64_t M, int64_t N, int64_t K) {
    XPU_TRY(check_gemm(M, N, K));
    XPU_NONNULL(a); XPU_NONNULL(b); XPU_NONNULL(c);
    XPU_TRY(ensure_device());
    return launched(gemm_i32(as_stream(stream), a, K, b, K, c, N, int(M), int(N), int(K)),
                    "int8_gemm");
}

int xpuint8_int8_gemm_nn_stream(const void* stream, const int8_t* a, const int8_t* b, int32_t* c,
                                int64_t M, int64_t N, int64_t K, int8_t* work) {
    XPU_TRY(check_gemm(M, N, K));
    XPU_NONNULL(a); XPU_NONNULL(b); XPU_NONNULL(c); XPU_NONNULL(work);
    XPU_TRY(ensure_device());
    hipStream_t st = as_stream(stream);
    XPU_TRY(launched(transpose_i8(st, b, work, K, N), "int8_gemm_nn (transpose)"));
    return launched(gemm_i32(st, a, K, work, K, c, N, int(M), int(N), int(K)), "int8_gemm_nn");
}

int xpuint8_linear_gemm_stream(const void* stream, const int8_t* xq, const float* x_scale,
                               const int8_t* w8, const float* w_scale, const void* bias,
                               int32_t bias_bf16, void* out, int64_t M, int64_t N, int64_t K) {
    XPU_TRY(check_epilogue(M, N));
    XPU_TRY(check_gemm(M, N, K));
    XPU_NONNULL(xq); XPU_NONNULL(x_scale); XPU_NONNULL(w8); XPU_NONNULL(w_scale);
    XPU_NONNULL(out);
    XPU_ALIGNED_OPT(bias);
    if (bias_bf16 != 0 && bias_bf16 != 1) return fail(2, "bias_bf16 must be 0 or 1");
    XPU_TRY(ensure_device());
    const float* b32 = bias_bf16 ? nullptr : static_cast<const float*>(bias);
    const uint16_t* b16 = bias_bf16 ? static_cast<const uint16_t*>(bias) : nullptr;
    return launched(gemm_dequant(as_stream(stream), xq, K, w8, K, out, N, x_scale, w_scale, b32,
                                 b16, int(M), int(N), int(K)),
                    "linear_gemm");
}

int xpuint8_linear_gemm_tiled_stream(const void* stream, const int8_t* xq, const float* x_scale,
                                     const int8_t* w8, const float* w_scale, const void* bias,
                                     int32_t bias_bf16, void* out, int64_t M, int64_t N,
                                     int64_t K) {
    XPU_TRY(check_rows(M, K));
    XPU_TRY(check_epilogue(M, N));
    XPU_TRY(check_gemm(M, N, K));
    XPU_NONNULL(xq); XPU_NONNULL(x_scale); XPU_NONNULL(w8); XPU_NONNULL(w_scale);
    XPU_NONNULL(out);
    XPU_ALIGNED_OPT(bias);
    if (bias_bf16 != 0 && bias_bf16 != 1) return fail(2, "bias_bf16 must be 0 or 1");
    XPU_TRY(ensure_device());
    const float* b32 = bias_bf16 ? nullptr : static_cast<const float*>(bias);
    const uint16_t* b16 = bias_bf16 ? static_cast<const uint16_t*>(bias) : nullptr;
    hipStream_t st = as_stream(stream);
    if (pp_applies(int(M), int(N), int(K), false))
        return launched(gemm_dequant_pp_xt(st, xq, w8, K, out, N, x_scale, w_scale, b32, b16,
                                           int(M), int(N), int(K)),
                        "linear_gemm_tiled");
    if (splitk_applies(int(M), int(N), int(K)) && gemm_slices(int(M), int(N), int(K)) == 0)
        return launched(gemm_dequant_xt(st, xq, w8, K, out, N, x_scale, w_scale, b32, b16,
                                        int(M), int(N), int(K)),
                        "linear_gemm_tiled");
    return fail(2, "linear_gemm_tiled: this shape does not read x in the block layout");
}

int64_t xpuint8_linear_workspace_size(int64_t M, int64_t N, int64_t K) {
    if (check_rows(M, K) != 0 || check_epilogue(M, N) != 0 || check_gemm(M, N, K) != 0) return -1;
    return int64_t(linear_work_bytes(M, N, K));
}

int xpuint8_linear_stream(const void* stream, const void* x, const int8_t* w8,
                          const float* w_scale, const void* bias, int32_t bias_bf16, void* out,
                          int64_t M, int64_t N, int64_t K, void* work, int64_t work_bytes) {
    XPU_TRY(linear_check(x, w8, w_scale, bias, bias_bf16, out, M, N, K, work, work_bytes));
    XPU_TRY(ensure_device());
    return linear_run(as_stream(stream), x, w8, w_scale, bias, bias_bf16, out, M, N, K, work);
}

int64_t xpuint8_packed_weight_bytes(int64_t N, int64_t K) {
    if (N <= 0 || K <= 0 || N % 16 != 0 || K % 16 != 0 || N > kMaxDim || K > kMaxK) return -1;
    return tiled_bytes(N, K);
}

int xpuint8_pack_weight_stream(const void* stream, const int8_t* w8, int8_t* packed, int64_t N,
                               int64_t K) {
    if (N <= 0 || K <= 0 || N % 16 != 0 || K % 16 != 0)
        return fail(2, "pack_weight: N and K must be positive multiples of 16");
    if (N > kMaxDim || K > kMaxK) return fail(4, "pack_weight: K must be <= 131072 and N < 2^31");
    XPU_NONNULL(w8); XPU_NONNULL(packed);
    XPU_TRY(ensure_device());
    return launched(pack_weight(as_stream(stream), w8, packed, N, int(K)), "pack_weight");
}

int xpuint8_linear_packed_stream(const void* stream, const void* x, const int8_t* w8,
                                 const int8_t* w8_packed, const float* w_scale, const void* bias,
                                 int32_t bias_bf16, void* out, int64_t M, int64_t N, int64_t K,
                                 void* work, int64_t work_bytes) {
    XPU_TRY(linear_check(x, w8, w_scale, bias, bias_bf16, out, M, N, K, work, work_bytes));
    XPU_ALIGNED_OPT(w8_packed);
    XPU_TRY(ensure_device());
    return linear_run(as_stream(stream), x, w8, w_scale, bias, bias_bf16, out, M, N, K, work,
                      w8_packed);
}

int xpuint8_linear_residual_packed_stream(const void* stream, const void* x, const int8_t* w8,
                                          const int8_t* w8_packed, const float* w_scale,
                                          const void* bias, int32_t bias_bf16,
                                          const void* residual, const void* residual_scale,
                                          void* out, int64_t M, int64_t N, int64_t K, void* work,
                                          int64_t work_bytes) {
    XPU_TRY(linear_check(x, w8, w_scale, bias, bias_bf16, out, M, N, K, work, work_bytes));
    XPU_NONNULL(residual); XPU_NONNULL(residual_scale);
    XPU_ALIGNED_OPT(w8_packed);
    XPU_TRY(ensure_device());
    hipStream_t st = as_stream(stream);
    int8_t* q = static_cast<int8_t*>(work);
    float* xs = reinterpret_cast<float*>(static_cast<char*>(work) + linear_work_q_bytes(M, K));
    const float* b32 = bias_bf16 ? nullptr : static_cast<const float*>(bias);
    const uint16_t* b16 = bias_bf16 ? static_cast<const uint16_t*>(bias) : nullptr;
    // the kernels that read x in the MFMA block layout (and the packed weight)
    if (rowquant_can_tile(int(K)) &&
        (pp_applies(int(M), int(N), int(K), false) ||
         (splitk_applies(int(M), int(N), int(K)) && gemm_slices(int(M), int(N), int(K)) == 0))) {
        XPU_TRY(launched(convrot_quantize_tiled(st, x, q, xs, M, int(K)),
                         "linear_residual (quantize)"));
        return launched(gemm_dequant_residual_xt(st, q, w8_packed ? w8_packed : w8, K, out, N, xs,
                                                 w_scale, b32, b16, residual, N, residual_scale,
                                                 int(M), int(N), int(K), w8_packed != nullptr),
                        "linear_residual (gemm)");
    }
    XPU_TRY(launched(convrot_quantize(st, x, q, xs, M, int(K), 0), "linear_residual (quantize)"));
    return launched(gemm_dequant_residual(st, q, K, w8, K, out, N, xs, w_scale, b32, b16, residual,
                                          N, residual_scale, int(M), int(N), int(K)),
                    "linear_residual (gemm)");
}

int xpuint8_linear_acc_packed_stream(const void* stream, const void* x, const int8_t* w8,
                                     const int8_t* w8_packed, int32_t* acc, float* x_scale,
                                     int64_t M, int64_t N, int64_t K, void* work,
                                     int64_t work_bytes) {
    XPU_TRY(check_rows(M, K));
    XPU_TRY(check_gemm(M, N, K));
    XPU_NONNULL(x); XPU_NONNULL(w8); XPU_NONNULL(acc); XPU_NONNULL(x_scale); XPU_NONNULL(work);
    XPU_ALIGNED_OPT(w8_packed);
    if (work_bytes < int64_t(linear_work_q_bytes(M, K)))
        return fail(2, "work must hold xpuint8_linear_workspace_size(M, N, K) bytes");
    XPU_TRY(ensure_device());
    hipStream_t st = as_stream(stream);
    int8_t* q = static_cast<int8_t*>(work);
    if (rowquant_can_tile(int(K)) && pp_applies(int(M), int(N), int(K), false)) {
        XPU_TRY(launched(convrot_quantize_tiled(st, x, q, x_scale, M, int(K)),
                         "linear_acc (quantize)"));
        return launched(gemm_i32_pp_xt(st, q, w8_packed ? w8_packed : w8, K, acc, N, int(M),
                                       int(N), int(K), w8_packed != nullptr),
                        "linear_acc (gemm)");
    }
    XPU_TRY(launched(convrot_quantize(st, x, q, x_scale, M, int(K), 0), "linear_acc (quantize)"));
    return launched(gemm_i32(st, q, K, w8, K, acc, N, int(M), int(N), int(K)), "linear_acc (gemm)");
}

int xpuint8_linear_gemm_packed_stream(const void* stream, const int8_t* xq, const float* x_scale,
                                      const int8_t* w8_packed, const float* w_scale,
                                      const void* bias, int32_t bias_bf16, void* out, int64_t M,
                                      int64_t N, int64_t K) {
    XPU_TRY(check_rows(M, K));
    XPU_TRY(check_epilogue(M, N));
    XPU_TRY(check_gemm(M, N, K));
    XPU_NONNULL(xq); XPU_NONNULL(x_scale); XPU_NONNULL(w8_packed); XPU_NONNULL(w_scale);
    XPU_NONNULL(out);
    XPU_ALIGNED_OPT(bias);
    if (bias_bf16 != 0 && bias_bf16 != 1) return fail(2, "bias_bf16 must be 0 or 1");
    XPU_TRY(ensure_device());
    const float* b32 = bias_bf16 ? nullptr : static_cast<const float*>(bias);
    const uint16_t* b16 = bias_bf16 ? static_cast<const uint16_t*>(bias) : nullptr;
    hipStream_t st = as_stream(stream);
    if (pp_applies(int(M), int(N), int(K), false))
        return launched(gemm_dequant_pp_xt(st, xq, w8_packed, 0, out, N, x_scale, w_scale, b32,
                                           b16, int(M), int(N), int(K), true),
                        "linear_gemm_packed");
    if (splitk_applies(int(M), int(N), int(K)) && gemm_slices(int(M), int(N), int(K)) == 0)
        return launched(gemm_dequant_xt(st, xq, w8_packed, 0, out, N, x_scale, w_scale, b32, b16,
                                        int(M), int(N), int(K), true),
                        "linear_gemm_packed");
    if (skinny_applies(int(M), false) && gemm_slices(int(M), int(N), int(K)) == 0)
        return launched(gemm_dequant_skinny_xt(st, xq, w8_packed, out, N, x_scale, w_scale, b32,
                                               b16, int(M), int(N), int(K)),
                        "linear_gemm_packed");
    return fail(2, "linear_gemm_packed: this shape does not read the block layouts");
}

int64_t xpuint8_ffn_workspace_size(int64_t M, int64_t inner, int64_t K, int32_t activation) {
    if (ffn_check(M, inner, K, activation) != 0) return -1;
    return int64_t(ffn_work_bytes(M, inner, K));
}

int xpuint8_ffn_stream(const void* stream, const void* x, const int8_t* up_w8,
                       const float* up_scale, const int8_t* down_w8, const float* down_scale,
                       const void* bias, int32_t bias_bf16, void* out, int64_t M, int64_t inner,
                       int64_t K, int32_t activation, void* work, int64_t work_bytes) {
    XPU_TRY(ffn_args_check(x, up_w8, up_scale, down_w8, down_scale, bias, bias_bf16, out, M,
                           inner, K, activation, work, work_bytes));
    XPU_TRY(ensure_device());
    return ffn_run(as_stream(stream), x, up_w8, nullptr, up_scale, down_w8, nullptr, down_scale,
                   bias, bias_bf16, out, M, inner, K, activation, work);
}

int xpuint8_ffn_packed_stream(const void* stream, const void* x, const int8_t* up_w8,
                              const int8_t* up_packed, const float* up_scale,
                              const int8_t* down_w8, const int8_t* down_packed,
                              const float* down_scale, const void* bias, int32_t bias_bf16,
                              void* out, int64_t M, int64_t inner, int64_t K, int32_t activation,
                              void* work, int64_t work_bytes) {
    XPU_TRY(ffn_args_check(x, up_w8, up_scale, down_w8, down_scale, bias, bias_bf16, out, M,
                           inner, K, activation, work, work_bytes));
    XPU_ALIGNED_OPT(up_packed);
    XPU_ALIGNED_OPT(down_packed);
    XPU_TRY(ensure_device());
    return ffn_run(as_stream(stream), x, up_w8, up_packed, up_scale, down_w8, down_packed,
                   down_scale, bias, bias_bf16, out, M, inner, K, activation, work);
}

int xpuint8_linear_gemm_residual_stream(const void* stream, const int8_t* xq,
                                        const float* x_scale, const int8_t* w8,
                                        const float* w_scale, const void* bias, int32_t bias_bf16,
                                        const void* residual, const void* residual_scale,
                                        void* out, int64_t M, int64_t N, int64_t K) {
    XPU_TRY(check_epilogue(M, N));
    XPU_TRY(check_gemm(M, N, K));
    XPU_NONNULL(xq); XPU_NONNULL(x_scale); XPU_NONNULL(w8); XPU_NONNULL(w_scale);
    XPU_NONNULL(residual); XPU_NONNULL(residual_scale); XPU_NONNULL(out);
    XPU_ALIGNED_OPT(bias);
    if (bias_bf16 != 0 && bias_bf16 != 1) return fail(2, "bias_bf16 must be 0 or 1");
    XPU_TRY(ensure_device());
    const float* b32 = bias_bf16 ? nullptr : static_cast<const float*>(bias);
    const uint16_t* b16 = bias_bf16 ? static_cast<const uint16_t*>(bias) : nullptr;
    return launched(gemm_dequant_residual(as_stream(stream), xq, K, w8, K, out, N, x_scale, w_scale,
                                          b32, b16, residual, N, residual_scale, int(M), int(N),
                                          int(K)),
                    "linear_gemm_residual");
}

int xpuint8_ffn_up_stream(const void* stream, const int8_t* xq, const float* x_scale,
                          const int8_t* w8, const float* w_scale, void* out, int64_t M, int64_t N,
                          int64_t K, int32_t activation) {
    if (activation != 3 && activation != 4 && activation != 5)
        return fail(6, "ffn_up supports activation 3 (situ), 4 (GEGLU) or 5 (GELU-erf)");
    const int64_t rows = act_paired(activation) ? 2 * N : N;   // weight rows
    XPU_TRY(check_epilogue(M, N));
    XPU_TRY(check_gemm(M, rows, K));
    XPU_NONNULL(xq); XPU_NONNULL(x_scale); XPU_NONNULL(w8); XPU_NONNULL(w_scale);
    XPU_NONNULL(out);
    XPU_TRY(ensure_device());
    return launched(gemm_act(as_stream(stream), xq, K, w8, K, out, N, x_scale, w_scale, int(M),
                             int(N), int(K), activation),
                    "ffn_up");
}

int xpuint8_dx_gemm_stream(const void* stream, const int8_t* q, const float* a, const int8_t* w8,
                           void* dx, int64_t M, int64_t N, int64_t K, int8_t* work) {
    // q [M,N] @ w8 [N,K] -> dx [M,K]; the contraction runs over N
    XPU_TRY(check_gemm(M, K, N));
    XPU_NONNULL(q); XPU_NONNULL(a); XPU_NONNULL(w8); XPU_NONNULL(dx); XPU_NONNULL(work);
    XPU_TRY(ensure_device());
    hipStream_t st = as_stream(stream);
    XPU_TRY(launched(transpose_i8(st, w8, work, N, K), "dx_gemm (transpose)"));
    return launched(gemm_dequant(st, q, N, work, N, dx, K, a, nullptr, nullptr, nullptr, int(M), int(K),
                                 int(N)),
                    "dx_gemm");
}

int64_t xpuint8_column_sum_workspace_size(int64_t M, int64_t N) {
    if (check_epilogue(M, N) != 0) return -1;
    return colsum_work_bytes(M, N);
}

int xpuint8_column_sum_stream(const void* stream, const void* x, void* out, int64_t M, int64_t N,
                              void* work, int64_t work_bytes) {
    XPU_TRY(check_epilogue(M, N));
    XPU_NONNULL(x); XPU_NONNULL(out); XPU_NONNULL(work);
    if (work_bytes < colsum_work_bytes(M, N))
        return fail(2, "work must hold xpuint8_column_sum_workspace_size(M, N) bytes");
    XPU_TRY(ensure_device());
    return launched(column_sum_bf16(as_stream(stream), x, out, M, int(N), static_cast<float*>(work)),
                    "column_sum");
}

int64_t xpuint8_linear_dx_int8_workspace_size(int64_t M, int64_t N, int64_t K) {
    if (check_dx(M, N, K) != 0) return -1;
    return int64_t(dx_work_layout(M, N, K).total);
}

int xpuint8_linear_dx_int8_stream(const void* stream, const void* dy, const float* w_scale,
                                  const int8_t* w8, void* dx, int64_t M, int64_t N, int64_t K,
                                  void* work, int64_t work_bytes) {
    XPU_TRY(check_dx(M, N, K));
    XPU_NONNULL(dy); XPU_NONNULL(w_scale); XPU_NONNULL(w8); XPU_NONNULL(dx); XPU_NONNULL(work);
    if (work_bytes < int64_t(dx_work_layout(M, N, K).total))
        return fail(2, "work must hold xpuint8_linear_dx_int8_workspace_size(M, N, K) bytes");
    XPU_TRY(ensure_device());
    return dx_chain(as_stream(stream), dy, w_scale, w8, dx, M, N, K, static_cast<char*>(work));
}

int64_t xpuint8_packed_weight_nn_bytes(int64_t N, int64_t K) {
    if (N <= 0 || K <= 0 || N % 16 != 0 || K % 32 != 0 || N > kMaxK || K > kMaxDim) return -1;
    return packed_nn_bytes(N, K);
}

int xpuint8_pack_weight_nn_stream(const void* stream, const int8_t* w8, int8_t* packed, int64_t N,
                                  int64_t K) {
    if (N <= 0 || K <= 0 || N % 16 != 0 || K % 32 != 0)
        return fail(2, "pack_weight_nn: N must be a positive multiple of 16 and K of 32");
    if (N > kMaxK || K > kMaxDim) return fail(4, "pack_weight_nn: N must be <= 131072 and K < 2^31");
    XPU_NONNULL(w8); XPU_NONNULL(packed);
    XPU_TRY(ensure_device());
    return launched(pack_weight_nn(as_stream(stream), w8, packed, N, int(K)), "pack_weight_nn");
}

int xpuint8_linear_dx_int8_packed_stream(const void* stream, const void* dy, const float* w_scale,
                                         const int8_t* w8, const int8_t* w8_packed_nn, void* dx,
                                         int64_t M, int64_t N, int64_t K, void* work,
                                         int64_t work_bytes) {
    XPU_TRY(check_dx(M, N, K));
    XPU_NONNULL(dy); XPU_NONNULL(w_scale); XPU_NONNULL(w8); XPU_NONNULL(dx); XPU_NONNULL(work);
    XPU_ALIGNED_OPT(w8_packed_nn);
    if (work_bytes < int64_t(dx_work_layout(M, N, K).total))
        return fail(2, "work must hold xpuint8_linear_dx_int8_workspace_size(M, N, K) bytes");
    XPU_TRY(ensure_device());
    return dx_chain(as_stream(stream), dy, w_scale, w8, dx, M, N, K, static_cast<char*>(work),
                    w8_packed_nn);
}

int64_t xpuint8_linear_backward_int8_workspace_size(int64_t M, int64_t N, int64_t K) {
    if (check_dx(M, N, K) != 0) return -1;
    const size_t dx = (dx_work_layout(M, N, K).total + 255) & ~size_t(255);
    return int64_t(dx + size_t(colsum_work_bytes(M, N)));
}

int xpuint8_linear_backward_int8_stream(const void* stream, const void* dy, const float* w_scale,
                                        const int8_t* w8, const int8_t* w8_packed_nn, void* dx,
                                        void* dbias, int32_t dbias_fp32, int64_t M, int64_t N,
                                        int64_t K, void* work, int64_t work_bytes) {
    XPU_TRY(check_dx(M, N, K));
    XPU_NONNULL(dy); XPU_NONNULL(w_scale); XPU_NONNULL(w8); XPU_NONNULL(dx); XPU_NONNULL(work);
    XPU_ALIGNED_OPT(w8_packed_nn);
    XPU_ALIGNED_OPT(dbias);
    if (dbias_fp32 != 0 && dbias_fp32 != 1) return fail(2, "dbias_fp32 must be 0 or 1");
    const size_t dxw = (dx_work_layout(M, N, K).total + 255) & ~size_t(255);
    if (work_bytes < int64_t(dxw + size_t(colsum_work_bytes(M, N))))
        return fail(2, "work must hold xpuint8_linear_backward_int8_workspace_size(M, N, K) bytes");
    XPU_TRY(ensure_device());
    hipStream_t st = as_stream(stream);
    char* w = static_cast<char*>(work);
    if (dbias)
        XPU_TRY(launched(column_sum_bf16(st, dy, dbias, M, int(N), reinterpret_cast<float*>(w + dxw),
                                         dbias_fp32 != 0),
                         "linear_backward_int8 (column sum)"));
    return dx_chain(st, dy, w_scale, w8, dx, M, N, K, w, w8_packed_nn);
}

int xpuint8_linear_dx_int8_noalloc_stream(const void* stream, const void* dy,
                                          const float* w_scale, const int8_t* w8, void* dx,
                                          int64_t M, int64_t N, int64_t K) {
    XPU_TRY(check_dx(M, N, K));
    XPU_NONNULL(dy); XPU_NONNULL(w_scale); XPU_NONNULL(w8); XPU_NONNULL(dx);
    const size_t need = dx_work_layout(M, N, K).total;
    if (need > kScratchBytes)
        return fail(4, "linear_dx_int8_noalloc: this shape needs " + std::to_string(need) +
                           " bytes of workspace, above the library's fixed 64 MiB "
                           "(67108864 bytes); use xpuint8_linear_dx_int8_stream with a "
                           "caller workspace");
    XPU_TRY(ensure_device());
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || g_scratch[dev] == nullptr)
        return fail(5, "linear_dx_int8_noalloc: no scratch address for the current device");
    return dx_chain(as_stream(stream), dy, w_scale, w8, dx, M, N, K, g_scratch[dev]);
}

int xpuint8_linear_dw_stream(const void* stream, const void* dy, const void* x, void* dw,
                             int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || N <= 0 || K <= 0) return fail(2, "M, N and K must be positive");
    if (N % 16 != 0 || K % 16 != 0) return fail(2, "N and K must be multiples of 16");
    if (M > kMaxDim || N > kMaxDim || K > kMaxDim) return fail(4, "M, N and K must be < 2^31");
    XPU_NONNULL(dy); XPU_NONNULL(x); XPU_NONNULL(dw);
    XPU_TRY(ensure_device());
    return launched(gemm_bf16_tn(as_stream(stream), dy, N, x, K, dw, K, int(M), int(N), int(K)),
                    "linear_dw");
}

static int check_linear_dx(int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || N <= 0 || K <= 0) return fail(2, "M, N and K must be positive");
    if (N % 16 != 0 || K % 16 != 0) return fail(2, "N and K must be multiples of 16");
    if (M > kMaxDim || N > kMaxDim || K > kMaxDim) return fail(4, "M, N and K must be < 2^31");
    return 0;
}

int64_t xpuint8_linear_dx_workspace_size(int64_t M, int64_t N, int64_t K) {
    if (check_linear_dx(M, N, K) != 0) return -1;
    const int nsl = bf16_nn_slices(int(M), int(N), int(K));
    return nsl > 0 ? int64_t(nsl) * M * K * 4 : 0;
}

int xpuint8_linear_dx_stream(const void* stream, const void* dy, const void* w, void* dx,
                             int64_t M, int64_t N, int64_t K, void* work, int64_t work_bytes) {
    XPU_TRY(check_linear_dx(M, N, K));
    XPU_NONNULL(dy); XPU_NONNULL(w); XPU_NONNULL(dx); XPU_ALIGNED_OPT(work);
    XPU_TRY(ensure_device());
    // a small batch with a workspace: the contraction split across blocks
    const int nsl = bf16_nn_slices(int(M), int(N), int(K));
    if (nsl > 0 && work != nullptr && work_bytes >= int64_t(nsl) * M * K * 4)
        return launched(gemm_bf16_nn_slices(as_stream(stream), dy, N, w, K, dx, K, int(M), int(N),
                                            int(K), static_cast<float*>(work), nsl),
                        "linear_dx");
    return launched(gemm_bf16_nn(as_stream(stream), dy, N, w, K, dx, K, int(M), int(N), int(K)),
                    "linear_dx");
}

// The workspace of xpuint8_linear_backward_dense_stream: the dequantized
// weight bf16 [N, K], the column sums' partials, and (for a contraction split
// across blocks) the bf16 GEMM's fp32 partials, each on a 256-byte boundary.
struct DenseBwdWork {
    size_t wd, colsum, part, total;
};
static DenseBwdWork dense_bwd_layout(int64_t M, int64_t N, int64_t K) {
    auto up = [](int64_t b) { return (size_t(b) + 255) & ~size_t(255); };
    DenseBwdWork w;
    w.wd = 0;
    w.colsum = up(2 * N * K);
    w.part = w.colsum + up(colsum_work_bytes(M, N));
    const int nsl = bf16_nn_slices(int(M), int(N), int(K));
    w.total = w.part + (nsl > 0 ? size_t(nsl) * size_t(M) * size_t(K) * 4 : 0);
    return w;
}

int64_t xpuint8_linear_backward_dense_workspace_size(int64_t M, int64_t N, int64_t K) {
    if (check_rows(N, K) != 0 || check_linear_dx(M, N, K) != 0) return -1;
    return int64_t(dense_bwd_layout(M, N, K).total);
}

int xpuint8_linear_backward_dense_stream(const void* stream, const void* dy, const int8_t* w8,
                                         const float* w_scale, void* dx, void* dbias,
                                         int32_t dbias_fp32, int64_t M, int64_t N, int64_t K,
                                         void* work, int64_t work_bytes) {
    XPU_TRY(check_rows(N, K));                  // the weight's rotation: K % 256
    XPU_TRY(check_linear_dx(M, N, K));
    XPU_NONNULL(dy); XPU_NONNULL(w8); XPU_NONNULL(w_scale); XPU_NONNULL(dx); XPU_NONNULL(work);
    XPU_ALIGNED_OPT(dbias);
    if (dbias_fp32 != 0 && dbias_fp32 != 1) return fail(2, "dbias_fp32 must be 0 or 1");
    const DenseBwdWork L = dense_bwd_layout(M, N, K);
    if (work_bytes < int64_t(L.total))
        return fail(2, "work must hold xpuint8_linear_backward_dense_workspace_size(M, N, K) bytes");
    XPU_TRY(ensure_device());
    hipStream_t st = as_stream(stream);
    char* w = static_cast<char*>(work);
    if (dbias)
        XPU_TRY(launched(column_sum_bf16(st, dy, dbias, M, int(N),
                                         reinterpret_cast<float*>(w + L.colsum), dbias_fp32 != 0),
                         "linear_backward_dense (column sum)"));
    void* wd = w + L.wd;
    XPU_TRY(launched(dequant_weight(st, w8, w_scale, wd, N, int(K)),
                     "linear_backward_dense (dequant_weight)"));
    if (const int nsl = bf16_nn_slices(int(M), int(N), int(K)))
        return launched(gemm_bf16_nn_slices(st, dy, N, wd, K, dx, K, int(M), int(N), int(K),
                                            reinterpret_cast<float*>(w + L.part), nsl),
                        "linear_backward_dense (gemm)");
    return launched(gemm_bf16_nn(st, dy, N, wd, K, dx, K, int(M), int(N), int(K)),
                    "linear_backward_dense (gemm)");
}

// ------------------------------------------------------------- rms + rope
int xpuint8_rms_rope_dequant_stream(const void* stream, const int32_t* acc, int64_t acc_stride_b,
                                    int64_t acc_stride_s, int64_t acc_stride_h,
                                    const float* x_scale, int64_t xs_stride_b,
                                    int64_t xs_stride_s, const float* w_scale, const float* freqs,
                                    int64_t f_stride_b, int64_t f_stride_s, int64_t f_stride_dim,
                                    int64_t f_stride_rot, int64_t f_stride_pair, int64_t f_batch,
                                    int64_t f_seq, const float* scale, void* out, int64_t B,
                                    int64_t S, int64_t H, int64_t D, float epsilon,
                                    int32_t split_half) {
    if (B <= 0 || S <= 0 || H <= 0) return fail(2, "B, S and H must be positive");
    if (D < 2 || D > 256 || D % 2 != 0) return fail(2, "D must be even and in [2, 256]");
    if (B * S > kMaxDim || H * D > kMaxDim || B * S * H > kMaxDim)
        return fail(4, "B*S*H rows must be < 2^31");
    if (f_batch != 1 && f_batch != B) return fail(2, "freqs_cis batch must be 1 or B");
    if (f_seq != 1 && f_seq != S) return fail(2, "freqs_cis sequence length must be 1 or S");
    if (!(epsilon >= 0.0f)) return fail(2, "epsilon must be >= 0");
    XPU_NONNULL(acc); XPU_NONNULL(x_scale); XPU_NONNULL(w_scale); XPU_NONNULL(freqs);
    XPU_NONNULL(scale); XPU_NONNULL(out);
    XPU_TRY(ensure_device());
    return launched(rms_rope_dequant(as_stream(stream), acc, acc_stride_b, acc_stride_s,
                                     acc_stride_h, x_scale, xs_stride_b, xs_stride_s, w_scale,
                                     freqs, f_stride_b, f_stride_s, f_stride_dim, f_stride_rot,
                                     f_stride_pair, f_batch, f_seq, scale, out, B, S, int(H),
                                     int(D), epsilon, split_half != 0),
                    "rms_rope_dequant");
}

// ------------------------------------------------------ prepare / row quant
int xpuint8_prepare_weight_stream(const void* stream, const void* w, int8_t* q, float* scale,
                                  int64_t N, int64_t K) {
    XPU_TRY(check_rows(N, K));
    XPU_NONNULL(w); XPU_NONNULL(q); XPU_NONNULL(scale);
    XPU_TRY(ensure_device());
    return launched(prepare_weight(as_stream(stream), w, q, scale, N, int(K)), "prepare_weight");
}

int xpuint8_quantize_row_stream(const void* stream, const void* x, const float* col_scale,
                                int8_t* q, float* scale, int64_t M, int64_t N) {
    XPU_TRY(check_epilogue(M, N));
    if (N > kMaxK) return fail(4, "rows longer than 131072 are not supported");
    XPU_NONNULL(x); XPU_NONNULL(q); XPU_NONNULL(scale);
    XPU_ALIGNED_OPT(col_scale);
    XPU_TRY(ensure_device());
    return launched(quantize_row(as_stream(stream), x, col_scale, q, scale, M, int(N)),
                    "quantize_row");
}

int xpuint8_activation_table(int32_t id, uint16_t* out) {
    if (id < 0 || id >= kNumTables) return fail(6, "table id must be 0..6");
    XPU_NONNULL(out);
    std::memcpy(out, host_activation_tables() + size_t(id) * kTabSize, sizeof(uint16_t) * kTabSize);
    return 0;
}

}  // extern "C"
