// The weight gradient of a linear on CDNA4 bf16 MFMA (v_mfma_f32_16x16x32_bf16):
//
//   dw[n, k] = sum_m dy[m, n] * x[m, k]      dy bf16 [R, N], x bf16 [R, K]
//
// fp32 accumulation, one bf16 rounding (RNE) at the store: the reference's
// linear_dw, dy^T @ x in bf16 (python/xpu_kernels/int8/ops.py:207-238).
//
// Both operands are contracted along their *rows*, while an MFMA operand
// fragment wants 8 consecutive reduction values per lane.  The tiles therefore
// go into LDS exactly as they lie in memory (row-major, direct global->LDS
// loads), and the fragments come out with gfx950's transposing LDS read
// ds_read_b64_tr_b16.  Within each group of 16 lanes, lane j supplies the
// address of 4 consecutive bf16 and lane i = 4a + b receives element b of the
// vectors supplied by lanes a, a+4, a+8, a+12.  So when lane j points at row
// j/4, columns 4(j%4)..+3 of a 4 x 16 block, lane i receives column i of the
// 4 rows -- a transposed 4 x 16 read.  Two such reads (rows +0..3 and +4..7)
// give lane l the 8 reduction values m = 8(l/16)..+7 of operand row l%16,
// the fragment layout of the 16x16x32 MFMA.
//
// D = A * B with A from x (D rows = k) and B from dy (D columns = n), so lane
// l of a 16x16 block holds D[4(l/16)+i][l%16]: four consecutive k of one dw
// row, stored as one 8-byte write.
#include "common.hpp"
#include "kernels.hpp"

namespace xpuint8 {
namespace {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef short v8s __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

// 16 zero bytes: the DMA source for reduction rows past R.
__device__ __attribute__((aligned(16))) int8_t g_zero_line[16];

constexpr int kStepRows = 32;                // reduction rows per MFMA step
constexpr int kRegion = kStepRows * 256;     // 32 rows x 128 bf16 columns = 8 KB

// A region row is 256 bytes = 16 chunks of 16 bytes, i.e. one pass over the
// 64 four-byte LDS banks; chunk c of row r sits at position c ^ swz(r).  A
// transposing read touches 16 rows, 8g + 4h + q (g, q = 0..3), and two
// adjacent chunks (8 banks) in each: swz takes 8 distinct even values over
// (q, g & 1), so the rows' chunk pairs cover all 64 banks twice -- the
// minimum two cycles for the read's 512 bytes.
__device__ __forceinline__ int swz(int r) { return 2 * ((r & 3) | (((r >> 3) & 1) << 2)); }

__device__ __forceinline__ void dma16(const int8_t* gsrc, int8_t* ldst) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_global_load_lds(gsrc, (__attribute__((address_space(3))) void*)ldst, 16, 0,
                                     0);
#endif
}

// The transposing read, issued as inline assembly.  Written with the builtin,
// the compiler must assume the read may see LDS that a pending direct-to-LDS
// load writes, and waits for *all* outstanding loads before it -- including
// the stage just issued, which removes the pipelining.  Here the ring's own
// vmcnt waits (before each barrier) order the loads; the reads' completion is
// awaited by lds_wait() below before any fragment is used.
__device__ __forceinline__ uint32_t lds_addr(const int8_t* p) {
    return static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const int8_t*)p));
}
__device__ __forceinline__ v4s tr_read(uint32_t addr) {
    v4s r;
    asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r) : "v"(addr));
    return r;
}

__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v2f{lo, hi}, v2bf));
}

// s_waitcnt immediate waiting for vmcnt <= n only.
__host__ __device__ constexpr int vmcnt_imm(int n) {
    return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8);
}

// One 128 (k) x 128 (n) tile per block of 4 waves (2 x 2, 64 x 64 each); the
// reduction runs in steps of 32 rows through a ring of STAGES LDS stages (x
// region, then dy region), filled STAGES-1 steps ahead.
template <int STAGES>
__global__ __launch_bounds__(256, 2) void gemm_bf16_tn_kernel(
    const uint16_t* __restrict__ X, int64_t ldx, const uint16_t* __restrict__ Y, int64_t ldy,
    uint16_t* __restrict__ out, int64_t ldo, int R, int K, int N, int tiles_k, int tiles_n) {
    constexpr int BKD = 128, BND = 128;                 // D rows (k), D columns (n) per tile
    constexpr int TM = 4, TN = 4;                       // 16x16 blocks per wave
    constexpr int STAGE = 2 * kRegion;
    __shared__ __attribute__((aligned(1024))) int8_t smem[STAGES * STAGE];

    const int tiles = tiles_k * tiles_n;
    int t = blockIdx.x;
    if (tiles % 8 == 0) t = (t % 8) * (tiles / 8) + t / 8;   // each XCD a contiguous range
    const int k0 = (t % tiles_k) * BKD, n0 = (t / tiles_k) * BND;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave >> 1, wn = wave & 1;

    // DMA: a stage is 16 blocks of 1 KB (4 rows x 256 bytes): blocks 0..7 the
    // x region, 8..15 the dy region; wave w brings blocks w, w+4, w+8, w+12.
    // Lane l fills row r = 4*(b%8) + l/16, position l%16, i.e. source chunk
    // (l%16) ^ swz(r).  Columns past K / N repeat a valid chunk (their results
    // are not stored); rows past R read zeros.
    const int8_t* src[4];
    int srow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int b = wave + 4 * i;
        srow[i] = 4 * (b & 7) + (lane >> 4);
        const int dchunk = (lane & 15) ^ swz(srow[i]);
        if (i < 2) {
            const int col = min(k0 + dchunk * 8, K - 8);
            src[i] = reinterpret_cast<const int8_t*>(X + col);
        } else {
            const int col = min(n0 + dchunk * 8, N - 8);
            src[i] = reinterpret_cast<const int8_t*>(Y + col);
        }
    }
    auto issue = [&](int buf, int step) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = step * kStepRows + srow[i];
            const int64_t ld = i < 2 ? ldx : ldy;
            const int8_t* p = row < R ? src[i] + int64_t(row) * ld * 2 : g_zero_line;
            dma16(p, smem + buf * STAGE + (wave + 4 * i) * 1024);
        }
    };

    // transposing-read offsets: lane l (group g, index j) reads row
    // 8g + 4h + j/4 (h = 0, 1), 8 bytes at column 16*blk + 4*(j%4)
    const int g = lane >> 4, j = lane & 15;
    uint32_t roff[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) roff[h] = (8 * g + 4 * h + (j >> 2)) * 256 + 8 * (j & 1);
    const int cpair = (j & 3) >> 1;             // chunk within the block's two
    const int rs = swz(8 * g + (j >> 2));       // swz of the rows read (h does not change it)
    const uint32_t sbase = lds_addr(smem);
    // fragment halves: lo = reduction rows +0..3, hi = +4..7 of the lane's 8
    auto frag_read = [&](uint32_t region, int blk, v4s& lo, v4s& hi) {
        const uint32_t pos = ((2 * blk + cpair) ^ rs) * 16;
        lo = tr_read(region + roff[0] + pos);
        hi = tr_read(region + roff[1] + pos);
    };
    auto join = [](const v4s& lo, const v4s& hi) {
        const v8s v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        return __builtin_bit_cast(v8bf, v);
    };

    v4f acc[TN][TM];
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
        for (int b = 0; b < TM; ++b) acc[a][b] = v4f{0.f, 0.f, 0.f, 0.f};

    const int RS = (R + kStepRows - 1) / kStepRows;
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
        if (s < RS) issue(s, s);
#pragma clang loop unroll(disable)
    for (int st = 0; st < RS; ++st) {
        const int later = min(RS - 1 - st, STAGES - 2);
        if (later >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(8));
        else if (later == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(4));
        else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        __builtin_amdgcn_s_barrier();
        // the buffer refilled now was read at step st-1, before this barrier
        if (st + STAGES - 1 < RS) issue((st + STAGES - 1) % STAGES, st + STAGES - 1);
        const uint32_t sb = sbase + (st % STAGES) * STAGE;
        v4s al[TM], ah[TM], bl[TN], bh[TN];
#pragma unroll
        for (int b = 0; b < TM; ++b) frag_read(sb, wm * TM + b, al[b], ah[b]);
#pragma unroll
        for (int a = 0; a < TN; ++a) frag_read(sb + kRegion, wn * TN + a, bl[a], bh[a]);
        // every read has landed before any fragment is used (the operands tie
        // the fragments to this wait, so no use can be scheduled above it)
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(al[0]), "+v"(al[1]), "+v"(al[2]), "+v"(al[3]), "+v"(ah[0]),
                       "+v"(ah[1]), "+v"(ah[2]), "+v"(ah[3]), "+v"(bl[0]), "+v"(bl[1]),
                       "+v"(bl[2]), "+v"(bl[3]), "+v"(bh[0]), "+v"(bh[1]), "+v"(bh[2]),
                       "+v"(bh[3]));
        v8bf af[TM], bf[TN];
#pragma unroll
        for (int b = 0; b < TM; ++b) af[b] = join(al[b], ah[b]);
#pragma unroll
        for (int a = 0; a < TN; ++a) bf[a] = join(bl[a], bh[a]);
#pragma unroll
        for (int a = 0; a < TN; ++a)
#pragma unroll
            for (int b = 0; b < TM; ++b)
                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[b], bf[a], acc[a][b], 0, 0, 0);
    }

    // lane l of block (a, b): dw row n = n0 + 64 wn + 16a + l%16,
    // columns k = k0 + 64 wm + 16b + 4(l/16) .. +3
#pragma unroll
    for (int a = 0; a < TN; ++a) {
        const int n = n0 + wn * 64 + 16 * a + (lane & 15);
        if (n >= N) continue;
#pragma unroll
        for (int b = 0; b < TM; ++b) {
            const int k = k0 + wm * 64 + 16 * b + 4 * (lane >> 4);
            if (k < K) {
                const v4f v = acc[a][b];
                *reinterpret_cast<uint2*>(out + int64_t(n) * ldo + k) =
                    make_uint2(cvt_pk_bf16(v[0], v[1]), cvt_pk_bf16(v[2], v[3]));
            }
        }
    }
}

// The activation gradient of a linear with a bf16 weight, the dense-mode dx:
//
//   out[m, k] = sum_n dy[m, n] * w[n, k]      dy bf16 [M, N], w bf16 [N, K]
//
// (python/xpu_kernels/int8/ops.py:194-204, dy @ w).  The weight is contracted
// along its rows, like both operands above, and goes through the same x
// region and transposing reads (D rows = k).  dy is contracted along its
// contiguous dimension: its region holds 128 rows (m) of one 32-element
// (64-byte) step, and lane l's B fragment, dy[m][8(l/16)..+7] of row
// m = l%16 of a block, is one plain 16-byte read.  Chunk c of region row r
// sits at position c ^ swz_dy(r); the 16 rows a read touches then cover the
// 64 banks exactly once.  Lane l of a 16x16 block holds D[4(l/16)+i][l%16]:
// four consecutive k of one output row, one 8-byte store.
__device__ __forceinline__ int swz_dy(int r) { return (r >> 2) & 3; }

__device__ __forceinline__ v8bf plain_read(uint32_t addr) {
    v8s r;
    asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(addr));
    return __builtin_bit_cast(v8bf, r);
}

template <int STAGES>
__global__ __launch_bounds__(256, 2) void gemm_bf16_nn_kernel(
    const uint16_t* __restrict__ W, int64_t ldw, const uint16_t* __restrict__ Y, int64_t ldy,
    uint16_t* __restrict__ out, int64_t ldo, int R, int K, int M, int tiles_k, int tiles_m) {
    constexpr int BKD = 128, BMD = 128;                 // D rows (k), D columns (m) per tile
    constexpr int TM = 4, TN = 4;                       // 16x16 blocks per wave
    constexpr int STAGE = 2 * kRegion;
    __shared__ __attribute__((aligned(1024))) int8_t smem[STAGES * STAGE];

    const int tiles = tiles_k * tiles_m;
    int t = blockIdx.x;
    if (tiles % 8 == 0) t = (t % 8) * (tiles / 8) + t / 8;   // each XCD a contiguous range
    const int k0 = (t % tiles_k) * BKD, m0 = (t / tiles_k) * BMD;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave >> 1, wn = wave & 1;

    // DMA: blocks 0..7 of a stage are the weight region (as in the TN kernel:
    // 4 rows x 256 bytes each), blocks 8..15 the dy region (16 rows x 64
    // bytes each).  Lane l of a dy block fills row r = 16*(b-8) + l/4,
    // position l%4, i.e. chunk (l%4) ^ swz_dy(r) of the step: columns past R
    // read zeros, rows past M repeat the last row (not stored).
    const int8_t* src[4];
    int srow[4];
    int scol[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int b = wave + 4 * i;
        if (i < 2) {
            srow[i] = 4 * (b & 7) + (lane >> 4);
            const int dchunk = (lane & 15) ^ swz(srow[i]);
            const int col = min(k0 + dchunk * 8, K - 8);
            src[i] = reinterpret_cast<const int8_t*>(W + col);
            scol[i] = 0;
        } else {
            const int r = 16 * (b - 8) + (lane >> 2);
            srow[i] = r;
            const int m = min(m0 + r, M - 1);
            src[i] = reinterpret_cast<const int8_t*>(Y + int64_t(m) * ldy);
            scol[i] = 8 * ((lane & 3) ^ swz_dy(r));
        }
    }
    auto issue = [&](int buf, int step) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int8_t* p;
            if (i < 2) {
                const int row = step * kStepRows + srow[i];
                p = row < R ? src[i] + int64_t(row) * ldw * 2 : g_zero_line;
            } else {
                const int col = step * kStepRows + scol[i];
                p = col < R ? src[i] + int64_t(col) * 2 : g_zero_line;
            }
            dma16(p, smem + buf * STAGE + (wave + 4 * i) * 1024);
        }
    };

    // weight fragments: the TN kernel's transposing reads
    const int g = lane >> 4, j = lane & 15;
    uint32_t roff[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) roff[h] = (8 * g + 4 * h + (j >> 2)) * 256 + 8 * (j & 1);
    const int cpair = (j & 3) >> 1;
    const int rs = swz(8 * g + (j >> 2));
    const uint32_t sbase = lds_addr(smem);
    auto frag_read = [&](uint32_t region, int blk, v4s& lo, v4s& hi) {
        const uint32_t pos = ((2 * blk + cpair) ^ rs) * 16;
        lo = tr_read(region + roff[0] + pos);
        hi = tr_read(region + roff[1] + pos);
    };
    auto join = [](const v4s& lo, const v4s& hi) {
        const v8s v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        return __builtin_bit_cast(v8bf, v);
    };
    // dy fragments: row 16*blk + j of the region, chunk g
    const uint32_t dyoff = j * 64 + ((g ^ swz_dy(j)) * 16);

    v4f acc[TN][TM];
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
        for (int b = 0; b < TM; ++b) acc[a][b] = v4f{0.f, 0.f, 0.f, 0.f};

    const int RS = (R + kStepRows - 1) / kStepRows;
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
        if (s < RS) issue(s, s);
#pragma clang loop unroll(disable)
    for (int st = 0; st < RS; ++st) {
        const int later = min(RS - 1 - st, STAGES - 2);
        if (later >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(8));
        else if (later == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(4));
        else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        __builtin_amdgcn_s_barrier();
        if (st + STAGES - 1 < RS) issue((st + STAGES - 1) % STAGES, st + STAGES - 1);
        const uint32_t sb = sbase + (st % STAGES) * STAGE;
        v4s al[TM], ah[TM];
        v8bf bf[TN];
#pragma unroll
        for (int b = 0; b < TM; ++b) frag_read(sb, wm * TM + b, al[b], ah[b]);
#pragma unroll
        for (int a = 0; a < TN; ++a) bf[a] = plain_read(sb + kRegion + (wn * TN + a) * 1024 + dyoff);
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(al[0]), "+v"(al[1]), "+v"(al[2]), "+v"(al[3]), "+v"(ah[0]),
                       "+v"(ah[1]), "+v"(ah[2]), "+v"(ah[3]), "+v"(bf[0]), "+v"(bf[1]),
                       "+v"(bf[2]), "+v"(bf[3]));
        v8bf af[TM];
#pragma unroll
        for (int b = 0; b < TM; ++b) af[b] = join(al[b], ah[b]);
#pragma unroll
        for (int a = 0; a < TN; ++a)
#pragma unroll
            for (int b = 0; b < TM; ++b)
                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[b], bf[a], acc[a][b], 0, 0, 0);
    }

    // lane l of block (a, b): output row m = m0 + 64 wn + 16a + l%16,
    // columns k = k0 + 64 wm + 16b + 4(l/16) .. +3
#pragma unroll
    for (int a = 0; a < TN; ++a) {
        const int m = m0 + wn * 64 + 16 * a + (lane & 15);
        if (m >= M) continue;
#pragma unroll
        for (int b = 0; b < TM; ++b) {
            const int k = k0 + wm * 64 + 16 * b + 4 * (lane >> 4);
            if (k < K) {
                const v4f v = acc[a][b];
                *reinterpret_cast<uint2*>(out + int64_t(m) * ldo + k) =
                    make_uint2(cvt_pk_bf16(v[0], v[1]), cvt_pk_bf16(v[2], v[3]));
            }
        }
    }
}

// ---------------------------------------------------------------- split K
// Narrow outputs with a long contraction: the dense dx (C5: M = 4096 rows,
// K = 1280 outputs, R = 5120 contraction rows) and dW (N = 5120 rows, K = 1280,
// R = 4096).  There the 128 x 128 tiles above make 320 (400) blocks for 256
// CUs, and the CUs that run two of them set the time.  Here one block of 8
// waves owns a BB x 160 tile of out[b, k] (256 tiles at C5 for both), in two
// teams of 4 (2 x 2 waves of BB/2 x 80): team t owns half of the 32-row
// contraction steps through its own ring of S LDS stages, and the teams
// alternate between MFMAs and data movement every half step, so that on each
// SIMD one wave feeds the matrix core while the other reads fragments and
// issues loads:
//   A(s): team 0 runs its step s;  team 1 reads its step s's fragments and
//         issues its loads for step s + S - 1
//   B(s): team 1 runs its step s;  team 0 reads its step s + 1's fragments
//         and issues its loads for step s + S - 1
// with one s_barrier between phases.  D = A * B with A from the operand
// contracted along its rows, a[r, k] (dx: the weight; dW: x), and B from
// b (dx: dy[m, r], contracted along its contiguous dimension, BB = 128; dW,
// YT: dy[r, n], contracted along its rows, BB = 160).  A stage holds
//   for A, 10 blocks of 16 rows (contraction) x 32 columns (64 bytes), block
//     2cg + rb for rows 16rb.. and columns 32cg..: 16-byte chunk c of row r
//     at chunk 4r + (c ^ ((r >> 2) & 2)).  One direct-to-LDS load fills a
//     block from 16 row segments of 64 bytes (measured 8% faster at C5 than
//     32 rows x 32 bytes), and the two transposing reads of a fragment (rows
//     8g + 4h + q of the step, g, q = 0..3, 32 bytes each) cover the 64 banks
//     twice, the two-cycle minimum for their 512 bytes;
//   for B, the same (YT), or 8 blocks of 16 rows (m) x 64 bytes (one step of
//     32 bf16): chunk c of row r at position c ^ ((r >> 1) & 3), lane l's
//     fragment (row l%16, elements 8(l/16)..+7) one 16-byte read.
// The fp32 sums of the two halves meet in LDS (each team adds the other's
// partial for its share of the B blocks: IEEE addition is commutative, so the
// sum does not depend on which team forms it), and each team rounds and
// stores its share.  Lane l of block (a, b) holds D[4(l/16)+i][l%16]: four
// consecutive k of one output row, one 8-byte store.
__device__ __forceinline__ int swz_y(int r, int c) { return c ^ ((r >> 1) & 3); }
// chunk (16 bytes) of row r, chunk c within a 16-row x 64-byte block
__device__ __forceinline__ int chunk_at(int r, int c) { return 4 * r + (c ^ ((r >> 2) & 2)); }

template <int OFF>
__device__ __forceinline__ v4s tr_read_at(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
    v4s r;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
    return r;
}
template <int OFF>
__device__ __forceinline__ v8s plain_read_at(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
    v8s r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
    return r;
}

// SL: contraction slice blockIdx.y of a split across blocks (dense dx only):
// R is the slice's length, A's rows and Y's columns are offset to it, and the
// slice's fp32 partial sums go to (float*)out + blockIdx.y * sl_stride
// instead of the bf16 output.
template <int S, bool YT, bool SL = false>
__global__ __launch_bounds__(512, 1) void gemm_bf16_splitk_kernel(
    const uint16_t* __restrict__ A, int64_t lda, const uint16_t* __restrict__ Y, int64_t ldy,
    uint16_t* __restrict__ out, int64_t ldo, int R, int K, int NBR, int tiles_b, int tiles_k,
    int64_t sl_stride = 0) {
    static_assert(!SL || !YT, "contraction slices for the dense dx");
    if constexpr (SL) {
        A += int64_t(blockIdx.y) * R * lda;
        Y += int64_t(blockIdx.y) * R;
    }
    constexpr int BK = 160, TK = 5;                     // A side: k columns, blocks per wave
    constexpr int TB = YT ? 5 : 4, BB = 32 * TB;        // B side: blocks per wave, tile rows
    constexpr int AB = BK / 16, YB = BB / 16, NB = AB + YB;
    // block order in a stage: dy's blocks first (measured faster at C5 than
    // after the A operand's: 61.0 against 63.9 us for the dx, 59.8 against
    // 61.0 for dW)
    constexpr int A0 = YB, Y0 = 0;
    constexpr int PER = (NB + 3) / 4, REM = NB % 4;
    constexpr int STAGE = NB * 1024, RING = S * STAGE;
    constexpr int OWN0 = (TB + 1) / 2;                  // team 0 owns B blocks 0..OWN0-1
    static_assert(2 * RING >= 4 * TK * TB * 1024, "the exchanged partial sums fit");
    static_assert(2 * RING <= 160 * 1024, "LDS");
    __shared__ __attribute__((aligned(1024))) int8_t smem[2 * RING];

    // tile grid over the 8 XCDs (block b on XCD b % 8): each XCD a gx x
    // (8 / gx) block of tiles, gx chosen so that it reads the fewest operand
    // rows and columns
    int tbi = blockIdx.x % tiles_b, tki = blockIdx.x / tiles_b;
    {
        int best = 0, cost = 0;
        for (int gx = 1; gx <= 8; gx *= 2) {
            const int gy = 8 / gx;
            if (tiles_b % gx || tiles_k % gy) continue;
            const int c = (tiles_b / gx) * BB + (tiles_k / gy) * BK;
            if (!best || c < cost) best = gx, cost = c;
        }
        if (best) {
            const int x = blockIdx.x % 8, j = blockIdx.x / 8;
            const int lb = tiles_b / best, lk = tiles_k / (8 / best);
            tbi = (x % best) * lb + j % lb;
            tki = (x / best) * lk + j / lb;
        }
    }
    const int b0 = tbi * BB, k0 = tki * BK;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int team = wave >> 2, wt = wave & 3;
    const int wb = wt >> 1, wk = wt & 1;
    int8_t* const ring = smem + team * RING;

    const int RT = R / kStepRows, RH = (RT + 1) / 2;   // team 0 takes the first RH steps
    const int st0 = team * RH, nst = min(RT, st0 + RH) - st0;

    // DMA: wave wt brings blocks wt, wt + 4, ... of its team's stages.  Byte offsets from a wave-uniform base; a step adds 32
    // rows (row-contracted operands) or 64 bytes (dy of the dx).  Rows past
    // the output edge repeat the last row, columns past it a valid chunk
    // (neither is stored).
    const int8_t* const abase = reinterpret_cast<const int8_t*>(A + k0);
    const int8_t* const ybase =
        reinterpret_cast<const int8_t*>(YT ? Y + b0 : Y + int64_t(b0) * ldy);
    int off[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int j = min(wt + 4 * i, NB - 1);
        // row-contracted blocks: lane l fills chunk l of the block, i.e. row
        // r = l/4, chunk (l%4) ^ ((r >> 2) & 2) (an involution of l%4)
        const int r = lane >> 2, c = (lane & 3) ^ ((r >> 2) & 2);
        const bool isa = j >= A0 && j < A0 + AB;
        if (isa) {
            const int jj = j - A0, row = 16 * (jj & 1) + r;
            off[i] = row * int(lda) * 2 + (min(k0 + 32 * (jj >> 1) + 8 * c, K - 8) - k0) * 2;
        } else if constexpr (YT) {
            const int jj = j - Y0, row = 16 * (jj & 1) + r;
            off[i] = row * int(ldy) * 2 + (min(b0 + 32 * (jj >> 1) + 8 * c, NBR - 8) - b0) * 2;
        } else {
            const int rr = lane >> 2, c = swz_y(rr, lane & 3);
            off[i] = (min(b0 + 16 * (j - Y0) + rr, NBR - 1) - b0) * int(ldy) * 2 + 16 * c;
        }
    }
    const bool full_share = REM == 0 || wt < REM;
    auto issue = [&](int s) {
        const int step = st0 + s;
        int8_t* const st = ring + (s % S) * STAGE;
        const uint32_t arow = uint32_t(step * kStepRows) * uint32_t(lda) * 2u;
        const uint32_t yrow = YT ? uint32_t(step * kStepRows) * uint32_t(ldy) * 2u
                                 : uint32_t(step * 64);
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            if (i == PER - 1 && !full_share) break;
            const int j = wt + 4 * i;
            const int8_t* p = (j >= A0 && j < A0 + AB) ? abase + uint64_t(uint32_t(off[i]) + arow)
                                                       : ybase + uint64_t(uint32_t(off[i]) + yrow);
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

    // fragment addresses within a stage.  Transposing reads of row-contracted
    // blocks: for the 16-column block at column kc of the tile, lane j of
    // group g reads step row 8g + 4h + j/4, 8 bytes at column kc + 4(j%4);
    // plain 16-byte reads for dy of the dx.
    const int g = lane >> 4, j = lane & 15;
    auto tr_off = [&](int first, int kc, int h) {
        const int cg = kc >> 5, half = (kc >> 4) & 1;
        const int R = 8 * g + 4 * h + (j >> 2), rb = R >> 4, r = R & 15;
        const int c = 2 * half + ((j & 3) >> 1);
        return uint32_t((first + 2 * cg + rb) * 1024 + 16 * chunk_at(r, c) + 8 * (j & 1));
    };
    uint32_t aoffs[TK][2], yoffs[YT ? TB : 1][2];
#pragma unroll
    for (int a = 0; a < TK; ++a)
#pragma unroll
        for (int h = 0; h < 2; ++h) aoffs[a][h] = tr_off(A0, wk * (BK / 2) + 16 * a, h);
    if constexpr (YT) {
#pragma unroll
        for (int b = 0; b < TB; ++b)
#pragma unroll
            for (int h = 0; h < 2; ++h) yoffs[b][h] = tr_off(Y0, wb * (BB / 2) + 16 * b, h);
    }
    const uint32_t yoff = (Y0 + wb * TB) * 1024 + j * 64 + swz_y(j, g) * 16;
    const uint32_t rbase = lds_addr(ring);

    v4f acc[TK][TB];
#pragma unroll
    for (int a = 0; a < TK; ++a)
#pragma unroll
        for (int b = 0; b < TB; ++b) acc[a][b] = v4f{0.f, 0.f, 0.f, 0.f};
    v4s al[TK], ah[TK];
    v4s yl[YT ? TB : 1], yh[YT ? TB : 1];
    v8s yf[YT ? 1 : TB];
    auto read_frags = [&](int s) {
        const uint32_t sb = rbase + (s % S) * STAGE;
        auto rda = [&](auto I) {
            constexpr int a = decltype(I)::value;
            if constexpr (a < TK) {
                al[a] = tr_read_at<0>(sb + aoffs[a][0]);
                ah[a] = tr_read_at<0>(sb + aoffs[a][1]);
            }
        };
        auto rdb = [&](auto I) {
            constexpr int b = decltype(I)::value;
            if constexpr (b < TB) {
                if constexpr (YT) {
                    yl[b] = tr_read_at<0>(sb + yoffs[b][0]);
                    yh[b] = tr_read_at<0>(sb + yoffs[b][1]);
                } else {
                    yf[b] = plain_read_at<b * 1024>(sb + yoff);
                }
            }
        };
        rda(std::integral_constant<int, 0>{});
        rda(std::integral_constant<int, 1>{});
        rda(std::integral_constant<int, 2>{});
        rda(std::integral_constant<int, 3>{});
        rda(std::integral_constant<int, 4>{});
        rdb(std::integral_constant<int, 0>{});
        rdb(std::integral_constant<int, 1>{});
        rdb(std::integral_constant<int, 2>{});
        rdb(std::integral_constant<int, 3>{});
        rdb(std::integral_constant<int, 4>{});
    };
    auto join = [](const v4s& lo, const v4s& hi) {
        const v8s v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        return __builtin_bit_cast(v8bf, v);
    };
    auto compute = [&]() {
        // every read has landed before any fragment is used (the operands tie
        // the fragments to this wait)
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(al[0]), "+v"(al[1]), "+v"(al[2]), "+v"(al[3]), "+v"(al[4]),
                       "+v"(ah[0]), "+v"(ah[1]), "+v"(ah[2]), "+v"(ah[3]), "+v"(ah[4]));
        if constexpr (YT) {
            asm volatile("" : "+v"(yl[0]), "+v"(yl[1]), "+v"(yl[2]), "+v"(yl[3]), "+v"(yl[4]),
                              "+v"(yh[0]), "+v"(yh[1]), "+v"(yh[2]), "+v"(yh[3]), "+v"(yh[4]));
        } else {
            asm volatile("" : "+v"(yf[0]), "+v"(yf[1]), "+v"(yf[2]), "+v"(yf[3]));
        }
        v8bf bfr[TB];
#pragma unroll
        for (int b = 0; b < TB; ++b) {
            if constexpr (YT) bfr[b] = join(yl[b], yh[b]);
            else bfr[b] = __builtin_bit_cast(v8bf, yf[b]);
        }
#pragma unroll
        for (int a = 0; a < TK; ++a) {
            const v8bf af = join(al[a], ah[a]);
#pragma unroll
            for (int b = 0; b < TB; ++b)
                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bfr[b], acc[a][b], 0, 0, 0);
        }
    };
    auto barrier = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };

    for (int s = 0; s < S - 1; ++s)
        if (s < nst) issue(s);
    if (nst > 0) wait_batches(min(S - 2, nst - 1));
    barrier();
    if (team == 0) {
        if (nst > 0) read_frags(0);
        barrier();
#pragma clang loop unroll(disable)
        for (int s = 0; s < RH; ++s) {
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
        for (int s = 0; s < RH; ++s) {
            if (s < nst) read_frags(s);                         // A(s)
            if (s + S - 1 < nst) issue(s + S - 1);
            barrier();
            if (s < nst) compute();                             // B(s)
            if (s + 1 < nst) wait_batches(min(S - 2, nst - 2 - s));
            barrier();
        }
    }

    // exchange: each team gives the other its partial sums of the B blocks
    // the other owns (team 0 owns blocks 0 .. OWN0-1 of each wave, team 1 the
    // rest).  Team t's given blocks fill its own region of LDS, [wave][a][b]
    // x 64 lanes; constant block indices in each branch keep the
    // accumulators in registers.
    __syncthreads();
    v4f* const xchg = reinterpret_cast<v4f*>(smem);
    constexpr int CNT0 = TB - OWN0, CNT1 = OWN0;        // blocks given by team 0, 1
    auto slot = [&](auto T, int a, int b) {
        constexpr int t = decltype(T)::value;
        constexpr int first = t == 0 ? OWN0 : 0, cnt = t == 0 ? CNT0 : CNT1;
        constexpr int region = t == 0 ? 0 : 4 * TK * CNT0;
        return ((region + (wt * TK + a) * cnt + (b - first)) * 64) + lane;
    };
    auto finish = [&](auto T) {
        constexpr int t = decltype(T)::value;
        constexpr int lo = t == 0 ? 0 : OWN0, hi = t == 0 ? OWN0 : TB;   // owned blocks
        constexpr std::integral_constant<int, t> self{};
        constexpr std::integral_constant<int, 1 - t> other{};
#pragma unroll
        for (int a = 0; a < TK; ++a)
#pragma unroll
            for (int b = 0; b < TB; ++b)
                if (b < lo || b >= hi) xchg[slot(self, a, b)] = acc[a][b];
        __syncthreads();
#pragma unroll
        for (int a = 0; a < TK; ++a)
#pragma unroll
            for (int b = lo; b < hi; ++b) acc[a][b] += xchg[slot(other, a, b)];
        // lane l of block (a, b): output row b0 + (BB/2) wb + 16b + l%16,
        // columns k0 + 80 wk + 16a + 4(l/16) .. +3
#pragma unroll
        for (int b = lo; b < hi; ++b) {
            const int row = b0 + wb * (BB / 2) + 16 * b + (lane & 15);
            if (row >= NBR) continue;
#pragma unroll
            for (int a = 0; a < TK; ++a) {
                const int k = k0 + wk * 80 + 16 * a + 4 * (lane >> 4);
                if (k < K) {
                    const v4f v = acc[a][b];
                    if constexpr (SL)
                        *reinterpret_cast<v4f*>(reinterpret_cast<float*>(out) +
                                                int64_t(blockIdx.y) * sl_stride +
                                                int64_t(row) * ldo + k) = v;
                    else
                        *reinterpret_cast<uint2*>(out + int64_t(row) * ldo + k) =
                            make_uint2(cvt_pk_bf16(v[0], v[1]), cvt_pk_bf16(v[2], v[3]));
                }
            }
        }
    };
    if (team == 0) finish(std::integral_constant<int, 0>{});
    else finish(std::integral_constant<int, 1>{});
}

// out[m, k] = bf16(sum over s of part[s][m, k]), the slices added in order in
// fp32; four columns per thread (K % 4 == 0), grid-stride.
__global__ __launch_bounds__(256) void sum_slices_bf16_kernel(const float* __restrict__ part,
                                                              int nsl, int64_t sl_stride,
                                                              uint16_t* __restrict__ out,
                                                              int64_t ldo, int64_t M, int64_t K) {
    const int64_t q = K / 4, total = M * q;
    for (int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
         t += int64_t(gridDim.x) * blockDim.x) {
        const int64_t m = t / q, k = (t - m * q) * 4;
        const float* p = part + m * K + k;
        float4 v = *reinterpret_cast<const float4*>(p);
        for (int s = 1; s < nsl; ++s) {
            const float4 w = *reinterpret_cast<const float4*>(p + s * sl_stride);
            v.x = v.x + w.x; v.y = v.y + w.y; v.z = v.z + w.z; v.w = v.w + w.w;
        }
        *reinterpret_cast<uint2*>(out + m * ldo + k) =
            make_uint2(cvt_pk_bf16(v.x, v.y), cvt_pk_bf16(v.z, v.w));
    }
}

}  // namespace

// Whether a product takes the split-K kernel: a contraction of whole 32-row
// steps long enough for two teams, and enough bb x 160 tiles to fill the chip
// where 128 x 128 tiles would leave a ragged second round.  (The byte offsets
// of the row-contracted operands, up to R rows, stay below 2^32.)
static bool bf16_splitk_applies(int nb, int bb, int R, int K, int64_t lda, int64_t ldy, bool yt) {
    if (nb <= 64 || R % kStepRows || R < 2048 || K % 8 || (yt && nb % 8)) return false;
    if (int64_t(R) * lda * 2 >= (int64_t(1) << 32)) return false;
    if (yt && int64_t(R) * ldy * 2 >= (int64_t(1) << 32)) return false;
    const int64_t tiles = int64_t((nb + bb - 1) / bb) * ((K + 159) / 160);
    return tiles >= 128 && tiles <= 256;
}

// Contraction slices of the dense dx (dy [M, N] . w [N, K]) split across
// blocks, when its 128 x 160 tiles are too few for the split-K kernel (below
// 128): the fewest power-of-two slices giving at least 192 blocks, each slice
// a whole number of 32-row steps and at least 1024 rows; 0 when none applies.
int bf16_nn_slices(int M, int N, int K) {
    if (M <= 64 || K % 8 || N % kStepRows) return 0;
    const int64_t tiles = int64_t((M + 127) / 128) * ((K + 159) / 160);
    if (tiles >= 128) return 0;
    int s = 1;
    while (tiles * s < 192 && (N / kStepRows) % (2 * s) == 0 && N / (2 * s) >= 1024) s *= 2;
    if (s == 1) return 0;
    // the split-K kernel's 32-bit byte offsets: a slice's rows of w (N / s
    // rows of K) and a 128-row block of dy (rows of N); beyond them the
    // unsplit kernel takes the shape
    if (int64_t(N / s) * K * 2 >= (int64_t(1) << 32) || 128 * int64_t(N) * 2 >= (int64_t(1) << 31))
        return 0;
    return s;
}

hipError_t gemm_bf16_nn_slices(hipStream_t st, const void* dy, int64_t ldy, const void* w,
                               int64_t ldw, void* out, int64_t ldo, int M, int N, int K,
                               float* part, int nsl) {
    const int tm = (M + 127) / 128, tk = (K + 159) / 160;
    hipLaunchKernelGGL((gemm_bf16_splitk_kernel<4, false, true>),
                       dim3(unsigned(tm * tk), unsigned(nsl)), dim3(512), 0, st,
                       static_cast<const uint16_t*>(w), ldw, static_cast<const uint16_t*>(dy), ldy,
                       reinterpret_cast<uint16_t*>(part), int64_t(K), N / nsl, K, M, tm, tk,
                       int64_t(M) * K);
    if (const hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    int64_t blocks = (int64_t(M) * (K / 4) + 255) / 256;
    if (blocks > (int64_t(1) << 20)) blocks = int64_t(1) << 20;
    hipLaunchKernelGGL(sum_slices_bf16_kernel, dim3(unsigned(blocks)), dim3(256), 0, st, part, nsl,
                       int64_t(M) * K, static_cast<uint16_t*>(out), ldo, int64_t(M), int64_t(K));
    return hipGetLastError();
}

hipError_t gemm_bf16_nn(hipStream_t st, const void* dy, int64_t ldy, const void* w, int64_t ldw,
                        void* out, int64_t ldo, int M, int N, int K) {
    if (bf16_splitk_applies(M, 128, N, K, ldw, ldy, false)) {
        const int tm = (M + 127) / 128, tk = (K + 159) / 160;
        hipLaunchKernelGGL((gemm_bf16_splitk_kernel<4, false>), dim3(unsigned(tm * tk)), dim3(512),
                           0, st, static_cast<const uint16_t*>(w), ldw,
                           static_cast<const uint16_t*>(dy), ldy, static_cast<uint16_t*>(out), ldo,
                           N, K, M, tm, tk);
        return hipGetLastError();
    }
    const int tiles_k = (K + 127) / 128, tiles_m = (M + 127) / 128;
    hipLaunchKernelGGL((gemm_bf16_nn_kernel<2>), dim3(unsigned(tiles_k * tiles_m)), dim3(256), 0,
                       st, static_cast<const uint16_t*>(w), ldw, static_cast<const uint16_t*>(dy),
                       ldy, static_cast<uint16_t*>(out), ldo, N, K, M, tiles_k, tiles_m);
    return hipGetLastError();
}

hipError_t gemm_bf16_tn(hipStream_t st, const void* dy, int64_t ldy, const void* x, int64_t ldx,
                        void* dw, int64_t ldo, int R, int N, int K) {
    constexpr int STAGES_TN = 4;                // 2 x 4 x 20 KB of LDS
    if (bf16_splitk_applies(N, 160, R, K, ldx, ldy, true)) {
        const int tn = (N + 159) / 160, tk = (K + 159) / 160;
        hipLaunchKernelGGL((gemm_bf16_splitk_kernel<STAGES_TN, true>), dim3(unsigned(tn * tk)),
                           dim3(512), 0, st, static_cast<const uint16_t*>(x), ldx,
                           static_cast<const uint16_t*>(dy), ldy, static_cast<uint16_t*>(dw), ldo,
                           R, K, N, tn, tk);
        return hipGetLastError();
    }
    const int tiles_k = (K + 127) / 128, tiles_n = (N + 127) / 128;
    // two stages (one in flight): measured fastest at the C5 shape (75 us vs
    // 83-86 us for three to five), the smaller LDS footprint leaving room for
    // more resident blocks per CU
    hipLaunchKernelGGL((gemm_bf16_tn_kernel<2>), dim3(unsigned(tiles_k * tiles_n)), dim3(256), 0,
                       st, static_cast<const uint16_t*>(x), ldx, static_cast<const uint16_t*>(dy),
                       ldy, static_cast<uint16_t*>(dw), ldo, R, K, N, tiles_k, tiles_n);
    return hipGetLastError();
}

}  // namespace xpuint8
