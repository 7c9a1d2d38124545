// W8A8 projection for gfx950: the engine's linear() with a QuantizedWeight
// (operator/linear.hpp:106-132). Input rows are quantized per row (quantize_rows,
// quant.hpp:112-133, by the per-token kernel), the int8 rows times the int8
// weight [out, in] are exact int32 sums on v_mfma_i32_32x32x32_i8, and the
// epilogue applies y = float(sum) * (row_scale * weight_scale) (+ bias), the
// engine's float steps in its order, each rounded on its own (no contraction),
// so the outputs are bit-identical.
//
// Tiling: a workgroup of 4 waves owns a 128 x 128 output tile; each wave a
// 64 x 64 quarter as 2 x 2 blocks of 32 x 32. K advances 64 bytes per step through
// kStages LDS stages filled by direct-to-LDS buffer loads issued kStages - 1 steps
// ahead, so a step's matrix work never waits on memory latency (no staging
// registers, no LDS store instructions). Workgroups are numbered so that each XCD
// (which receives every eighth workgroup) takes a contiguous run of tiles, rows of
// tiles sharing their input rows in that XCD's L2.
#include <algorithm>
#include <cmath>
#include <cstdlib>

#include "reef_common.hpp"

namespace reef {
namespace {

constexpr int kGemmThreads = 256;
constexpr int kXcds = 8;
#ifndef REEF_GEMM_BN
#define REEF_GEMM_BN 128
#endif
#ifndef REEF_GEMM_BK
#define REEF_GEMM_BK 128
#endif
#ifndef REEF_GEMM_STAGES
#define REEF_GEMM_STAGES 2
#endif
constexpr int kBM = 128, kBN = REEF_GEMM_BN;  // output tile: rows x out features
constexpr int kBK = REEF_GEMM_BK;             // bytes of K per step
constexpr int kStages = REEF_GEMM_STAGES;
constexpr int kABytes = kBM * kBK, kBBytes = kBN * kBK;  // operand tiles of one stage
constexpr int kChunks = kBK / 16;             // 16-byte chunks per tile row
constexpr int kRowsPerBlock = 1024 / kBK;     // tile rows per 1 KB direct load

struct GemmArgs {
    const int8_t *x;  // [rows, in] quantized rows, row stride in
    const float *xs;  // [rows]
    const int8_t *w;  // [out, in]
    const float *ws;  // [out]
    const float *bias;  // [out] or null
    float *y;
    int64_t y_stride;
    int32_t rows, in, out;
    int32_t m_tiles, n_tiles;
    uint32_t *status;
};

// Chunk c (16 bytes) of tile row r sits at 16 * (c ^ s(r)) in the row, s(r) the row
// bits above those that already separate rows within 256 bytes: the 16 lanes that
// read one chunk column of 16 consecutive rows hit 16 distinct bank groups.
__device__ __forceinline__ int chunk_pos(int r, int c) {
    constexpr int rows256 = 256 / kBK;  // rows whose chunks c fall in distinct bank groups
    return c ^ ((r / rows256) & (kChunks - 1));
}

// One BM x BN output tile at (m0, n0) (128 x 128, 128 x 64 or 64 x 64): 4 waves
// in a 2 x 2 grid, each wave BM/2 x BN/2 in 32 x 32 blocks; the operand tiles of
// one stage are BM x kBK (A) then BN x kBK (B) from the start of `smem`'s stage.
template <int BM, int BN>
__device__ __forceinline__ void gemm_tile(const GemmArgs &a, int m0, int n0,
                                          int8_t (*smem)[kABytes + kBBytes]) {
    constexpr int MI = BM / 64, NJ = BN / 64;          // 32-wide blocks per wave
    constexpr int TA = BM * kBK, TB = BN * kBK;        // operand tiles of a stage
    constexpr int PA = TA / 1024 / 4, PB = TB / 1024 / 4;  // 1 KB blocks per wave
    static_assert(PA >= 1 && PB >= 1 && TA + TB <= kABytes + kBBytes, "tile fits a stage");
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int col = lane & 31, grp = lane >> 5;

    // Direct loads: wave w fills 1 KB blocks w, w + 4, ... of each operand tile;
    // lane L of block b writes tile row kRowsPerBlock b + L / kChunks at position
    // L % kChunks, which holds chunk chunk_pos(row, L % kChunks). Rows past the end
    // and chunks past `in` read zeros: their offset is set beyond the buffer.
    const uint32_t xbytes = (uint32_t)((int64_t)a.rows * a.in);
    const uint32_t wbytes = (uint32_t)((int64_t)a.out * a.in);
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(a.x, xbytes);
    const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(a.w, wbytes);
    uint32_t aoff[PA], boff[PB];
    // (every block row of a wave has the same chunk position, so one k offset each)
    const int kch = 16 * chunk_pos(kRowsPerBlock * wave + lane / kChunks, lane % kChunks);
#pragma unroll
    for (int i = 0; i < PA; ++i) {
        const int r = kRowsPerBlock * (wave + 4 * i) + lane / kChunks;
        aoff[i] = m0 + r < a.rows ? (uint32_t)((int64_t)(m0 + r) * a.in + kch) : xbytes;
    }
#pragma unroll
    for (int i = 0; i < PB; ++i) {
        const int r = kRowsPerBlock * (wave + 4 * i) + lane / kChunks;
        boff[i] = n0 + r < a.out ? (uint32_t)((int64_t)(n0 + r) * a.in + kch) : wbytes;
    }
    const int steps = (a.in + kBK - 1) / kBK;
    auto issue = [&](int s) {  // K step s (clamped to the last) into stage s % kStages
        const int k0 = min(s, steps - 1) * kBK;
        int8_t *sa = smem[s % kStages];
        int8_t *sb = sa + TA;
        const bool in_k = k0 + kch < a.in;
#pragma unroll
        for (int i = 0; i < PA; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xr, (__attribute__((address_space(3))) void *)(sa + 1024 * (wave + 4 * i)), 16,
                in_k ? aoff[i] : xbytes, k0, 0, 0);
#pragma unroll
        for (int i = 0; i < PB; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                wr, (__attribute__((address_space(3))) void *)(sb + 1024 * (wave + 4 * i)), 16,
                in_k ? boff[i] : wbytes, k0, 0, 0);
    };

    // Operand reads: row (BM/2) wm + 32 i + col (A) or (BN/2) wn + 32 j + col (B),
    // chunk 2 ks + grp; the swizzle depends on bits 2-3 of the row, i.e. of col.
    int rpos[kBK / 32];
#pragma unroll
    for (int ks = 0; ks < kBK / 32; ++ks) rpos[ks] = 16 * chunk_pos(col, 2 * ks + grp);
    const int arow = ((BM / 2) * wm + col) * kBK, brow = ((BN / 2) * wn + col) * kBK;

    i32x16 acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = i32x16{};

#pragma unroll
    for (int s = 0; s < kStages - 1; ++s) issue(s);
    for (int k = 0; k < steps; ++k) {
        // Each wave has issued PA + PB loads per step; those of the kStages - 2 later
        // steps may still be in flight, this step's must have landed. (s_waitcnt
        // fields: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8; 0xf70 leaves
        // the other two unconstrained.)
        constexpr int kInFlight = (PA + PB) * (kStages - 2);
        static_assert(kInFlight < 64, "vmcnt fits");
        __builtin_amdgcn_s_waitcnt(0xf70 | (kInFlight & 15) | ((kInFlight >> 4) << 14));
        // All waves' loads of step k are in LDS and their reads of step k - 1 are
        // done (consumed by the matrix instructions), so stage (k - 1) is free. A
        // bare barrier: __syncthreads() would also wait for every load in flight.
        __builtin_amdgcn_s_barrier();
        issue(k + kStages - 1);
        const int8_t *sa = smem[k % kStages];
        const int8_t *sb = sa + TA;
#pragma unroll
        for (int ks = 0; ks < kBK / 32; ++ks) {
            i32x4 aop[MI], bop[NJ];
#pragma unroll
            for (int i = 0; i < MI; ++i)
                aop[i] = *reinterpret_cast<const i32x4 *>(sa + arow + 32 * i * kBK + rpos[ks]);
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                bop[j] = *reinterpret_cast<const i32x4 *>(sb + brow + 32 * j * kBK + rpos[ks]);
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j) acc[i][j] = mfma_32x32x32_i8(aop[i], bop[j], acc[i][j]);
        }
    }
    // The trailing loads of the clamped last steps must land before the workgroup's
    // LDS can be handed to another workgroup.
    __builtin_amdgcn_s_waitcnt(0xf70);

    // Epilogue: lane holds output column n0 + (BN/2) wn + 32 j + col and, in
    // register 4 q + e, row m0 + (BM/2) wm + 32 i + 8 q + 4 grp + e.
    bool bad = false;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int n = n0 + (BN / 2) * wn + 32 * j + col;
        if (n >= a.out) continue;
        const float wsc = a.ws[n];
        const float bn = a.bias ? a.bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + (BM / 2) * wm + 32 * i + 8 * (r >> 2) + 4 * grp + (r & 3);
                if (m >= a.rows) continue;
                float v;
                {
#pragma clang fp contract(off)
                    const float scale = a.xs[m] * wsc;  // safe_multiply(row, column)
                    v = (float)acc[i][j][r] * scale;    // safe_multiply(sum, scale)
                    if (a.bias) v = v + bn;             // add_bias: safe_add
                }
                bad |= !__builtin_isfinite(v);
                a.y[(int64_t)m * a.y_stride + n] = v;
            }
    }
    if (bad) flag_status(a.status, REEF_STATUS_BIT_OVERFLOW);
}

// Workgroups [0, n_big) take the 128 x 128 tiles [0, n_big) in tile order (tiles
// along `out` fastest). When there are a few more tiles than compute units, the
// remaining tiles are cut into `pieces` (4: 64 x 64 quadrants, 2: 128 x 64 halves),
// one workgroup each, so that every compute unit holds one large tile and at most
// one piece instead of some holding two large tiles while the others idle.
// Workgroup i runs on XCD i % 8: each XCD gets a contiguous run of the large
// tiles and of the pieces.
__global__ __launch_bounds__(kGemmThreads, 2) void gemm_w8a8_kernel(GemmArgs a, int n_big,
                                                                    int pieces) {
    static_assert(kBN == kBM, "square tiles");
    __shared__ __attribute__((aligned(16))) int8_t smem[kStages][kABytes + kBBytes];  // [stage] A, B
    const int g = (int)blockIdx.x;
    auto xcd_rank = [](int i, int count) {
        const int x = i % kXcds, per = count / kXcds, rem = count % kXcds;
        return x * per + min(x, rem) + i / kXcds;
    };
    if (g < n_big) {
        const int t = xcd_rank(g, n_big);
        gemm_tile<kBM, kBN>(a, t / a.n_tiles * kBM, t % a.n_tiles * kBN, smem);
    } else if (pieces == 4) {
        const int s = xcd_rank(g - n_big, (int)gridDim.x - n_big);
        const int t = n_big + s / 4, q = s % 4;
        gemm_tile<kBM / 2, kBN / 2>(a, t / a.n_tiles * kBM + (kBM / 2) * (q >> 1),
                                    t % a.n_tiles * kBN + (kBN / 2) * (q & 1), smem);
    } else {
        const int s = xcd_rank(g - n_big, (int)gridDim.x - n_big);
        const int t = n_big + s / 2, q = s % 2;
        gemm_tile<kBM, kBN / 2>(a, t / a.n_tiles * kBM, t % a.n_tiles * kBN + (kBN / 2) * q, smem);
    }
}

reef_status launch_gemm(const int8_t *xq, const float *xs, int64_t rows, int64_t in,
                        const int8_t *w, const float *ws, const float *bias, int64_t out,
                        float *y, int64_t y_stride, uint32_t *status, hipStream_t stream) {
    GemmArgs a;
    a.x = xq;
    a.xs = xs;
    a.w = w;
    a.ws = ws;
    a.bias = bias;
    a.y = y;
    a.y_stride = y_stride;
    a.rows = (int32_t)rows;
    a.in = (int32_t)in;
    a.out = (int32_t)out;
    a.n_tiles = (int32_t)ceil_div(out, kBN);
    a.m_tiles = (int32_t)ceil_div(rows, kBM);
    a.status = status;
    const int64_t tiles = (int64_t)a.m_tiles * a.n_tiles;
    // A few more tiles than compute units: the tiles past one per unit go as
    // pieces, so the grid is at most two workgroups per unit: quadrants for up to a
    // quarter more tiles, halves for up to half more. (Measured on 4096 x 8192 ->
    // 1280, 320 tiles: 64.5 us against 70.4 with quadrants; cut into quadrants, 384
    // tiles queue and lose: 84.9 against 80.7 us.)
    const int64_t cus = compute_units();
    const int64_t extra = tiles - cus;
    const int pieces = extra <= 0         ? 1
                       : 4 * extra <= cus ? 4
                       : 2 * extra <= cus ? 2
                                          : 1;
    const int64_t n_big = pieces > 1 ? cus : tiles;
    const int64_t grid = n_big + pieces * (tiles - n_big);
    hipLaunchKernelGGL(gemm_w8a8_kernel, dim3((unsigned)grid), dim3(kGemmThreads), 0, stream, a,
                       (int)n_big, pieces);
    return launch_status();
}

reef_status validate_gemm(const void *x, const float *xs, int64_t rows, int64_t in,
                          const int8_t *w, const float *ws, int64_t out, float *y,
                          int64_t y_stride) {
    if (!x || !xs || !w || !ws || !y || rows <= 0 || in <= 0 || out <= 0 || y_stride < out)
        return REEF_INVALID_ARGUMENT;
    if (in % 16 != 0 || !aligned(w, 16)) return REEF_UNSUPPORTED;
    if (rows * in >= (int64_t(1) << 31) || out * in >= (int64_t(1) << 31) ||
        ceil_div(rows, kBM) * ceil_div(out, kBN) >= (int64_t(1) << 31))
        return REEF_UNSUPPORTED;
    return REEF_OK;
}

}  // namespace
}  // namespace reef

using namespace reef;

extern "C" size_t reef_linear_w8a8_workspace_bytes(int64_t rows, int64_t in_features) {
    if (rows <= 0 || in_features <= 0) return 0;
    // quantized rows (16-byte aligned), then one scale per row
    return (size_t)(ceil_div(rows * in_features, 16) * 16 + rows * 4);
}

extern "C" reef_status reef_gemm_w8a8(const int8_t *xq, const float *x_scales, int64_t rows,
                                      int64_t in_features, const int8_t *weight,
                                      const float *w_scales, const float *bias,
                                      int64_t out_features, float *y, int64_t y_row_stride,
                                      uint32_t *status_word, hipStream_t stream) {
    const reef_status s = validate_gemm(xq, x_scales, rows, in_features, weight, w_scales,
                                        out_features, y, y_row_stride);
    if (s != REEF_OK) return s;
    if (!aligned(xq, 16)) return REEF_UNSUPPORTED;
    return launch_gemm(xq, x_scales, rows, in_features, weight, w_scales, bias, out_features, y,
                       y_row_stride, status_word, stream);
}

extern "C" reef_status reef_linear_w8a8(const float *x, int64_t rows, int64_t in_features,
                                        int64_t x_row_stride, const int8_t *weight,
                                        const float *w_scales, const float *bias,
                                        int64_t out_features, float *y, int64_t y_row_stride,
                                        void *workspace, size_t workspace_bytes,
                                        uint32_t *status_word, hipStream_t stream) {
    reef_status s = validate_gemm(x, w_scales, rows, in_features, weight, w_scales, out_features,
                                  y, y_row_stride);
    if (s != REEF_OK) return s;
    if (!workspace || !aligned(workspace, 16) ||
        workspace_bytes < reef_linear_w8a8_workspace_bytes(rows, in_features))
        return REEF_INVALID_ARGUMENT;
    int8_t *xq = static_cast<int8_t *>(workspace);
    float *xs = reinterpret_cast<float *>(xq + ceil_div(rows * in_features, 16) * 16);
    s = reef_quantize_int8_per_token(x, rows, in_features, x_row_stride, xq, xs, status_word,
                                     stream);
    if (s != REEF_OK) return s;
    return launch_gemm(xq, xs, rows, in_features, weight, w_scales, bias, out_features, y,
                       y_row_stride, status_word, stream);
}
