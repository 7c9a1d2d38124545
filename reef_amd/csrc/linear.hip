// W8A8 projection for gfx950: the engine's linear() with a QuantizedWeight
// (operator/linear.hpp:106-132). Input rows are quantized per row (quantize_rows,
// quant.hpp:112-133, by the per-token kernel), the int8 rows times the int8
// weight [out, in] are exact int32 sums on v_mfma_i32_32x32x32_i8, and the
// epilogue applies y = float(sum) * (row_scale * weight_scale) (+ bias), the
// engine's float steps in its order, each rounded on its own (no contraction),
// so the outputs are bit-identical.
//
// Tiling: a workgroup of 4 waves owns a 128 x 128 output tile; each wave a
// 64 x 64 quarter as 2 x 2 blocks of 32 x 32. The K loop steps 64 bytes at a time
// through two LDS stages, loads for the next step in flight during this one.
#include <algorithm>
#include <cmath>

#include "reef_common.hpp"

namespace reef {
namespace {

constexpr int kGemmThreads = 256;
constexpr int kBM = 128, kBN = 128, kBK = 64;
constexpr int kRowBytes = kBK + 16;  // LDS row stride: rows r and r + 8 share no banks
constexpr int kTileBytes = kBM * kRowBytes;

struct GemmArgs {
    const int8_t *x;  // [rows, in] quantized rows, row stride in
    const float *xs;  // [rows]
    const int8_t *w;  // [out, in]
    const float *ws;  // [out]
    const float *bias;  // [out] or null
    float *y;
    int64_t y_stride;
    int32_t rows, in, out;
    int32_t n_tiles;  // output tiles along out
    uint32_t *status;
};

__global__ __launch_bounds__(kGemmThreads, 2) void gemm_w8a8_kernel(GemmArgs a) {
    __shared__ __attribute__((aligned(16))) int8_t smem[2][2][kTileBytes];  // [stage][A|B]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int col = lane & 31, grp = lane >> 5;
    const int tm = (int)blockIdx.x / a.n_tiles, tn = (int)blockIdx.x % a.n_tiles;
    const int m0 = tm * kBM, n0 = tn * kBN;

    // Loads: each thread moves two 16-byte chunks of A and two of B per K step:
    // chunk c = tid + 256 j is row c / 4, bytes (c % 4) * 16. Rows past the end and
    // bytes past `in` read zeros (buffer resource bounds).
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(a.x, (uint32_t)((int64_t)a.rows * a.in));
    const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(a.w, (uint32_t)((int64_t)a.out * a.in));
    uint32_t aoff[2], boff[2];
    int dst[2];
    bool a_ok[2], b_ok[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int c = tid + kGemmThreads * j, r = c >> 2, kb = (c & 3) * 16;
        a_ok[j] = m0 + r < a.rows;
        b_ok[j] = n0 + r < a.out;
        aoff[j] = (uint32_t)((int64_t)(a_ok[j] ? m0 + r : 0) * a.in + kb);
        boff[j] = (uint32_t)((int64_t)(b_ok[j] ? n0 + r : 0) * a.in + kb);
        dst[j] = r * kRowBytes + kb;
    }
    i32x4 ra[2], rb[2];
    auto load = [&](int k0) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            // a k offset past `in` (the last partial step) reads zeros
            const bool in_k = k0 + (int)((tid + kGemmThreads * j) & 3) * 16 < a.in;
            ra[j] = (a_ok[j] && in_k) ? __builtin_amdgcn_raw_buffer_load_b128(xr, aoff[j], k0, 0)
                                      : i32x4{0, 0, 0, 0};
            rb[j] = (b_ok[j] && in_k) ? __builtin_amdgcn_raw_buffer_load_b128(wr, boff[j], k0, 0)
                                      : i32x4{0, 0, 0, 0};
        }
    };
    auto store = [&](int stage) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            *reinterpret_cast<i32x4 *>(&smem[stage][0][dst[j]]) = ra[j];
            *reinterpret_cast<i32x4 *>(&smem[stage][1][dst[j]]) = rb[j];
        }
    };

    i32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = i32x16{};

    const int steps = (a.in + kBK - 1) / kBK;
    load(0);
    store(0);
    __syncthreads();
    for (int s = 0; s < steps; ++s) {
        const int stage = s & 1;
        if (s + 1 < steps) load((s + 1) * kBK);
        const int8_t *sa = smem[stage][0];
        const int8_t *sb = smem[stage][1];
#pragma unroll
        for (int ks = 0; ks < kBK / 32; ++ks) {
            i32x4 aop[2], bop[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                aop[i] = *reinterpret_cast<const i32x4 *>(
                    sa + (64 * wm + 32 * i + col) * kRowBytes + 32 * ks + 16 * grp);
                bop[i] = *reinterpret_cast<const i32x4 *>(
                    sb + (64 * wn + 32 * i + col) * kRowBytes + 32 * ks + 16 * grp);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = mfma_32x32x32_i8(aop[i], bop[j], acc[i][j]);
        }
        if (s + 1 < steps) store(stage ^ 1);
        __syncthreads();
    }

    // Epilogue: lane holds output column n0 + 64 wn + 32 j + col and, in register
    // 4 q + e, row m0 + 64 wm + 32 i + 8 q + 4 grp + e.
    bool bad = false;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = n0 + 64 * wn + 32 * j + col;
        if (n >= a.out) continue;
        const float wsc = a.ws[n];
        const float bn = a.bias ? a.bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + 64 * wm + 32 * i + 8 * (r >> 2) + 4 * grp + (r & 3);
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
    a.status = status;
    const int64_t tiles = ceil_div(rows, kBM) * a.n_tiles;
    hipLaunchKernelGGL(gemm_w8a8_kernel, dim3((unsigned)tiles), dim3(kGemmThreads), 0, stream, a);
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
