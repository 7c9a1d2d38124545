// int8 quantization kernels: the rule of quant.hpp:51-81 (scale = max|x| / 127,
// or 1 when every value is 0; code = clamp(nearbyint(x / scale), +-127)) at
// per-tensor, per-head and per-token (quantize_rows, quant.hpp:112-133)
// granularity. Codes and scales are bit-identical to the engine's: the largest
// magnitude is an exact reduction, and the division and the round-to-nearest-
// even are single correctly rounded IEEE operations.
//
// Every kernel here is bound by HBM bandwidth: 4 bytes read and 1 byte written
// per element (per-tensor and per-head scales need the whole tensor's maximum
// first, so those read the input twice; the second read usually hits the
// 256 MB last-level cache).
#include "reef_common.hpp"

namespace reef {
namespace {

constexpr int kQuantThreads = 256;

// Largest magnitudes are reduced as the bit patterns of |x|: for non-negative
// floats the unsigned order of the bits is the float order, and any Inf or NaN
// (>= 0x7f800000) wins, which the quantize pass reports as non-finite input.
__device__ __forceinline__ uint32_t mag_bits(float x) { return __float_as_uint(x) & 0x7fffffffu; }

__global__ void zero_words(uint32_t *words, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) words[i] = 0u;
}

__device__ __forceinline__ void block_max_to(uint32_t m, uint32_t *dst) {
    __shared__ uint32_t partial[kQuantThreads / kWave];
    m = wave_max_u32(m);
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    if (lane == 0) partial[wave] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t r = partial[0];
        for (int w = 1; w < kQuantThreads / kWave; ++w) r = r > partial[w] ? r : partial[w];
        atomicMax(dst, r);
    }
}

// ---- per tensor: flat array of n values ------------------------------------------------

__global__ __launch_bounds__(kQuantThreads) void tensor_max(const float *__restrict__ x, int64_t n,
                                                            uint32_t *max_bits) {
    uint32_t m = 0;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t n4 = n / 4;
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
        const float4 v = x4[i];
        uint32_t a = mag_bits(v.x), b = mag_bits(v.y), c = mag_bits(v.z), d = mag_bits(v.w);
        a = a > b ? a : b;
        c = c > d ? c : d;
        a = a > c ? a : c;
        m = m > a ? m : a;
    }
    for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint32_t a = mag_bits(x[i]);
        m = m > a ? m : a;
    }
    block_max_to(m, max_bits);
}

__global__ __launch_bounds__(kQuantThreads) void tensor_quantize(const float *__restrict__ x,
                                                                 int64_t n, const uint32_t *max_bits,
                                                                 int8_t *__restrict__ q,
                                                                 uint32_t *status) {
    const float scale = int8_scale(__uint_as_float(*max_bits));
    bool bad = false;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t n4 = n / 4;
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
        const float4 v = x4[i];
        bad |= !(__builtin_isfinite(v.x) && __builtin_isfinite(v.y) && __builtin_isfinite(v.z) &&
                 __builtin_isfinite(v.w));
        char4 c;
        c.x = quantize_int8(v.x, scale);
        c.y = quantize_int8(v.y, scale);
        c.z = quantize_int8(v.z, scale);
        c.w = quantize_int8(v.w, scale);
        reinterpret_cast<char4 *>(q)[i] = c;
    }
    for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        bad |= !__builtin_isfinite(x[i]);
        q[i] = quantize_int8(x[i], scale);
    }
    if (bad) flag_status(status, REEF_STATUS_BIT_NON_FINITE);
}

// Converts reduced maxima (bit patterns, in place) into scales.
__global__ void finalize_scales(float *scales, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) scales[i] = int8_scale(__uint_as_float(reinterpret_cast<uint32_t *>(scales)[i]));
}

// ---- per head: x [B, H, S, D] with strides; scale per head over (B, S, D) ---------------

struct HeadView {
    const float *x;
    int64_t sb, sh, st;  // element strides of batch, head, token
    int64_t batch, tokens, dim;
};

__device__ __forceinline__ const float *head_row(const HeadView &v, int64_t h, int64_t row) {
    const int64_t b = row / v.tokens, t = row - b * v.tokens;
    return v.x + b * v.sb + h * v.sh + t * v.st;
}

template <bool VEC>
__global__ __launch_bounds__(kQuantThreads) void head_max(HeadView v, uint32_t *max_bits) {
    const int64_t h = blockIdx.y;
    const int64_t rows = v.batch * v.tokens;
    const int64_t per_row = VEC ? v.dim / 4 : v.dim;
    const int64_t total = rows * per_row;
    uint32_t m = 0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = i / per_row, col = i - row * per_row;
        const float *r = head_row(v, h, row);
        if (VEC) {
            const float4 x = reinterpret_cast<const float4 *>(r)[col];
            uint32_t a = mag_bits(x.x), b = mag_bits(x.y), c = mag_bits(x.z), d = mag_bits(x.w);
            a = a > b ? a : b;
            c = c > d ? c : d;
            a = a > c ? a : c;
            m = m > a ? m : a;
        } else {
            const uint32_t a = mag_bits(r[col]);
            m = m > a ? m : a;
        }
    }
    block_max_to(m, max_bits + h);
}

template <bool VEC>
__global__ __launch_bounds__(kQuantThreads) void head_quantize(HeadView v, const uint32_t *max_bits,
                                                               int64_t heads, int8_t *__restrict__ q,
                                                               uint32_t *status) {
    const int64_t h = blockIdx.y;
    const float scale = int8_scale(__uint_as_float(max_bits[h]));
    const int64_t rows = v.batch * v.tokens;
    const int64_t per_row = VEC ? v.dim / 4 : v.dim;
    const int64_t total = rows * per_row;
    bool bad = false;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = i / per_row, col = i - row * per_row;
        const int64_t b = row / v.tokens, t = row - b * v.tokens;
        const float *r = head_row(v, h, row);
        int8_t *out = q + ((b * heads + h) * v.tokens + t) * v.dim;
        if (VEC) {
            const float4 x = reinterpret_cast<const float4 *>(r)[col];
            bad |= !(__builtin_isfinite(x.x) && __builtin_isfinite(x.y) &&
                     __builtin_isfinite(x.z) && __builtin_isfinite(x.w));
            char4 c;
            c.x = quantize_int8(x.x, scale);
            c.y = quantize_int8(x.y, scale);
            c.z = quantize_int8(x.z, scale);
            c.w = quantize_int8(x.w, scale);
            reinterpret_cast<char4 *>(out)[col] = c;
        } else {
            bad |= !__builtin_isfinite(r[col]);
            out[col] = quantize_int8(r[col], scale);
        }
    }
    if (bad) flag_status(status, REEF_STATUS_BIT_NON_FINITE);
}

// ---- per token (quantize_rows): one wave per row -----------------------------------------

template <bool VEC>
__global__ __launch_bounds__(kQuantThreads) void token_quantize(const float *__restrict__ x,
                                                                int64_t rows, int64_t width,
                                                                int64_t row_stride,
                                                                int8_t *__restrict__ q,
                                                                float *__restrict__ scales,
                                                                uint32_t *status) {
    const int lane = threadIdx.x % kWave;
    const int64_t row = (int64_t)blockIdx.x * (kQuantThreads / kWave) + threadIdx.x / kWave;
    if (row >= rows) return;
    const float *r = x + row * row_stride;
    int8_t *out = q + row * width;
    const int64_t n = VEC ? width / 4 : width;
    uint32_t m = 0;
    for (int64_t i = lane; i < n; i += kWave) {
        if (VEC) {
            const float4 v = reinterpret_cast<const float4 *>(r)[i];
            uint32_t a = mag_bits(v.x), b = mag_bits(v.y), c = mag_bits(v.z), d = mag_bits(v.w);
            a = a > b ? a : b;
            c = c > d ? c : d;
            a = a > c ? a : c;
            m = m > a ? m : a;
        } else {
            const uint32_t a = mag_bits(r[i]);
            m = m > a ? m : a;
        }
    }
    m = wave_max_u32(m);
    const float scale = int8_scale(__uint_as_float(m));
    bool bad = m >= 0x7f800000u;
    for (int64_t i = lane; i < n; i += kWave) {
        if (VEC) {
            const float4 v = reinterpret_cast<const float4 *>(r)[i];
            char4 c;
            c.x = quantize_int8(v.x, scale);
            c.y = quantize_int8(v.y, scale);
            c.z = quantize_int8(v.z, scale);
            c.w = quantize_int8(v.w, scale);
            reinterpret_cast<char4 *>(out)[i] = c;
        } else {
            out[i] = quantize_int8(r[i], scale);
        }
    }
    if (lane == 0) {
        scales[row] = scale;
        if (bad) flag_status(status, REEF_STATUS_BIT_NON_FINITE);
    }
}

__global__ __launch_bounds__(kQuantThreads) void dequantize(const int8_t *__restrict__ q, int64_t n,
                                                            int64_t group,
                                                            const float *__restrict__ scales,
                                                            float *__restrict__ x) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        x[i] = (float)q[i] * scales[i / group];
    }
}

int grid_for(int64_t work_items, int64_t cap = 4096) {
    int64_t g = ceil_div(work_items, kQuantThreads);
    if (g < 1) g = 1;
    return (int)(g < cap ? g : cap);
}

}  // namespace
}  // namespace reef

using namespace reef;

extern "C" reef_status reef_quantize_int8_per_tensor(const float *x, int64_t n, int8_t *q,
                                                     float *scale, uint32_t *status_word,
                                                     hipStream_t stream) {
    if (n <= 0 || !x || !q || !scale || !aligned(x, 16) || !aligned(q, 4))
        return REEF_INVALID_ARGUMENT;
    uint32_t *bits = reinterpret_cast<uint32_t *>(scale);
    hipLaunchKernelGGL(zero_words, dim3(1), dim3(64), 0, stream, bits, (int64_t)1);
    const int grid = grid_for(n / 4 + 1);
    hipLaunchKernelGGL(tensor_max, dim3(grid), dim3(kQuantThreads), 0, stream, x, n, bits);
    hipLaunchKernelGGL(tensor_quantize, dim3(grid), dim3(kQuantThreads), 0, stream, x, n,
                       (const uint32_t *)bits, q, status_word);
    hipLaunchKernelGGL(finalize_scales, dim3(1), dim3(64), 0, stream, scale, (int64_t)1);
    return launch_status();
}

extern "C" reef_status reef_quantize_int8_per_head(const float *x, int64_t batch, int64_t heads,
                                                   int64_t tokens, int64_t head_dim,
                                                   const reef_strides *xs, int8_t *q,
                                                   float *scales, uint32_t *status_word,
                                                   hipStream_t stream) {
    if (!x || !q || !scales || batch <= 0 || heads <= 0 || tokens <= 0 || head_dim <= 0 ||
        heads > 65535)
        return REEF_INVALID_ARGUMENT;
    HeadView v;
    v.x = x;
    v.sb = xs ? xs->batch : heads * tokens * head_dim;
    v.sh = xs ? xs->head : tokens * head_dim;
    v.st = xs ? xs->token : head_dim;
    v.batch = batch;
    v.tokens = tokens;
    v.dim = head_dim;
    if (v.sb < 0 || v.sh < 0 || v.st < 0) return REEF_INVALID_ARGUMENT;
    const bool vec = head_dim % 4 == 0 && v.sb % 4 == 0 && v.sh % 4 == 0 && v.st % 4 == 0 &&
                     aligned(x, 16) && aligned(q, 4);
    uint32_t *bits = reinterpret_cast<uint32_t *>(scales);
    hipLaunchKernelGGL(zero_words, dim3((unsigned)ceil_div(heads, 64)), dim3(64), 0, stream, bits,
                       heads);
    const int64_t per_head = batch * tokens * (vec ? head_dim / 4 : head_dim);
    // Enough blocks to fill the 256 compute units several times over.
    const int64_t want = ceil_div(2048, heads);
    const dim3 grid((unsigned)std::min<int64_t>(want, grid_for(per_head)), (unsigned)heads);
    if (vec) {
        hipLaunchKernelGGL(head_max<true>, grid, dim3(kQuantThreads), 0, stream, v, bits);
        hipLaunchKernelGGL(head_quantize<true>, grid, dim3(kQuantThreads), 0, stream, v,
                           (const uint32_t *)bits, heads, q, status_word);
    } else {
        hipLaunchKernelGGL(head_max<false>, grid, dim3(kQuantThreads), 0, stream, v, bits);
        hipLaunchKernelGGL(head_quantize<false>, grid, dim3(kQuantThreads), 0, stream, v,
                           (const uint32_t *)bits, heads, q, status_word);
    }
    hipLaunchKernelGGL(finalize_scales, dim3((unsigned)ceil_div(heads, 64)), dim3(64), 0, stream,
                       scales, heads);
    return launch_status();
}

extern "C" reef_status reef_quantize_int8_per_token(const float *x, int64_t rows, int64_t width,
                                                    int64_t row_stride, int8_t *q, float *scales,
                                                    uint32_t *status_word, hipStream_t stream) {
    if (!x || !q || !scales || rows <= 0 || width <= 0 || row_stride < width)
        return REEF_INVALID_ARGUMENT;
    const bool vec = width % 4 == 0 && row_stride % 4 == 0 && aligned(x, 16) && aligned(q, 4);
    const dim3 grid((unsigned)ceil_div(rows, kQuantThreads / kWave));
    if (vec) {
        hipLaunchKernelGGL(token_quantize<true>, grid, dim3(kQuantThreads), 0, stream, x, rows,
                           width, row_stride, q, scales, status_word);
    } else {
        hipLaunchKernelGGL(token_quantize<false>, grid, dim3(kQuantThreads), 0, stream, x, rows,
                           width, row_stride, q, scales, status_word);
    }
    return launch_status();
}

extern "C" reef_status reef_dequantize_int8(const int8_t *q, int64_t n, int64_t group,
                                            const float *scales, float *x, hipStream_t stream) {
    if (!q || !scales || !x || n <= 0 || group <= 0) return REEF_INVALID_ARGUMENT;
    hipLaunchKernelGGL(dequantize, dim3(grid_for(n)), dim3(kQuantThreads), 0, stream, q, n, group,
                       scales, x);
    return launch_status();
}

extern "C" reef_status reef_read_status_word(uint32_t *status_word, int clear,
                                             hipStream_t stream) {
    if (!status_word) return REEF_INVALID_ARGUMENT;
    uint32_t word = 0;
    if (hipMemcpyAsync(&word, status_word, sizeof word, hipMemcpyDeviceToHost, stream) !=
            hipSuccess ||
        hipStreamSynchronize(stream) != hipSuccess)
        return REEF_HIP_ERROR;
    if (clear) {
        hipLaunchKernelGGL(zero_words, dim3(1), dim3(64), 0, stream, status_word, (int64_t)1);
        if (hipGetLastError() != hipSuccess) return REEF_HIP_ERROR;
    }
    if (word & REEF_STATUS_BIT_NON_FINITE) return REEF_NON_FINITE_INPUT;
    if (word & REEF_STATUS_BIT_CAPACITY) return REEF_CAPACITY;
    if (word & (REEF_STATUS_BIT_BAD_PAGE | REEF_STATUS_BIT_BAD_LENGTH))
        return REEF_INVALID_ARGUMENT;
    return REEF_OK;
}
