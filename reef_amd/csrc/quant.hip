// int8 quantization kernels: the rule of quant.hpp:51-81 (scale = max|x| / 127,
// or 1 when every value is 0; code = clamp(nearbyint(x / scale), +-127)) at
// per-tensor, per-head and per-token (quantize_rows, quant.hpp:112-133)
// granularity. Codes and scales are bit-identical to the engine's: the largest
// magnitude is an exact reduction, and the division and the round-to-nearest-
// even are single correctly rounded IEEE operations.
//
// Every kernel here is bound by HBM bandwidth: 4 bytes read and 1 byte written
// per element (per-tensor and per-head scales need the whole tensor's maximum
// first, so those read the input twice). Streams larger than the last-level cache
// use non-temporal accesses: nothing of them is found in a cache again, and
// without the allocation they run a quarter to a third faster (a per-head
// quantize of 4 x 32 x 8192 x 128 floats, 537 MB: 214 against 277 us; a
// dequantize to 537 MB of floats: 97 against 157 us). Smaller ones use ordinary
// accesses, and the second read of a two-pass scale finds much of the first in
// the 256 MB last-level cache.
#include "reef_common.hpp"

namespace reef {
namespace {

constexpr int kQuantThreads = 256;
// Inputs (or outputs) beyond these sizes are streamed with non-temporal accesses:
// one-pass kernels beyond the 256 MB last-level cache, the two-pass per-tensor and
// per-head scales beyond 384 MB (at 268 MB the second read still finds enough of
// the first in the cache: 97 against 108 us with non-temporal loads).
constexpr int64_t kStreamBytes = int64_t(256) << 20;
constexpr int64_t kStreamBytesTwoPass = int64_t(384) << 20;

template <bool NT>
__device__ __forceinline__ float4 load4(const float4 *p) {
    if constexpr (NT) {
        const f32x4 t = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
        return float4{t[0], t[1], t[2], t[3]};
    } else {
        return *p;
    }
}

// Codes of quantize_int8 for a group of values that share one scale, from
// y = x * rcp(scale) instead of the IEEE quotient t = x / scale: |x| <= 127 scale
// bounds |t| by 127 (1 + 2^-24); rcp is within 1 ulp and the product is rounded
// once, so |y - t| < 2^-15.4, and t's own rounding adds under 2^-16.9: y lies
// within 3.1e-5 of the engine's quotient. Unless y is within 2^-14 of a
// half-integer, rint(y) is the engine's code. When any lane of the wave has such
// a value (about 1.2e-4 per value), or the scale is below 2^-125 or not finite,
// the active lanes of the wave take IEEE quotients for the whole group (one
// ballot; lanes that do not call it take no part).
template <int N>
__device__ __forceinline__ void quantize_group(const float (&x)[N], float scale,
                                               int8_t (&code)[N]) {
    const float rs = __builtin_amdgcn_rcpf(scale);
    bool near = !(scale >= 0x1p-125f && scale <= 3.4028235e38f);
    float r[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const float y = x[i] * rs;
        r[i] = __builtin_rintf(y);
        near |= __builtin_fabsf(y - r[i]) > 0.5f - 0x1p-14f;
    }
    if (__builtin_amdgcn_ballot_w64(near) != 0) {
#pragma unroll
        for (int i = 0; i < N; ++i) r[i] = __builtin_rintf(x[i] / scale);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const float c = r[i] < -127.0f ? -127.0f : (r[i] > 127.0f ? 127.0f : r[i]);
        code[i] = (int8_t)(int)c;
    }
}

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
#pragma unroll 4
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
#pragma unroll 4
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
//
// Block (x, h) walks a contiguous range of the head's B * S rows. A row of D values
// is VEC ? D / 4 float4 : D floats wide; `tpr` threads share a row (all 256 when a
// row is wider than the block) and 256 / tpr rows are in flight per step, with
// 32-bit index arithmetic per row rather than per element.

struct HeadView {
    const float *x;
    int64_t sb, sh, st;  // element strides of batch, head, token
    int32_t batch, tokens, dim;
    int32_t per_row;        // VEC ? dim / 4 : dim
    int32_t tpr;            // threads per row: min(per_row rounded up to a power of 2, 256)
    int32_t rows_per_block;
};

__device__ __forceinline__ const float *head_row(const HeadView &v, int64_t h, int32_t row) {
    const int32_t b = row / v.tokens, t = row - b * v.tokens;
    return v.x + b * v.sb + h * v.sh + t * v.st;
}

template <bool VEC>
__device__ __forceinline__ uint32_t max_of(const float *r, int32_t col) {
    if (VEC) {
        const float4 x = reinterpret_cast<const float4 *>(r)[col];
        uint32_t a = mag_bits(x.x), b = mag_bits(x.y), c = mag_bits(x.z), d = mag_bits(x.w);
        a = a > b ? a : b;
        c = c > d ? c : d;
        return a > c ? a : c;
    }
    return mag_bits(r[col]);
}

template <bool VEC>
__global__ __launch_bounds__(kQuantThreads) void head_max(HeadView v, uint32_t *max_bits) {
    const int64_t h = blockIdx.y;
    const int32_t rows = v.batch * v.tokens;
    const int32_t r0 = blockIdx.x * v.rows_per_block;
    const int32_t r1 = min(rows, r0 + v.rows_per_block);
    const int32_t lane_row = threadIdx.x / v.tpr, lane_col = threadIdx.x % v.tpr;
    const int32_t step = kQuantThreads / v.tpr;
    uint32_t m = 0;
#pragma unroll 4
    for (int32_t row = r0 + lane_row; row < r1; row += step) {
        const float *r = head_row(v, h, row);
        for (int32_t col = lane_col; col < v.per_row; col += v.tpr) {
            const uint32_t a = max_of<VEC>(r, col);
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
    const int32_t rows = v.batch * v.tokens;
    const int32_t r0 = blockIdx.x * v.rows_per_block;
    const int32_t r1 = min(rows, r0 + v.rows_per_block);
    const int32_t lane_row = threadIdx.x / v.tpr, lane_col = threadIdx.x % v.tpr;
    const int32_t step = kQuantThreads / v.tpr;
    bool bad = false;
#pragma unroll 4
    for (int32_t row = r0 + lane_row; row < r1; row += step) {
        const int32_t b = row / v.tokens, t = row - b * v.tokens;
        const float *r = v.x + b * v.sb + h * v.sh + t * v.st;
        int8_t *out = q + ((b * heads + h) * v.tokens + t) * v.dim;
        for (int32_t col = lane_col; col < v.per_row; col += v.tpr) {
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
    }
    if (bad) flag_status(status, REEF_STATUS_BIT_NON_FINITE);
}

// Flat form for heads whose tokens are contiguous (token stride == head_dim, both
// multiples of 4): slice (b, h) is tokens * dim consecutive floats. Block (x, h, b)
// streams float4 [x * chunk, (x + 1) * chunk) of its slice, kFlatUnroll independent
// loads in flight per thread, no per-row index arithmetic. No atomics (atomic maxima
// into the scales array serialize: the heads' words share one cache line); every
// block's largest magnitude goes to partial words kept in the output buffer q,
// which the quantize pass overwrites afterwards. Two launches when every chunk of
// q holds the batch * blocks partials of its head ("spread"): the max pass writes
// its word into the chunk of every block of the same head, and each quantize block
// reduces the words in its own chunk (the same maximum, so the same scale, in every
// block of a head) before it overwrites that chunk, which no other block reads.
// Otherwise three: the partials go to the front of q, one block per head reduces
// them and writes the scale, and the quantize pass reads the scales.
struct FlatHeads {
    const float *x;
    int64_t sb, sh;      // element strides of batch and head
    int64_t slice4;      // float4 per (batch, head) slice
    int64_t chunk4;      // float4 per block
    int32_t heads, batch, blocks;  // blocks per slice
};

constexpr int kFlatUnroll = 4;
// Blocks of a flat launch over `bytes` of input: about 8 per compute unit (128 KB of
// loads in flight per unit); 4 per unit for streams beyond the cache, which run
// non-temporal (q, k and v of 4x32x8192x128 per head: 640 against 667 us).
inline int64_t flat_blocks(int64_t bytes) { return bytes > kStreamBytesTwoPass ? 1024 : 2048; }

__device__ __forceinline__ uint32_t block_max(uint32_t m) {  // the result on thread 0
    __shared__ uint32_t partial[kQuantThreads / kWave];
    m = wave_max_u32(m);
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    if (lane == 0) partial[wave] = m;
    __syncthreads();
    uint32_t r = partial[0];
    for (int w = 1; w < kQuantThreads / kWave; ++w) r = r > partial[w] ? r : partial[w];
    return r;
}

// Word offset in q of the chunk of block (x, h, b).
__device__ __forceinline__ int64_t chunk_word(const FlatHeads &f, int b, int h, int x) {
    return ((int64_t)b * f.heads + h) * f.slice4 + (int64_t)x * f.chunk4;
}

template <bool kSpread, bool NT>
__global__ __launch_bounds__(kQuantThreads) void head_max_flat(FlatHeads f, uint32_t *partials) {
    const int h = blockIdx.y, b = blockIdx.z;
    const float4 *x = reinterpret_cast<const float4 *>(f.x + b * f.sb + h * f.sh);
    const int64_t i0 = (int64_t)blockIdx.x * f.chunk4;
    const int64_t i1 = min(f.slice4, i0 + f.chunk4);
    uint32_t m = 0;
    for (int64_t i = i0 + threadIdx.x; i < i1; i += kQuantThreads * kFlatUnroll) {
        float4 v[kFlatUnroll];
#pragma unroll
        for (int u = 0; u < kFlatUnroll; ++u) {
            const int64_t j = i + u * kQuantThreads;
            v[u] = j < i1 ? load4<NT>(x + j) : float4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int u = 0; u < kFlatUnroll; ++u) {
            uint32_t a = mag_bits(v[u].x), c = mag_bits(v[u].y), d = mag_bits(v[u].z),
                     e = mag_bits(v[u].w);
            a = a > c ? a : c;
            d = d > e ? d : e;
            a = a > d ? a : d;
            m = m > a ? m : a;
        }
    }
    m = block_max(m);
    if (kSpread) {
        // partials is q: word b * blocks + x of the chunk of every block of head h
        const int n = f.batch * f.blocks;
        for (int i = threadIdx.x; i < n; i += kQuantThreads)
            partials[chunk_word(f, i / f.blocks, h, i % f.blocks) + b * f.blocks + blockIdx.x] = m;
    } else if (threadIdx.x == 0) {
        partials[((int64_t)h * f.batch + b) * f.blocks + blockIdx.x] = m;
    }
}

// One block per head: the largest of its partials, then the head's scale.
__global__ __launch_bounds__(kQuantThreads) void head_scale_flat(FlatHeads f,
                                                                 const uint32_t *partials,
                                                                 float *scales) {
    const int h = blockIdx.x;
    const int n = f.batch * f.blocks;
    uint32_t m = 0;
    for (int i = threadIdx.x; i < n; i += kQuantThreads) {
        const uint32_t a = partials[(int64_t)h * n + i];
        m = m > a ? m : a;
    }
    m = block_max(m);
    if (threadIdx.x == 0) scales[h] = int8_scale(__uint_as_float(m));
}

// kSpread: the scale comes from the partial words in this block's own chunk of q
// (written by the max pass), and block (0, h, 0) stores it to scales[h].
template <bool kSpread, bool NT>
__global__ __launch_bounds__(kQuantThreads) void head_quantize_flat(FlatHeads f, float *scales,
                                                                    int8_t *__restrict__ q,
                                                                    uint32_t *status) {
    const int h = blockIdx.y, b = blockIdx.z;
    float scale;
    if (kSpread) {
        const uint32_t *words = reinterpret_cast<const uint32_t *>(q) + chunk_word(f, b, h, blockIdx.x);
        uint32_t m = 0;
        for (int i = threadIdx.x; i < f.batch * f.blocks; i += kQuantThreads) {
            const uint32_t a = words[i];
            m = m > a ? m : a;
        }
        // every thread's reads are consumed before block_max's barrier, so the
        // chunk may be overwritten after it
        m = block_max(m);
        scale = int8_scale(__uint_as_float(m));
        if (b == 0 && blockIdx.x == 0 && threadIdx.x == 0) scales[h] = scale;
    } else {
        scale = scales[h];
    }
    const float4 *x = reinterpret_cast<const float4 *>(f.x + b * f.sb + h * f.sh);
    char4 *out = reinterpret_cast<char4 *>(q) + ((int64_t)b * f.heads + h) * f.slice4;
    const int64_t i0 = (int64_t)blockIdx.x * f.chunk4;
    const int64_t i1 = min(f.slice4, i0 + f.chunk4);
    bool bad = false;
    for (int64_t i = i0 + threadIdx.x; i < i1; i += kQuantThreads * kFlatUnroll) {
        float4 v[kFlatUnroll];
#pragma unroll
        for (int u = 0; u < kFlatUnroll; ++u) {
            const int64_t j = i + u * kQuantThreads;
            v[u] = j < i1 ? load4<NT>(x + j) : float4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        float xs[4 * kFlatUnroll];
#pragma unroll
        for (int u = 0; u < kFlatUnroll; ++u) {
            bad |= !(__builtin_isfinite(v[u].x) && __builtin_isfinite(v[u].y) &&
                     __builtin_isfinite(v[u].z) && __builtin_isfinite(v[u].w));
            xs[4 * u] = v[u].x;
            xs[4 * u + 1] = v[u].y;
            xs[4 * u + 2] = v[u].z;
            xs[4 * u + 3] = v[u].w;
        }
        int8_t c[4 * kFlatUnroll];
        quantize_group(xs, scale, c);  // the lanes past i1 hold zeros
#pragma unroll
        for (int u = 0; u < kFlatUnroll; ++u) {
            const int64_t j = i + u * kQuantThreads;
            if (j < i1) out[j] = char4{c[4 * u], c[4 * u + 1], c[4 * u + 2], c[4 * u + 3]};
        }
    }
    if (bad) flag_status(status, REEF_STATUS_BIT_NON_FINITE);
}

// ---- per token (quantize_rows) --------------------------------------------------------------
//
// Fast form for rows of at most 256 float4 (width % 4 == 0): LPR lanes per row hold
// the row's float4 in registers (PER each), so the row is read once; 64 / LPR rows
// per wave and row group. The largest magnitude is reduced over the LPR lanes of the
// row. Streams beyond the cache take row_groups groups per wave whose loads are all
// issued before the first group is reduced (4 float4 in flight per lane: 1M rows of
// 128 in 126 against 149 us); smaller inputs one group per wave (more, shorter
// waves: 65536 rows of 128 in 10.9 against 12.8 us).
__host__ __device__ constexpr int row_groups(int per, bool nt) {
    return nt && per < 4 ? 4 / per : 1;
}

template <int LPR, int PER, bool NT>
__global__ __launch_bounds__(kQuantThreads) void token_quantize_regs(
    const float *__restrict__ x, int64_t rows, int32_t w4, int64_t row_stride,
    int8_t *__restrict__ q, float *__restrict__ scales, uint32_t *status) {
    constexpr int RPW = kWave / LPR;  // rows per wave and group
    constexpr int G = row_groups(PER, NT);
    const int lane = threadIdx.x % kWave, sub = lane / LPR, l = lane % LPR;
    const int64_t wave_id = (int64_t)blockIdx.x * (kQuantThreads / kWave) + threadIdx.x / kWave;
    float4 v[G][PER];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int64_t row = (wave_id * G + g) * RPW + sub;
        const bool live = row < rows;
        const float4 *r = reinterpret_cast<const float4 *>(x + (live ? row : 0) * row_stride);
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int col = l + j * LPR;
            v[g][j] = (live && col < w4) ? load4<NT>(r + col) : float4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int64_t row = (wave_id * G + g) * RPW + sub;
        uint32_t m = 0;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            uint32_t a = mag_bits(v[g][j].x), b = mag_bits(v[g][j].y), c = mag_bits(v[g][j].z),
                     d = mag_bits(v[g][j].w);
            a = a > b ? a : b;
            c = c > d ? c : d;
            a = a > c ? a : c;
            m = m > a ? m : a;
        }
#pragma unroll
        for (int o = LPR / 2; o > 0; o >>= 1) {
            const uint32_t w = (uint32_t)__shfl_xor((int)m, o);
            m = m > w ? m : w;
        }
        const float scale = int8_scale(__uint_as_float(m));
        float xs[4 * PER];
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            xs[4 * j] = v[g][j].x;
            xs[4 * j + 1] = v[g][j].y;
            xs[4 * j + 2] = v[g][j].z;
            xs[4 * j + 3] = v[g][j].w;
        }
        int8_t c[4 * PER];
        quantize_group(xs, scale, c);
        if (row < rows) {
            char4 *out = reinterpret_cast<char4 *>(q + row * (int64_t)w4 * 4);
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                const int col = l + j * LPR;
                if (col < w4) out[col] = char4{c[4 * j], c[4 * j + 1], c[4 * j + 2], c[4 * j + 3]};
            }
            if (l == 0) {
                scales[row] = scale;
                if (m >= 0x7f800000u) flag_status(status, REEF_STATUS_BIT_NON_FINITE);
            }
        }
    }
}

// Wide rows (256 < width / 4 <= 256 * PER): one block per row, PER float4 per
// thread held in registers, the largest magnitude reduced across the block.
template <int PER, bool NT>
__global__ __launch_bounds__(kQuantThreads) void token_quantize_wide(
    const float *__restrict__ x, int32_t w4, int64_t row_stride, int8_t *__restrict__ q,
    float *__restrict__ scales, uint32_t *status) {
    __shared__ uint32_t partial[kQuantThreads / kWave];
    const int64_t row = blockIdx.x;
    const float4 *r = reinterpret_cast<const float4 *>(x + row * row_stride);
    float4 v[PER];
    uint32_t m = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int col = threadIdx.x + j * kQuantThreads;
        v[j] = col < w4 ? load4<NT>(r + col) : float4{0.0f, 0.0f, 0.0f, 0.0f};
        uint32_t a = mag_bits(v[j].x), b = mag_bits(v[j].y), c = mag_bits(v[j].z),
                 d = mag_bits(v[j].w);
        a = a > b ? a : b;
        c = c > d ? c : d;
        a = a > c ? a : c;
        m = m > a ? m : a;
    }
    m = wave_max_u32(m);
    if (threadIdx.x % kWave == 0) partial[threadIdx.x / kWave] = m;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kQuantThreads / kWave; ++w) m = m > partial[w] ? m : partial[w];
    const float scale = int8_scale(__uint_as_float(m));
    float xs[4 * PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        xs[4 * j] = v[j].x;
        xs[4 * j + 1] = v[j].y;
        xs[4 * j + 2] = v[j].z;
        xs[4 * j + 3] = v[j].w;
    }
    int8_t c[4 * PER];
    quantize_group(xs, scale, c);
    char4 *out = reinterpret_cast<char4 *>(q + row * (int64_t)w4 * 4);
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int col = threadIdx.x + j * kQuantThreads;
        if (col < w4) out[col] = char4{c[4 * j], c[4 * j + 1], c[4 * j + 2], c[4 * j + 3]};
    }
    if (threadIdx.x == 0) {
        scales[row] = scale;
        if (m >= 0x7f800000u) flag_status(status, REEF_STATUS_BIT_NON_FINITE);
    }
}

// General form: one wave per row, the row read twice.
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
    uint32_t m = 0;
    for (int64_t i = lane; i < width; i += kWave) {
        const uint32_t a = mag_bits(r[i]);
        m = m > a ? m : a;
    }
    m = wave_max_u32(m);
    const float scale = int8_scale(__uint_as_float(m));
    for (int64_t i = lane; i < width; i += kWave) out[i] = quantize_int8(r[i], scale);
    if (lane == 0) {
        scales[row] = scale;
        if (m >= 0x7f800000u) flag_status(status, REEF_STATUS_BIT_NON_FINITE);
    }
}

// x[i] = float(q[i]) * scales[i / group]. VEC: 4 values per thread (group % 4 == 0,
// n a whole number of groups); `tpr` threads per group, 256 / tpr groups per step.
template <bool VEC, bool NT>
__global__ __launch_bounds__(kQuantThreads) void dequantize(const int8_t *__restrict__ q, int64_t n,
                                                            int64_t group, int32_t tpr,
                                                            const float *__restrict__ scales,
                                                            float *__restrict__ x) {
    const int64_t groups = (n + group - 1) / group;
    const int64_t per = VEC ? group / 4 : group;
    const int32_t lane_g = threadIdx.x / tpr, lane_c = threadIdx.x % tpr;
    const int64_t step = (int64_t)gridDim.x * (kQuantThreads / tpr);
#pragma unroll 4
    for (int64_t g = (int64_t)blockIdx.x * (kQuantThreads / tpr) + lane_g; g < groups; g += step) {
        const float s = scales[g];
        if (VEC) {
            const char4 *src = reinterpret_cast<const char4 *>(q + g * group);
            float4 *dst = reinterpret_cast<float4 *>(x + g * group);
            for (int64_t c = lane_c; c < per; c += tpr) {
                const char4 v = src[c];
                const f32x4 o = {(float)v.x * s, (float)v.y * s, (float)v.z * s, (float)v.w * s};
                if constexpr (NT)
                    __builtin_nontemporal_store(o, reinterpret_cast<f32x4 *>(dst + c));
                else
                    *reinterpret_cast<f32x4 *>(dst + c) = o;
            }
        } else {
            const int64_t e1 = min(n, (g + 1) * group);
            for (int64_t i = g * group + lane_c; i < e1; i += tpr) x[i] = (float)q[i] * s;
        }
    }
}

// The flat kernels over f (q 4-byte aligned, at least 4 * batch * heads * blocks
// bytes): two launches when the shortest chunk of q holds a head's batch * blocks
// partial words, three otherwise.
template <bool NT>
void launch_flat_nt(const FlatHeads &f, int8_t *q, float *scales, uint32_t *status,
                    hipStream_t stream) {
    uint32_t *partials = reinterpret_cast<uint32_t *>(q);
    const dim3 grid((unsigned)f.blocks, (unsigned)f.heads, (unsigned)f.batch);
    const int64_t last4 = f.slice4 - (int64_t)(f.blocks - 1) * f.chunk4;  // shortest chunk
    if ((int64_t)f.batch * f.blocks <= std::min<int64_t>(last4, 512)) {
        hipLaunchKernelGGL((head_max_flat<true, NT>), grid, dim3(kQuantThreads), 0, stream, f,
                           partials);
        hipLaunchKernelGGL((head_quantize_flat<true, NT>), grid, dim3(kQuantThreads), 0, stream, f,
                           scales, q, status);
        return;
    }
    hipLaunchKernelGGL((head_max_flat<false, NT>), grid, dim3(kQuantThreads), 0, stream, f,
                       partials);
    hipLaunchKernelGGL(head_scale_flat, dim3((unsigned)f.heads), dim3(kQuantThreads), 0, stream,
                       f, (const uint32_t *)partials, scales);
    hipLaunchKernelGGL((head_quantize_flat<false, NT>), grid, dim3(kQuantThreads), 0, stream, f,
                       scales, q, status);
}

void launch_flat(const FlatHeads &f, int8_t *q, float *scales, uint32_t *status,
                 hipStream_t stream) {
    if (16 * f.slice4 * f.batch * f.heads > kStreamBytesTwoPass)
        launch_flat_nt<true>(f, q, scales, status, stream);
    else
        launch_flat_nt<false>(f, q, scales, status, stream);
}

// The register and wide forms (width % 4 == 0, w4 = width / 4 <= 8 * kQuantThreads).
template <bool NT>
void launch_rows(const float *x, int64_t rows, int64_t w4, int64_t row_stride, int8_t *q,
                 float *scales, uint32_t *status_word, hipStream_t stream) {
    if (w4 <= 4 * kWave) {
        // lanes per row: the smallest power of two >= w4 (up to 64), then up to 4
        // float4 per lane
        int lpr = 1;
        while (lpr < w4 && lpr < kWave) lpr *= 2;
        const int per = w4 <= kWave ? 1 : w4 <= 2 * kWave ? 2 : 4;  // float4 per lane
        const int64_t rows_per_block =
            (int64_t)(kWave / lpr) * row_groups(per, NT) * (kQuantThreads / kWave);
        const dim3 grid((unsigned)ceil_div(rows, rows_per_block));
#define REEF_TOKEN_LAUNCH(L, P)                                                               \
    hipLaunchKernelGGL((token_quantize_regs<L, P, NT>), grid, dim3(kQuantThreads), 0, stream, \
                       x, rows, (int32_t)w4, row_stride, q, scales, status_word)
        switch (lpr) {
        case 1: REEF_TOKEN_LAUNCH(1, 1); break;
        case 2: REEF_TOKEN_LAUNCH(2, 1); break;
        case 4: REEF_TOKEN_LAUNCH(4, 1); break;
        case 8: REEF_TOKEN_LAUNCH(8, 1); break;
        case 16: REEF_TOKEN_LAUNCH(16, 1); break;
        case 32: REEF_TOKEN_LAUNCH(32, 1); break;
        default:
            if (per == 1) REEF_TOKEN_LAUNCH(64, 1);
            else if (per == 2) REEF_TOKEN_LAUNCH(64, 2);
            else REEF_TOKEN_LAUNCH(64, 4);
        }
#undef REEF_TOKEN_LAUNCH
    } else {
        const dim3 grid((unsigned)rows);
        if (w4 <= 2 * kQuantThreads)
            hipLaunchKernelGGL((token_quantize_wide<2, NT>), grid, dim3(kQuantThreads), 0,
                               stream, x, (int32_t)w4, row_stride, q, scales, status_word);
        else if (w4 <= 4 * kQuantThreads)
            hipLaunchKernelGGL((token_quantize_wide<4, NT>), grid, dim3(kQuantThreads), 0,
                               stream, x, (int32_t)w4, row_stride, q, scales, status_word);
        else
            hipLaunchKernelGGL((token_quantize_wide<8, NT>), grid, dim3(kQuantThreads), 0,
                               stream, x, (int32_t)w4, row_stride, q, scales, status_word);
    }
}

}  // namespace
}  // namespace reef

using namespace reef;

extern "C" reef_status reef_quantize_int8_per_tensor(const float *x, int64_t n, int8_t *q,
                                                     float *scale, uint32_t *status_word,
                                                     hipStream_t stream) {
    if (n <= 0 || !x || !q || !scale || !aligned(x, 16) || !aligned(q, 4))
        return REEF_INVALID_ARGUMENT;
    if (n % 4 == 0) {
        // One flat slice: the per-head kernels with a single head.
        FlatHeads f;
        f.x = x;
        f.sb = f.sh = 0;
        f.slice4 = n / 4;
        f.heads = f.batch = 1;
        const int64_t per_slice = std::max<int64_t>(
            1, std::min<int64_t>(flat_blocks(4 * n), ceil_div(f.slice4, kQuantThreads * kFlatUnroll)));
        f.chunk4 = ceil_div(f.slice4, per_slice);
        f.blocks = (int32_t)ceil_div(f.slice4, f.chunk4);
        if (4 * (int64_t)f.blocks <= n) {
            launch_flat(f, q, scale, status_word, stream);
            return launch_status();
        }
    }
    uint32_t *bits = reinterpret_cast<uint32_t *>(scale);
    hipLaunchKernelGGL(zero_words, dim3(1), dim3(64), 0, stream, bits, (int64_t)1);
    const int grid = (int)std::max<int64_t>(1, std::min<int64_t>(1024, ceil_div(n / 4 + 1, kQuantThreads * 8)));
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
    if (batch * tokens >= (int64_t(1) << 31) || head_dim >= (int64_t(1) << 24))
        return REEF_UNSUPPORTED;
    HeadView v;
    v.x = x;
    v.sb = xs ? xs->batch : heads * tokens * head_dim;
    v.sh = xs ? xs->head : tokens * head_dim;
    v.st = xs ? xs->token : head_dim;
    v.batch = (int32_t)batch;
    v.tokens = (int32_t)tokens;
    v.dim = (int32_t)head_dim;
    if (v.sb < 0 || v.sh < 0 || v.st < 0) return REEF_INVALID_ARGUMENT;
    const bool vec = head_dim % 4 == 0 && v.sb % 4 == 0 && v.sh % 4 == 0 && v.st % 4 == 0 &&
                     aligned(x, 16) && aligned(q, 4);
    v.per_row = (int32_t)(vec ? head_dim / 4 : head_dim);
    v.tpr = 1;
    while (v.tpr < v.per_row && v.tpr < kQuantThreads) v.tpr *= 2;
    if (vec && v.st == head_dim && batch <= 65535) {
        // Contiguous tokens: flat float4 streams, about flat_blocks() blocks in all,
        // at least 16 KB of input each; the partial maxima (4 bytes per block) fit
        // in q when q holds at least that many bytes.
        FlatHeads f;
        f.x = x;
        f.sb = v.sb;
        f.sh = v.sh;
        f.slice4 = tokens * head_dim / 4;
        f.heads = (int32_t)heads;
        f.batch = (int32_t)batch;
        const int64_t per_slice =
            std::max<int64_t>(1, std::min(ceil_div(flat_blocks(16 * f.slice4 * batch * heads),
                                                   batch * heads),
                                          ceil_div(f.slice4, kQuantThreads * kFlatUnroll)));
        f.chunk4 = ceil_div(f.slice4, per_slice);
        f.blocks = (int32_t)ceil_div(f.slice4, f.chunk4);
        const int64_t partial_bytes = 4 * batch * heads * (int64_t)f.blocks;
        if (partial_bytes <= batch * heads * tokens * head_dim && aligned(q, 4)) {
            launch_flat(f, q, scales, status_word, stream);
            return launch_status();
        }
    }
    uint32_t *bits = reinterpret_cast<uint32_t *>(scales);
    hipLaunchKernelGGL(zero_words, dim3((unsigned)ceil_div(heads, 64)), dim3(64), 0, stream, bits,
                       heads);
    // About 1024 blocks in all (4 per compute unit), each a run of whole rows of
    // at least 8 values per thread.
    const int64_t rows = batch * tokens;
    const int64_t rows_min = std::max<int64_t>(1, ceil_div(kQuantThreads * 8, v.per_row));
    const int64_t blocks_per_head =
        std::max<int64_t>(1, std::min<int64_t>(ceil_div(1024, heads), ceil_div(rows, rows_min)));
    v.rows_per_block = (int32_t)ceil_div(rows, blocks_per_head);
    const dim3 grid((unsigned)ceil_div(rows, v.rows_per_block), (unsigned)heads);
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
    const int64_t w4 = width / 4;
    if (vec && (w4 <= 4 * kWave || (w4 <= 8 * kQuantThreads && rows < (int64_t(1) << 31)))) {
        if (4 * rows * row_stride > kStreamBytes)
            launch_rows<true>(x, rows, w4, row_stride, q, scales, status_word, stream);
        else
            launch_rows<false>(x, rows, w4, row_stride, q, scales, status_word, stream);
    } else {
        const dim3 grid((unsigned)ceil_div(rows, kQuantThreads / kWave));
        hipLaunchKernelGGL(token_quantize, grid, dim3(kQuantThreads), 0, stream, x, rows, width,
                           row_stride, q, scales, status_word);
    }
    return launch_status();
}

extern "C" reef_status reef_dequantize_int8(const int8_t *q, int64_t n, int64_t group,
                                            const float *scales, float *x, hipStream_t stream) {
    if (!q || !scales || !x || n <= 0 || group <= 0) return REEF_INVALID_ARGUMENT;
    const bool vec = group % 4 == 0 && n % group == 0 && aligned(q, 4) && aligned(x, 16);
    const int64_t per = vec ? group / 4 : group;
    int tpr = 1;
    while (tpr < per && tpr < kQuantThreads) tpr *= 2;
    const int64_t groups = ceil_div(n, group);
    const int64_t blocks =
        std::max<int64_t>(1, std::min<int64_t>(1024, ceil_div(groups, kQuantThreads / tpr)));
    const dim3 grid((unsigned)blocks);
    if (vec && 4 * n > kStreamBytes)  // outputs no cache keeps: stored non-temporally
        hipLaunchKernelGGL((dequantize<true, true>), grid, dim3(kQuantThreads), 0, stream, q, n,
                           group, tpr, scales, x);
    else if (vec)
        hipLaunchKernelGGL((dequantize<true, false>), grid, dim3(kQuantThreads), 0, stream, q, n,
                           group, tpr, scales, x);
    else
        hipLaunchKernelGGL((dequantize<false, false>), grid, dim3(kQuantThreads), 0, stream, q, n,
                           group, tpr, scales, x);
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
    if (word & REEF_STATUS_BIT_OVERFLOW) return REEF_OVERFLOW;
    if (word & (REEF_STATUS_BIT_BAD_PAGE | REEF_STATUS_BIT_BAD_LENGTH))
        return REEF_INVALID_ARGUMENT;
    return REEF_OK;
}
