// KV-cache append for the int8 decode cache (gfx950).
//
// The engine's Attention::append_kv_cache (attention.hpp:290-352) copies the
// whole fp32 cache into a new buffer on every call, one (batch, head) block at a
// time, so that the new positions land at the end of each block. Here the cache
// is preallocated to its capacity and stays in place. One workgroup fills one
// 16-token cache page of one (sequence, KV head) with the new tokens that fall
// in it: each wave quantizes key and value rows (quantize_rows,
// quant.hpp:112-133, bit-identical codes and scales) into LDS, K token-major and
// V already transposed, and the page then leaves in 16-byte stores, whole pages
// as they are laid out in the cache (K [16, D], V [D, 16], the layout the decode
// kernel reads). The capacity check of attention.hpp:321-327 becomes a status
// bit, since the lengths live on the device.
#include "reef_common.hpp"

namespace reef {
namespace {

constexpr int kPage = 16;
constexpr int kAppendThreads = 256;  // 4 waves per (batch, kv head, cache page)
constexpr int kAppendWaves = kAppendThreads / kWave;

struct AppendArgs {
    const float *k, *v;
    int64_t k_sb, k_sh, k_st, v_sb, v_sh, v_st;
    const int32_t *start;
    int32_t batch, kv_heads, new_tokens, max_context;
    int8_t *k_dst, *v_dst;
    float *ks_dst, *vs_dst;
    const int32_t *table;  // paged only
    int32_t max_blocks, num_pages;
    uint32_t *status;
};

// Largest |x| of the wave's row as IEEE bits (a NaN has the largest bits).
__device__ __forceinline__ uint32_t mag(float x) { return __float_as_uint(x) & 0x7fffffffu; }

// Quantizes the row of D values at src (lane holds channels lane + 64 j) and
// stores the codes through store(d, code); returns the scale.
template <int D, typename Store>
__device__ __forceinline__ float quantize_row(const float *src, int lane, bool &bad, Store store) {
    constexpr int PER = D / kWave;
    float x[PER];
    uint32_t m = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        x[j] = src[lane + kWave * j];
        const uint32_t b = mag(x[j]);
        m = m > b ? m : b;
    }
    m = wave_max_u32(m);
    bad = m >= 0x7f800000u;
    const float scale = int8_scale(__uint_as_float(m));
#pragma unroll
    for (int j = 0; j < PER; ++j) store(lane + kWave * j, quantize_int8(x[j], scale));
    return scale;
}

template <int D, bool PAGED>
__global__ __launch_bounds__(kAppendThreads) void kv_append(AppendArgs a) {
    __shared__ __attribute__((aligned(16))) int8_t sK[kPage * D];   // [slot][channel]
    __shared__ __attribute__((aligned(16))) int8_t sVT[D * kPage];  // [channel][slot]
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int b = blockIdx.z, kvh = blockIdx.y;
    const int start = a.start[b];
    // attention.hpp:321-327: the whole append of a sequence fits or none of it is written.
    if (start < 0 || start > a.max_context - a.new_tokens) {
        if (blockIdx.x == 0 && kvh == 0 && tid == 0)
            flag_status(a.status, start < 0 ? REEF_STATUS_BIT_BAD_LENGTH : REEF_STATUS_BIT_CAPACITY);
        return;
    }
    // This workgroup's page and the positions [p_lo, p_hi) of new tokens in it.
    const int page_idx = start / kPage + (int)blockIdx.x;
    const int p_lo = max(start, page_idx * kPage);
    const int p_hi = min(start + a.new_tokens, (page_idx + 1) * kPage);
    if (p_lo >= p_hi) return;  // past the appended range (uniform over the workgroup)
    int64_t page_base;  // index of this (page, kv head) in units of 16-token pages
    if (PAGED) {
        const int page = a.table[(int64_t)b * a.max_blocks + page_idx];
        if (page < 0 || page >= a.num_pages) {
            if (tid == 0) flag_status(a.status, REEF_STATUS_BIT_BAD_PAGE);
            return;
        }
        page_base = (int64_t)page * a.kv_heads + kvh;
    } else {
        page_base = ((int64_t)b * a.kv_heads + kvh) * (a.max_context / kPage) + page_idx;
    }
    // Wave w quantizes slots w, w + 4, w + 8, w + 12 of the page.
    bool bad = false;
#pragma unroll
    for (int i = 0; i < kPage / kAppendWaves; ++i) {
        const int slot = wave + kAppendWaves * i;
        const int pos = page_idx * kPage + slot;
        if (pos < p_lo || pos >= p_hi) continue;  // wave-uniform
        const int t = pos - start;
        bool bad_k, bad_v;
        const float ks = quantize_row<D>(a.k + b * a.k_sb + kvh * a.k_sh + (int64_t)t * a.k_st,
                                         lane, bad_k, [&](int d, int8_t c) { sK[slot * D + d] = c; });
        const float vs = quantize_row<D>(a.v + b * a.v_sb + kvh * a.v_sh + (int64_t)t * a.v_st,
                                         lane, bad_v, [&](int d, int8_t c) { sVT[d * kPage + slot] = c; });
        if (lane == 0) {
            a.ks_dst[page_base * kPage + slot] = ks;
            a.vs_dst[page_base * kPage + slot] = vs;
        }
        bad |= bad_k || bad_v;
    }
    if (bad && lane == 0) flag_status(a.status, REEF_STATUS_BIT_NON_FINITE);
    __syncthreads();
    int8_t *kpage = a.k_dst + page_base * kPage * D;
    int8_t *vpage = a.v_dst + page_base * D * kPage;
    if (p_hi - p_lo == kPage) {
        // A whole page: 16-byte copies of both LDS images.
        for (int o = 16 * tid; o < kPage * D; o += 16 * kAppendThreads) {
            *reinterpret_cast<i32x4 *>(kpage + o) = *reinterpret_cast<const i32x4 *>(sK + o);
            *reinterpret_cast<i32x4 *>(vpage + o) = *reinterpret_cast<const i32x4 *>(sVT + o);
        }
    } else {
        // A partial page (the first or last of the append): only its new slots
        // change; the others hold earlier tokens.
        const int s_lo = p_lo - page_idx * kPage, s_hi = p_hi - page_idx * kPage;
        for (int o = tid; o < kPage * D; o += kAppendThreads) {
            const int ks = o / D, vs = o % kPage;
            if (ks >= s_lo && ks < s_hi) kpage[o] = sK[o];
            if (vs >= s_lo && vs < s_hi) vpage[o] = sVT[o];
        }
    }
}

// After the writes: context_lens[b] = start[b] + new_tokens for every sequence
// that had room (the others keep their length).
__global__ void advance_lengths(const int32_t *start, int32_t batch, int32_t new_tokens,
                                int32_t max_context, int32_t *lens) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= batch) return;
    const int s = start[b];
    if (s >= 0 && s <= max_context - new_tokens) lens[b] = s + new_tokens;
}

reef_status prepare(const reef_kv_append_params *p, const float *k_new, const reef_strides *ks,
                    const float *v_new, const reef_strides *vs, const int32_t *start,
                    const void *k_dst, const void *v_dst, const float *k_scales,
                    const float *v_scales, AppendArgs &a) {
    if (!p || !k_new || !v_new || !start || !k_dst || !v_dst || !k_scales || !v_scales)
        return REEF_INVALID_ARGUMENT;
    if (p->batch <= 0 || p->kv_heads <= 0 || p->head_dim <= 0 || p->new_tokens <= 0 ||
        p->max_context <= 0 || p->max_context % kPage != 0)
        return REEF_INVALID_ARGUMENT;
    // attention.hpp:321-327: an append longer than the whole cache can never fit.
    if (p->new_tokens > p->max_context) return REEF_CAPACITY;
    if (p->head_dim != 64 && p->head_dim != 128) return REEF_UNSUPPORTED;
    // (grid: pages x kv heads x batch)
    if (p->max_context >= (int64_t(1) << 30) || p->batch > 65535 || p->kv_heads > 65535)
        return REEF_UNSUPPORTED;
    const int64_t D = p->head_dim, H = p->kv_heads, T = p->new_tokens;
    const auto strides = [&](const reef_strides *s, int64_t &sb, int64_t &sh, int64_t &st) {
        sb = s ? s->batch : H * T * D;
        sh = s ? s->head : T * D;
        st = s ? s->token : D;
        return sb >= 0 && sh >= 0 && st >= 0;
    };
    if (!strides(ks, a.k_sb, a.k_sh, a.k_st) || !strides(vs, a.v_sb, a.v_sh, a.v_st))
        return REEF_INVALID_ARGUMENT;
    a.k = k_new;
    a.v = v_new;
    a.start = start;
    a.batch = (int32_t)p->batch;
    a.kv_heads = (int32_t)H;
    a.new_tokens = (int32_t)T;
    a.max_context = (int32_t)p->max_context;
    a.k_dst = (int8_t *)k_dst;
    a.v_dst = (int8_t *)v_dst;
    a.ks_dst = (float *)k_scales;
    a.vs_dst = (float *)v_scales;
    a.table = nullptr;
    a.max_blocks = 0;
    a.num_pages = 0;
    return REEF_OK;
}

template <bool PAGED>
reef_status launch(const reef_kv_append_params *p, AppendArgs &a, int32_t *context_lens,
                   uint32_t *status_word, hipStream_t stream) {
    a.status = status_word;
    // pages an append of new_tokens can touch: ceil(new_tokens / 16) + 1 when it
    // starts inside a page
    const dim3 grid((unsigned)(ceil_div(p->new_tokens, kPage) + 1), (unsigned)p->kv_heads,
                    (unsigned)p->batch);
    if (p->head_dim == 128)
        hipLaunchKernelGGL((kv_append<128, PAGED>), grid, dim3(kAppendThreads), 0, stream, a);
    else
        hipLaunchKernelGGL((kv_append<64, PAGED>), grid, dim3(kAppendThreads), 0, stream, a);
    if (hipGetLastError() != hipSuccess) return REEF_HIP_ERROR;
    if (context_lens) {
        hipLaunchKernelGGL(advance_lengths, dim3((unsigned)ceil_div(p->batch, 256)), dim3(256), 0,
                           stream, a.start, a.batch, a.new_tokens, a.max_context, context_lens);
    }
    return launch_status();
}

}  // namespace
}  // namespace reef

using namespace reef;

extern "C" reef_status reef_kv_append_int8(const reef_kv_append_params *p, const float *k_new,
                                           const reef_strides *k_strides, const float *v_new,
                                           const reef_strides *v_strides,
                                           const int32_t *start_positions, int8_t *k_cache,
                                           int8_t *v_cache, float *k_scales, float *v_scales,
                                           int32_t *context_lens, uint32_t *status_word,
                                           hipStream_t stream) {
    AppendArgs a;
    const reef_status s = prepare(p, k_new, k_strides, v_new, v_strides, start_positions, k_cache,
                                  v_cache, k_scales, v_scales, a);
    if (s != REEF_OK) return s;
    return launch<false>(p, a, context_lens, status_word, stream);
}

extern "C" reef_status reef_kv_append_int8_paged(
    const reef_kv_append_params *p, const float *k_new, const reef_strides *k_strides,
    const float *v_new, const reef_strides *v_strides, const int32_t *start_positions,
    const int32_t *block_table, int64_t max_blocks_per_seq, int64_t num_pages, int8_t *k_pages,
    int8_t *v_pages, float *k_scale_pages, float *v_scale_pages, int32_t *context_lens,
    uint32_t *status_word, hipStream_t stream) {
    AppendArgs a;
    const reef_status s = prepare(p, k_new, k_strides, v_new, v_strides, start_positions, k_pages,
                                  v_pages, k_scale_pages, v_scale_pages, a);
    if (s != REEF_OK) return s;
    if (!block_table || max_blocks_per_seq <= 0 || num_pages <= 0 ||
        max_blocks_per_seq * kPage < p->max_context || num_pages >= (int64_t(1) << 31) ||
        max_blocks_per_seq >= (int64_t(1) << 26))
        return REEF_INVALID_ARGUMENT;
    a.table = block_table;
    a.max_blocks = (int32_t)max_blocks_per_seq;
    a.num_pages = (int32_t)num_pages;
    return launch<true>(p, a, context_lens, status_word, stream);
}
