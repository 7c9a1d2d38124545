// KV-cache append for the int8 decode cache (gfx950).
//
// The engine's Attention::append_kv_cache (attention.hpp:290-352) copies the
// whole fp32 cache into a new buffer on every call, one (batch, head) block at a
// time, so that the new positions land at the end of each block. Here the cache
// is preallocated to its capacity and stays in place. One workgroup fills one
// 16-token cache page of one (sequence, KV head) with the new tokens that fall
// in it: each wave quantizes key and value rows (quantize_rows,
// quant.hpp:112-133, bit-identical codes and scales) into token-major LDS
// images, and the page then leaves in 16-byte stores, whole pages as they are
// laid out in the cache (K [16, D], V transposed to [D, 16] on the way out: the
// layout the decode kernel reads). The capacity check of attention.hpp:321-327 becomes a status
// bit, since the lengths live on the device.
#include "reef_common.hpp"

namespace reef {
namespace {

constexpr int kPage = 16;
constexpr int kAppendThreads = 256;  // 4 waves per (batch, kv head, cache page)

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

// Largest |x| as IEEE bits (a NaN has the largest bits).
__device__ __forceinline__ uint32_t mag(float x) { return __float_as_uint(x) & 0x7fffffffu; }

// Largest v over the LPR (8 or 16) lanes of this lane's group, in every lane of it:
// a group is (part of) one 16-lane DPP row, reduced by the quad swaps, the mirrored
// half row and (16 lanes) the mirrored row.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_max(uint32_t v) {
    const uint32_t w = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
    return v > w ? v : w;
}

template <int LPR>
__device__ __forceinline__ uint32_t group_max_u32(uint32_t v) {
    v = dpp_max<0xB1>(v);   // quad_perm [1, 0, 3, 2]
    v = dpp_max<0x4E>(v);   // quad_perm [2, 3, 0, 1]
    v = dpp_max<0x141>(v);  // row_half_mirror
    if (LPR == 16) v = dpp_max<0x140>(v);  // row_mirror
    return v;
}

// Each wave quantizes 8 rows of the page (quantize_rows, quant.hpp:112-133): waves 0
// and 1 the keys of slots 0-7 and 8-15, waves 2 and 3 the values. A row is spread
// over LPR = D / 8 lanes holding 8 consecutive channels each, so a wave takes
// 64 / LPR rows at once and a row's maximum is a reduction within a DPP row.
//
// The codes are rint(x / scale) clamped to +-127 with the engine's IEEE quotient,
// computed as y = x * rcp(scale): the quotient t satisfies |t| <= 127 (1 + 2^-24)
// since |x| <= max, rcp is within 1 ulp, and the product is rounded once, so
// |y - t| < 2^-15.4, and t's own rounding adds under 2^-16.9: y lies within 3.1e-5
// of the IEEE quotient. Unless y is within 2^-14 of a half-integer, rint(y) is the
// engine's code. When any lane of the wave has such a value (rare: about 1.2e-4
// per value), or a row is not finite or its scale is tiny, the wave redoes the
// pass with IEEE divisions.
template <int D, bool PAGED, bool VEC>
__global__ __launch_bounds__(kAppendThreads) void kv_append(AppendArgs a) {
    constexpr int LPR = D / 8, RPW = kWave / LPR, PASSES = 8 / RPW;
    // Both images token-major ([slot][channel]): 8-byte code writes with no bank
    // conflicts. The value page is transposed to [channel][slot] as it is stored.
    __shared__ __attribute__((aligned(16))) int8_t sK[kPage * D];
    __shared__ __attribute__((aligned(16))) int8_t sV[kPage * D];
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
    const bool is_v = wave >= 2;  // wave-uniform
    const float *src = is_v ? a.v + b * a.v_sb + kvh * a.v_sh : a.k + b * a.k_sb + kvh * a.k_sh;
    const int64_t st = is_v ? a.v_st : a.k_st;
    float *scale_dst = (is_v ? a.vs_dst : a.ks_dst) + page_base * kPage;
    const int g = lane / LPR, li = lane % LPR;
    // Every pass's loads are issued before any row is reduced.
    float x[PASSES][8];
    bool valid[PASSES];
#pragma unroll
    for (int pass = 0; pass < PASSES; ++pass) {
        const int slot = 8 * (wave & 1) + RPW * pass + g;
        const int pos = page_idx * kPage + slot;
        valid[pass] = pos >= p_lo && pos < p_hi;
        // rows outside the page's new range read new token 0 (always present) and
        // are zeroed afterwards: the loads need no branch
        const float *row = src + (int64_t)(valid[pass] ? pos - start : 0) * st + 8 * li;
        if (VEC) {
            const f32x4 lo4 = *reinterpret_cast<const f32x4 *>(row);
            const f32x4 hi4 = *reinterpret_cast<const f32x4 *>(row + 4);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                x[pass][j] = lo4[j];
                x[pass][4 + j] = hi4[j];
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) x[pass][j] = row[j];
        }
    }
#pragma unroll
    for (int pass = 0; pass < PASSES; ++pass) {
#pragma unroll
        for (int j = 0; j < 8; ++j) x[pass][j] = valid[pass] ? x[pass][j] : 0.0f;
    }
    bool bad = false;
#pragma unroll
    for (int pass = 0; pass < PASSES; ++pass) {
        const int slot = 8 * (wave & 1) + RPW * pass + g;
        if (__builtin_amdgcn_ballot_w64(valid[pass]) == 0) continue;  // wave-uniform
        uint32_t m = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) m = m > mag(x[pass][j]) ? m : mag(x[pass][j]);
        m = group_max_u32<LPR>(m);
        const bool row_bad = m >= 0x7f800000u;
        const float scale = int8_scale(__uint_as_float(m));
        const float rs = __builtin_amdgcn_rcpf(scale);
        bool near = row_bad || !(scale >= 0x1p-125f);
        float qf[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float y = x[pass][j] * rs;
            qf[j] = __builtin_rintf(y);
            near |= __builtin_fabsf(y - qf[j]) > 0.5f - 0x1p-14f;
        }
        if (__builtin_amdgcn_ballot_w64(near && valid[pass]) != 0) {  // rare: IEEE quotients
#pragma unroll
            for (int j = 0; j < 8; ++j) qf[j] = __builtin_rintf(x[pass][j] / scale);
        }
        uint32_t c[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float r = qf[j] < -127.0f ? -127.0f : (qf[j] > 127.0f ? 127.0f : qf[j]);
            c[j] = (uint32_t)(int32_t)r & 0xffu;
        }
        if (valid[pass]) {
            bad |= row_bad;
            const uint32_t w0 = c[0] | c[1] << 8 | c[2] << 16 | c[3] << 24;
            const uint32_t w1 = c[4] | c[5] << 8 | c[6] << 16 | c[7] << 24;
            *reinterpret_cast<uint2 *>((is_v ? sV : sK) + slot * D + 8 * li) = make_uint2(w0, w1);
            if (li == 0) scale_dst[slot] = scale;
        }
    }
    if (bad) flag_status(a.status, REEF_STATUS_BIT_NON_FINITE);
    __syncthreads();
    int8_t *kpage = a.k_dst + page_base * kPage * D;
    int8_t *vpage = a.v_dst + page_base * D * kPage;
    if (p_hi - p_lo == kPage) {
        // A whole page: threads [0, D) copy the key image in 16-byte chunks; thread
        // 128 + c gathers channel c's 16 slots of the value image (consecutive lanes
        // read consecutive bytes) into the transposed page row [c][0..15].
        if (tid < kPage * D / 16) {
            *reinterpret_cast<i32x4 *>(kpage + 16 * tid) = *reinterpret_cast<const i32x4 *>(sK + 16 * tid);
        } else if (tid >= 128 && tid < 128 + D) {
            const int ch = tid - 128;
            uint32_t w[4];
#pragma unroll
            for (int q = 0; q < 4; ++q)
                w[q] = (uint32_t)(uint8_t)sV[(4 * q) * D + ch] |
                       (uint32_t)(uint8_t)sV[(4 * q + 1) * D + ch] << 8 |
                       (uint32_t)(uint8_t)sV[(4 * q + 2) * D + ch] << 16 |
                       (uint32_t)(uint8_t)sV[(4 * q + 3) * D + ch] << 24;
            *reinterpret_cast<i32x4 *>(vpage + kPage * ch) =
                i32x4{(int32_t)w[0], (int32_t)w[1], (int32_t)w[2], (int32_t)w[3]};
        }
    } else {
        // A partial page (the first or last of the append): only its new slots
        // change; the others hold earlier tokens.
        const int s_lo = p_lo - page_idx * kPage, s_hi = p_hi - page_idx * kPage;
        for (int o = tid; o < kPage * D; o += kAppendThreads) {
            const int ks = o / D, vs = o % kPage;
            if (ks >= s_lo && ks < s_hi) kpage[o] = sK[o];
            if (vs >= s_lo && vs < s_hi) vpage[o] = sV[vs * D + o / kPage];
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
    // 16-byte row loads when every new row starts 16-byte aligned
    const bool vec = aligned(a.k, 16) && aligned(a.v, 16) && a.k_sb % 4 == 0 && a.k_sh % 4 == 0 &&
                     a.k_st % 4 == 0 && a.v_sb % 4 == 0 && a.v_sh % 4 == 0 && a.v_st % 4 == 0;
    if (p->head_dim == 128) {
        if (vec) hipLaunchKernelGGL((kv_append<128, PAGED, true>), grid, dim3(kAppendThreads), 0, stream, a);
        else hipLaunchKernelGGL((kv_append<128, PAGED, false>), grid, dim3(kAppendThreads), 0, stream, a);
    } else {
        if (vec) hipLaunchKernelGGL((kv_append<64, PAGED, true>), grid, dim3(kAppendThreads), 0, stream, a);
        else hipLaunchKernelGGL((kv_append<64, PAGED, false>), grid, dim3(kAppendThreads), 0, stream, a);
    }
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
