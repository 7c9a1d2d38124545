// Prefill over the int8 decode cache (gfx950): chunked and multi-turn prompts.
//
// The engine's Attention::forward with query_len > 1 on a non-empty cache appends
// the chunk's keys and values first and then runs context() over every cached key,
// with query_start = key_len - query_len (attention.hpp:354-372, :415): a second
// prompt chunk attends over the first one's keys. The cache here is the decode
// format (contiguous [B, Hkv, L, D] keys and transposed [D, 16] value pages, or a
// paged pool with a block table, per-token scales), which the prefill kernels do
// not read. One gather launch copies the kv_len cached tokens of every (sequence,
// kv head) into token-major int8 rows and per-token scales in the workspace, page
// by page (the values transposed back through LDS); the prefill entry point then
// runs over them with per-token K/V scales, on the balanced schedule when the
// chunk has fewer 128-row query tiles than the GPU has compute units (its
// workspace is the first part of this one). The gather moves 2 (D + 4) bytes per
// cached token and kv head each way, small beside the chunk's attention.
#include "reef_common.hpp"

namespace reef {

int64_t prefill_balanced_bytes(const reef_attention_params &p);  // prefill.hip

namespace {

constexpr int kPage = 16;
constexpr int kGatherThreads = 256;

struct GatherArgs {
    const int8_t *k, *v;     // contiguous cache or page pool
    const float *ks, *vs;
    const int32_t *table;    // paged only (null: contiguous)
    int32_t kv_heads, kv_len, max_context, max_blocks, num_pages;
    int8_t *k_out, *v_out;   // [B, Hkv, kv_len, D]
    float *ks_out, *vs_out;  // [B, Hkv, kv_len]
    uint32_t *status;
};

// One workgroup per (cache page, sequence x kv head): the page's live tokens (the
// first kv_len of the sequence) move to the token-major rows. A page number
// outside [0, num_pages) sets BAD_PAGE and yields zero codes and scales.
template <int D>
__global__ __launch_bounds__(kGatherThreads) void gather_cache(GatherArgs a) {
    constexpr int CH = D / 16;  // 16-byte chunks per row
    __shared__ int8_t sT[kPage][D];
    const int pg = blockIdx.x;
    const int item = blockIdx.y;  // b * kv_heads + kvh
    const int b = item / a.kv_heads, kvh = item - b * a.kv_heads;
    const int t0 = pg * kPage;
    const int n = min(kPage, a.kv_len - t0);
    const int tid = threadIdx.x;

    const int8_t *kp, *vp;
    const float *ksp, *vsp;
    bool ok = true;
    if (a.table) {
        int page = a.table[(int64_t)b * a.max_blocks + pg];
        ok = page >= 0 && page < a.num_pages;
        if (!ok) page = 0;
        const int64_t slot = (int64_t)page * a.kv_heads + kvh;
        kp = a.k + slot * (kPage * D);
        vp = a.v + slot * (kPage * D);
        ksp = a.ks + slot * kPage;
        vsp = a.vs + slot * kPage;
    } else {
        const int64_t tok = (int64_t)item * a.max_context + t0;
        kp = a.k + tok * D;
        vp = a.v + tok * D;  // the [D, 16] pages of a sequence are contiguous in order
        ksp = a.ks + tok;
        vsp = a.vs + tok;
    }
    if (!ok && tid == 0) flag_status(a.status, REEF_STATUS_BIT_BAD_PAGE);
    const int64_t row0 = (int64_t)item * a.kv_len + t0;

    // Keys: rows are already token-major; chunk c of row r.
    if (tid < kPage * CH) {
        const int r = tid / CH, c = tid % CH;
        if (r < n) {
            const i32x4 w = ok ? *reinterpret_cast<const i32x4 *>(kp + r * D + 16 * c)
                               : i32x4{0, 0, 0, 0};
            *reinterpret_cast<i32x4 *>(a.k_out + (row0 + r) * D + 16 * c) = w;
        }
    }
    // Values: channel d's 16 tokens are one 16-byte row of the page; through LDS
    // to token-major rows.
    if (tid < D) {
        const i32x4 w = ok ? *reinterpret_cast<const i32x4 *>(vp + tid * kPage)
                           : i32x4{0, 0, 0, 0};
        const int8_t *bytes = reinterpret_cast<const int8_t *>(&w);
#pragma unroll
        for (int t = 0; t < kPage; ++t) sT[t][tid] = bytes[t];
    }
    if (tid < n) {
        a.ks_out[row0 + tid] = ok ? ksp[tid] : 0.0f;
        a.vs_out[row0 + tid] = ok ? vsp[tid] : 0.0f;
    }
    __syncthreads();
    if (tid < kPage * CH) {
        const int r = tid / CH, c = tid % CH;
        if (r < n)
            *reinterpret_cast<i32x4 *>(a.v_out + (row0 + r) * D + 16 * c) =
                *reinterpret_cast<const i32x4 *>(&sT[r][16 * c]);
    }
}

int64_t round256(int64_t n) { return ceil_div(n, 256) * 256; }

// Workspace layout: the prefill's balanced-schedule workspace (item counters, zero
// between calls, and part slots), then the gathered keys and values (int8 rows),
// key scales and value scales.
struct CacheWorkspace {
    int64_t balanced, k, v, ks, vs, total;
};

CacheWorkspace cache_workspace(const reef_attention_params *p) {
    const int64_t rows = p->batch * p->kv_heads * p->kv_len;
    CacheWorkspace w;
    w.balanced = round256(prefill_balanced_bytes(*p));
    w.k = w.balanced;
    w.v = w.k + round256(rows * p->head_dim);
    w.ks = w.v + round256(rows * p->head_dim);
    w.vs = w.ks + round256(rows * 4);
    w.total = w.vs + round256(rows * 4);
    return w;
}

}  // namespace
}  // namespace reef

using namespace reef;

extern "C" size_t reef_attention_prefill_cache_workspace_bytes(const reef_attention_params *p) {
    if (!p || p->batch <= 0 || p->kv_heads <= 0 || p->kv_len <= 0 ||
        (p->head_dim != 64 && p->head_dim != 128))
        return 0;
    return (size_t)cache_workspace(p).total;
}

extern "C" reef_status reef_attention_prefill_int8_cache(
    const reef_attention_params *p, const int8_t *q, const reef_strides *q_strides,
    const float *q_scales, const int8_t *k_cache, const int8_t *v_cache, const float *k_scales,
    const float *v_scales, int64_t max_context, const int32_t *block_table,
    int64_t max_blocks_per_seq, int64_t num_pages, float *out, const reef_strides *out_strides,
    void *workspace, size_t workspace_bytes, uint32_t *status_word, hipStream_t stream) {
    if (!p || !q || !q_scales || !k_cache || !v_cache || !k_scales || !v_scales || !out)
        return REEF_INVALID_ARGUMENT;
    if (p->batch <= 0 || p->q_heads <= 0 || p->kv_heads <= 0 || p->q_len <= 0 ||
        p->kv_len <= 0 || p->q_heads % p->kv_heads != 0 || p->query_start < 0 ||
        p->query_start + p->q_len > p->kv_len || p->kv_granularity != REEF_SCALE_PER_TOKEN)
        return REEF_INVALID_ARGUMENT;
    if (p->head_dim != 64 && p->head_dim != 128) return REEF_UNSUPPORTED;
    if (p->kv_len >= (int64_t(1) << 30) || p->batch * p->kv_heads > 65535 ||
        p->q_heads > 65535 || p->batch > 65535)
        return REEF_UNSUPPORTED;
    if (!aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(k_scales, 4) ||
        !aligned(v_scales, 4))
        return REEF_INVALID_ARGUMENT;
    if (block_table) {
        if (num_pages <= 0 || num_pages >= (int64_t(1) << 31) ||
            max_blocks_per_seq * kPage < p->kv_len || max_blocks_per_seq >= (int64_t(1) << 30))
            return REEF_INVALID_ARGUMENT;
    } else {
        if (max_context < p->kv_len || max_context % kPage != 0 ||
            max_context >= (int64_t(1) << 30))
            return REEF_INVALID_ARGUMENT;
    }
    const CacheWorkspace w = cache_workspace(p);
    if (!workspace || !aligned(workspace, 256) || (int64_t)workspace_bytes < w.total)
        return REEF_INVALID_ARGUMENT;

    char *base = static_cast<char *>(workspace);
    GatherArgs g;
    g.k = k_cache;
    g.v = v_cache;
    g.ks = k_scales;
    g.vs = v_scales;
    g.table = block_table;
    g.kv_heads = (int32_t)p->kv_heads;
    g.kv_len = (int32_t)p->kv_len;
    g.max_context = (int32_t)(block_table ? 0 : max_context);
    g.max_blocks = (int32_t)(block_table ? max_blocks_per_seq : 0);
    g.num_pages = (int32_t)(block_table ? num_pages : 0);
    g.k_out = reinterpret_cast<int8_t *>(base + w.k);
    g.v_out = reinterpret_cast<int8_t *>(base + w.v);
    g.ks_out = reinterpret_cast<float *>(base + w.ks);
    g.vs_out = reinterpret_cast<float *>(base + w.vs);
    g.status = status_word;
    const dim3 grid((unsigned)ceil_div(p->kv_len, kPage), (unsigned)(p->batch * p->kv_heads));
    if (p->head_dim == 128)
        hipLaunchKernelGGL(gather_cache<128>, grid, dim3(kGatherThreads), 0, stream, g);
    else
        hipLaunchKernelGGL(gather_cache<64>, grid, dim3(kGatherThreads), 0, stream, g);
    if (launch_status() != REEF_OK) return REEF_HIP_ERROR;
    return reef_attention_prefill_int8(p, q, q_strides, g.k_out, nullptr, g.v_out, nullptr,
                                       q_scales, g.ks_out, g.vs_out, out, out_strides, workspace,
                                       (size_t)w.balanced, stream);
}
