// Decode attention over an int8 KV cache for gfx950: one query token per
// sequence, all query heads of a KV head group served by one wave, the keys
// split across waves (flash-decoding), partial (max, sum, output) combined by
// a log-sum-exp pass.
//
// The engine's decode step is Attention::forward with query_len = 1
// (attention.hpp:354-372): context() sees every cached key, query_start =
// key_len - 1 (:415). Per (sequence, query head) this computes
//   s_j = float(int32 q . k_j) * (s_q * s_k[j]) * softmax_scale,
//   out = sum_j softmax(s)_j * float(v_j) * s_v[j].
//
// The kernel streams the cache straight from HBM into registers (no LDS): each
// lane issues 16-byte loads that are exactly its matrix-instruction operands.
//   * S^T = K . q^T on v_mfma_i32_16x16x64_i8: a 16-key x 16-head block per
//     instruction; lane group g of the output holds keys 16g + 4t + i, i.e. the
//     whole 16-token page g of the 64-key block.
//   * out^T = V^T . P^T on v_mfma_f32_16x16x32_f16: P comes from the score
//     registers unchanged (page g's 16 keys are lane group g's P operand), and V
//     pages are stored transposed ([D, 16] per page), so a lane's V operand for
//     one channel and 16 keys is one 16-byte load, converted exactly to fp16.
//     The head stays in lane % 16 from scores to output.
// Only G = q_heads / kv_heads of the 16 instruction columns are live (4 for
// 4:1 grouping); the instructions are far from the bound, HBM is.
#include <algorithm>
#include <cmath>
#include <mutex>

#include "reef_common.hpp"

namespace reef {
namespace {

constexpr int kDecodeWaves = 4;          // waves per workgroup, one split each
constexpr int kBlockKeys = 64;           // keys per inner step (4 pages)
constexpr int kPage = 16;                // tokens per page

struct DecodeArgs {
    const int8_t *q;
    const float *qs;
    const int8_t *k;        // contiguous cache or page pool
    const int8_t *v;
    const float *ks, *vs;
    const int32_t *block_table;  // paged only
    const int32_t *context_lens; // may be null
    uint32_t *counters;     // one per (sequence, kv head); zero between launches
    float *slots;           // [B * Hkv, groups] parts (DecodeSlot), with groups > 1
    uint32_t *status;
    int32_t batch, q_heads, kv_heads, group;
    int32_t max_context, window, splits;
    int32_t groups;  // partials per (sequence, head): one per workgroup of 4 splits
    int32_t max_blocks, num_pages;               // paged only
    int32_t q_gran;
    float score_scale;  // softmax_scale * log2(e)
};

// Page number of page_idx of sequence b from the block table (paged only), read
// ahead of the page's data: pages at or past n_pages (the sequence's
// ceil(len / 16)) are not looked up.
template <bool PAGED>
__device__ __forceinline__ int table_page(const DecodeArgs &a, int b, int page_idx, int n_pages) {
    if (!PAGED || page_idx >= n_pages) return 0;
    return a.block_table[(int64_t)b * a.max_blocks + page_idx];
}

// Addresses of one 16-token page of (sequence b, kv head kvh), `page` its number
// from table_page. Pages at or past n_pages point at a safe page and are dead. A
// page number outside [0, num_pages) is an error.
struct PageRef {
    const int8_t *k;   // [16, D]
    const int8_t *vt;  // [D, 16]
    const float *ks, *vs;  // [16]
    bool live;  // holds keys of this sequence
    bool ok;    // false: the block table held an out-of-range page number
};

template <int D, bool PAGED>
__device__ __forceinline__ PageRef page_ref(const DecodeArgs &a, int b, int kvh, int page_idx,
                                            int n_pages, int page) {
    PageRef r;
    const bool in_seq = page_idx < n_pages;
    if (PAGED) {
        const bool valid = page >= 0 && page < a.num_pages;
        r.ok = valid || !in_seq;
        r.live = in_seq && valid;
        if (!valid) page = 0;
        const int64_t slot = (int64_t)page * a.kv_heads + kvh;
        r.k = a.k + slot * (kPage * D);
        r.vt = a.v + slot * (kPage * D);
        r.ks = a.ks + slot * kPage;
        r.vs = a.vs + slot * kPage;
    } else {
        r.ok = true;
        r.live = in_seq;
        const int64_t seq = (int64_t)b * a.kv_heads + kvh;
        const int64_t tok = seq * a.max_context + (int64_t)(in_seq ? page_idx : 0) * kPage;
        r.k = a.k + tok * D;
        r.vt = a.v + tok * D;  // pages of [D, 16] are contiguous in the same order
        r.ks = a.ks + tok;
        r.vs = a.vs + tok;
    }
    return r;
}

// int8 x 16 (one 16-byte word) -> two fp16 x 8 operands, exactly. After the XOR a
// byte holds u = b + 128; a byte permute puts each u under the exponent byte 0x64,
// which reads as the fp16 1024 + u, and subtracting 1152 leaves b. Five
// instructions per 4 values.
__device__ __forceinline__ void int8x16_to_f16(i32x4 w, f16x8 &lo, f16x8 &hi) {
    const f16x2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t u = (uint32_t)w[j] ^ 0x80808080u;
        const f16x2 a = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias;
        const f16x2 c = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias;
        f16x8 &dst = j < 2 ? lo : hi;
        const int e = 4 * (j & 1);
        dst[e] = a[0];
        dst[e + 1] = a[1];
        dst[e + 2] = c[0];
        dst[e + 3] = c[1];
    }
}

// A 16-byte load of the streamed cache; NT marks it non-temporal (read once: a
// contiguous cache is not re-read within a step, and keeping it out of the caches
// measured faster there).
template <bool NT>
__device__ __forceinline__ i32x4 load_stream(const i32x4 *p) {
    return NT ? __builtin_nontemporal_load(p) : *p;
}

// One 64-key block in registers: the operands of both matrix products and,
// per lane, the K and V scale of key 16 grp + col (the 16 lanes of a group
// hold the 16 scales of its page, handed around with shuffles).
template <int D>
struct DecodeBlock {
    i32x4 k[4][D / 64];
    i32x4 v[D / 16];
    float ks, vs;
    bool live;
};

// A wave's running state over its keys: max (log2 units), row sum, the value
// normalizer s_run and the accumulator in units of s_run.
template <int D>
struct DecodeRun {
    float m_run, l_run, s_run, inv_s;
    f32x4 acc[D / 16];
};

// 8-byte elements of one workgroup's part in the workspace: the output in
// [element][lane] order, then (max, sum).
template <int D>
struct DecodeSlot {
    static constexpr int O = 2 * (D / 16);
    static constexpr int ELEMS = (O + 1) * kWave;
};

template <int D>
__device__ __forceinline__ void reset_run(DecodeRun<D> &r) {
    r.m_run = -INFINITY;
    r.l_run = 0.0f;
    r.s_run = 0.0f;
    r.inv_s = 0.0f;
#pragma unroll
    for (int d = 0; d < D / 16; ++d) r.acc[d] = f32x4{};
}

// Block-table entries of the block at key kb, read one block ahead of the
// block's data so that the data loads never wait on a table load: lane l holds
// entry l % 4 of the block's 4 pages, handed to the lanes that need it.
template <bool PAGED>
__device__ __forceinline__ int fetch_pages(const DecodeArgs &a, int b, int kb, int n_pages, int lane) {
    return table_page<PAGED>(a, b, kb / kPage + (lane & 3), n_pages);
}

// Issues the loads of the block at key kb (pages: from fetch_pages).
template <int D, bool PAGED>
__device__ __forceinline__ void load_block(const DecodeArgs &a, int b, int kvh, int kb, int n_pages,
                                           int pages, int col, int grp, DecodeBlock<D> &x,
                                           bool &bad_page) {
    constexpr int KS = D / 64, DB = D / 16;
    const int page0 = kb / kPage;
    // K rows for the score instruction: row m = col of block t is key
    // 16 (m / 4) + 4t + (m % 4), in page m / 4.
    const PageRef kp = page_ref<D, PAGED>(a, b, kvh, page0 + (col >> 2), n_pages,
                                          PAGED ? __shfl(pages, col >> 2) : 0);
    // This lane group's page for scales, P and V.
    const PageRef gp = page_ref<D, PAGED>(a, b, kvh, page0 + grp, n_pages,
                                          PAGED ? __shfl(pages, grp) : 0);
    bad_page |= !gp.ok;
    x.live = gp.live;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int s = 0; s < KS; ++s)
            x.k[t][s] = load_stream<!PAGED>(reinterpret_cast<const i32x4 *>(
                kp.k + (4 * t + (col & 3)) * D + 64 * s + 16 * grp));
#pragma unroll
    for (int d = 0; d < DB; ++d)
        x.v[d] = load_stream<!PAGED>(reinterpret_cast<const i32x4 *>(gp.vt + (16 * d + col) * kPage));
    x.ks = gp.ks[col];
    x.vs = gp.vs[col];
}

// Scores, online softmax and P.V of one block for keys [lo, k_end).
template <int D>
__device__ __forceinline__ void block_math(const DecodeBlock<D> &cur, int kb, int lo, int k_end,
                                           const i32x4 (&qop)[D / 64], float c, int lane,
                                           DecodeRun<D> &st) {
    constexpr int KS = D / 64, DB = D / 16;
    const int grp = lane >> 4;
    const auto &kop = cur.k;
    const auto &vop = cur.v;
    const int row0 = lane & ~15;  // first lane of this lane group
    float ksc[16], vsc[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        ksc[r] = __shfl(cur.ks, row0 + r);
        vsc[r] = __shfl(cur.vs, row0 + r);
    }
    const bool live_g = cur.live;

    float x[16];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        i32x4 s = {0, 0, 0, 0};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) s = mfma_16x16x64_i8(kop[t][ks], qop[ks], s);
#pragma unroll
        for (int i = 0; i < 4; ++i) x[4 * t + i] = (float)s[i] * (c * ksc[4 * t + i]);
    }
    // Blocks wholly inside [lo, k_end) on live pages skip the masks. In the
    // others, keys outside or on a dead page take no part: score -inf and
    // value scale 0 (the cache past a sequence's end may hold anything).
    const bool full = kb >= lo && kb + kBlockKeys <= k_end && __all(live_g);
    float vv[16];
    if (full) {
#pragma unroll
        for (int r = 0; r < 16; ++r) vv[r] = vsc[r];
    } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = kb + 16 * grp + r;
            const bool vis = key >= lo && key < k_end && live_g;
            if (!vis) x[r] = -INFINITY;
            vv[r] = vis ? vsc[r] : 0.0f;
        }
    }
    float mt = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    float vmax = fmaxf(fmaxf(vv[0], vv[1]), fmaxf(vv[2], vv[3]));
#pragma unroll
    for (int r = 4; r < 16; r += 2) {
        mt = fmaxf(mt, fmaxf(x[r], x[r + 1]));
        vmax = fmaxf(vmax, fmaxf(vv[r], vv[r + 1]));
    }
    mt = fmaxf(mt, __shfl_xor(mt, 16));
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    vmax = fmaxf(vmax, __shfl_xor(vmax, 16));
    vmax = fmaxf(vmax, __shfl_xor(vmax, 32));

    // Lazy rescale: the running max moves only when a head's block max exceeds
    // it by more than 2^8, and the value normalizer s_run (values accumulate in
    // units of s_run, the largest value scale so far) only when a value scale
    // exceeds it 16-fold, so p * v_scale / s_run stays below 2^12 in fp16.
    if (__any(mt > st.m_run + 8.0f || vmax > st.s_run * 16.0f)) {
        const float m_new = fmaxf(st.m_run, mt);
        const float s_new = fmaxf(st.s_run, vmax);
        const float alpha = st.m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(st.m_run - m_new);
        const float alpha_o = s_new > 0.0f ? alpha * (st.s_run / s_new) : alpha;
        st.inv_s = s_new > 0.0f ? 1.0f / s_new : 0.0f;
        st.m_run = m_new;
        st.s_run = s_new;
        st.l_run *= alpha;
#pragma unroll
        for (int d = 0; d < DB; ++d) st.acc[d] *= alpha_o;
    }
    const float m_use = st.m_run == -INFINITY ? 0.0f : st.m_run;

    // P operand: lane group g's keys 16g + 8h + e for the two halves h.
    f16x8 pop[2];
    float lp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(x[r] - m_use);
        lp[r & 3] += p;
        pop[r >> 3][r & 7] = (_Float16)(p * (vv[r] * st.inv_s));
    }
    st.l_run += (lp[0] + lp[1]) + (lp[2] + lp[3]);
    // out^T = V^T . P^T: the output column is the head (lane % 16), the lane
    // that owns the head's running max, so the rescale above is per lane.
#pragma unroll
    for (int d = 0; d < DB; ++d) {
        f16x8 v0, v1;
        int8x16_to_f16(vop[d], v0, v1);
        st.acc[d] = mfma_16x16x32_f16(v0, pop[0], st.acc[d]);
        st.acc[d] = mfma_16x16x32_f16(v1, pop[1], st.acc[d]);
    }
}

// The q^T operand of query head `head` of sequence b (zeros for dead heads) and
// its log2-domain score factor.
template <int D>
__device__ __forceinline__ float load_query(const DecodeArgs &a, int b, int head, bool head_ok,
                                            int grp, i32x4 (&qop)[D / 64]) {
    const int8_t *qrow = a.q + ((int64_t)b * a.q_heads + (head_ok ? head : 0)) * D;
#pragma unroll
    for (int s = 0; s < D / 64; ++s)
        qop[s] = head_ok ? *reinterpret_cast<const i32x4 *>(qrow + 64 * s + 16 * grp)
                         : i32x4{0, 0, 0, 0};
    float cq = 0.0f;
    if (head_ok) {
        cq = a.q_gran == REEF_SCALE_PER_TENSOR ? a.qs[0]
             : a.q_gran == REEF_SCALE_PER_HEAD ? a.qs[head]
                                                : a.qs[(int64_t)b * a.q_heads + head];
    }
    return cq * a.score_scale;
}

// Keys [k_begin, k_end) of (sequence b, kv head kvh) in steps of k_step, the next
// block's loads (and the table entries of the one after) issued before the
// current block is computed.
template <int D, bool PAGED>
__device__ __forceinline__ void run_keys(const DecodeArgs &a, int b, int kvh, int lo, int k_begin,
                                         int k_end, int k_step, int n_pages,
                                         const i32x4 (&qop)[D / 64], float c, int lane,
                                         DecodeRun<D> &st, bool &bad_page) {
    const int col = lane & 15, grp = lane >> 4;
    DecodeBlock<D> cur, nxt;
    if (k_begin < k_end)
        load_block<D, PAGED>(a, b, kvh, k_begin, n_pages,
                             fetch_pages<PAGED>(a, b, k_begin, n_pages, lane), col, grp, cur,
                             bad_page);
    int pg_next = fetch_pages<PAGED>(a, b, k_begin + k_step, n_pages, lane);
    for (int kb = k_begin; kb < k_end; kb += k_step) {
        const bool more = kb + k_step < k_end;
        const int pg_after = fetch_pages<PAGED>(a, b, kb + 2 * k_step, n_pages, lane);
        if (more) load_block<D, PAGED>(a, b, kvh, kb + k_step, n_pages, pg_next, col, grp, nxt, bad_page);
        pg_next = pg_after;
        block_math<D>(cur, kb, lo, k_end, qop, c, lane, st);
        if (more) cur = nxt;
    }
}

template <int D, bool PAGED>
__global__ __launch_bounds__(kDecodeWaves * 64, 2) void decode_kernel(DecodeArgs a, float *out) {
    constexpr int DB = D / 16;   // 16-wide output blocks
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int split = blockIdx.x * kDecodeWaves + wave;
    const int kvh = blockIdx.y, b = blockIdx.z;
    // Every wave reaches the workgroup merge below, so none returns early; a wave
    // past the last split, or whose split holds no keys, contributes nothing.
    const bool in_range = split < a.splits;

    const int head = kvh * a.group + col;   // this lane's query head (live if col < group)
    const bool head_ok = col < a.group;

    int len = a.context_lens ? a.context_lens[b] : a.max_context;
    if (len < 1 || len > a.max_context) {
        if (split == 0 && lane == 0) flag_status(a.status, REEF_STATUS_BIT_BAD_LENGTH);
        len = 0;
    }
    const int lo = a.window > 0 ? max(0, len - a.window) : 0;
    // Split s takes the 64-key blocks first + s, first + s + splits, ...: at any
    // moment the splits of a sequence read neighbouring blocks, which keeps the
    // DRAM accesses of the waves running together close.
    const int k_step = a.splits * kBlockKeys;
    const int k_begin = (lo / kBlockKeys + split) * kBlockKeys;
    const int k_end = in_range ? len : 0;
    const int n_pages = (len + kPage - 1) / kPage;

    i32x4 qop[D / 64];
    const float c = load_query<D>(a, b, head, head_ok, grp, qop);
    DecodeRun<D> st;
    reset_run<D>(st);
    bool bad_page = false;
    run_keys<D, PAGED>(a, b, kvh, lo, k_begin, k_end, k_step, n_pages, qop, c, lane, st, bad_page);
    float m_run = st.m_run, l_run = st.l_run, s_run = st.s_run;
    f32x4 acc[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) acc[d] = st.acc[d];
    if (bad_page) flag_status(a.status, REEF_STATUS_BIT_BAD_PAGE);

    // Row sums: this lane holds head col's partial over its 16 keys per block.
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);

    // The workgroup's 4 splits merge in LDS (log-sum-exp) into one part. Waves 1..3
    // hand over (max, sum, accumulator in value units) in a lane-linear layout;
    // wave 0 merges.
    __shared__ f32x4 sO[kDecodeWaves - 1][DB][kWave];
    __shared__ float2 sML[kDecodeWaves - 1][kWave];
    if (wave > 0) {
#pragma unroll
        for (int d = 0; d < DB; ++d) sO[wave - 1][d][lane] = acc[d] * s_run;
        sML[wave - 1][lane] = float2{m_run, l_run};
    }
    __syncthreads();
    if (wave > 0) return;
    float mw[kDecodeWaves], lw[kDecodeWaves];
    mw[0] = m_run;
    lw[0] = l_run;
#pragma unroll
    for (int w = 1; w < kDecodeWaves; ++w) {
        const float2 x = sML[w - 1][lane];
        mw[w] = x.x;
        lw[w] = x.y;
    }
    float m = mw[0];
#pragma unroll
    for (int w = 1; w < kDecodeWaves; ++w) m = fmaxf(m, mw[w]);
    float e[kDecodeWaves], l = 0.0f;
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) {
        e[w] = mw[w] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw[w] - m);
        l += lw[w] * e[w];
    }
    // acc[d][i] is (channel 16 d + 4 grp + i, head col): this part's output in
    // absolute value units.
    f32x4 o[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) {
        o[d] = acc[d] * (s_run * e[0]);
#pragma unroll
        for (int w = 1; w < kDecodeWaves; ++w) o[d] += sO[w - 1][d][lane] * e[w];
    }

    // With more than one workgroup per (sequence, kv head), every part writes
    // (max, sum, output) to its workspace slot with device-coherent atomic stores,
    // releases them at agent scope and counts itself in on the item's counter (an
    // acquire-release increment); the last part acquires at agent scope, merges
    // the slots in part order (its own from registers, explicit fused
    // multiply-adds: the same result whichever part finishes last), stores the
    // output and resets the counter. No second kernel combines splits.
    const int parts = a.groups;
    bool store = parts == 1;
    if (parts > 1) {
        const int item = b * a.kv_heads + kvh;
        const int self = blockIdx.x;
        uint64_t *slots = reinterpret_cast<uint64_t *>(a.slots) +
                          (int64_t)item * parts * DecodeSlot<D>::ELEMS;
        uint64_t *so = slots + (int64_t)self * DecodeSlot<D>::ELEMS;
        auto pack = [](float x0, float x1) {
            return (uint64_t)__float_as_uint(x0) | ((uint64_t)__float_as_uint(x1) << 32);
        };
#pragma unroll
        for (int d = 0; d < DB; ++d) {
            __hip_atomic_store(so + (2 * d) * kWave + lane, pack(o[d][0], o[d][1]),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(so + (2 * d + 1) * kWave + lane, pack(o[d][2], o[d][3]),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __hip_atomic_store(so + DecodeSlot<D>::O * kWave + lane, pack(m, l), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");  // the slot before the count
        uint32_t ticket = 0;
        if (lane == 0)
            ticket = __hip_atomic_fetch_add(a.counters + item, 1u, __ATOMIC_ACQ_REL,
                                            __HIP_MEMORY_SCOPE_AGENT);
        ticket = __shfl(ticket, 0);
        if (ticket != (uint32_t)(parts - 1)) return;
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");  // the other parts' slots
        if (lane == 0)
            __hip_atomic_store(a.counters + item, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        auto get = [](const uint64_t *q) {
            return __hip_atomic_load(const_cast<uint64_t *>(q), __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
        };
        auto lo32 = [](uint64_t v) { return __uint_as_float((uint32_t)v); };
        auto hi32 = [](uint64_t v) { return __uint_as_float((uint32_t)(v >> 32)); };
        float mt = m;
        for (int p = 0; p < parts; ++p)
            if (p != self)
                mt = fmaxf(mt, lo32(get(slots + (int64_t)p * DecodeSlot<D>::ELEMS +
                                        DecodeSlot<D>::O * kWave + lane)));
        float lt = 0.0f;
        f32x4 tot[DB];
#pragma unroll
        for (int d = 0; d < DB; ++d) tot[d] = f32x4{};
        for (int p = 0; p < parts; ++p) {
            float mp, lp;
            f32x4 op[DB];
            if (p == self) {
                mp = m;
                lp = l;
#pragma unroll
                for (int d = 0; d < DB; ++d) op[d] = o[d];
            } else {
                const uint64_t *sl = slots + (int64_t)p * DecodeSlot<D>::ELEMS;
                const uint64_t ml = get(sl + DecodeSlot<D>::O * kWave + lane);
                mp = lo32(ml);
                lp = hi32(ml);
#pragma unroll
                for (int d = 0; d < DB; ++d) {
                    const uint64_t v0 = get(sl + (2 * d) * kWave + lane);
                    const uint64_t v1 = get(sl + (2 * d + 1) * kWave + lane);
                    op[d] = f32x4{lo32(v0), hi32(v0), lo32(v1), hi32(v1)};
                }
            }
            const float wp = mp == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mp - mt);
            lt = __builtin_fmaf(wp, lp, lt);
#pragma unroll
            for (int d = 0; d < DB; ++d)
#pragma unroll
                for (int i = 0; i < 4; ++i) tot[d][i] = __builtin_fmaf(wp, op[d][i], tot[d][i]);
        }
#pragma unroll
        for (int d = 0; d < DB; ++d) o[d] = tot[d];
        l = lt;
        store = true;
    }
    // A sequence with no keys (a bad length) ends with l = 0 and stores zeros.
    if (store && head_ok) {
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        float *orow = out + ((int64_t)b * a.q_heads + head) * D;
#pragma unroll
        for (int d = 0; d < DB; ++d) *reinterpret_cast<f32x4 *>(orow + 16 * d + 4 * grp) = o[d] * inv;
    }
}

__global__ void pack_v_pages(const int8_t *__restrict__ v_tokens, int64_t pages, int32_t dim,
                             int8_t *__restrict__ v_pages) {
    // One thread per (page, channel): gathers 16 bytes with stride dim.
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= pages * dim) return;
    const int64_t page = i / dim;
    const int d = (int)(i % dim);
    const int8_t *src = v_tokens + page * kPage * dim + d;
    int8_t buf[kPage];
#pragma unroll
    for (int t = 0; t < kPage; ++t) buf[t] = src[(int64_t)t * dim];
    *reinterpret_cast<i32x4 *>(v_pages + (page * dim + d) * kPage) =
        *reinterpret_cast<const i32x4 *>(buf);
}

int default_splits(const reef_decode_params *p) {
    if (p->num_splits > 0) return p->num_splits;
    const int64_t blocks = ceil_div(p->max_context, kBlockKeys);
    const int64_t pairs = p->batch * p->kv_heads;
    // About 1024 waves (4 per compute unit) with 16 KB of cache in flight each
    // keep HBM busy; more add per-split start-up and merge work. At least one
    // full workgroup (4 splits) per sequence, at least 4 blocks (256 keys) per
    // split. Measured on MI355X, 128 x 8q/1kv ragged paged: 43 us at 8 splits,
    // 45 us at 16; 4 x 8kv x 32768: 53 us at 32, 61 us at 64.
    int64_t s = std::max<int64_t>(kDecodeWaves, ceil_div(1024, pairs));
    s = std::min<int64_t>(s, ceil_div(blocks, 4));
    return (int)std::max<int64_t>(1, s);
}

reef_status validate_params(const reef_decode_params *p, const int8_t *q, const float *q_scales,
                            float *out) {
    if (!p || !q || !q_scales || !out) return REEF_INVALID_ARGUMENT;
    if (p->batch <= 0 || p->q_heads <= 0 || p->kv_heads <= 0 || p->max_context <= 0 ||
        p->q_heads % p->kv_heads != 0 || p->window < 0 || p->num_splits < 0 ||
        p->max_context % kPage != 0 || !std::isfinite(p->softmax_scale) ||
        (p->q_granularity != REEF_SCALE_PER_TENSOR && p->q_granularity != REEF_SCALE_PER_HEAD &&
         p->q_granularity != REEF_SCALE_PER_TOKEN))
        return REEF_INVALID_ARGUMENT;
    if (p->head_dim != 64 && p->head_dim != 128) return REEF_UNSUPPORTED;
    if (p->q_heads / p->kv_heads > 16 || p->kv_heads > 65535 || p->batch > 65535 ||
        p->max_context >= (int64_t(1) << 30))
        return REEF_UNSUPPORTED;
    if (!aligned(q, 16) || !aligned(out, 4)) return REEF_INVALID_ARGUMENT;
    return REEF_OK;
}

reef_status validate(const reef_decode_params *p, const int8_t *q, const float *q_scales,
                     float *out, void *workspace, size_t workspace_bytes) {
    const reef_status st = validate_params(p, q, q_scales, out);
    if (st != REEF_OK) return st;
    if (!workspace || !aligned(workspace, 16) ||
        workspace_bytes < reef_attention_decode_workspace_bytes(p))
        return REEF_INVALID_ARGUMENT;
    return REEF_OK;
}

// Workspace: one counter per (sequence, kv head), then, with more than one
// workgroup (4 splits) per sequence, one part slot per workgroup.
int64_t counter_bytes(const reef_decode_params *p) {
    return ceil_div(p->batch * p->kv_heads * 4, 256) * 256;
}

int64_t workspace_bytes(const reef_decode_params *p) {
    const int64_t groups = ceil_div(default_splits(p), kDecodeWaves);
    const int64_t slot = (p->head_dim == 128 ? DecodeSlot<128>::ELEMS : DecodeSlot<64>::ELEMS) * 8;
    return counter_bytes(p) + (groups > 1 ? p->batch * p->kv_heads * groups * slot : 0);
}

template <bool PAGED>
reef_status launch_decode(const reef_decode_params *p, DecodeArgs &a, float *out, void *workspace,
                          hipStream_t stream) {
    a.batch = (int32_t)p->batch;
    a.q_heads = (int32_t)p->q_heads;
    a.kv_heads = (int32_t)p->kv_heads;
    a.group = (int32_t)(p->q_heads / p->kv_heads);
    a.max_context = (int32_t)p->max_context;
    a.window = (int32_t)std::min<int64_t>(p->window, INT32_MAX);
    a.q_gran = p->q_granularity;
    a.score_scale = p->softmax_scale * kLog2e;
    const int splits = default_splits(p);
    a.splits = splits;
    a.groups = (int32_t)ceil_div(splits, kDecodeWaves);
    a.counters = static_cast<uint32_t *>(workspace);
    a.slots = reinterpret_cast<float *>(static_cast<char *>(workspace) + counter_bytes(p));
    const dim3 grid((unsigned)a.groups, (unsigned)p->kv_heads, (unsigned)p->batch);
    if (p->head_dim == 128)
        hipLaunchKernelGGL((decode_kernel<128, PAGED>), grid, dim3(64 * kDecodeWaves), 0, stream, a,
                           out);
    else
        hipLaunchKernelGGL((decode_kernel<64, PAGED>), grid, dim3(64 * kDecodeWaves), 0, stream, a,
                           out);
    return launch_status();
}

}  // namespace
}  // namespace reef

using namespace reef;

extern "C" size_t reef_attention_decode_workspace_bytes(const reef_decode_params *p) {
    if (!p || p->batch <= 0 || p->q_heads <= 0 || p->kv_heads <= 0 || p->head_dim <= 0 ||
        p->max_context <= 0)
        return 0;
    return (size_t)workspace_bytes(p);
}

extern "C" reef_status reef_attention_decode_int8(const reef_decode_params *p, const int8_t *q,
                                                  const float *q_scales, const int8_t *k_cache,
                                                  const int8_t *v_cache, const float *k_scales,
                                                  const float *v_scales,
                                                  const int32_t *context_lens, float *out,
                                                  void *workspace, size_t workspace_bytes,
                                                  uint32_t *status_word, hipStream_t stream) {
    reef_status st = validate(p, q, q_scales, out, workspace, workspace_bytes);
    if (st != REEF_OK) return st;
    if (!k_cache || !v_cache || !k_scales || !v_scales || !aligned(k_cache, 16) ||
        !aligned(v_cache, 16) || !aligned(k_scales, 16) || !aligned(v_scales, 16))
        return REEF_INVALID_ARGUMENT;
    DecodeArgs a = {};
    a.q = q;
    a.qs = q_scales;
    a.k = k_cache;
    a.v = v_cache;
    a.ks = k_scales;
    a.vs = v_scales;
    a.context_lens = context_lens;
    a.status = status_word;
    return launch_decode<false>(p, a, out, workspace, stream);
}

namespace reef {
namespace {

// The allocation-free paged decode keeps its workspace (counters and part slots)
// in this file-scope array: one copy per GPU, held until the process ends, shared
// by every call on that GPU. In host code `scratch` is a stand-in symbol, not a
// device address: scratch_address() resolves the device address once per device
// (with that device current) and every use goes through it.
constexpr int64_t kScratchBytes = int64_t(8) << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
void *scratch_ptr[kMaxDevices];

void *scratch_address() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(scratch_mutex);
    if (!scratch_ptr[dev]) {
        void *ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
        scratch_ptr[dev] = ptr;
    }
    return scratch_ptr[dev];
}

__global__ void clear_words(uint32_t *words, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        words[i] = 0;
}

}  // namespace
}  // namespace reef

extern "C" reef_status reef_attention_decode_int8_paged(
    const reef_decode_params *p, const int8_t *q, const float *q_scales, const int8_t *k_pages,
    const int8_t *v_pages, const float *k_scale_pages, const float *v_scale_pages,
    const int32_t *block_table, int64_t max_blocks_per_seq, int64_t num_pages,
    const int32_t *context_lens, float *out, void *workspace, size_t workspace_bytes,
    uint32_t *status_word, hipStream_t stream) {
    reef_status st = validate(p, q, q_scales, out, workspace, workspace_bytes);
    if (st != REEF_OK) return st;
    if (!k_pages || !v_pages || !k_scale_pages || !v_scale_pages || !block_table ||
        !context_lens || num_pages <= 0 || num_pages >= (int64_t(1) << 31) ||
        max_blocks_per_seq * kPage < p->max_context || max_blocks_per_seq >= (int64_t(1) << 30) ||
        !aligned(k_pages, 16) || !aligned(v_pages, 16) || !aligned(k_scale_pages, 16) ||
        !aligned(v_scale_pages, 16))
        return REEF_INVALID_ARGUMENT;
    DecodeArgs a = {};
    a.q = q;
    a.qs = q_scales;
    a.k = k_pages;
    a.v = v_pages;
    a.ks = k_scale_pages;
    a.vs = v_scale_pages;
    a.block_table = block_table;
    a.context_lens = context_lens;
    a.status = status_word;
    a.max_blocks = (int32_t)max_blocks_per_seq;
    a.num_pages = (int32_t)num_pages;
    return launch_decode<true>(p, a, out, workspace, stream);
}

extern "C" reef_status reef_attention_decode_int8_paged_noalloc(
    const reef_decode_params *p, const int8_t *q, const float *q_scales, const int8_t *k_pages,
    const int8_t *v_pages, const float *k_scale_pages, const float *v_scale_pages,
    const int32_t *block_table, int64_t max_blocks_per_seq, int64_t num_pages,
    const int32_t *context_lens, float *out, uint32_t *status_word, hipStream_t stream) {
    // Shapes and pointers are checked before the scratch address is looked up.
    const reef_status st = validate_params(p, q, q_scales, out);
    if (st != REEF_OK) return st;
    const int64_t need = workspace_bytes(p);
    if (need > kScratchBytes) return REEF_UNSUPPORTED;  // beyond the fixed scratch array
    void *ws = scratch_address();
    if (!ws) return REEF_HIP_ERROR;
    // The counters must start at zero; a fill kernel (no memset node under graph
    // capture) clears them. The part slots are written before they are read.
    const int64_t words = counter_bytes(p) / 4;
    hipLaunchKernelGGL(clear_words, dim3((unsigned)std::min<int64_t>(ceil_div(words, 256), 1024)),
                       dim3(256), 0, stream, static_cast<uint32_t *>(ws), words);
    if (hipGetLastError() != hipSuccess) return REEF_HIP_ERROR;
    return reef_attention_decode_int8_paged(p, q, q_scales, k_pages, v_pages, k_scale_pages,
                                            v_scale_pages, block_table, max_blocks_per_seq,
                                            num_pages, context_lens, out, ws, (size_t)need,
                                            status_word, stream);
}

extern "C" reef_status reef_kv_pack_v_pages(const int8_t *v_tokens, int64_t pages,
                                            int64_t head_dim, int8_t *v_pages,
                                            hipStream_t stream) {
    if (!v_tokens || !v_pages || pages <= 0 || head_dim <= 0 || head_dim > 65536 ||
        !aligned(v_pages, 16))
        return REEF_INVALID_ARGUMENT;
    const int64_t n = pages * head_dim;
    hipLaunchKernelGGL(pack_v_pages, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, stream,
                       v_tokens, pages, (int32_t)head_dim, v_pages);
    return launch_status();
}
