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

constexpr int kDecodeWaves = 4;          // waves per workgroup
constexpr int kBlockKeys = 64;           // keys per inner step (4 pages)
constexpr int kPage = 16;                // tokens per page
constexpr int kPlanItems = 2048;         // items whose block offsets a workgroup plans in LDS
constexpr int kWgPerCu = 2;              // resident workgroups per compute unit (at most)

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
    int32_t max_context, window;
    int32_t items;  // batch * kv_heads: one (sequence, kv head) each
    int32_t wgs;    // workgroups of the launch
    int32_t flat;   // 1: the launch's keys are dealt out by 64-key blocks, 0: by items
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
    // it by more than 2^6, and the value normalizer s_run (values accumulate in
    // units of s_run / 2^8, s_run the largest value scale so far) only when a value
    // scale exceeds it 2-fold, so the weight p * v_scale * 2^8 / s_run stays below
    // 2^15 in fp16, and above its subnormals (hi and lo keep 11 bits each) wherever
    // its share of the row sum (of p itself) exceeds 2^-21.
    if (__any(mt > st.m_run + 6.0f || vmax > st.s_run * 2.0f)) {
        const float m_new = fmaxf(st.m_run, mt);
        const float s_new = fmaxf(st.s_run, vmax);
        const float alpha = st.m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(st.m_run - m_new);
        const float alpha_o = s_new > 0.0f ? alpha * (st.s_run / s_new) : alpha;
        st.inv_s = s_new > 0.0f ? 256.0f / s_new : 0.0f;
        st.m_run = m_new;
        st.s_run = s_new;
        st.l_run *= alpha;
#pragma unroll
        for (int d = 0; d < DB; ++d) st.acc[d] *= alpha_o;
    }
    const float m_use = st.m_run == -INFINITY ? 0.0f : st.m_run;

    // P operand: lane group g's keys 16g + 8h + e for the two halves h, each weight
    // p * v_scale / s_run split into an fp16 part and the fp16 of its remainder
    // (22 significant bits together: one fp16 alone moves an output by up to
    // 2^-12 of the values' magnitude, about 1e-3 for |v| ~ 4). The products run
    // on both; the row sum stays the fp32 sum of p.
    f16x8 pop[2], plo[2];
    float lp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(x[r] - m_use);
        lp[r & 3] += p;
        const float w = p * (vv[r] * st.inv_s);
        const _Float16 hi = (_Float16)w;
        pop[r >> 3][r & 7] = hi;
        plo[r >> 3][r & 7] = (_Float16)(w - (float)hi);
    }
    st.l_run += (lp[0] + lp[1]) + (lp[2] + lp[3]);
    // out^T = V^T . P^T: the output column is the head (lane % 16), the lane
    // that owns the head's running max, so the rescale above is per lane.
#pragma unroll
    for (int d = 0; d < DB; ++d) {
        f16x8 v0, v1;
        int8x16_to_f16(vop[d], v0, v1);
        st.acc[d] = mfma_16x16x32_f16(v0, pop[0], st.acc[d]);
        st.acc[d] = mfma_16x16x32_f16(v0, plo[0], st.acc[d]);
        st.acc[d] = mfma_16x16x32_f16(v1, pop[1], st.acc[d]);
        st.acc[d] = mfma_16x16x32_f16(v1, plo[1], st.acc[d]);
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
// current block is computed. The first block is loaded into `nxt` and copied,
// like every later one: the current block's registers are then always written
// by copies, never by loads still in flight, so computing it waits for nothing
// the next block's loads are doing.
template <int D, bool PAGED>
__device__ __forceinline__ void run_keys(const DecodeArgs &a, int b, int kvh, int lo, int k_begin,
                                         int k_end, int k_step, int n_pages,
                                         const i32x4 (&qop)[D / 64], float c, int lane,
                                         DecodeRun<D> &st, bool &bad_page) {
    const int col = lane & 15, grp = lane >> 4;
    DecodeBlock<D> cur, nxt;
    if (k_begin < k_end) {
        load_block<D, PAGED>(a, b, kvh, k_begin, n_pages,
                             fetch_pages<PAGED>(a, b, k_begin, n_pages, lane), col, grp, nxt,
                             bad_page);
        cur = nxt;
    }
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

// Keys of one item (sequence b = item / kv_heads): its length (0 if the length is
// out of range), the first visible key, and its 64-key blocks from the block that
// holds that key. An item with no keys still counts one block, so that some
// workgroup stores its (zero) output.
struct ItemKeys {
    int len, lo, first_block, blocks;
    bool bad;
};

__device__ __forceinline__ ItemKeys item_keys(const DecodeArgs &a, int item) {
    ItemKeys r;
    const int b = item / a.kv_heads;
    int len = a.context_lens ? a.context_lens[b] : a.max_context;
    r.bad = len < 1 || len > a.max_context;
    if (r.bad) len = 0;
    r.len = len;
    r.lo = a.window > 0 ? max(0, len - a.window) : 0;
    r.first_block = r.lo / kBlockKeys;
    r.blocks = len > 0 ? (len + kBlockKeys - 1) / kBlockKeys - r.first_block : 1;
    return r;
}

// sOff[i] = blocks of items 0 .. i-1, for i <= items (a workgroup-wide scan).
__device__ void plan_blocks(const DecodeArgs &a, int32_t *sOff, int32_t *sWave) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) sOff[0] = 0;
    int32_t run = 0;
    for (int base = 0; base < a.items; base += 64 * kDecodeWaves) {
        const int i = base + tid;
        int32_t x = i < a.items ? item_keys(a, i).blocks : 0;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int32_t y = __shfl_up(x, o);
            if (lane >= o) x += y;
        }
        if (lane == 63) sWave[wave] = x;
        __syncthreads();
        int32_t before = run;
        for (int w = 0; w < kDecodeWaves; ++w) {
            if (w < wave) before += sWave[w];
            run += sWave[w];
        }
        if (i < a.items) sOff[i + 1] = before + x;
        __syncthreads();
    }
}

// Workgroup g of G owns units [start(g), start(g + 1)) of the T units (64-key
// blocks of all items, or items), start(g) = g T / G; unit u lies in workgroup
// ((u + 1) G - 1) / T.
__device__ __forceinline__ int64_t wg_start(int64_t g, int64_t T, int64_t G) { return g * T / G; }
__device__ __forceinline__ int wg_of(int64_t u, int64_t T, int64_t G) {
    return (int)(((u + 1) * G - 1) / T);
}

// Log-sum-exp merge of the waves' (max, sum, output in absolute value units)
// through LDS, in wave order; the result is valid in wave 0. The caller places a
// barrier between this and the next use of sO / sML.
template <int D>
__device__ __forceinline__ void merge_waves(float &m, float &l, f32x4 (&o)[D / 16],
                                            f32x4 (*sO)[D / 16][kWave], float2 *sML, int wave,
                                            int lane) {
    constexpr int DB = D / 16;
#pragma unroll
    for (int d = 0; d < DB; ++d) sO[wave][d][lane] = o[d];
    sML[wave * kWave + lane] = float2{m, l};
    __syncthreads();
    if (wave != 0) return;
    float mw[kDecodeWaves], lw[kDecodeWaves];
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) {
        const float2 x = sML[w * kWave + lane];
        mw[w] = x.x;
        lw[w] = x.y;
    }
    float mt = mw[0];
#pragma unroll
    for (int w = 1; w < kDecodeWaves; ++w) mt = fmaxf(mt, mw[w]);
    float lt = 0.0f;
    f32x4 ot[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) ot[d] = f32x4{};
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) {
        const float e = mw[w] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw[w] - mt);
        lt = __builtin_fmaf(e, lw[w], lt);
#pragma unroll
        for (int d = 0; d < DB; ++d) {
            const f32x4 x = sO[w][d][lane];
#pragma unroll
            for (int i = 0; i < 4; ++i) ot[d][i] = __builtin_fmaf(e, x[i], ot[d][i]);
        }
    }
    m = mt;
    l = lt;
#pragma unroll
    for (int d = 0; d < DB; ++d) o[d] = ot[d];
}

// Balanced decode. The launch's work is the keys of all items (sequence, kv head)
// cut into 64-key blocks; each item counts at least one block. With at most
// kPlanItems items, every workgroup computes the prefix of the items' block counts
// (from the context lengths, in LDS) and takes an equal run of blocks, whatever
// the lengths; otherwise it takes an equal run of whole items. Within a run, each
// item's part is one segment: the 4 waves take its blocks in turn (wave w: blocks
// w, w + 4, ...), keep a flash-decoding running state and merge in LDS. An item
// inside one workgroup's run is stored directly. An item spread over several
// workgroups leaves one part per workgroup (the first or the last segment of a
// run) in the workspace; the last part to arrive merges them all. A paged launch
// places two workgroups on a compute unit, a contiguous one one (decode_wgs).
template <int D, bool PAGED>
__global__ __launch_bounds__(kDecodeWaves * 64, PAGED ? kWgPerCu : 1) void decode_kernel(
    DecodeArgs a, float *out) {
    constexpr int DB = D / 16;   // 16-wide output blocks
    __shared__ int32_t sOff[kPlanItems + 1];
    __shared__ int32_t sWave[kDecodeWaves];
    __shared__ f32x4 sO[kDecodeWaves][DB][kWave];
    __shared__ float2 sML[kDecodeWaves * kWave];
    __shared__ uint32_t sLast;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, grp = lane >> 4;
    const int g = blockIdx.x;
    const int64_t G = a.wgs;

    // Without context lengths every item holds max_context keys: the same block
    // count, so the prefix is i * nb and no plan is needed.
    const bool same = a.context_lens == nullptr;
    const int64_t nb = same ? item_keys(a, 0).blocks : 0;
    if (a.flat && !same) plan_blocks(a, sOff, sWave);
    // Values read from LDS arrive in vector registers; every one of them is uniform
    // over the workgroup, and moving them to scalar registers keeps the loop control
    // and the addresses scalar.
    const int64_t T = !a.flat ? a.items
                      : same  ? a.items * nb
                              : __builtin_amdgcn_readfirstlane(sOff[a.items]);
    auto unit_of = [&](int item) -> int64_t {
        return !a.flat ? item : same ? item * nb : __builtin_amdgcn_readfirstlane(sOff[item]);
    };
    const int64_t u0 = wg_start(g, T, G), u1 = wg_start(g + 1, T, G);
    if (u0 >= u1) return;  // no units for this workgroup (uniform)
    // First item of the run: the last item whose first unit is <= u0.
    int item = (int)(a.flat && same ? u0 / nb : u0);
    if (a.flat && !same) {
        int lo_i = 0, hi_i = a.items - 1;
        while (lo_i < hi_i) {
            const int mid = (lo_i + hi_i + 1) >> 1;
            if (sOff[mid] <= u0) lo_i = mid; else hi_i = mid - 1;
        }
        item = __builtin_amdgcn_readfirstlane(lo_i);
    }

    for (;;) {
        const int64_t p_begin = unit_of(item), p_end = unit_of(item + 1);
        ItemKeys ik = item_keys(a, item);
        // The item is the workgroup's: its length moves to a scalar register.
        ik.len = __builtin_amdgcn_readfirstlane(ik.len);
        ik.lo = __builtin_amdgcn_readfirstlane(ik.lo);
        ik.first_block = __builtin_amdgcn_readfirstlane(ik.first_block);
        ik.blocks = __builtin_amdgcn_readfirstlane(ik.blocks);
        const int b = item / a.kv_heads, kvh = item % a.kv_heads;
        // This segment's blocks of the item (local numbering).
        const int s_blk = a.flat ? (int)(max(u0, p_begin) - p_begin) : 0;
        const int e_blk = a.flat ? (int)(min(u1, p_end) - p_begin) : ik.blocks;
        if (ik.bad && s_blk == 0 && threadIdx.x == 0)
            flag_status(a.status, REEF_STATUS_BIT_BAD_LENGTH);

        const int head = kvh * a.group + col;   // this lane's query head (live if col < group)
        const bool head_ok = col < a.group;
        const int k_begin = (ik.first_block + s_blk + wave) * kBlockKeys;
        const int k_end = min(ik.len, (ik.first_block + e_blk) * kBlockKeys);
        const int n_pages = (ik.len + kPage - 1) / kPage;
        i32x4 qop[D / 64];
        const float c = load_query<D>(a, b, head, head_ok, grp, qop);
        DecodeRun<D> st;
        reset_run<D>(st);
        bool bad_page = false;
        run_keys<D, PAGED>(a, b, kvh, ik.lo, k_begin, k_end, kDecodeWaves * kBlockKeys, n_pages,
                           qop, c, lane, st, bad_page);
        if (bad_page) flag_status(a.status, REEF_STATUS_BIT_BAD_PAGE);
        // Row sums: this lane holds head col's partial over its 16 keys per block.
        float l = st.l_run;
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        float m = st.m_run;
        f32x4 o[DB];
#pragma unroll
        for (int d = 0; d < DB; ++d) o[d] = st.acc[d] * (st.s_run * (1.0f / 256.0f));
        merge_waves<D>(m, l, o, sO, sML, wave, lane);

        // Workgroups holding a part of this item: the non-empty ones in gf .. gl.
        // With T >= G every workgroup owns at least one unit; with fewer units than
        // workgroups each non-empty one owns exactly one.
        const int gf = a.flat ? wg_of(p_begin, T, G) : g;
        const int gl = a.flat ? wg_of(p_end - 1, T, G) : g;
        const int parts = T >= G ? gl - gf + 1 : (int)(p_end - p_begin);
        if (wave == 0) {
            if (parts == 1) {
                // A sequence with no keys (a bad length) ends with l = 0 and stores zeros.
                if (head_ok) {
                    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
                    float *orow = out + ((int64_t)b * a.q_heads + head) * D;
#pragma unroll
                    for (int d = 0; d < DB; ++d)
                        *reinterpret_cast<f32x4 *>(orow + 16 * d + 4 * grp) = o[d] * inv;
                }
            } else {
                // Part slot: 0 for the first segment of this run, 1 for the last. The
                // slots are written with agent-scope atomic stores (coherent at the
                // device level, beneath the per-XCD L2s), which have completed
                // (vmcnt 0) before the item's counter counts this part in; the part
                // that counts last reads the slots with agent-scope atomic loads
                // issued after its count returned. Every access to the shared data is
                // device-coherent, so no L2 write-back or invalidate is needed.
                const int slot = p_begin <= u0 ? 0 : 1;
                uint64_t *so = reinterpret_cast<uint64_t *>(a.slots) +
                               ((int64_t)g * 2 + slot) * DecodeSlot<D>::ELEMS;
                auto pack = [](float x0, float x1) {
                    return (uint64_t)__float_as_uint(x0) | ((uint64_t)__float_as_uint(x1) << 32);
                };
                if (head_ok) {
#pragma unroll
                    for (int d = 0; d < DB; ++d) {
                        part_store(so + (2 * d) * kWave + lane, pack(o[d][0], o[d][1]));
                        part_store(so + (2 * d + 1) * kWave + lane, pack(o[d][2], o[d][3]));
                    }
                    part_store(so + DecodeSlot<D>::O * kWave + lane, pack(m, l));
                }
                part_stores_done();
                uint32_t ticket = 0;
                if (lane == 0) ticket = part_count(a.counters + item);
                ticket = __shfl(ticket, 0);
                if (lane == 0) sLast = ticket == (uint32_t)(parts - 1) ? 1u : 0u;
            }
        }
        __syncthreads();  // frees sO / sML, publishes sLast
        if (parts > 1 && __builtin_amdgcn_readfirstlane(sLast)) {
            // Every wave merges the parts gf + wave, gf + wave + 4, ... in order, then
            // the waves merge in LDS: the same result whichever part arrived last.
            const int64_t first_start = wg_start(gf, T, G);
            float mp_run = -INFINITY, lp_run = 0.0f;
            f32x4 op_run[DB];
#pragma unroll
            for (int d = 0; d < DB; ++d) op_run[d] = f32x4{};
            auto get = [](const uint64_t *q) { return part_load(q); };
            auto lo32 = [](uint64_t v) { return __uint_as_float((uint32_t)v); };
            auto hi32 = [](uint64_t v) { return __uint_as_float((uint32_t)(v >> 32)); };
            part_claimed();
            if (head_ok) {
                for (int gg = gf + wave; gg <= gl; gg += kDecodeWaves) {
                    if (wg_start(gg, T, G) == wg_start(gg + 1, T, G)) continue;  // empty
                    const int slot = gg == gf && first_start < p_begin ? 1 : 0;
                    const uint64_t *sl = reinterpret_cast<const uint64_t *>(a.slots) +
                                         ((int64_t)gg * 2 + slot) * DecodeSlot<D>::ELEMS;
                    const uint64_t ml = get(sl + DecodeSlot<D>::O * kWave + lane);
                    f32x4 op[DB];
#pragma unroll
                    for (int d = 0; d < DB; ++d) {
                        const uint64_t v0 = get(sl + (2 * d) * kWave + lane);
                        const uint64_t v1 = get(sl + (2 * d + 1) * kWave + lane);
                        op[d] = f32x4{lo32(v0), hi32(v0), lo32(v1), hi32(v1)};
                    }
                    const float mp = lo32(ml), lp = hi32(ml);
                    const float mn = fmaxf(mp_run, mp);
                    const float er = mp_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mp_run - mn);
                    const float ep = mp == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mp - mn);
                    lp_run = __builtin_fmaf(ep, lp, lp_run * er);
#pragma unroll
                    for (int d = 0; d < DB; ++d)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            op_run[d][i] = __builtin_fmaf(ep, op[d][i], op_run[d][i] * er);
                    mp_run = mn;
                }
            }
            merge_waves<D>(mp_run, lp_run, op_run, sO, sML, wave, lane);
            if (wave == 0) {
                if (lane == 0) part_reset(a.counters + item);
                if (head_ok) {
                    const float inv = lp_run > 0.0f ? 1.0f / lp_run : 0.0f;
                    float *orow = out + ((int64_t)b * a.q_heads + head) * D;
#pragma unroll
                    for (int d = 0; d < DB; ++d)
                        *reinterpret_cast<f32x4 *>(orow + 16 * d + 4 * grp) = op_run[d] * inv;
                }
            }
            __syncthreads();  // frees sO / sML
        }
        if (p_end >= u1) break;
        ++item;
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

// Whether the launch deals out 64-key blocks (the items' prefix fits the LDS plan
// and the block count of the largest possible launch fits 31 bits).
bool flat_plan(const reef_decode_params *p) {
    const int64_t items = p->batch * p->kv_heads;
    return items <= kPlanItems && items * ceil_div(p->max_context, kBlockKeys) < (int64_t(1) << 31);
}

// Workgroups of the launch. A paged cache: two per compute unit (8 waves, each
// with 16 KB of cache in flight: the 2 KB pages scatter the loads, and the second
// workgroup's requests keep HBM busy). A contiguous cache streams at full bandwidth
// with one per compute unit (one wave per SIMD); a second one only adds an
// imbalance, its waves' loads being served behind the older workgroup's (its runs
// ended up to 20 % later), and one per unit measured 6 % faster at 64 x 8kv x 4096
// (the paged 128 x 8q/1kv ragged workload 2 % slower). Either way at most one per
// unit of work (a workgroup that takes several items in turn pays each item's
// start-up and merge latency once more: 128 one-block items took 66 us on 8
// workgroups, 8 us on 128). num_splits > 0 asks for that many waves per item on
// average instead.
int64_t decode_wgs(const reef_decode_params *p, bool paged) {
    const int64_t items = p->batch * p->kv_heads;
    const int64_t units = flat_plan(p) ? items * ceil_div(p->max_context, kBlockKeys) : items;
    const int64_t g = p->num_splits > 0 ? ceil_div(items * p->num_splits, kDecodeWaves)
                                        : (paged ? kWgPerCu : 1) * compute_units();
    return std::max<int64_t>(1, std::min<int64_t>(std::min(g, units), 1 << 20));
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
        p->batch * p->kv_heads > INT32_MAX ||
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

// Workspace: a fixed region of kPlanItems counters (one per (sequence, kv head);
// only a launch that deals out blocks, with at most kPlanItems items, counts
// parts), then, for such a launch, two part slots per workgroup (the first and
// the last segment of its run). Counter i sits at the same place whatever the
// shape of the call, and every launch leaves the counters it used at zero, so one
// zero-filled workspace serves calls of any shape; the slots are written before
// they are read.
constexpr int64_t kCounterBytes = kPlanItems * 4;

int64_t counter_bytes(const reef_decode_params *) { return kCounterBytes; }

int64_t workspace_bytes(const reef_decode_params *p) {
    const int64_t slot = (p->head_dim == 128 ? DecodeSlot<128>::ELEMS : DecodeSlot<64>::ELEMS) * 8;
    // Sized for the larger (paged) launch, so that one workspace serves both forms.
    return counter_bytes(p) + (flat_plan(p) ? decode_wgs(p, true) * 2 * slot : 0);
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
    a.items = (int32_t)(p->batch * p->kv_heads);
    a.flat = flat_plan(p) ? 1 : 0;
    a.wgs = (int32_t)decode_wgs(p, PAGED);
    a.counters = static_cast<uint32_t *>(workspace);
    a.slots = reinterpret_cast<float *>(static_cast<char *>(workspace) + counter_bytes(p));
    const dim3 grid((unsigned)a.wgs);
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
constexpr int64_t kScratchBytes = int64_t(16) << 20;
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
