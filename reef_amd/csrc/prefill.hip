// Prefill / general int8 flash attention for gfx950.
//
// Replaces the per-head loop of Attention::context (attention.hpp:374-432,
// attend_head :117-123 with causal_visibility :82-100) by one launch over every
// (batch, head, 128-query tile). Scores are exact int32 sums on the int8
// matrix cores (v_mfma_i32_32x32x32_i8), dequantized as float(acc) * (s_q * s_k)
// (the order of operator/linear.hpp:125-127) times softmax_scale, then an fp32
// online softmax; P.V runs on v_mfma_f32_32x32x16_f16 with P split into fp16 hi + lo
// parts (22 bits) and the int8 values converted exactly to fp16.
//
// Work layout (one workgroup = 4 waves = 128 query rows):
//   * each wave owns 32 query rows and computes S^T = K . Q^T, so a lane holds
//     one query (lane % 32) and 16 keys of every 32-key block: the row max and
//     row sum are in-lane plus one exchange with lane ^ 32, and the rescale of
//     the output accumulator is one multiplier per lane;
//   * K tiles (64 keys) are staged in LDS with their rows permuted so that
//     lane group g of the score output holds keys [16g, 16g + 16) of each 32-key
//     block in order; those registers are then directly the P operand of the
//     P.V instruction, whose value operand is a transposed fp16 V tile in LDS;
//   * tiles above the causal diagonal (or outside the window) are skipped, and
//     masking runs only on tiles that cross a boundary.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <type_traits>

#include "prefill_packed.hpp"

namespace reef {


namespace {

constexpr int kBM = 128;  // query rows per workgroup
constexpr int kBN = 64;   // keys per tile
constexpr int kThreads = 256;
constexpr int kXcds = 8;  // workgroup i of a launch runs on XCD i % 8

struct PrefillArgs {
    const int8_t *q, *k, *v;
    const float *qs, *ks, *vs;
    float *out;
    int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st, o_sb, o_sh, o_st;
    int32_t batch, q_heads, kv_heads, q_len, kv_len;
    int32_t query_start, window;
    float score_scale;  // softmax_scale * log2(e)
    int32_t q_gran, kv_gran;
    int32_t q_tiles;
    int32_t zigzag;  // pair heavy and light tiles in grids that fit at once
};

// Precision of P: these kernels always split P into fp16 hi + lo parts (22 bits).
// Choosing one fp16 P per item, for items whose dequantized values stay within
// kHiOnlyMax, cost more than it saved: the choice needs the item's value scale
// before its first tile, and a kernel holding both bodies allocates registers for
// the larger one (1x32x2048x128 balanced: 71.0 us against 66.4 with hi + lo
// everywhere), while real heads have values above 1 and take hi + lo anyway.

// Balanced schedule: the steps (item, key tile) of all items, items in (batch,
// head, query tile) order and each item's tiles in key order, are cut into G
// equal ranges, one per workgroup of the grid. An item that a range boundary
// cuts is computed in parts; every part leaves its (running max, row sum,
// unnormalized output) in a slot of the workspace, and the part that finishes
// last (an item counter says which) merges the slots in part order, so the
// result does not depend on the order the parts finish in.
struct StreamArgs {
    int64_t units;       // steps of all items
    int64_t per_head;    // steps of one (batch, head)
    uint32_t *counters;  // one per item; zero between launches (the merging part resets it)
    float *slots;        // 2 G partial results
};

// One part of an item in the balanced schedule.
struct StreamPart {
    int parts;      // parts of the item (1: the whole item, no merge)
    int slot;       // this part's slot
    int item;       // counter index
    int first_wg;   // logical workgroup of the item's first part
    int64_t item_u0;  // first step of the item
};

enum PrefillMode { kWhole = 0, kSplit = 1, kStream = 2, kSplitStream = 3 };

template <int D>
struct StreamSlot {  // floats of one partial result: output in lane order, then (max, sum)
    static constexpr int O_FLOATS = 4 * (D / 32) * 4 * kWave * 4;
    static constexpr int FLOATS = O_FLOATS + 4 * kWave * 2;
};

// Row m of a 32-row score block holds key sigma(m) = 16 ((m >> 2) & 1) +
// 4 (m >> 3) + (m & 3), so that output register r = 4j + i of lane group g is
// key 16g + r.
__device__ __forceinline__ int key_of_score_row(int m) {
    return 16 * ((m >> 2) & 1) + 4 * (m >> 3) + (m & 3);
}

// One 32 x 32 block of int32 scores S^T = K . Q^T over head_dim D. krow points at
// the K row of key sigma(lane % 32) (LDS or global); qop holds this lane's query
// row, 16 bytes per 32-wide reduction step. Shared by the flash kernel and the
// bit-exact score hook.
template <int D>
__device__ __forceinline__ i32x16 score_tile(const i32x4 (&qop)[D / 32], const int8_t *krow,
                                             int grp) {
    i32x16 s = {};
#pragma unroll
    for (int t = 0; t < D / 32; ++t) {
        const i32x4 kop = *reinterpret_cast<const i32x4 *>(krow + 32 * t + 16 * grp);
        s = mfma_32x32x32_i8(kop, qop[t], s);
    }
    return s;
}

template <int D>
__device__ __forceinline__ void load_q_operand(i32x4 (&qop)[D / 32], const int8_t *qrow, bool ok,
                                               int grp) {
#pragma unroll
    for (int t = 0; t < D / 32; ++t) {
        qop[t] = ok ? *reinterpret_cast<const i32x4 *>(qrow + 32 * t + 16 * grp) : i32x4{0, 0, 0, 0};
    }
}

__device__ __forceinline__ float scale_of(const float *s, int gran, int b, int h, int t, int heads,
                                          int tokens) {
    if (gran == REEF_SCALE_PER_TENSOR) return s[0];
    if (gran == REEF_SCALE_PER_HEAD) return s[h];
    return s[((int64_t)b * heads + h) * tokens + t];
}

// Two fp16 of keys (key0, key1) at one channel, packed [key0, key1], from the
// int8 byte `sel` of words w0 (key0) and w1 (key1): each half is one
// v_cvt_f16_i16 reading the sign-extended byte through a sub-dword operand
// select (exact: every int8 is an fp16 integer), the second write keeping the
// first half.
#define REEF_CVT_PAIR(SEL)                                                                     \
    asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_" #SEL \
        "\n\tv_cvt_f16_i16_sdwa %0, sext(%2) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE "        \
        "src0_sel:BYTE_" #SEL                                                                  \
        : "=&v"(r)                                                                             \
        : "v"(w0), "v"(w1))
__device__ __forceinline__ uint32_t int8_pair_to_f16(uint32_t w0, uint32_t w1, int sel) {
    uint32_t r;
    switch (sel) {  // a constant once the caller's loop is unrolled
    case 0: REEF_CVT_PAIR(0); break;
    case 1: REEF_CVT_PAIR(1); break;
    case 2: REEF_CVT_PAIR(2); break;
    default: REEF_CVT_PAIR(3); break;
    }
    return r;
}
#undef REEF_CVT_PAIR

__device__ __forceinline__ int floor_div(int a, int b) {  // b > 0
    return a >= 0 ? a / b : -((-a + b - 1) / b);
}

// Key tiles of query tile `tile`: the tiles from the one holding the first key
// any row of the tile sees through the one holding the last.
__device__ __forceinline__ int tile_steps(const PrefillArgs &a, int tile, int &kt_first) {
    const int q0 = tile * kBM;
    const int r_last = min(q0 + kBM, a.q_len) - 1;
    const int key_lo = a.window > 0 ? max(0, a.query_start + q0 + 1 - a.window) : 0;
    const int key_hi = min(a.query_start + r_last, a.kv_len - 1);
    kt_first = key_lo / kBN * kBN;
    return (key_hi - kt_first) / kBN + 1;
}

// Sum of tile_steps over the query tiles t < T, for T < q_tiles (every such tile
// is full). With query_start + q_len <= kv_len the last key of tile t is
// query_start + 128 t + 127, in tile 2 t + (query_start + 127) / 64; with a window
// the first is max(0, query_start + 128 t + 1 - window), in tile
// 2 t + floor((query_start + 1 - window) / 64) once t reaches t0.
__device__ __forceinline__ int64_t steps_before(const PrefillArgs &a, int T) {
    const int64_t t = T;
    int64_t s = t + t * (t - 1) + (int64_t)((a.query_start + 127) / 64) * t;
    if (a.window > 0) {
        const int t0 = max(0, floor_div(a.window - a.query_start - 1, kBM) + 1);
        if (T > t0)
            s -= (t - t0) * (t + t0 - 1) +
                 (int64_t)floor_div(a.query_start + 1 - a.window, kBN) * (t - t0);
    }
    return s;
}

// The balanced schedule visits a head's query tiles heaviest and lightest in
// turn: z = 0, 1, 2, 3, ... is tile Q - 1, 0, Q - 2, 1, ..., so that the steps
// of neighbouring tiles add up to about the same, and a workgroup's range holds
// one or two parts of items rather than several light items.
__device__ __forceinline__ int zigzag_tile(int q_tiles, int z) {
    return (z & 1) ? z >> 1 : q_tiles - 1 - (z >> 1);
}

// Steps of the first Z tiles of a head in that order (Z < q_tiles): the Z/2
// lightest and the Z - Z/2 heaviest.
__device__ __forceinline__ int64_t steps_before_zigzag(const PrefillArgs &a, int64_t per_head,
                                                       int Z) {
    if (Z == 0) return 0;
    return per_head - steps_before(a, a.q_tiles - (Z + 1) / 2) + steps_before(a, Z / 2);
}

// Work items are (query tile, batch x head), ranked heaviest first: the causal
// rows of the last tile see the most keys.
__device__ __forceinline__ void item_coords(const PrefillArgs &a, int rank, int &tile, int &b,
                                            int &h) {
    const int pairs = a.batch * a.q_heads;
    tile = a.q_tiles - 1 - rank / pairs;
    const int bh = rank % pairs;
    b = bh / a.q_heads;
    h = bh % a.q_heads;
}

// Rank of this workgroup's item in the one-item-per-workgroup kernel. With
// zig-zag on, the second half of the grid takes ranks in reverse, so that the
// two workgroups a compute unit receives in a grid that fits at once are a heavy
// and a light tile.
__device__ __forceinline__ int grid_rank(const PrefillArgs &a) {
    const int L = blockIdx.x, N = gridDim.x;
    if (!a.zigzag) return L;
    const int half = (N + 1) / 2;
    return L < half ? L : N - 1 - (L - half);
}

// LDS of one prefill workgroup: two stages (the tile being computed and the next
// one being filled) of a K tile and a transposed fp16 V tile.
template <int D>
struct PrefillLds {
    static constexpr int KSTRIDE = D + 16;        // bytes per K row
    static constexpr int VSTRIDE = kBN * 2 + 16;  // bytes per transposed-V row
    static constexpr int K_BYTES = kBN * KSTRIDE, V_BYTES = D * VSTRIDE;
    static constexpr int BYTES = 2 * (K_BYTES + V_BYTES);
};


// SPLIT: the workgroup is two groups of 4 waves over the same 128 query rows;
// group 0 takes the first half of the key tiles and group 1 the second half, each
// with its own LDS stages, and group 0 merges both partial results at the end.
// This halves the longest sequential chain of a workgroup, which balances causal
// grids that fit the GPU at once.
//
// MODE kWhole and kStream compute key tiles [c0, c1) of the item (kWhole: all of
// them); kStream parts of a cut item merge through the workspace (StreamArgs).
// kSplitStream: the two groups of SPLIT split the key tiles [c0, c1) of a kStream
// part, merge in LDS, and group 0 goes on as kStream (group 1 joins its barriers).
template <int D, bool KV_TOKEN, int MODE>
__device__ __forceinline__ void prefill_body(const PrefillArgs &a, int tile, int b, int h, int c0,
                                             int c1, int8_t *smem_all,
                                             float (*sScale)[KV_TOKEN ? 2 * kBN + 1 : 1],
                                             const StreamArgs &sa, const StreamPart &sp,
                                             uint32_t *sTicket) {
    constexpr bool SPLIT = MODE == kSplit || MODE == kSplitStream;
    constexpr bool STREAM = MODE == kStream || MODE == kSplitStream;
    static_assert(!SPLIT || !KV_TOKEN, "the split kernels have no per-token K/V scales");
    constexpr int KSTRIDE = PrefillLds<D>::KSTRIDE, VSTRIDE = PrefillLds<D>::VSTRIDE;
    constexpr int DB = D / 32;  // 32-wide output blocks
    constexpr int K_BYTES = PrefillLds<D>::K_BYTES, V_BYTES = PrefillLds<D>::V_BYTES;
    constexpr int KLOADS = kBN * D / 16 / kThreads;  // 16-byte K loads per thread
    constexpr int VBLOCKS = (kBN / 4) * (D / 8);     // 4-key x 8-channel V blocks
    constexpr float kLazy = 8.0f;  // rescale only when a row max grows by > 2^8
    // p = exp2(s - m_run + kShift): the row sums and the merges carry the same factor
    // 2^kShift, which cancels; it keeps a p of weight above 2^-21 of the row's
    // largest out of the fp16 subnormals (so hi and lo keep 11 bits each; below, each
    // p is off by at most 2^-25, under 2^-32 of the row sum), and every p below
    // 2^(kLazy + kShift) = 2^15.
    constexpr float kShift = 7.0f;

    const int tid = threadIdx.x & (kThreads - 1), lane = tid & 63;
    // The wave index is the same on every lane; saying so lets every per-wave
    // decision below be a scalar branch instead of predicated vector code.
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int group = SPLIT ? __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 8) : 0;
    int8_t *smem = smem_all + group * PrefillLds<D>::BYTES;
    const int col = lane & 31, grp = lane >> 5;
    const int kvh = h / (a.q_heads / a.kv_heads);
    const int q0 = tile * kBM;
    const int row = q0 + wave * 32 + col;
    const bool row_ok = row < a.q_len;

    // Visible keys of this lane's row: [lo, hi].
    const int pos = a.query_start + row;
    const int lo = a.window > 0 ? max(0, pos + 1 - a.window) : 0;
    const int hi = min(pos, a.kv_len - 1);
    // Of the workgroup and of the wave.
    const int r_last = min(q0 + kBM, a.q_len) - 1;
    const int key_lo = a.window > 0 ? max(0, a.query_start + q0 + 1 - a.window) : 0;
    const int key_hi = min(a.query_start + r_last, a.kv_len - 1);
    const int w_first = q0 + wave * 32;
    const int w_last = min(w_first + 31, a.q_len - 1);
    const bool wave_active = w_first < a.q_len;
    const int wk_lo = a.window > 0 ? max(0, a.query_start + w_first + 1 - a.window) : 0;
    const int wk_hi = min(a.query_start + w_last, a.kv_len - 1);
    // Keys every row of the wave sees.
    const int full_lo = a.window > 0 ? a.query_start + w_last + 1 - a.window : 0;
    const int full_hi = min(a.query_start + w_first, a.kv_len - 1);

    const int8_t *kbase = a.k + b * a.k_sb + kvh * a.k_sh;
    const int8_t *vbase = a.v + b * a.v_sb + kvh * a.v_sh;

    // ---- staging: global -> registers (next tile) -> LDS ----------------------------
    i32x4 kreg[KLOADS];
    uint2 vreg[4];
    float ks_reg = 0.0f, vs_reg = 0.0f;
    // This thread's V block (if tid < VBLOCKS): keys 4 vkg..+3, channels 8 vdg..+7. Key
    // groups vary fastest, so the 16 lanes storing one transposed row write 128
    // contiguous bytes (rows 8 channels apart would all hit the same banks).
    const int vkg = tid % (kBN / 4), vdg = tid / (kBN / 4);
    // Loads go through buffer resources over this (batch, kv head)'s rows. The tile
    // offset is added to the per-lane offset (the range check covers the per-lane
    // offset, not the scalar one), so keys past kv_len read zeros (every tile
    // reaching past kv_len is masked anyway; a zero scale never wins a maximum).
    const __amdgpu_buffer_rsrc_t krsrc =
        buffer_rsrc(kbase, (uint32_t)((int64_t)(a.kv_len - 1) * a.k_st + D));
    const __amdgpu_buffer_rsrc_t vrsrc =
        buffer_rsrc(vbase, (uint32_t)((int64_t)(a.kv_len - 1) * a.v_st + D));
    // K chunk j of this thread: LDS row krow[j] (rows are 144 bytes, so rows r and
    // r + 8 fill the 64 banks together; they share each 16-lane store group),
    // holding key kkey of the tile, bytes kch * 16.
    uint32_t koff[KLOADS];
    int kdst[KLOADS];
#pragma unroll
    for (int j = 0; j < KLOADS; ++j) {
        const int slot = (tid + j * kThreads) / (D / 16), kch = tid % (D / 16);
        const int row = (slot & ~9) | ((slot & 1) << 3) | ((slot >> 3) & 1);
        const int kkey = ((row >> 5) << 5) + key_of_score_row(row & 31);
        koff[j] = (uint32_t)(kkey * a.k_st + kch * 16);
        kdst[j] = row * KSTRIDE + kch * 16;
    }
    uint32_t voff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) voff[i] = (uint32_t)((4 * vkg + i) * a.v_st + 8 * vdg);
    const int64_t srow = ((int64_t)b * a.kv_heads + kvh) * a.kv_len;
    const __amdgpu_buffer_rsrc_t ksrsrc = buffer_rsrc(a.ks + srow, (uint32_t)a.kv_len * 4u);
    const __amdgpu_buffer_rsrc_t vsrsrc = buffer_rsrc(a.vs + srow, (uint32_t)a.kv_len * 4u);
    auto load_tile = [&](int kt) {
        const uint32_t ks_off = (uint32_t)__builtin_amdgcn_readfirstlane((int)(kt * a.k_st));
        const uint32_t vs_off = (uint32_t)__builtin_amdgcn_readfirstlane((int)(kt * a.v_st));
#pragma unroll
        for (int j = 0; j < KLOADS; ++j)
            kreg[j] = __builtin_amdgcn_raw_buffer_load_b128(krsrc, koff[j] + ks_off, 0, 0);
        if (tid < VBLOCKS) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const auto w = __builtin_amdgcn_raw_buffer_load_b64(vrsrc, voff[i] + vs_off, 0, 0);
                vreg[i] = uint2{w[0], w[1]};
            }
        }
        if (KV_TOKEN && wave == 0) {
            ks_reg = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(ksrsrc, (lane + kt) * 4, 0, 0));
            vs_reg = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(vsrsrc, (lane + kt) * 4, 0, 0));
        }
    };
    auto store_tile = [&](int buf) {
        int8_t *sK = smem + buf * (K_BYTES + V_BYTES);
        int8_t *sVT = sK + K_BYTES;
#pragma unroll
        for (int j = 0; j < KLOADS; ++j) *reinterpret_cast<i32x4 *>(sK + kdst[j]) = kreg[j];
        if (tid < VBLOCKS) {
            const uint32_t w[4][2] = {{vreg[0].x, vreg[0].y}, {vreg[1].x, vreg[1].y},
                                      {vreg[2].x, vreg[2].y}, {vreg[3].x, vreg[3].y}};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t k01 = int8_pair_to_f16(w[0][j >> 2], w[1][j >> 2], j & 3);
                const uint32_t k23 = int8_pair_to_f16(w[2][j >> 2], w[3][j >> 2], j & 3);
                *reinterpret_cast<uint2 *>(sVT + (8 * vdg + j) * VSTRIDE + 4 * vkg * 2) =
                    uint2{k01, k23};
            }
        }
        if (KV_TOKEN && wave == 0) {
            sScale[buf][lane] = ks_reg;
            sScale[buf][kBN + lane] = vs_reg;
            const float m = wave_max(vs_reg);
            if (lane == 0) sScale[buf][2 * kBN] = m;
        }
    };

    // The first tile, the query operand and the scales are independent loads:
    // all of them are in flight before anything waits for one.
    const int kt_first = key_lo / kBN * kBN;
    const int n_all = (key_hi - kt_first) / kBN + 1;
    // This group's tiles: [kt0, kt0 + n_tiles * kBN); both groups run n_iter steps.
    int n_iter, kt0, n_tiles;
    if (SPLIT) {
        const int s0 = MODE == kSplitStream ? c0 : 0;
        const int n_seg = (MODE == kSplitStream ? min(c1, n_all) : n_all) - s0;
        n_iter = (n_seg + 1) / 2;
        kt0 = kt_first + (s0 + (group ? n_iter : 0)) * kBN;
        n_tiles = group ? n_seg - n_iter : n_iter;
    } else {
        kt0 = kt_first + c0 * kBN;
        n_tiles = min(c1, n_all) - c0;
        n_iter = n_tiles;
    }
    if (n_tiles > 0) load_tile(kt0);
    i32x4 qop[D / 32];
    load_q_operand<D>(qop, a.q + b * a.q_sb + h * a.q_sh + (int64_t)(row_ok ? row : 0) * a.q_st,
                      row_ok, grp);
    const float cq = row_ok ? scale_of(a.qs, a.q_gran, b, h, row, a.q_heads, a.q_len) : 0.0f;
    const float ck = KV_TOKEN ? 1.0f : scale_of(a.ks, a.kv_gran, b, kvh, 0, a.kv_heads, a.kv_len);
    const float cv = KV_TOKEN ? 1.0f : scale_of(a.vs, a.kv_gran, b, kvh, 0, a.kv_heads, a.kv_len);
    // log2-domain score per unit of int32 accumulator
    const float c = cq * ck * a.score_scale;

    float m_run = -INFINITY, m_sh = -INFINITY, l_run = 0.0f, s_run = 0.0f, inv_s = 0.0f;
    f32x16 acc[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) acc[d] = f32x16{};

    // One tile of scores, online softmax and P.V for this wave's 32 rows.
    auto tile_math = [&](const int kt, const int buf, auto mask_tag) {  // wave-uniform
            const int8_t *sK = smem + buf * (K_BYTES + V_BYTES);
            constexpr bool need_mask = decltype(mask_tag)::value;
            const int8_t *sVT = sK + K_BYTES;
            i32x16 sc[2];
#pragma unroll
            for (int u = 0; u < 2; ++u)
                sc[u] = score_tile<D>(qop, sK + (32 * u + col) * KSTRIDE, grp);

            // Tile max of the log2-domain scores, masked keys excluded.
            float mt;
            float x[KV_TOKEN ? 32 : 1];
            if (KV_TOKEN) {
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int key = kt + 32 * u + 16 * grp + r;
                        float xv = (float)sc[u][r] * (c * sScale[buf][32 * u + 16 * grp + r]);
                        if constexpr (need_mask) {
                            if (key < lo || key > hi) xv = -INFINITY;
                        }
                        x[16 * u + r] = xv;
                    }
                mt = x[0];
#pragma unroll
                for (int r = 1; r < 32; ++r) mt = fmaxf(mt, x[r]);
            } else {
                if constexpr (need_mask) {
#pragma unroll
                    for (int u = 0; u < 2; ++u)
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int key = kt + 32 * u + 16 * grp + r;
                            if (key < lo || key > hi) sc[u][r] = INT32_MIN;
                        }
                }
                int mi = sc[0][0];
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int r = (u == 0 ? 1 : 0); r < 16; ++r) mi = max(mi, sc[u][r]);
                // c > 0, so the largest float score is c times the largest integer.
                mt = mi == INT32_MIN ? -INFINITY : (float)mi * c;
            }
            mt = xor32_max(mt);
            float svt = 0.0f;
            bool grow = mt > m_run + kLazy;
            if constexpr (KV_TOKEN) {
                svt = sScale[buf][2 * kBN];
                grow = grow || svt > s_run * 2.0f;
            }
            // Lazy rescale: the running max only moves when some row's max grows by
            // more than 2^kLazy (exp values stay <= 2^8, well inside fp16).
            if (__any(grow)) {
                const float m_new = fmaxf(m_run, mt);
                float alpha = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
                float alpha_o = alpha;
                if (KV_TOKEN) {
                    // Values accumulate in units of s_run / 2^6, s_run the largest value
                    // scale so far (within a factor 2), so that p * v_scale * 2^6 / s_run
                    // stays below 2^15 in fp16 and above its subnormals where its weight
                    // counts (the row sum is of p itself).
                    const float s_new = fmaxf(s_run, svt);
                    alpha_o = s_new > 0.0f ? alpha * (s_run / s_new) : alpha;
                    inv_s = s_new > 0.0f ? 64.0f / s_new : 0.0f;
                    s_run = s_new;
                }
                m_run = m_new;
                m_sh = KV_TOKEN ? m_new : m_new - kShift;
                l_run *= alpha;
#pragma unroll
                for (int d = 0; d < DB; ++d) acc[d] *= alpha_o;
            }

            f16x8 phi[2][2], plo[2][2];
            // The tile's weights are summed on their own and then added to the running
            // sum once: small weights added one by one to a large running sum would
            // each lose their low bits.
            float l_tile = 0.0f;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
#pragma unroll
                for (int s = 0; s < 2; ++s) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int r = 8 * s + e;
                        float p;
                        if (KV_TOKEN) {
                            // A row with nothing visible yet keeps m_run = -inf.
                            p = __builtin_amdgcn_exp2f(x[16 * u + r] - m_sh);
                            if constexpr (need_mask) {
                                if (x[16 * u + r] == -INFINITY) p = 0.0f;
                            }
                        } else {
                            p = __builtin_amdgcn_exp2f(__builtin_fmaf((float)sc[u][r], c, -m_sh));
                            if constexpr (need_mask) {
                                if (sc[u][r] == INT32_MIN) p = 0.0f;
                            }
                        }
                        if (KV_TOKEN) l_tile += p;
                        const float pv =
                            KV_TOKEN ? p * (sScale[buf][kBN + 32 * u + 16 * grp + r] * inv_s) : p;
                        const _Float16 hi16 = (_Float16)pv;
                        phi[u][s][e] = hi16;
                        plo[u][s][e] = (_Float16)(pv - (float)hi16);
                    }
                    if (!KV_TOKEN) {
                        // Row sum of the fp16 probabilities the P.V product uses, two
                        // per instruction, accumulated in fp32.
                        const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
                        for (int e = 0; e < 8; e += 2) {
                            const f16x2 pr = {phi[u][s][e], phi[u][s][e + 1]};
                            l_tile = __builtin_amdgcn_fdot2(pr, one, l_tile, false);
                            const f16x2 pl = {plo[u][s][e], plo[u][s][e + 1]};
                            l_tile = __builtin_amdgcn_fdot2(pl, one, l_tile, false);
                        }
                    }
                }
            }
            l_run += l_tile;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    f16x8 vop[DB];
#pragma unroll
                    for (int d = 0; d < DB; ++d)
                        vop[d] = *reinterpret_cast<const f16x8 *>(
                            sVT + (32 * d + col) * VSTRIDE + (32 * u + 16 * grp + 8 * s) * 2);
#pragma unroll
                    for (int d = 0; d < DB; ++d) {
                        acc[d] = mfma_32x32x16_f16(vop[d], phi[u][s], acc[d]);
                        acc[d] = mfma_32x32x16_f16(vop[d], plo[u][s], acc[d]);
                    }
                }
            }
            };

    // One pipeline step: this tile's math while the next tile's loads (issued at the
    // end of the previous step) are in flight, then its LDS stores. With
    // `every_row` the tile is inside the visible range of every row of the
    // workgroup, so no wave skips it or masks it: such steps run in
    // a loop of their own with a single code path, which keeps the output
    // accumulators in place (merging the masked and unmasked versions of a tile
    // would copy all of them on every step).
    auto step = [&](const int it, auto every_row_tag) {
        constexpr bool every_row = decltype(every_row_tag)::value;
        const int kt = kt0 + it * kBN;
        const int buf = it & 1;
        if constexpr (every_row) {
            tile_math(kt, buf, std::false_type{});
        } else {
            const bool mine = it < n_tiles;  // uniform over the group
            if (mine && wave_active && kt <= wk_hi && kt + kBN - 1 >= wk_lo) {  // wave-uniform
                // Tiles inside every row's visible range take the path without masks.
                if (kt + kBN - 1 <= full_hi && kt >= full_lo)
                    tile_math(kt, buf, std::false_type{});
                else
                    tile_math(kt, buf, std::true_type{});
            }
        }
        if (it + 1 < n_tiles) store_tile(buf ^ 1);
        // The registers are free again: the loads of the tile after next fly through
        // the barrier and the whole next step.
        if (it + 2 < n_tiles) load_tile(kt + 2 * kBN);
        __syncthreads();
    };
    // Steps [it_a, it_b): tiles every row of the workgroup sees whole. Rows past
    // q_len (a partial last query tile) compute on zero queries and store nothing.
    const int wg_full_lo = a.window > 0 ? a.query_start + r_last + 1 - a.window : 0;
    const int wg_full_hi = min(a.query_start + q0, a.kv_len - 1);
    // Clamped to n_iter: with a window the first fully visible tile can lie past this
    // group's tiles, and both groups of a split workgroup must run n_iter steps (one
    // barrier each).
    const int it_a = min(n_iter, max(0, wg_full_lo - kt0 + kBN - 1) / kBN);
    const int span = wg_full_hi + 1 - kt0;  // keys from kt0 through wg_full_hi
    const int it_b = max(it_a, min(n_tiles, span > 0 ? span / kBN : 0));

    if (n_tiles > 0) store_tile(0);
    if (n_tiles > 1) load_tile(kt0 + kBN);
    __syncthreads();
    int it = 0;
    for (; it < it_a; ++it) step(it, std::false_type{});
    for (; it < it_b; ++it) step(it, std::true_type{});
    for (; it < n_iter; ++it) step(it, std::false_type{});

    float l_tot = xor32_sum(l_run);
    if (SPLIT) {
        // Group 1 hands (running max, row sum, accumulator) to group 0 through LDS,
        // in a lane-linear layout (conflict-free 16-byte accesses).
        f32x4 *xo = reinterpret_cast<f32x4 *>(smem_all);
        float2 *xml = reinterpret_cast<float2 *>(smem_all + 4 * DB * 4 * kWave * 16);
        if (group == 1) {
#pragma unroll
            for (int d = 0; d < DB; ++d)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    xo[((wave * DB + d) * 4 + j) * kWave + lane] =
                        f32x4{acc[d][4 * j], acc[d][4 * j + 1], acc[d][4 * j + 2], acc[d][4 * j + 3]};
            xml[wave * kWave + lane] = float2{m_run, l_tot};
        }
        __syncthreads();
        if (group == 1) {
            // the two barriers of group 0's part store and count below
            if (MODE == kSplitStream && sp.parts > 1) {
                __syncthreads();
                __syncthreads();
            }
            return;
        }
        const float2 other = xml[wave * kWave + lane];
        const float m = fmaxf(m_run, other.x);
        const float w0 = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m);
        const float w1 = other.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(other.x - m);
        l_tot = l_tot * w0 + other.y * w1;
#pragma unroll
        for (int d = 0; d < DB; ++d)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f32x4 o = xo[((wave * DB + d) * 4 + j) * kWave + lane];
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[d][4 * j + i] = acc[d][4 * j + i] * w0 + o[i] * w1;
            }
        m_run = m;  // the merged state's maximum (a kSplitStream part stores it)
    }
    if (KV_TOKEN && MODE == kStream) {
        // Parts merge in absolute value units: the accumulator leaves the units of
        // s_run (the largest value scale this part saw) here.
#pragma unroll
        for (int d = 0; d < DB; ++d)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[d][i] *= s_run * (1.0f / 64.0f);
        s_run = 64.0f;
    }
    if (STREAM && sp.parts > 1) {
        // Leave this part in its slot (every lane: rows past q_len hold finite
        // values), then count the part in; the last part of the item merges. Every
        // access to a slot is a device-coherent atomic (agent scope: written through
        // to, and read from, the memory side beneath the per-XCD L2s); each thread
        // waits until its slot stores have completed before the barrier that
        // precedes the count, and the merging part reads the slots only after its
        // count returned. The same protocol as the decode merge. Release and acquire
        // fences at agent scope compile to a write-back and an invalidation of the
        // whole XCD L2 (buffer_wbl2 / buffer_inv), which every other workgroup on
        // the XCD then pays in K and V misses: 106 against 57 us on 1x32x2048x128.
        constexpr int SF = StreamSlot<D>::FLOATS, OF = StreamSlot<D>::O_FLOATS;
        constexpr int E = DB * 8;  // 8-byte elements of output per lane
        auto pack = [](float x, float y) {
            return (uint64_t)__float_as_uint(x) | ((uint64_t)__float_as_uint(y) << 32);
        };
        auto put = [](uint64_t *p, uint64_t v) { part_store(p, v); };
        auto get = [](const uint64_t *p) { return part_load(p); };
        // Element e of wave w, lane l at [(w E + e) 64 + l]: each store is 512
        // contiguous bytes.
        uint64_t *so = reinterpret_cast<uint64_t *>(sa.slots + (int64_t)sp.slot * SF);
#pragma unroll
        for (int d = 0; d < DB; ++d)
#pragma unroll
            for (int e = 0; e < 8; ++e)
                put(so + (wave * E + d * 8 + e) * kWave + lane,
                    pack(acc[d][2 * e], acc[d][2 * e + 1]));
        put(so + OF / 2 + wave * kWave + lane, pack(m_run, l_tot));
        part_stores_done();
        __syncthreads();
        if (tid == 0) *sTicket = part_count(sa.counters + sp.item);
        __syncthreads();
        if (*sTicket != (uint32_t)(sp.parts - 1)) return;
        part_claimed();
        if (tid == 0) part_reset(sa.counters + sp.item);  // ready for the next launch
        // Parts in order: part p is workgroup first_wg + p; the first part sits in
        // its workgroup's second slot when that range began before the item.
        auto slot_of = [&](int p) {
            const int L = sp.first_wg + p;
            const bool second = p == 0 && (int64_t)L * sa.units / gridDim.x < sp.item_u0;
            return reinterpret_cast<const uint64_t *>(sa.slots +
                                                      (int64_t)(2 * L + (second ? 1 : 0)) * SF);
        };
        // Every part, this one included, comes from its slot, folded in part order (a
        // running log-sum-exp with explicit fused multiply-adds: the same roundings
        // whichever part merges), kMergeAhead parts' loads in flight at a time.
        constexpr int kMergeAhead = 2;
        float m = -INFINITY, l = 0.0f;
        f32x16 tot[DB];
#pragma unroll
        for (int d = 0; d < DB; ++d) tot[d] = f32x16{};
        auto fold = [&](float mp, float lp, auto &&value) {
            const float mn = fmaxf(m, mp);
            const float er = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - mn);
            const float ep = mp == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mp - mn);
            l = __builtin_fmaf(ep, lp, l * er);
#pragma unroll
            for (int d = 0; d < DB; ++d)
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    tot[d][i] = __builtin_fmaf(ep, value(d, i), tot[d][i] * er);
            m = mn;
        };
        for (int p0 = 0; p0 < sp.parts; p0 += kMergeAhead) {
            uint64_t ml[kMergeAhead], v[kMergeAhead][DB * 8];
#pragma unroll
            for (int j = 0; j < kMergeAhead; ++j) {
                const int p = p0 + j;
                if (p >= sp.parts) continue;
                const uint64_t *sl = slot_of(p);
                ml[j] = get(sl + OF / 2 + wave * kWave + lane);
#pragma unroll
                for (int e = 0; e < DB * 8; ++e) v[j][e] = get(sl + (wave * E + e) * kWave + lane);
            }
#pragma unroll
            for (int j = 0; j < kMergeAhead; ++j) {
                const int p = p0 + j;
                if (p >= sp.parts) continue;
                fold(__uint_as_float((uint32_t)ml[j]), __uint_as_float((uint32_t)(ml[j] >> 32)),
                     [&](int d, int i) {
                         const uint64_t w = v[j][d * 8 + i / 2];
                         return __uint_as_float((uint32_t)(i & 1 ? w >> 32 : w));
                     });
            }
        }
#pragma unroll
        for (int d = 0; d < DB; ++d) acc[d] = tot[d];
        l_tot = l;
    }
    if (!row_ok) return;
    const float norm = (KV_TOKEN ? s_run * (1.0f / 64.0f) : cv) / l_tot;
    float *orow = a.out + b * a.o_sb + h * a.o_sh + (int64_t)row * a.o_st;
#pragma unroll
    for (int d = 0; d < DB; ++d) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f32x4 o;
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = acc[d][4 * j + i] * norm;
            *reinterpret_cast<f32x4 *>(orow + 32 * d + 8 * j + 4 * grp) = o;
        }
    }
}

// Persistent form of the split kernel: one workgroup per compute unit takes the
// items of round r = 0, 1, ... at index r * G + blockIdx.x, the odd rounds in
// reverse order, so that with heaviest-first ranks every workgroup's sum of work
// is about the same. A workgroup's next item starts while the stores of its last
// one drain.
template <int D>
__global__ __launch_bounds__(2 * kThreads, 1) void prefill_split_kernel(PrefillArgs a, int items) {
    static_assert(4 * (D / 32) * 4 * kWave * 16 + 4 * kWave * 8 <= 2 * PrefillLds<D>::BYTES,
                  "merge buffer fits in the stages");
    __shared__ __attribute__((aligned(16))) int8_t smem[2 * PrefillLds<D>::BYTES];
    __shared__ float sScale[2][1];
    const int G = gridDim.x;
    for (int r = 0;; ++r) {
        const int item = (r & 1) ? (r + 1) * G - 1 - (int)blockIdx.x : r * G + (int)blockIdx.x;
        if (item >= items) {
            if (r * G >= items) break;
            continue;  // a reversed last round with fewer items than workgroups
        }
        int tile, b, h;
        item_coords(a, item, tile, b, h);
        prefill_body<D, false, kSplit>(a, tile, b, h, 0, 0, smem, sScale, StreamArgs{},
                                       StreamPart{}, nullptr);
        __syncthreads();  // the next item's stages overwrite the merge buffer
    }
}

template <int D, bool KV_TOKEN>
__global__ __launch_bounds__(kThreads, 1) void prefill_kernel(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) int8_t smem[PrefillLds<D>::BYTES];
    __shared__ float sScale[2][KV_TOKEN ? 2 * kBN + 1 : 1];
    int tile, b, h;
    item_coords(a, grid_rank(a), tile, b, h);
    prefill_body<D, KV_TOKEN, kWhole>(a, tile, b, h, 0, INT32_MAX, smem, sScale, StreamArgs{},
                                      StreamPart{}, nullptr);
}

// Balanced schedule (StreamArgs): workgroup g works through the steps
// [L G^-1 units, (L + 1) G^-1 units) of logical workgroup L, where the G / 8
// workgroups that run on one XCD (hardware workgroup g goes to XCD g % 8) hold
// consecutive L, so an XCD's L2 sees a few heads, not all of them. GROUPS 2: the
// workgroup is two 4-wave groups that split each part's key tiles (kSplitStream).
template <int D, bool KV_TOKEN, int GROUPS>
__global__ __launch_bounds__(GROUPS * kThreads, 1) void prefill_stream_kernel(
    PrefillArgs a, StreamArgs sa) {
    static_assert(GROUPS == 1 || (GROUPS == 2 && !KV_TOKEN), "two groups: no per-token scales");
    static_assert(GROUPS == 1 || 4 * (D / 32) * 4 * kWave * 16 + 4 * kWave * 8 <=
                                     2 * PrefillLds<D>::BYTES,
                  "merge buffer fits in the stages");
    constexpr int MODE = GROUPS == 2 ? kSplitStream : kStream;
    __shared__ __attribute__((aligned(16))) int8_t smem[GROUPS * PrefillLds<D>::BYTES];
    __shared__ float sScale[2][KV_TOKEN ? 2 * kBN + 1 : 1];
    __shared__ uint32_t sTicket;
    const int G = gridDim.x, g = blockIdx.x;
    const int x = g % kXcds, per = G / kXcds, rem = G % kXcds;
    const int L = x * per + min(x, rem) + g / kXcds;
    int64_t u = (int64_t)L * sa.units / G;
    const int64_t u_end = (int64_t)(L + 1) * sa.units / G;
    // Locate the first step (the grid has at most one workgroup per step, so the
    // range is not empty): (batch, head), then the tile's place in the head's
    // order by bisection over the closed-form prefix sums.
    int bh = (int)(u / sa.per_head);
    int64_t r = u - (int64_t)bh * sa.per_head;
    int lo = 0, hi = a.q_tiles - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (steps_before_zigzag(a, sa.per_head, mid) <= r) lo = mid;
        else hi = mid - 1;
    }
    int z = lo;
    int c0 = (int)(r - steps_before_zigzag(a, sa.per_head, z));
    const int64_t W = sa.units;
    auto wg_of = [&](int64_t unit) { return (int)(((unit + 1) * G - 1) / W); };
    bool first = true;
    while (u < u_end) {
        const int tile = zigzag_tile(a.q_tiles, z);
        int kt_first;
        const int n = tile_steps(a, tile, kt_first);
        const int c1 = (int)(c0 + (u_end - u) < n ? c0 + (u_end - u) : n);
        StreamPart sp;
        sp.item_u0 = u - c0;
        sp.first_wg = wg_of(sp.item_u0);
        sp.parts = wg_of(sp.item_u0 + n - 1) - sp.first_wg + 1;
        sp.slot = 2 * L + (first ? 0 : 1);
        sp.item = bh * a.q_tiles + tile;
        prefill_body<D, KV_TOKEN, MODE>(a, tile, bh / a.q_heads, bh % a.q_heads, c0, c1, smem,
                                        sScale, sa, sp, &sTicket);
        u += c1 - c0;
        c0 = 0;
        first = false;
        if (++z == a.q_tiles) {
            z = 0;
            ++bh;
        }
        __syncthreads();  // the next item's first stage reuses the LDS
    }
}

// Bit-exact hook: the int32 score accumulators, through score_tile. One wave
// per 32 x 32 block of (query, key).
template <int D>
__global__ __launch_bounds__(64) void qk_scores_kernel(const int8_t *__restrict__ q,
                                                       const int8_t *__restrict__ k, int32_t batch,
                                                       int32_t q_heads, int32_t kv_heads,
                                                       int32_t q_len, int32_t kv_len,
                                                       int32_t *__restrict__ acc) {
    const int lane = threadIdx.x, col = lane & 31, grp = lane >> 5;
    const int q0 = blockIdx.x * 32, k0 = blockIdx.y * 32;
    const int bh = blockIdx.z, b = bh / q_heads, h = bh % q_heads;
    const int kvh = h / (q_heads / kv_heads);
    const int row = q0 + col;
    i32x4 qop[D / 32];
    load_q_operand<D>(qop, q + (((int64_t)b * q_heads + h) * q_len + (row < q_len ? row : 0)) * D,
                      row < q_len, grp);
    const int key = k0 + key_of_score_row(col);
    // Keys past the end read key 0 (in bounds); their scores are not stored.
    const int8_t *krow =
        k + (((int64_t)b * kv_heads + kvh) * kv_len + (key < kv_len ? key : 0)) * D;
    const i32x16 s = score_tile<D>(qop, krow, grp);
    if (row >= q_len) return;
    int32_t *out = acc + (((int64_t)b * q_heads + h) * q_len + row) * kv_len;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int kk = k0 + 16 * grp + r;
        if (kk < kv_len) out[kk] = s[r];
    }
}

bool valid_int8_strides(const reef_strides *s, const void *base) {
    if (!aligned(base, 16)) return false;
    if (!s) return true;
    return s->batch >= 0 && s->head >= 0 && s->token >= 0 && s->batch % 16 == 0 &&
           s->head % 16 == 0 && s->token % 16 == 0;
}

bool valid_granularity(int32_t g) {
    return g == REEF_SCALE_PER_TENSOR || g == REEF_SCALE_PER_HEAD || g == REEF_SCALE_PER_TOKEN;
}

int64_t floor_div_host(int64_t a, int64_t b) { return a >= 0 ? a / b : -((-a + b - 1) / b); }

// Host copies of tile_steps / steps_before (query tiles of 128 rows, key tiles of 64).
int64_t host_tile_steps(const reef_attention_params &p, int64_t tile) {
    const int64_t q0 = tile * kBM, r_last = std::min(q0 + kBM, p.q_len) - 1;
    const int64_t key_lo = p.window > 0 ? std::max<int64_t>(0, p.query_start + q0 + 1 - p.window) : 0;
    const int64_t key_hi = std::min(p.query_start + r_last, p.kv_len - 1);
    const int64_t kt_first = key_lo / kBN * kBN;
    return (key_hi - kt_first) / kBN + 1;
}

int64_t host_steps_before(const reef_attention_params &p, int64_t t) {
    int64_t s = t + t * (t - 1) + ((p.query_start + 127) / 64) * t;
    if (p.window > 0) {
        const int64_t t0 = std::max<int64_t>(0, floor_div_host(p.window - p.query_start - 1, kBM) + 1);
        if (t > t0)
            s -= (t - t0) * (t + t0 - 1) + floor_div_host(p.query_start + 1 - p.window, kBN) * (t - t0);
    }
    return s;
}

// Bound on the balanced schedule's grid (two part slots per workgroup are sized for
// it): two 4-wave workgroups per compute unit.
int64_t stream_groups() { return 2 * compute_units(); }

// The balanced schedule's workspace layout is the same for every call: a fixed
// region of counters (one per item, up to kStreamMaxItems items), then part slots
// sized for head_dim 128. Counter i sits at the same place whatever the shape of
// the call, and every launch leaves its counters at zero, so one zero-filled
// workspace serves calls of any shape (the slots are written before they are read).
constexpr int64_t kCounterWords = 65536;
constexpr int64_t kQueueWords = 16;  // the last words: the packed schedule's item queue
constexpr int64_t kStreamMaxItems = kCounterWords - kQueueWords;
constexpr int64_t kStreamMinSteps = 8;  // steps per workgroup of the balanced kernels
constexpr int64_t kStreamCounterBytes = kCounterWords * 4;

int64_t stream_items(const reef_attention_params &p) {
    return ceil_div(p.q_len, kBM) * p.q_heads * p.batch;
}

int64_t stream_slot_floats() { return StreamSlot<128>::FLOATS; }
static_assert(StreamSlot<128>::FLOATS == kPartSlotFloats, "the packed schedule's slots");


}  // namespace
}  // namespace reef

using namespace reef;

namespace reef {
namespace {
// Workspace: the balanced schedule's counters and slots, then (head_dim 128) the
// packed schedule's value image, 256-byte aligned.
int64_t balanced_bytes(const reef_attention_params &) {
    return ceil_div(kStreamCounterBytes + 2 * stream_groups() * stream_slot_floats() * 4, 256) * 256;
}
int64_t packed_bytes(const reef_attention_params &p) {
    return p.head_dim == 128 && p.kv_heads > 0 && p.kv_len > 0
               ? packed_image_bytes(p.batch, p.kv_heads, p.kv_len)
               : 0;
}
// The packed schedule is the library's choice for grids with at least one
// (light, heavy) pair of 256-row query tiles per compute unit; on smaller grids
// the one-item kernel was measured faster (1x32x2048: 53 against 80 us).
bool packed_by_default(const reef_attention_params &p) {
    const int64_t pairs = (ceil_div(p.q_len, 256) + 1) / 2 * p.batch * p.q_heads;
    return pairs >= compute_units();
}
}  // namespace

// The balanced schedule's workspace bytes (counters and part slots), for the
// prefill over the cache.
int64_t prefill_balanced_bytes(const reef_attention_params &p) { return balanced_bytes(p); }

}  // namespace reef

extern "C" size_t reef_attention_prefill_workspace_bytes(const reef_attention_params *p) {
    if (!p || p->batch <= 0 || p->q_heads <= 0 || p->q_len <= 0 ||
        (p->head_dim != 64 && p->head_dim != 128))
        return 0;
    return (size_t)(balanced_bytes(*p) + packed_bytes(*p));
}

extern "C" reef_status reef_attention_prefill_int8(
    const reef_attention_params *p, const int8_t *q, const reef_strides *q_strides,
    const int8_t *k, const reef_strides *k_strides, const int8_t *v, const reef_strides *v_strides,
    const float *q_scales, const float *k_scales, const float *v_scales, float *out,
    const reef_strides *out_strides, void *workspace, size_t workspace_bytes,
    hipStream_t stream) {
    if (!p || !q || !k || !v || !q_scales || !k_scales || !v_scales || !out)
        return REEF_INVALID_ARGUMENT;
    const int64_t D = p->head_dim;
    if (p->batch <= 0 || p->q_heads <= 0 || p->kv_heads <= 0 || p->q_len <= 0 ||
        p->kv_len <= 0 || D <= 0 || p->q_heads % p->kv_heads != 0 || p->query_start < 0 ||
        p->window < 0 || p->query_start + p->q_len > p->kv_len ||
        !valid_granularity(p->q_granularity) || !valid_granularity(p->kv_granularity) ||
        !std::isfinite(p->softmax_scale) || !(p->softmax_scale > 0.0f))
        return REEF_INVALID_ARGUMENT;
    if (p->kv_len >= (int64_t(1) << 30) || p->window >= (int64_t(1) << 30) ||
        p->q_heads > 65535 || p->batch > 65535)
        return REEF_UNSUPPORTED;
    if (D != 64 && D != 128) return REEF_UNSUPPORTED;
    {
        // Per-head K/V slices are addressed with 32-bit offsets.
        const int64_t kst = k_strides ? k_strides->token : D, vst = v_strides ? v_strides->token : D;
        if ((p->kv_len - 1) * std::max(kst, vst) + D >= (int64_t(1) << 31)) return REEF_UNSUPPORTED;
    }
    if (!valid_int8_strides(q_strides, q) || !valid_int8_strides(k_strides, k) ||
        !valid_int8_strides(v_strides, v) || !aligned(out, 16))
        return REEF_INVALID_ARGUMENT;
    if (out_strides && (out_strides->batch % 4 || out_strides->head % 4 ||
                        out_strides->token % 4 || out_strides->batch < 0 ||
                        out_strides->head < 0 || out_strides->token < 0))
        return REEF_INVALID_ARGUMENT;

    PrefillArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.qs = q_scales;
    a.ks = k_scales;
    a.vs = v_scales;
    a.out = out;
    const int64_t Hq = p->q_heads, Hkv = p->kv_heads, Sq = p->q_len, Skv = p->kv_len;
    a.q_sb = q_strides ? q_strides->batch : Hq * Sq * D;
    a.q_sh = q_strides ? q_strides->head : Sq * D;
    a.q_st = q_strides ? q_strides->token : D;
    a.k_sb = k_strides ? k_strides->batch : Hkv * Skv * D;
    a.k_sh = k_strides ? k_strides->head : Skv * D;
    a.k_st = k_strides ? k_strides->token : D;
    a.v_sb = v_strides ? v_strides->batch : Hkv * Skv * D;
    a.v_sh = v_strides ? v_strides->head : Skv * D;
    a.v_st = v_strides ? v_strides->token : D;
    a.o_sb = out_strides ? out_strides->batch : Hq * Sq * D;
    a.o_sh = out_strides ? out_strides->head : Sq * D;
    a.o_st = out_strides ? out_strides->token : D;
    a.batch = (int32_t)p->batch;
    a.q_heads = (int32_t)Hq;
    a.kv_heads = (int32_t)Hkv;
    a.q_len = (int32_t)Sq;
    a.kv_len = (int32_t)Skv;
    a.query_start = (int32_t)p->query_start;
    a.window = (int32_t)p->window;
    a.score_scale = p->softmax_scale * kLog2e;
    a.q_gran = p->q_granularity;
    a.kv_gran = p->kv_granularity;
    a.q_tiles = (int32_t)ceil_div(Sq, kBM);
    const int64_t items = a.q_tiles * Hq * p->batch;
    if (items >= (int64_t(1) << 31)) return REEF_UNSUPPORTED;
    const dim3 grid((unsigned)items);
    const bool tok = p->kv_granularity == REEF_SCALE_PER_TOKEN;
    if (workspace && !aligned(workspace, 256)) return REEF_INVALID_ARGUMENT;
    const uint32_t sched = p->flags & REEF_ATTN_SCHED_MASK;
    if (sched != REEF_ATTN_SCHED_AUTO && sched != REEF_ATTN_SCHED_ONE_ITEM &&
        sched != REEF_ATTN_SCHED_SPLIT && sched != REEF_ATTN_SCHED_BALANCED &&
        sched != REEF_ATTN_SCHED_PACKED)
        return REEF_INVALID_ARGUMENT;
    const int64_t bal_bytes = balanced_bytes(*p);
    const bool stream_ok = workspace && (int64_t)workspace_bytes >= bal_bytes &&
                           stream_items(*p) <= kStreamMaxItems;
    const bool packed_ok = D == 128 && !tok && workspace &&
                           (int64_t)workspace_bytes >= bal_bytes + packed_bytes(*p);
    if (sched == REEF_ATTN_SCHED_PACKED && !packed_ok) return REEF_INVALID_ARGUMENT;
    if (sched == REEF_ATTN_SCHED_PACKED && !packed_fits(*p)) return REEF_UNSUPPORTED;
    // The packed schedule takes whole query tiles from per-XCD queues on grids with
    // at least one (light, heavy) pair of tiles per compute unit (the library's choice
    // there), and, forced on smaller grids, equal runs of (tile, key tile) steps with
    // cut tiles merged through the balanced schedule's counters and slots (one counter
    // per tile; measured slower than the one-item and balanced kernels there: each
    // tile call and each merge costs 10-13 us of memory round trips). Outside its
    // limits AUTO falls back to the other schedules.
    const bool packed_large = packed_by_default(*p);
    const bool packed_runs_ok = stream_items(*p) <= kStreamMaxItems;
    if (sched == REEF_ATTN_SCHED_PACKED && !packed_large && !packed_runs_ok)
        return REEF_UNSUPPORTED;
    if (sched == REEF_ATTN_SCHED_PACKED ||
        (sched == REEF_ATTN_SCHED_AUTO && packed_ok && packed_fits(*p) && packed_large)) {
        const int64_t qst[3] = {a.q_sb, a.q_sh, a.q_st}, kst[3] = {a.k_sb, a.k_sh, a.k_st},
                      vst[3] = {a.v_sb, a.v_sh, a.v_st}, ost[3] = {a.o_sb, a.o_sh, a.o_st};
        PackedWork work;
        work.balanced = !packed_large && packed_runs_ok;
        work.queue = static_cast<uint32_t *>(workspace) + kStreamMaxItems;
        work.counters = static_cast<uint32_t *>(workspace);
        work.slots = reinterpret_cast<float *>(static_cast<char *>(workspace) + kStreamCounterBytes);
        return prefill_packed_launch(p, q, qst, k, kst, v, vst, q_scales, k_scales, v_scales, out,
                                     ost, static_cast<char *>(workspace) + bal_bytes, work, stream);
    }
    // The library takes the balanced schedule, which cuts the causal work of all
    // items into equal ranges, for grids of at most one 128-row tile per compute unit
    // (1x8q/1kv x4096x128: 63.6 us against 81.6 us with the split kernel and 92.5 us
    // with the one-item kernel). On larger grids, head_dim 128 takes the split
    // kernel, whose two 4-wave groups per workgroup halve each tile's key loop
    // (1x32x2048x128: 65.9 us against 82.0 us one-item and 66.0 us balanced;
    // 1x8q/1kv x8192x128: 195 against 278 us one-item),
    // and head_dim 64 the one-item kernel (1x32x4096x64: 150 us against 160 us split,
    // 4x32x4096x64: 541 against 582 us). Per-token K/V scales (which the split kernel
    // does not take) use the one-item kernel; small grids without a workspace, the
    // split kernel.
    if (sched == REEF_ATTN_SCHED_BALANCED && !stream_ok) return REEF_INVALID_ARGUMENT;
    if (sched == REEF_ATTN_SCHED_SPLIT && tok) return REEF_INVALID_ARGUMENT;
    if (sched == REEF_ATTN_SCHED_BALANCED ||
        (sched == REEF_ATTN_SCHED_AUTO && stream_ok && items <= compute_units())) {
        const int64_t per_head = host_steps_before(*p, a.q_tiles - 1) +
                                 host_tile_steps(*p, a.q_tiles - 1);
        StreamArgs sa;
        sa.per_head = per_head;
        sa.units = per_head * p->batch * Hq;
        sa.counters = static_cast<uint32_t *>(workspace);
        sa.slots = reinterpret_cast<float *>(static_cast<char *>(workspace) + kStreamCounterBytes);
        if (sa.units >= (int64_t(1) << 40)) return REEF_UNSUPPORTED;
        // No more workgroups than steps: every range holds at least one step, so the
        // workgroups between an item's first and last part each hold a part of it.
        // A workgroup holds a compute unit alone: at most one workgroup per unit, so
        // that every workgroup runs at once, and at least kStreamMinSteps steps per
        // workgroup, so that a short chunk of queries over a long prefix is cut into a
        // few parts per item (each merge reads its parts one after another).
        const dim3 sgrid((unsigned)std::min<int64_t>(
            std::max<int64_t>(1, std::min<int64_t>(compute_units(), sa.units / kStreamMinSteps)),
            sa.units));
        // Per-token K/V scales: one 4-wave group per workgroup; otherwise two groups
        // that split each part's key tiles (two waves per SIMD).
        if (tok) {
            if (D == 128)
                hipLaunchKernelGGL((prefill_stream_kernel<128, true, 1>), sgrid, dim3(kThreads), 0,
                                   stream, a, sa);
            else
                hipLaunchKernelGGL((prefill_stream_kernel<64, true, 1>), sgrid, dim3(kThreads), 0,
                                   stream, a, sa);
        } else {
            if (D == 128)
                hipLaunchKernelGGL((prefill_stream_kernel<128, false, 2>), sgrid,
                                   dim3(2 * kThreads), 0, stream, a, sa);
            else
                hipLaunchKernelGGL((prefill_stream_kernel<64, false, 2>), sgrid,
                                   dim3(2 * kThreads), 0, stream, a, sa);
        }
        return launch_status();
    }
    const bool split = sched == REEF_ATTN_SCHED_SPLIT ||
                       (sched == REEF_ATTN_SCHED_AUTO && !tok &&
                        (items <= compute_units() || D == 128));
    // The 4-wave kernel places two workgroups on each of the 256 compute units at
    // once; zig-zag pairs a heavy and a light tile there. The split kernel holds a
    // compute unit alone and takes the tiles heaviest first.
    a.zigzag = !split && items <= 2 * compute_units() ? 1 : 0;
    if (split) {
        const dim3 pgrid((unsigned)std::min<int64_t>(items, compute_units()));
        if (D == 128)
            hipLaunchKernelGGL(prefill_split_kernel<128>, pgrid, dim3(2 * kThreads), 0, stream, a,
                               (int)items);
        else
            hipLaunchKernelGGL(prefill_split_kernel<64>, pgrid, dim3(2 * kThreads), 0, stream, a,
                               (int)items);
        return launch_status();
    }
#define REEF_PREFILL_LAUNCH(DIM, TOK) \
    hipLaunchKernelGGL((prefill_kernel<DIM, TOK>), grid, dim3(kThreads), 0, stream, a)
    if (tok) {
        if (D == 128) REEF_PREFILL_LAUNCH(128, true);
        else REEF_PREFILL_LAUNCH(64, true);
    } else {
        if (D == 128) REEF_PREFILL_LAUNCH(128, false);
        else REEF_PREFILL_LAUNCH(64, false);
    }
#undef REEF_PREFILL_LAUNCH
    return launch_status();
}

extern "C" reef_status reef_qk_scores_i32(const int8_t *q, const int8_t *k, int64_t batch,
                                          int64_t q_heads, int64_t kv_heads, int64_t q_len,
                                          int64_t kv_len, int64_t head_dim, int32_t *acc,
                                          hipStream_t stream) {
    if (!q || !k || !acc || batch <= 0 || q_heads <= 0 || kv_heads <= 0 || q_len <= 0 ||
        kv_len <= 0 || q_heads % kv_heads != 0 || !aligned(q, 16) || !aligned(k, 16))
        return REEF_INVALID_ARGUMENT;
    if (head_dim != 64 && head_dim != 128) return REEF_UNSUPPORTED;
    if (batch * q_heads > 65535 || q_len >= (int64_t(1) << 30) || kv_len >= (int64_t(1) << 30))
        return REEF_UNSUPPORTED;
    const dim3 grid((unsigned)ceil_div(q_len, 32), (unsigned)ceil_div(kv_len, 32),
                    (unsigned)(batch * q_heads));
    if (head_dim == 128)
        hipLaunchKernelGGL(qk_scores_kernel<128>, grid, dim3(64), 0, stream, q, k, (int32_t)batch,
                           (int32_t)q_heads, (int32_t)kv_heads, (int32_t)q_len, (int32_t)kv_len,
                           acc);
    else
        hipLaunchKernelGGL(qk_scores_kernel<64>, grid, dim3(64), 0, stream, q, k, (int32_t)batch,
                           (int32_t)q_heads, (int32_t)kv_heads, (int32_t)q_len, (int32_t)kv_len,
                           acc);
    return launch_status();
}
