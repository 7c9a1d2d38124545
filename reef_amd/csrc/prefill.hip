// Prefill / general int8 flash attention for gfx950.
//
// Replaces the per-head loop of Attention::context (attention.hpp:374-432,
// attend_head :117-123 with causal_visibility :82-100) by one launch over every
// (batch, head, 128-query tile). Scores are exact int32 sums on the int8
// matrix cores (v_mfma_i32_32x32x32_i8), dequantized as float(acc) * (s_q * s_k)
// (the order of operator/linear.hpp:125-127) times softmax_scale, then an fp32
// online softmax; P.V runs on v_mfma_f32_32x32x16_f16 with P in fp16 (optionally
// split into hi + lo halves) and the int8 values converted exactly to fp16.
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

#include "reef_common.hpp"

namespace reef {
namespace {

constexpr int kBM = 128;  // query rows per workgroup
constexpr int kBN = 64;   // keys per tile
constexpr int kThreads = 256;

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

// Row m of a 32-row score block holds key sigma(m) = 16 ((m >> 2) & 1) +
// 4 (m >> 3) + (m & 3), so that output register r = 4j + i of lane group g is
// key 16g + r. Inverse: key kk -> row.
__device__ __forceinline__ int score_row_of_key(int kk) {
    return ((kk >> 2) & 3) * 8 + (kk >> 4) * 4 + (kk & 3);
}
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
template <int D, bool KV_TOKEN, bool PRECISE, bool SPLIT>
__device__ __forceinline__ void prefill_body(const PrefillArgs &a, int rank, int8_t *smem_all,
                                             float (*sScale)[KV_TOKEN ? 2 * kBN + 1 : 1]) {
    static_assert(!SPLIT || !KV_TOKEN, "the split kernel has no per-token K/V scales");
    constexpr int KSTRIDE = PrefillLds<D>::KSTRIDE, VSTRIDE = PrefillLds<D>::VSTRIDE;
    constexpr int DB = D / 32;  // 32-wide output blocks
    constexpr int K_BYTES = PrefillLds<D>::K_BYTES, V_BYTES = PrefillLds<D>::V_BYTES;
    constexpr int KLOADS = kBN * D / 16 / kThreads;  // 16-byte K loads per thread
    constexpr int VBLOCKS = (kBN / 4) * (D / 8);     // 4-key x 8-channel V blocks
    constexpr float kLazy = 8.0f;  // rescale only when a row max grows by > 2^8

    const int tid = threadIdx.x & (kThreads - 1), lane = tid & 63;
    // The wave index is the same on every lane; saying so lets every per-wave
    // decision below be a scalar branch instead of predicated vector code.
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int group = SPLIT ? __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 8) : 0;
    int8_t *smem = smem_all + group * PrefillLds<D>::BYTES;
    const int col = lane & 31, grp = lane >> 5;
    int tile, b, h;
    item_coords(a, rank, tile, b, h);
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
    // Loads go through buffer resources over this (batch, kv head)'s rows: the
    // per-lane offsets below never change, the tile offset is a scalar, and keys
    // past kv_len read zeros (every tile reaching past kv_len is masked anyway).
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
        const int ks_off = __builtin_amdgcn_readfirstlane((int)(kt * a.k_st));
        const int vs_off = __builtin_amdgcn_readfirstlane((int)(kt * a.v_st));
#pragma unroll
        for (int j = 0; j < KLOADS; ++j)
            kreg[j] = __builtin_amdgcn_raw_buffer_load_b128(krsrc, koff[j], ks_off, 0);
        if (tid < VBLOCKS) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const auto w = __builtin_amdgcn_raw_buffer_load_b64(vrsrc, voff[i], vs_off, 0);
                vreg[i] = uint2{w[0], w[1]};
            }
        }
        if (KV_TOKEN && wave == 0) {
            ks_reg = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(ksrsrc, lane * 4, kt * 4, 0));
            vs_reg = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(vsrsrc, lane * 4, kt * 4, 0));
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
    const int n_iter = SPLIT ? (n_all + 1) / 2 : n_all;
    const int kt0 = kt_first + (group ? n_iter * kBN : 0);
    const int n_tiles = group ? n_all - n_iter : n_iter;
    if (n_tiles > 0) load_tile(kt0);
    i32x4 qop[D / 32];
    load_q_operand<D>(qop, a.q + b * a.q_sb + h * a.q_sh + (int64_t)(row_ok ? row : 0) * a.q_st,
                      row_ok, grp);
    const float cq = row_ok ? scale_of(a.qs, a.q_gran, b, h, row, a.q_heads, a.q_len) : 0.0f;
    const float ck = KV_TOKEN ? 1.0f : scale_of(a.ks, a.kv_gran, b, kvh, 0, a.kv_heads, a.kv_len);
    const float cv = KV_TOKEN ? 1.0f : scale_of(a.vs, a.kv_gran, b, kvh, 0, a.kv_heads, a.kv_len);
    // log2-domain score per unit of int32 accumulator
    const float c = cq * ck * a.score_scale;

    float m_run = -INFINITY, l_run = 0.0f, s_run = 0.0f, inv_s = 0.0f;
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
            if (KV_TOKEN) {
                svt = sScale[buf][2 * kBN];
                grow = grow || svt > s_run * 16.0f;
            }
            // Lazy rescale: the running max only moves when some row's max grows by
            // more than 2^kLazy (exp values stay <= 2^8, well inside fp16).
            if (__any(grow)) {
                const float m_new = fmaxf(m_run, mt);
                float alpha = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
                float alpha_o = alpha;
                if (KV_TOKEN) {
                    // Values accumulate in units of s_run, the largest value scale so
                    // far, so that p * v_scale / s_run stays bounded in fp16.
                    const float s_new = fmaxf(s_run, svt);
                    alpha_o = s_new > 0.0f ? alpha * (s_run / s_new) : alpha;
                    inv_s = s_new > 0.0f ? 1.0f / s_new : 0.0f;
                    s_run = s_new;
                }
                m_run = m_new;
                l_run *= alpha;
#pragma unroll
                for (int d = 0; d < DB; ++d) acc[d] *= alpha_o;
            }

            f16x8 phi[2][2], plo[2][2];
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
                            p = __builtin_amdgcn_exp2f(x[16 * u + r] - m_run);
                            if constexpr (need_mask) {
                                if (x[16 * u + r] == -INFINITY) p = 0.0f;
                            }
                        } else {
                            p = __builtin_amdgcn_exp2f(__builtin_fmaf((float)sc[u][r], c, -m_run));
                            if constexpr (need_mask) {
                                if (sc[u][r] == INT32_MIN) p = 0.0f;
                            }
                        }
                        if (KV_TOKEN) l_run += p;
                        const float pv =
                            KV_TOKEN ? p * (sScale[buf][kBN + 32 * u + 16 * grp + r] * inv_s) : p;
                        const _Float16 hi16 = (_Float16)pv;
                        phi[u][s][e] = hi16;
                        if (PRECISE) plo[u][s][e] = (_Float16)(pv - (float)hi16);
                    }
                    if (!KV_TOKEN) {
                        // Row sum of the fp16 probabilities the P.V product uses, two
                        // per instruction, accumulated in fp32.
                        const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
                        for (int e = 0; e < 8; e += 2) {
                            const f16x2 pr = {phi[u][s][e], phi[u][s][e + 1]};
                            l_run = __builtin_amdgcn_fdot2(pr, one, l_run, false);
                            if (PRECISE) {
                                const f16x2 pl = {plo[u][s][e], plo[u][s][e + 1]};
                                l_run = __builtin_amdgcn_fdot2(pl, one, l_run, false);
                            }
                        }
                    }
                }
            }
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
                        if (PRECISE) acc[d] = mfma_32x32x16_f16(vop[d], plo[u][s], acc[d]);
                    }
                }
            }
            };

    // One pipeline step: the next tile's loads in flight during this tile's math,
    // then its LDS stores. With `every_row` the tile is inside the visible range of
    // every row of the workgroup, so no wave skips it or masks it: such steps run in
    // a loop of their own with a single code path, which keeps the output
    // accumulators in place (merging the masked and unmasked versions of a tile
    // would copy all of them on every step).
    auto step = [&](const int it, auto every_row_tag) {
        constexpr bool every_row = decltype(every_row_tag)::value;
        const int kt = kt0 + it * kBN;
        const int buf = it & 1;
        if (it + 1 < n_tiles) load_tile(kt + kBN);
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
        __syncthreads();
    };
    // Steps [it_a, it_b): tiles every row of the workgroup sees whole. Rows past
    // q_len (a partial last query tile) compute on zero queries and store nothing.
    const int wg_full_lo = a.window > 0 ? a.query_start + r_last + 1 - a.window : 0;
    const int wg_full_hi = min(a.query_start + q0, a.kv_len - 1);
    const int it_a = max(0, wg_full_lo - kt0 + kBN - 1) / kBN;
    const int span = wg_full_hi + 1 - kt0;  // keys from kt0 through wg_full_hi
    const int it_b = max(it_a, min(n_tiles, span > 0 ? span / kBN : 0));

    if (n_tiles > 0) store_tile(0);
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
        if (group == 1) return;
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
    }
    if (!row_ok) return;
    const float norm = (KV_TOKEN ? s_run : cv) / l_tot;
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
        prefill_body<D, false, false, true>(a, item, smem, sScale);
        __syncthreads();  // the next item's stages overwrite the merge buffer
    }
}

template <int D, bool KV_TOKEN, bool PRECISE>
__global__ __launch_bounds__(kThreads, (KV_TOKEN || PRECISE) ? 1 : 2) void prefill_kernel(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) int8_t smem[PrefillLds<D>::BYTES];
    __shared__ float sScale[2][KV_TOKEN ? 2 * kBN + 1 : 1];
    prefill_body<D, KV_TOKEN, PRECISE, false>(a, grid_rank(a), smem, sScale);
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

// Compute units of the current device (one split workgroup fits on each).
int64_t compute_units() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
        return 256;
    return n;
}

bool valid_granularity(int32_t g) {
    return g == REEF_SCALE_PER_TENSOR || g == REEF_SCALE_PER_HEAD || g == REEF_SCALE_PER_TOKEN;
}

}  // namespace
}  // namespace reef

using namespace reef;

extern "C" reef_status reef_attention_prefill_int8(
    const reef_attention_params *p, const int8_t *q, const reef_strides *q_strides,
    const int8_t *k, const reef_strides *k_strides, const int8_t *v, const reef_strides *v_strides,
    const float *q_scales, const float *k_scales, const float *v_scales, float *out,
    const reef_strides *out_strides, hipStream_t stream) {
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
    // Per-token K/V scales fold the value scale into P (p * s_v / max s_v) before its
    // fp16 rounding, which no longer cancels against the row sum; those launches
    // always split P into fp16 hi + lo parts to stay well inside the tolerance.
    const bool precise = (p->flags & REEF_ATTN_PRECISE_PV) != 0 || tok;
    // With no more items than compute units, the key split of the persistent
    // kernel is the only parallelism left to balance the causal work; with more,
    // two one-item workgroups per compute unit overlap each other's prologue and
    // epilogue better.
    const char *sp = getenv("REEF_PREFILL_SPLIT");
    const bool split =
        !tok && !precise && (sp ? atoi(sp) != 0 : items <= compute_units());
    // The 4-wave kernel places two workgroups on each of the 256 compute units at
    // once; zig-zag pairs a heavy and a light tile there. The split kernel holds a
    // compute unit alone and takes the tiles heaviest first.
    const char *zz = getenv("REEF_PREFILL_ZIGZAG");
    a.zigzag = zz ? atoi(zz) : (!split && items <= 512 ? 1 : 0);
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
#define REEF_PREFILL_LAUNCH(DIM, TOK, PREC)                                                  \
    hipLaunchKernelGGL((prefill_kernel<DIM, TOK, PREC>), grid, dim3(kThreads), 0, stream, a)
    if (D == 128) {
        if (tok) {
            if (precise) REEF_PREFILL_LAUNCH(128, true, true);
            else REEF_PREFILL_LAUNCH(128, true, false);
        } else {
            if (precise) REEF_PREFILL_LAUNCH(128, false, true);
            else REEF_PREFILL_LAUNCH(128, false, false);
        }
    } else {
        if (tok) {
            if (precise) REEF_PREFILL_LAUNCH(64, true, true);
            else REEF_PREFILL_LAUNCH(64, true, false);
        } else {
            if (precise) REEF_PREFILL_LAUNCH(64, false, true);
            else REEF_PREFILL_LAUNCH(64, false, false);
        }
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
