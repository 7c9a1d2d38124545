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

template <int D, bool KV_TOKEN, bool PRECISE>
__global__ __launch_bounds__(kThreads) void prefill_kernel(PrefillArgs a) {
    constexpr int KSTRIDE = D + 16;         // bytes per K row in LDS
    constexpr int VSTRIDE = kBN * 2 + 16;   // bytes per transposed-V row in LDS
    constexpr int DB = D / 32;              // 32-wide output blocks
    __shared__ __attribute__((aligned(16))) int8_t sK[kBN * KSTRIDE];
    __shared__ __attribute__((aligned(16))) int8_t sVT[D * VSTRIDE];
    __shared__ float sKS[KV_TOKEN ? kBN : 1], sVS[KV_TOKEN ? kBN : 1];
    __shared__ float sVmax;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, grp = lane >> 5;
    const int tile = a.q_tiles - 1 - (int)blockIdx.x;  // long causal rows first
    const int h = blockIdx.y, b = blockIdx.z;
    const int kvh = h / (a.q_heads / a.kv_heads);
    const int q0 = tile * kBM;
    const int row = q0 + wave * 32 + col;
    const bool row_ok = row < a.q_len;

    i32x4 qop[D / 32];
    load_q_operand<D>(qop, a.q + b * a.q_sb + h * a.q_sh + (int64_t)(row_ok ? row : 0) * a.q_st,
                      row_ok, grp);

    const float cq = row_ok ? scale_of(a.qs, a.q_gran, b, h, row, a.q_heads, a.q_len) : 0.0f;
    const float ck = KV_TOKEN ? 1.0f : scale_of(a.ks, a.kv_gran, b, kvh, 0, a.kv_heads, a.kv_len);
    const float cv = KV_TOKEN ? 1.0f : scale_of(a.vs, a.kv_gran, b, kvh, 0, a.kv_heads, a.kv_len);
    const float c = cq * ck * a.score_scale;

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

    float m_run = -INFINITY, l_run = 0.0f, s_run = 0.0f;
    f32x16 acc[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) acc[d] = f32x16{};

    for (int kt = key_lo / kBN * kBN; kt <= key_hi; kt += kBN) {
        __syncthreads();  // the previous tile's LDS reads are done
        // K tile -> LDS, rows permuted (score_row_of_key) within each 32-key block.
        for (int idx = tid; idx < kBN * D / 16; idx += kThreads) {
            const int kk = idx / (D / 16), ch = idx % (D / 16);
            const int key = kt + kk;
            i32x4 val = {0, 0, 0, 0};
            if (key < a.kv_len)
                val = *reinterpret_cast<const i32x4 *>(kbase + (int64_t)key * a.k_st + ch * 16);
            const int r = ((kk >> 5) << 5) + score_row_of_key(kk & 31);
            *reinterpret_cast<i32x4 *>(sK + r * KSTRIDE + ch * 16) = val;
        }
        // V tile -> LDS as fp16, transposed: row d holds the tile's 64 keys.
        for (int idx = tid; idx < (kBN / 4) * (D / 8); idx += kThreads) {
            const int kg = idx / (D / 8), dg = idx % (D / 8);
            uint2 w[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = kt + 4 * kg + i;
                w[i] = key < a.kv_len
                           ? *reinterpret_cast<const uint2 *>(vbase + (int64_t)key * a.v_st + 8 * dg)
                           : uint2{0u, 0u};
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                f16x4 h4;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t word = j < 4 ? w[i].x : w[i].y;
                    h4[i] = (_Float16)(int)(int8_t)(word >> (8 * (j & 3)));
                }
                *reinterpret_cast<f16x4 *>(sVT + (8 * dg + j) * VSTRIDE + 4 * kg * 2) = h4;
            }
        }
        if (KV_TOKEN && wave == 0) {
            const int key = kt + lane;
            const int64_t at = ((int64_t)b * a.kv_heads + kvh) * a.kv_len + key;
            const float ks = key < a.kv_len ? a.ks[at] : 0.0f;
            const float vs = key < a.kv_len ? a.vs[at] : 0.0f;
            sKS[lane] = ks;
            sVS[lane] = vs;
            const float m = wave_max(vs);
            if (lane == 0) sVmax = m;
        }
        __syncthreads();
        if (!wave_active || kt > wk_hi || kt + kBN - 1 < wk_lo) continue;  // wave-uniform
        const bool need_mask = !(kt + kBN - 1 <= full_hi && kt >= full_lo);

        i32x16 sc[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) sc[u] = score_tile<D>(qop, sK + (32 * u + col) * KSTRIDE, grp);

        float x[32];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float cs = KV_TOKEN ? c * sKS[32 * u + 16 * grp + r] : c;
                x[16 * u + r] = (float)sc[u][r] * cs;
            }
        }
        if (need_mask) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kt + 32 * u + 16 * grp + r;
                    if (key < lo || key > hi) x[16 * u + r] = -INFINITY;
                }
            }
        }
        float mt = x[0];
#pragma unroll
        for (int r = 1; r < 32; ++r) mt = fmaxf(mt, x[r]);
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float m_new = fmaxf(m_run, mt);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
        float alpha_o = alpha, inv_s = 1.0f;
        if (KV_TOKEN) {
            // Values are accumulated in units of s_run, the largest value scale
            // seen so far, so that p * v_scale / s_run stays in [0, 1].
            const float s_new = fmaxf(s_run, sVmax);
            alpha_o = s_new > 0.0f ? alpha * (s_run / s_new) : alpha;
            inv_s = s_new > 0.0f ? 1.0f / s_new : 0.0f;
            s_run = s_new;
        }
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int d = 0; d < DB; ++d) acc[d] *= alpha_o;

        f16x8 phi[2][2], plo[2][2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
#pragma unroll
            for (int s = 0; s < 2; ++s) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int r = 8 * s + e;
                    const float p = __builtin_amdgcn_exp2f(x[16 * u + r] - m_use);
                    l_run += p;
                    const float pv = KV_TOKEN ? p * (sVS[32 * u + 16 * grp + r] * inv_s) : p;
                    const _Float16 hi16 = (_Float16)pv;
                    phi[u][s][e] = hi16;
                    if (PRECISE) plo[u][s][e] = (_Float16)(pv - (float)hi16);
                }
            }
        }
#pragma unroll
        for (int d = 0; d < DB; ++d) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    const f16x8 vop = *reinterpret_cast<const f16x8 *>(
                        sVT + (32 * d + col) * VSTRIDE + (32 * u + 16 * grp + 8 * s) * 2);
                    acc[d] = mfma_32x32x16_f16(vop, phi[u][s], acc[d]);
                    if (PRECISE) acc[d] = mfma_32x32x16_f16(vop, plo[u][s], acc[d]);
                }
            }
        }
    }

    const float l_tot = l_run + __shfl_xor(l_run, 32);
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
        !std::isfinite(p->softmax_scale))
        return REEF_INVALID_ARGUMENT;
    if (p->kv_len >= (int64_t(1) << 30) || p->window >= (int64_t(1) << 30) ||
        p->q_heads > 65535 || p->batch > 65535)
        return REEF_UNSUPPORTED;
    if (D != 64 && D != 128) return REEF_UNSUPPORTED;
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

    const dim3 grid((unsigned)a.q_tiles, (unsigned)Hq, (unsigned)p->batch);
    const bool tok = p->kv_granularity == REEF_SCALE_PER_TOKEN;
    const bool precise = (p->flags & REEF_ATTN_PRECISE_PV) != 0;
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
