/*
 * CPU oracle for the int8 attention path: plain-C restatement of the Reef
 * engine's arithmetic. TEST INFRASTRUCTURE ONLY (see reef_oracle.h): the
 * shipped library never links or calls it.
 *
 * Citations are relative to inference-engine/reference/cpp/include/inference_engine/.
 * Build: -O3 -ffp-contract=off, no -ffast-math (oracle/Makefile). Loops that
 * the compiler vectorises do so across independent outputs only, so every
 * float sum still runs in the engine's order.
 */
#include "reef_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define RO_INT8_LIMIT 127 /* quant.hpp:30 kInt8Limit */

/* quant.hpp:51-57: max/127, or 1 when every value is zero. */
float ro_int8_scale(float max_magnitude) {
    return max_magnitude > 0.0f ? max_magnitude / (float)RO_INT8_LIMIT : 1.0f;
}

/* quant.hpp:68-81: nearbyint(value / scale) (ties to even), clamped to +-127.
 * Non-finite value or scale has no int8 code: the engine throws
 * std::invalid_argument, this returns RO_NON_FINITE. */
int ro_quantize_int8(float value, float scale, int8_t *out) {
    if (!isfinite(value) || !isfinite(scale)) {
        return RO_NON_FINITE;
    }
    const float limit = (float)RO_INT8_LIMIT;
    float rounded = nearbyintf(value / scale);
    /* std::clamp(rounded, -limit, limit) */
    if (rounded < -limit) {
        rounded = -limit;
    } else if (limit < rounded) {
        rounded = limit;
    }
    *out = (int8_t)rounded;
    return RO_OK;
}

/* quant.hpp:90-99: largest = std::max(largest, fabs(x)) from 0. std::max
 * keeps the first argument unless it is less than the second, so a NaN never
 * replaces the running value. */
float ro_row_max_magnitude(const float *row, size_t n) {
    float largest = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        const float m = fabsf(row[i]);
        if (largest < m) {
            largest = m;
        }
    }
    return largest;
}

static int quantize_span(const float *x, size_t n, float scale, int8_t *q) {
    int status = RO_OK;
    for (size_t i = 0; i < n; ++i) {
        if (ro_quantize_int8(x[i], scale, &q[i]) != RO_OK) {
            q[i] = 0;
            status = RO_NON_FINITE;
        }
    }
    return status;
}

/* quant.hpp:112-133: each row gets int8_scale(row_max_magnitude(row)). */
int ro_quantize_rows(const float *x, size_t rows, size_t width, int8_t *q, float *scales) {
    int status = RO_OK;
    for (size_t r = 0; r < rows; ++r) {
        const float scale = ro_int8_scale(ro_row_max_magnitude(x + r * width, width));
        scales[r] = scale;
        if (quantize_span(x + r * width, width, scale, q + r * width) != RO_OK) {
            status = RO_NON_FINITE;
        }
    }
    return status;
}

/* EXTENSION: the quant.hpp rule with one scale over the whole tensor. */
int ro_quantize_per_tensor(const float *x, size_t n, int8_t *q, float *scale) {
    *scale = ro_int8_scale(ro_row_max_magnitude(x, n));
    return quantize_span(x, n, *scale, q);
}

/* EXTENSION: x is [B, H, S, D]; head h's scale covers x[:, h, :, :]. */
int ro_quantize_per_head(const float *x, size_t B, size_t H, size_t S, size_t D, int8_t *q,
                         float *scales) {
    const size_t slab = S * D;
    int status = RO_OK;
    for (size_t h = 0; h < H; ++h) {
        float largest = 0.0f;
        for (size_t b = 0; b < B; ++b) {
            const float m = ro_row_max_magnitude(x + (b * H + h) * slab, slab);
            if (largest < m) {
                largest = m;
            }
        }
        scales[h] = ro_int8_scale(largest);
        for (size_t b = 0; b < B; ++b) {
            const size_t off = (b * H + h) * slab;
            if (quantize_span(x + off, slab, scales[h], q + off) != RO_OK) {
                status = RO_NON_FINITE;
            }
        }
    }
    return status;
}

/* The engine's dequantization of an int8 code, static_cast<float>(code) * scale
 * (tests/test_int8.cpp:182; quant.hpp:34: "row r of the real weight is
 * approximately values row r times scales[r]"): one correctly rounded product.
 * Value i uses scales[i / group] (group = row width for per-row scales, n for one
 * scale over the tensor). */
void ro_dequantize(const int8_t *q, size_t n, size_t group, const float *scales, float *x) {
    for (size_t i = 0; i < n; ++i) {
        x[i] = (float)q[i] * scales[i / group];
    }
}

/* math.hpp:34-67: x = k ln2 + r, Cephes expf polynomial for e^r, times 2^k.
 * Every step is one correctly rounded float operation, in the engine's
 * order; 2^k is assembled from its exponent field. */
float ro_exp_nonpositive(float x) {
    if (x < -87.0f) {
        return 0.0f;
    }
    const float k = ((x * 1.44269504088896341f) + 12582912.0f) - 12582912.0f;
    const float r = (x - (k * 0.693359375f)) - (k * -2.12194440e-4f);
    const float r2 = r * r;
    float poly = 1.9875691500E-4f;
    poly = (poly * r) + 1.3981999507E-3f;
    poly = (poly * r) + 8.3334519073E-3f;
    poly = (poly * r) + 4.1665795894E-2f;
    poly = (poly * r) + 1.6666665459E-1f;
    poly = (poly * r) + 5.0000001201E-1f;
    poly = ((poly * r2) + r) + 1.0f;
    const uint32_t bits = (uint32_t)((int32_t)k + 127) << 23;
    float scale;
    memcpy(&scale, &bits, sizeof scale);
    return poly * scale;
}

/* attention.hpp:88-98: row r sits at position query_start + r and sees keys
 * [window_start, position], window_start = position + 1 - window when a
 * window is set and position + 1 > window. */
int ro_visible(int64_t row, int64_t key, int64_t query_start, int64_t window) {
    const int64_t position = query_start + row;
    const int64_t start = (window > 0 && position + 1 > window) ? position + 1 - window : 0;
    return key >= start && key <= position;
}

/* tensor.hpp:179-192 with Scalar = int8, Accumulator = int32. Integer sums
 * are exact in any order; |acc| <= d * 127 * 128 never overflows for the
 * head sizes used (d <= 256). */
void ro_qk_i32(const int8_t *q, const int8_t *k, size_t sq, size_t sk, size_t d, int32_t *acc) {
    for (size_t i = 0; i < sq; ++i) {
        for (size_t j = 0; j < sk; ++j) {
            int32_t sum = 0;
            for (size_t c = 0; c < d; ++c) {
                sum += (int32_t)q[i * d + c] * (int32_t)k[j * d + c];
            }
            acc[i * sk + j] = sum;
        }
    }
}

/* activation.hpp:188-229 for one row: max over visible keys (std::max
 * semantics), e = exp_nonpositive(s - m), sum in key order, then e / sum.
 * Masked keys get exactly 0. */
int ro_masked_softmax_row(const float *scores, const uint8_t *vis, size_t n, float *out) {
    int any = 0;
    float m = 0.0f;
    for (size_t j = 0; j < n; ++j) {
        if (vis[j]) {
            m = any ? (m < scores[j] ? scores[j] : m) : scores[j];
            any = 1;
        }
    }
    if (!any) {
        return RO_INVALID;
    }
    float sum = 0.0f;
    for (size_t j = 0; j < n; ++j) {
        if (vis[j]) {
            const float e = ro_exp_nonpositive(scores[j] - m);
            out[j] = e;
            sum += e;
        } else {
            out[j] = 0.0f;
        }
    }
    for (size_t j = 0; j < n; ++j) {
        if (vis[j]) {
            out[j] /= sum;
        }
    }
    return RO_OK;
}

/* out[i][c] = sum over every key j, in order from 0, of p[i][j] * v[j][c]
 * (tensor.hpp:179-192 with float; masked keys contribute p = 0). The loop
 * over c is independent per output, so vectorising it keeps each sum's
 * order. */
static void probs_times_values(const float *p, const float *v, size_t sk, size_t d, float *out) {
    for (size_t c = 0; c < d; ++c) {
        out[c] = 0.0f;
    }
    for (size_t j = 0; j < sk; ++j) {
        const float pj = p[j];
        const float *vj = v + j * d;
        for (size_t c = 0; c < d; ++c) {
            out[c] += pj * vj[c];
        }
    }
}

/* attention.hpp:117-123: masked_softmax(q . k^T) . v, scores unscaled. */
int ro_attend_head_f32(const float *q, const float *k, const float *v, size_t sq, size_t sk,
                       size_t d, int64_t query_start, int64_t window, float *out) {
    float *scores = (float *)malloc(sk * sizeof(float));
    float *probs = (float *)malloc(sk * sizeof(float));
    uint8_t *vis = (uint8_t *)malloc(sk ? sk : 1);
    int status = RO_OK;
    for (size_t i = 0; i < sq && status == RO_OK; ++i) {
        for (size_t j = 0; j < sk; ++j) {
            float sum = 0.0f; /* tensor.hpp:184-190, in order over d */
            for (size_t c = 0; c < d; ++c) {
                sum += q[i * d + c] * k[j * d + c];
            }
            scores[j] = sum;
            vis[j] = (uint8_t)ro_visible((int64_t)i, (int64_t)j, query_start, window);
        }
        status = ro_masked_softmax_row(scores, vis, sk, probs);
        if (status == RO_OK) {
            probs_times_values(probs, v, sk, d, out + i * d);
        }
    }
    free(scores);
    free(probs);
    free(vis);
    return status;
}

/* int8.hpp:43-49: floor(value / 2^shift + 1/2) by arithmetic shifts. */
int32_t ro_rounding_shift(int32_t value, unsigned shift) {
    if (shift == 0) {
        return value;
    }
    return (value >> shift) + ((value >> (shift - 1)) & 1);
}

/* int8.hpp:56-60 */
int8_t ro_saturate_int8(int32_t value) {
    return (int8_t)(value < -128 ? -128 : (value > 127 ? 127 : value));
}

/* int8.hpp:156-164: entry d = lround(32768 * exp_nonpositive(-d * step)). */
void ro_exp_table(float step, uint16_t table[256]) {
    for (int d = 0; d < 256; ++d) {
        const float e = ro_exp_nonpositive(-(float)d * step);
        table[d] = (uint16_t)lroundf(32768.0f * e);
    }
}

/* int8.hpp:196-229 for one row. */
int ro_masked_softmax_int8_row(const int32_t *scores, const uint8_t *vis, size_t n,
                               unsigned shift, const uint16_t table[256], uint8_t *probs) {
    int any = 0;
    int32_t largest = 0;
    for (size_t k = 0; k < n; ++k) {
        if (vis[k]) {
            largest = any ? (largest < scores[k] ? scores[k] : largest) : scores[k];
            any = 1;
        }
    }
    if (!any) {
        return RO_INVALID;
    }
    uint32_t *weights = (uint32_t *)malloc((n ? n : 1) * sizeof(uint32_t));
    uint32_t sum = 0;
    for (size_t k = 0; k < n; ++k) {
        if (vis[k]) {
            const uint32_t d = (uint32_t)((largest - scores[k]) >> (int32_t)shift);
            weights[k] = table[d < 255u ? d : 255u];
            sum += weights[k];
        }
    }
    const uint32_t reciprocal = (255u << 16) / sum;
    for (size_t k = 0; k < n; ++k) {
        probs[k] = 0;
        if (vis[k]) {
            const uint32_t scaled = weights[k] * reciprocal;
            const uint32_t rounded = (scaled >> 16) + ((scaled >> 15) & 1u);
            probs[k] = (uint8_t)(rounded < 255u ? rounded : 255u);
        }
    }
    free(weights);
    return RO_OK;
}

/* int8.hpp:250-279: int32 scores, table softmax to uint8, uint8 . int8 sums
 * in int32, then saturate(rounding_shift(sum, out_shift)). */
int ro_attend_head_int8(const int8_t *q, const int8_t *k, const int8_t *v, size_t sq, size_t sk,
                        size_t d, int64_t query_start, int64_t window, unsigned score_shift,
                        const uint16_t table[256], unsigned out_shift, int8_t *out) {
    int32_t *scores = (int32_t *)malloc((sk ? sk : 1) * sizeof(int32_t));
    uint8_t *vis = (uint8_t *)malloc(sk ? sk : 1);
    uint8_t *probs = (uint8_t *)malloc(sk ? sk : 1);
    int status = RO_OK;
    for (size_t i = 0; i < sq && status == RO_OK; ++i) {
        ro_qk_i32(q + i * d, k, 1, sk, d, scores);
        for (size_t j = 0; j < sk; ++j) {
            vis[j] = (uint8_t)ro_visible((int64_t)i, (int64_t)j, query_start, window);
        }
        status = ro_masked_softmax_int8_row(scores, vis, sk, score_shift, table, probs);
        if (status != RO_OK) {
            break;
        }
        for (size_t c = 0; c < d; ++c) {
            int32_t sum = 0;
            for (size_t j = 0; j < sk; ++j) {
                sum += (int32_t)probs[j] * (int32_t)v[j * d + c];
            }
            out[i * d + c] = ro_saturate_int8(ro_rounding_shift(sum, out_shift));
        }
    }
    free(scores);
    free(vis);
    free(probs);
    return status;
}

static float scale_at(const float *scales, int32_t granularity, int64_t b, int64_t h, int64_t t,
                      int64_t heads, int64_t tokens) {
    switch (granularity) {
    case RO_GRAN_TENSOR:
        return scales[0];
    case RO_GRAN_HEAD:
        return scales[h];
    default:
        return scales[(b * heads + h) * tokens + t];
    }
}

/* EXTENSION: see reef_oracle.h. One (batch, query head) pair. */
static int attend_pair(const ro_attn_desc *a, int64_t b, int64_t h, const int8_t *q,
                       const int8_t *k, const int8_t *v, const float *qs, const float *ks,
                       const float *vs, float *out, int32_t *acc_out, int32_t *acc, float *s,
                       float *p, float *vdeq, uint8_t *vis) {
    const int64_t D = a->head_dim, Sq = a->q_len, Skv = a->kv_len;
    const int64_t group = a->q_heads / a->kv_heads;
    const int64_t kvh = h / group;
    const int8_t *qh = q + ((b * a->q_heads + h) * Sq) * D;
    const int8_t *kh = k + ((b * a->kv_heads + kvh) * Skv) * D;
    const int8_t *vh = v + ((b * a->kv_heads + kvh) * Skv) * D;
    float *oh = out + ((b * a->q_heads + h) * Sq) * D;

    /* Dequantized values: (float)v * v_scale, the engine's float tensor that
     * attend_head's P.V product reads. */
    for (int64_t j = 0; j < Skv; ++j) {
        const float sv = scale_at(vs, a->kv_granularity, b, kvh, j, a->kv_heads, Skv);
        for (int64_t c = 0; c < D; ++c) {
            vdeq[j * D + c] = (float)vh[j * D + c] * sv;
        }
    }
    for (int64_t i = 0; i < Sq; ++i) {
        ro_qk_i32(qh + i * D, kh, 1, (size_t)Skv, (size_t)D, acc);
        if (acc_out) {
            memcpy(acc_out + ((b * a->q_heads + h) * Sq + i) * Skv, acc,
                   (size_t)Skv * sizeof(int32_t));
        }
        const float sq = scale_at(qs, a->q_granularity, b, h, i, a->q_heads, Sq);
        for (int64_t j = 0; j < Skv; ++j) {
            const float sk = scale_at(ks, a->kv_granularity, b, kvh, j, a->kv_heads, Skv);
            s[j] = ((float)acc[j] * (sq * sk)) * a->softmax_scale;
            vis[j] = (uint8_t)ro_visible(i, j, a->query_start, a->window);
        }
        if (ro_masked_softmax_row(s, vis, (size_t)Skv, p) != RO_OK) {
            return RO_INVALID;
        }
        probs_times_values(p, vdeq, (size_t)Skv, (size_t)D, oh + i * D);
    }
    return RO_OK;
}

int ro_attention_int8(const ro_attn_desc *a, const int8_t *q, const int8_t *k, const int8_t *v,
                      const float *q_scales, const float *k_scales, const float *v_scales,
                      float *out, int32_t *acc_out) {
    if (a->batch <= 0 || a->q_heads <= 0 || a->kv_heads <= 0 || a->q_len <= 0 ||
        a->kv_len <= 0 || a->head_dim <= 0 || a->q_heads % a->kv_heads != 0 ||
        a->query_start < 0 || a->window < 0) {
        return RO_INVALID;
    }
    const int64_t pairs = a->batch * a->q_heads;
    const int64_t Skv = a->kv_len, D = a->head_dim;
    int status = RO_OK;
    const int threads = a->threads > 0 ? a->threads : 1;
#pragma omp parallel num_threads(threads)
    {
        int32_t *acc = (int32_t *)malloc((size_t)Skv * sizeof(int32_t));
        float *s = (float *)malloc((size_t)Skv * sizeof(float));
        float *p = (float *)malloc((size_t)Skv * sizeof(float));
        float *vdeq = (float *)malloc((size_t)(Skv * D) * sizeof(float));
        uint8_t *vis = (uint8_t *)malloc((size_t)Skv);
#pragma omp for schedule(dynamic, 1)
        for (int64_t pair = 0; pair < pairs; ++pair) {
            const int rc = attend_pair(a, pair / a->q_heads, pair % a->q_heads, q, k, v, q_scales,
                                       k_scales, v_scales, out, acc_out, acc, s, p, vdeq, vis);
            if (rc != RO_OK) {
#pragma omp atomic write
                status = rc;
            }
        }
        free(acc);
        free(s);
        free(p);
        free(vdeq);
        free(vis);
    }
    return status;
}
