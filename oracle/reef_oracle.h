/*
 * CPU oracle for the int8 attention path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the shipped library links, loads or
 * calls this code; only tests/, the smoke check and the CPU-baseline leg of
 * bench.py use it, and only as the checker.
 *
 * Each function restates one function of the Reef inference engine
 * (inference-engine/reference/cpp/include/inference_engine/...) in plain C,
 * performing the same IEEE operations in the same order, so that results are
 * identical bit for bit to the engine's. Build with -ffp-contract=off and
 * without -ffast-math, as the engine is (inference-engine/CMakeLists.txt:11-13).
 *
 * Functions marked EXTENSION have no engine counterpart: batch > 1, grouped
 * query heads, per-head / per-token scales, a softmax scale and the
 * composition of int8 scores with the float softmax. They are composed only of
 * restated engine steps, in the order the engine's W8A8 projection uses
 * (operator/linear.hpp:125-127 dequantizes as float(sum) * (s_row * s_col)).
 */
#ifndef REEF_ORACLE_H
#define REEF_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { RO_OK = 0, RO_INVALID = 1, RO_NON_FINITE = 2 };
/* Scale granularity: one scale per tensor, per head, or per (batch, head, token). */
enum { RO_GRAN_TENSOR = 0, RO_GRAN_HEAD = 1, RO_GRAN_TOKEN = 2 };

/* quant.hpp:51-57 */
float ro_int8_scale(float max_magnitude);
/* quant.hpp:68-81; returns RO_NON_FINITE where the engine throws. */
int ro_quantize_int8(float value, float scale, int8_t *out);
/* quant.hpp:90-99 */
float ro_row_max_magnitude(const float *row, size_t n);
/* quant.hpp:112-133: one scale per row of width values (per-token). */
int ro_quantize_rows(const float *x, size_t rows, size_t width, int8_t *q, float *scales);
/* EXTENSION: one scale over all n values (per-tensor), rule of quant.hpp. */
int ro_quantize_per_tensor(const float *x, size_t n, int8_t *q, float *scale);
/* EXTENSION: x is [B, H, S, D]; one scale per head over batch and tokens. */
int ro_quantize_per_head(const float *x, size_t B, size_t H, size_t S, size_t D, int8_t *q,
                         float *scales);

/* static_cast<float>(code) * scale (tests/test_int8.cpp:182), scales[i / group]. */
void ro_dequantize(const int8_t *q, size_t n, size_t group, const float *scales, float *x);

/* math.hpp:34-67 (Cephes expf polynomial, for x <= 0). */
float ro_exp_nonpositive(float x);

/* attention.hpp:82-100: 1 where query row `row` (at position query_start +
 * row) sees key `key`; window 0 means no window. */
int ro_visible(int64_t row, int64_t key, int64_t query_start, int64_t window);

/* tensor.hpp:179-246 with int8 inputs and an int32 accumulator:
 * acc[i][j] = sum over d of q[i][d] * k[j][d]. q is [sq, d], k is [sk, d]. */
void ro_qk_i32(const int8_t *q, const int8_t *k, size_t sq, size_t sk, size_t d, int32_t *acc);

/* activation.hpp:167-231 for one row of n scores; vis[j] != 0 where key j is
 * visible. Returns RO_INVALID for a row with no visible key. */
int ro_masked_softmax_row(const float *scores, const uint8_t *vis, size_t n, float *out);

/* attention.hpp:117-123 (attend_head): float head, no 1/sqrt(d). q [sq, d],
 * k and v [sk, d], out [sq, d]. */
int ro_attend_head_f32(const float *q, const float *k, const float *v, size_t sq, size_t sk,
                       size_t d, int64_t query_start, int64_t window, float *out);

/* Integer-only head, int8.hpp. */
int32_t ro_rounding_shift(int32_t value, unsigned shift); /* int8.hpp:43-49 */
int8_t ro_saturate_int8(int32_t value);                   /* int8.hpp:56-60 */
void ro_exp_table(float step, uint16_t table[256]);       /* int8.hpp:156-164 */
/* int8.hpp:180-232 for one row. */
int ro_masked_softmax_int8_row(const int32_t *scores, const uint8_t *vis, size_t n,
                               unsigned shift, const uint16_t table[256], uint8_t *probs);
/* int8.hpp:250-279 */
int ro_attend_head_int8(const int8_t *q, const int8_t *k, const int8_t *v, size_t sq, size_t sk,
                        size_t d, int64_t query_start, int64_t window, unsigned score_shift,
                        const uint16_t table[256], unsigned out_shift, int8_t *out);

/* EXTENSION: batched int8 attention with float softmax (the golden of the
 * int8 prefill and decode kernels).
 *
 * q is [B, Hq, Sq, D]; k and v are [B, Hkv, Skv, D], all int8, row-major.
 * Query head h reads key/value head h / (Hq / Hkv). Scales are indexed by
 * granularity: TENSOR [1], HEAD [H], TOKEN [B, H, S]. Per (b, h, row):
 *   acc[j] = sum_d q*k                                   (int32, exact)
 *   s[j]   = ((float)acc[j] * (q_scale * k_scale[j])) * softmax_scale
 *   p      = masked_softmax(s) over the keys ro_visible() admits
 *   out[c] = sum over every key j, in order, of p[j] * ((float)v[j][c] * v_scale[j])
 * softmax_scale = 1 gives the engine's unscaled scores (attention.hpp:102-106).
 * acc_out, if not NULL, receives acc as [B, Hq, Sq, Skv].
 * threads > 1 splits the (b, h) pairs across OpenMP threads; each pair is
 * computed the same way, so results do not depend on the thread count. */
typedef struct ro_attn_desc {
    int64_t batch, q_heads, kv_heads, q_len, kv_len, head_dim;
    int64_t query_start; /* position of query row 0; usually kv_len - q_len */
    int64_t window;      /* 0: global causal; else sliding window */
    float softmax_scale;
    int32_t q_granularity, kv_granularity;
    int32_t threads;
} ro_attn_desc;

int ro_attention_int8(const ro_attn_desc *desc, const int8_t *q, const int8_t *k, const int8_t *v,
                      const float *q_scales, const float *k_scales, const float *v_scales,
                      float *out, int32_t *acc_out);

#ifdef __cplusplus
}
#endif

#endif /* REEF_ORACLE_H */
