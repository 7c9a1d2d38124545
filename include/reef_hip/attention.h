/*
 * reef_hip: int8 attention for AMD MI355X (gfx950), C ABI.
 *
 * Drop-in device back end for the Reef engine's attention and quantization
 * operators (inference-engine/reference/cpp/include/inference_engine/). Every
 * entry point names the engine function whose arithmetic it follows, in the
 * way the engine's kernel ABI does (coral/include/reef_kernels/kernels.hpp:3-16):
 *
 *   - The caller owns every buffer; pointers are device pointers, arrays are
 *     row-major, and the innermost (head_dim / width) dimension is contiguous.
 *     Nothing here allocates or keeps hidden state, so calls are stream-ordered
 *     and re-entrant (kernels.hpp:13-14).
 *   - Where the engine throws, an entry point returns a status instead
 *     (kernels.hpp has no error path; host_if.hpp:24-30 uses status codes). All
 *     shape and argument checks run on the host before any launch.
 *   - Conditions only the device can see (non-finite values, out-of-range page
 *     numbers) set bits in an optional caller-owned device word (status_word);
 *     reef_read_status_word() waits for the stream and maps the word to a
 *     status. The C++ wrapper attention.hpp turns statuses into the engine's
 *     exception types.
 *
 * Scores follow the engine's W8A8 dequantization order
 * (operator/linear.hpp:125-127): s = float(int32 q.k) * (s_q * s_k), times
 * softmax_scale (1 reproduces the engine's unscaled attend_head,
 * attention.hpp:102-106; 1/sqrt(head_dim) is scaled dot-product attention).
 */
#ifndef REEF_HIP_ATTENTION_H
#define REEF_HIP_ATTENTION_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum reef_status {
    REEF_OK = 0,
    /* engine: std::invalid_argument for shapes and masks
     * (activation.hpp:178-181, 204-207; attention.hpp:293-318). */
    REEF_INVALID_ARGUMENT = 1,
    /* engine: std::invalid_argument from quantize_int8 (quant.hpp:72-74). */
    REEF_NON_FINITE_INPUT = 2,
    /* engine: std::length_error for the KV cache (attention.hpp:321-327). */
    REEF_CAPACITY = 3,
    /* a HIP runtime call failed. */
    REEF_HIP_ERROR = 4,
    /* well-formed but outside what the kernels implement (e.g. head_dim). */
    REEF_UNSUPPORTED = 5,
    /* engine: std::overflow_error from safe_multiply / safe_add (util.hpp:81-131). */
    REEF_OVERFLOW = 6
} reef_status;

/* Bits set in a status word by the kernels. */
#define REEF_STATUS_BIT_NON_FINITE 0x1u
#define REEF_STATUS_BIT_BAD_PAGE 0x2u
#define REEF_STATUS_BIT_BAD_LENGTH 0x4u
#define REEF_STATUS_BIT_CAPACITY 0x8u
#define REEF_STATUS_BIT_OVERFLOW 0x10u

typedef enum reef_scale_granularity {
    REEF_SCALE_PER_TENSOR = 0, /* one scale: scales[0] */
    REEF_SCALE_PER_HEAD = 1,   /* scales[head], over batch and tokens */
    REEF_SCALE_PER_TOKEN = 2   /* scales[(b * heads + head) * tokens + t] */
} reef_scale_granularity;

/* Element strides of a [batch, heads, tokens, head_dim] tensor whose head_dim
 * is contiguous. NULL means the packed layout {H*S*D, S*D, D}. The engine keeps
 * heads as [1, heads, len, head_dim] (attention.hpp:49-68); a projection
 * output [len, heads * head_dim] is {0, D, H*D}. */
typedef struct reef_strides {
    int64_t batch, head, token;
} reef_strides;

/* ---------------------------------------------------------------------------
 * Quantization (quant.hpp): scale = max|x| / 127 (1 when max is 0), code =
 * clamp(nearbyint(x / scale), -127, 127), IEEE division, ties to even. The
 * codes and scales are bit-identical to the engine's.
 */

/* The quant.hpp rule with one scale over all n values. scale: 1 float. */
reef_status reef_quantize_int8_per_tensor(const float *x, int64_t n, int8_t *q, float *scale,
                                          uint32_t *status_word, hipStream_t stream);

/* x: [B, H, S, D] with x_strides (NULL = packed); q: packed [B, H, S, D];
 * scales: [H], each over x[:, h, :, :]. */
reef_status reef_quantize_int8_per_head(const float *x, int64_t batch, int64_t heads,
                                        int64_t tokens, int64_t head_dim,
                                        const reef_strides *x_strides, int8_t *q, float *scales,
                                        uint32_t *status_word, hipStream_t stream);

/* quantize_rows (quant.hpp:112-133), the per-token quantizer of the W8A8
 * linear (linear.hpp:120): rows of width values, row r at x + r * row_stride;
 * q packed [rows, width]; scales [rows]. */
reef_status reef_quantize_int8_per_token(const float *x, int64_t rows, int64_t width,
                                         int64_t row_stride, int8_t *q, float *scales,
                                         uint32_t *status_word, hipStream_t stream);

/* Dequantize: x[i] = float(q[i]) * scale[i / group] (group = width for
 * per-token rows, n for per-tensor). */
reef_status reef_dequantize_int8(const int8_t *q, int64_t n, int64_t group, const float *scales,
                                 float *x, hipStream_t stream);

/* Waits for the stream, reads a status word written by the kernels and maps
 * it: 0 -> REEF_OK, NON_FINITE -> REEF_NON_FINITE_INPUT, CAPACITY ->
 * REEF_CAPACITY, OVERFLOW -> REEF_OVERFLOW, page/length bits ->
 * REEF_INVALID_ARGUMENT (first match in that order). Clears the word afterwards
 * when clear != 0. */
reef_status reef_read_status_word(uint32_t *status_word, int clear, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * W8A8 projection: linear() with a QuantizedWeight (operator/linear.hpp:106-132).
 * x [rows, in] fp32 (row r at x + r * x_row_stride) is quantized per row as
 * quantize_rows does (quant.hpp:112-133), multiplied by the int8 weight
 * [out, in] (row-major, the engine's layout) in exact int32, and
 * y[r, c] = float(sum) * (row_scale[r] * w_scales[c]) (+ bias[c]), the engine's
 * float steps in its order, each rounded on its own: bit-identical outputs. y is
 * fp32 [rows, out] with row stride y_row_stride. in must be a multiple of 16.
 * Non-finite input sets NON_FINITE; an infinite or NaN output sets OVERFLOW
 * (the engine's std::overflow_error). The workspace holds the quantized rows.
 */
size_t reef_linear_w8a8_workspace_bytes(int64_t rows, int64_t in_features);

reef_status reef_linear_w8a8(const float *x, int64_t rows, int64_t in_features,
                             int64_t x_row_stride, const int8_t *weight, const float *w_scales,
                             const float *bias, int64_t out_features, float *y,
                             int64_t y_row_stride, void *workspace, size_t workspace_bytes,
                             uint32_t *status_word, hipStream_t stream);

/* The product and epilogue alone, on rows already quantized (xq [rows, in] packed,
 * x_scales [rows]). */
reef_status reef_gemm_w8a8(const int8_t *xq, const float *x_scales, int64_t rows,
                           int64_t in_features, const int8_t *weight, const float *w_scales,
                           const float *bias, int64_t out_features, float *y,
                           int64_t y_row_stride, uint32_t *status_word, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Attention over int8 Q/K/V with an fp32 softmax and fp32 output.
 */

/* Attention flags. */
#define REEF_ATTN_PRECISE_PV 0x1u /* P.V with P split into fp16 hi + lo parts (22
                                     * bits) whatever the values. Without it the packed
                                     * schedule splits wherever a head's dequantized
                                     * values reach above 1 in magnitude, the other
                                     * schedules always; at or below 1 one fp16 P moves
                                     * an output by at most 2^-11 max|v_j - out| <=
                                     * 9.8e-4. Either
                                     * way each P carries an exponent offset that keeps
                                     * it out of the fp16 subnormals, so small weights
                                     * keep their precision */
/* Prefill work schedule (bits 4-6 of flags). AUTO lets the library choose from the
 * grid size and the workspace; the others force one schedule, for callers that
 * tune it and for tests that must reach every path. A forced schedule that the
 * call cannot use (BALANCED without a large enough workspace, SPLIT with PER_TOKEN
 * K/V scales, PACKED without head_dim 128, per-tensor or per-head K/V scales and a
 * workspace) returns REEF_INVALID_ARGUMENT, and PACKED outside the packed kernel's
 * limits REEF_UNSUPPORTED. AUTO takes PACKED for head_dim 128 with at least one
 * pair of 256-row query tiles per compute unit (and a workspace that holds the
 * image); BALANCED with a large enough workspace and at most one 128-row query tile
 * per compute unit; otherwise SPLIT for head_dim 128 and for small grids without a
 * workspace, ONE_ITEM for head_dim 64 and with PER_TOKEN K/V scales. Every schedule
 * splits P into hi + lo where the values need it. */
#define REEF_ATTN_SCHED_MASK 0x70u
#define REEF_ATTN_SCHED_AUTO 0x00u
#define REEF_ATTN_SCHED_ONE_ITEM 0x10u /* one 128-row query tile per workgroup */
#define REEF_ATTN_SCHED_SPLIT 0x20u    /* persistent workgroups; two 4-wave groups split
                                        * each tile's keys; hi + lo P */
#define REEF_ATTN_SCHED_BALANCED 0x30u /* equal (tile, key block) ranges per workgroup,
                                        * two 4-wave groups splitting each range's key
                                        * tiles (one with PER_TOKEN K/V scales); cut
                                        * tiles merge through the workspace; hi + lo P */
#define REEF_ATTN_SCHED_PACKED 0x40u   /* head_dim 128, per-tensor / per-head K and V
                                        * scales: V packed once into an fp16 image in the
                                        * workspace, 128-row query tiles, persistent
                                        * workgroups taking (light, heavy) tile pairs
                                        * from per-XCD queues in the workspace */

typedef struct reef_attention_params {
    int64_t batch, q_heads, kv_heads; /* q head h reads kv head h / (q_heads / kv_heads) */
    int64_t q_len, kv_len, head_dim;  /* head_dim 64 or 128 */
    int64_t query_start; /* position of query row 0; engine: kv_len - q_len (attention.hpp:415) */
    int64_t window;      /* 0: GlobalAttention; > 0: LocalAttention window (attention.hpp:223-261) */
    float softmax_scale;    /* > 0; scales must be positive, as the quantizers make them */
    int32_t q_granularity;  /* reef_scale_granularity of q_scales */
    int32_t kv_granularity; /* reef_scale_granularity of k_scales and v_scales */
    uint32_t flags;
} reef_attention_params;

/* Prefill / general attention: Attention::context (attention.hpp:374-432) for
 * every (batch, head) in one launch; per head, attend_head (:117-123) with
 * causal_visibility (:82-100). q [B, Hq, q_len, D], k and v [B, Hkv, kv_len, D],
 * out fp32 [B, Hq, q_len, D], each with optional strides. Requires
 * query_start + q_len <= kv_len, so that every row sees a key (the engine
 * throws for a row with none, activation.hpp:204-207).
 *
 * workspace (optional, 256-byte aligned, at least
 * reef_attention_prefill_workspace_bytes(p) bytes; NULL/0 allowed) holds the
 * counters (a fixed 256 KB region: the balanced schedule's, at most 65520 items of
 * 128 query rows, and the packed schedule's item queue) and partial results of the
 * balanced schedule and, for head_dim 128, the fp16 value image of the packed
 * schedule (2 bytes per V element). It must be zero-filled
 * before its first use; every call leaves the counters zero-filled, and the
 * counters sit at the same offsets for every shape, so one workspace serves calls
 * of any shape that it is large enough for. Without it the library uses the
 * schedules that need none. Calls that may run at the same time need separate
 * workspaces. */
size_t reef_attention_prefill_workspace_bytes(const reef_attention_params *p);

reef_status reef_attention_prefill_int8(const reef_attention_params *p, const int8_t *q,
                                        const reef_strides *q_strides, const int8_t *k,
                                        const reef_strides *k_strides, const int8_t *v,
                                        const reef_strides *v_strides, const float *q_scales,
                                        const float *k_scales, const float *v_scales, float *out,
                                        const reef_strides *out_strides, void *workspace,
                                        size_t workspace_bytes, hipStream_t stream);

/* Bit-exact hook: the int32 score accumulators q . k^T (tensor.hpp:210-246
 * with int8 inputs and int32 sums), computed by the same MFMA tile code as the
 * prefill kernel. acc: [B, Hq, q_len, kv_len] int32. Packed q and k. */
reef_status reef_qk_scores_i32(const int8_t *q, const int8_t *k, int64_t batch, int64_t q_heads,
                               int64_t kv_heads, int64_t q_len, int64_t kv_len, int64_t head_dim,
                               int32_t *acc, hipStream_t stream);

/* The same scores from the packed schedule's own kernel (head_dim 128; the
 * matmul<int8_t, int32_t> of tensor.hpp:210-246 on q . k^T): it runs one attention
 * over (q, k, v = k) in which every row sees every key, and stores every score
 * accumulator as its tile code reads it (keys staged in LDS in its permuted order,
 * accumulators relative to the running maximum), turned back into the plain int32
 * sum. acc: [B, Hq, q_len, kv_len] int32; packed q [B, Hq, q_len, 128] and k
 * [B, Hkv, kv_len, 128]; workspace: 256-byte aligned, zero-filled once (the launch
 * leaves it zero-filled where it must be), at least
 * reef_qk_scores_i32_packed_workspace_bytes() bytes (0: invalid sizes). A test hook. */
size_t reef_qk_scores_i32_packed_workspace_bytes(int64_t batch, int64_t q_heads,
                                                 int64_t kv_heads, int64_t q_len,
                                                 int64_t kv_len);
reef_status reef_qk_scores_i32_packed(const int8_t *q, const int8_t *k, int64_t batch,
                                      int64_t q_heads, int64_t kv_heads, int64_t q_len,
                                      int64_t kv_len, int32_t *acc, void *workspace,
                                      size_t workspace_bytes, hipStream_t stream);

/* Integer-only attention: attend_head_int8 (int8.hpp:250-279) for every (batch,
 * head) in one launch, bit-identical to the engine. Per row: int32 scores over the
 * visible keys, weights table[min((max - s) >> score_shift, 255)], probabilities
 * in [0, 255] from the integer reciprocal of their sum (masked_softmax_int8,
 * :180-232), out = saturate_int8(rounding_shift(sum p * v, out_shift)) (:43-60).
 * table: 256 uint16 on the device (exp_table(), :156-164). q, k, v int8
 * [B, H, S, D] with strides as for the prefill; out int8 [B, Hq, q_len, D].
 * p->softmax_scale, q_granularity, kv_granularity and flags are not used;
 * head_dim 32, 64 or 128; score_shift and out_shift at most 31. A row may see at
 * most 65536 keys (kv_len, or the window when shorter): beyond that the engine's
 * uint32 weight sum could wrap, and the call returns REEF_UNSUPPORTED. */
reef_status reef_attention_int8_integer(const reef_attention_params *p, const int8_t *q,
                                        const reef_strides *q_strides, const int8_t *k,
                                        const reef_strides *k_strides, const int8_t *v,
                                        const reef_strides *v_strides, uint32_t score_shift,
                                        const uint16_t *table, uint32_t out_shift, int8_t *out,
                                        const reef_strides *out_strides, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Decode over an int8 KV cache (one query token per sequence), split across
 * waves along the keys, partial results combined by log-sum-exp.
 *
 * KV cache format (int8 values, fp32 per-token-per-head scales). The cache is
 * cut into pages of 16 tokens. A K page is [16, D] (token-major, like the
 * engine's KvCache rows, attention.hpp:64-68). A V page is stored transposed,
 * [D, 16]: each of its D rows holds one channel of the 16 tokens, which is the
 * operand layout of the P.V matrix instruction. reef_kv_pack_v_pages() converts
 * token-major values into this layout and reef_kv_append_int8() writes it.
 *
 *   contiguous: k_cache [B, Hkv, L, D]; v_cache [B, Hkv, L/16, D, 16];
 *               k_scales, v_scales [B, Hkv, L]; L = max_context, a multiple of 16.
 *   paged:      k_pages [P, Hkv, 16, D]; v_pages [P, Hkv, D, 16];
 *               k_scale_pages, v_scale_pages [P, Hkv, 16];
 *               block_table [B, max_blocks_per_seq] int32 page numbers.
 * q: [B, Hq, D] int8 with q_scales by q_granularity (PER_TOKEN: [B, Hq]);
 * out: [B, Hq, D] fp32. context_lens: [B] int32 on the device (NULL: every
 * sequence holds max_context tokens). Query b sits at position
 * context_lens[b] - 1 and sees all earlier keys (or the last window).
 * A sequence whose length is outside [1, max_context], or a page number outside
 * [0, P), sets a status-word bit and yields zeros for that sequence.
 */
typedef struct reef_decode_params {
    int64_t batch, q_heads, kv_heads, head_dim; /* head_dim 64 or 128 */
    int64_t max_context;  /* tokens per sequence the cache can hold */
    int64_t window;       /* 0: global */
    float softmax_scale;
    int32_t q_granularity;
    int32_t num_splits;   /* 0: library choice; n > 0: about n waves per (sequence,
                             kv head) on average (ceil(B * Hkv * n / 4) workgroups) */
    uint32_t flags;
} reef_decode_params;

/* Bytes of device workspace the decode entry points need for params. The launch
 * deals the keys of all (sequence, kv head) items out to its workgroups in equal
 * runs of 64-key blocks, whatever the context lengths (with at most 2048 items;
 * beyond that, in equal runs of whole items). The workspace holds a fixed 8 KB
 * region of counters (one per item, at the same offset for every shape) and two
 * partial-result slots per workgroup; an item whose keys span several workgroups
 * is merged by the last of them inside the same launch. The workspace must be
 * zero-filled before its first use; every call leaves it ready for the next call of
 * any shape it is large enough for (no refill). Calls that may run at the same
 * time need separate workspaces. */
size_t reef_attention_decode_workspace_bytes(const reef_decode_params *p);

reef_status reef_attention_decode_int8(const reef_decode_params *p, const int8_t *q,
                                       const float *q_scales, const int8_t *k_cache,
                                       const int8_t *v_cache, const float *k_scales,
                                       const float *v_scales, const int32_t *context_lens,
                                       float *out, void *workspace, size_t workspace_bytes,
                                       uint32_t *status_word, hipStream_t stream);

reef_status reef_attention_decode_int8_paged(
    const reef_decode_params *p, const int8_t *q, const float *q_scales, const int8_t *k_pages,
    const int8_t *v_pages, const float *k_scale_pages, const float *v_scale_pages,
    const int32_t *block_table, int64_t max_blocks_per_seq, int64_t num_pages,
    const int32_t *context_lens, float *out, void *workspace, size_t workspace_bytes,
    uint32_t *status_word, hipStream_t stream);

/* Allocation-free form of reef_attention_decode_int8_paged, with no counterpart in
 * the reference: for callers that cannot allocate or pass device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The
 * split-merge workspace is a fixed 16 MiB array inside the library, one per GPU,
 * held until the process ends; a call whose workspace
 * (reef_attention_decode_workspace_bytes) would exceed it returns REEF_UNSUPPORTED
 * before any launch. Each call clears the counters it uses with a small fill
 * kernel on `stream`, then runs the same kernels as the workspace entry point
 * (bit-identical outputs). Every call on one GPU shares that array: calls that
 * overlap on one GPU (other streams, other host threads) race and must not run
 * concurrently. Nothing is allocated or freed. */
reef_status reef_attention_decode_int8_paged_noalloc(
    const reef_decode_params *p, const int8_t *q, const float *q_scales, const int8_t *k_pages,
    const int8_t *v_pages, const float *k_scale_pages, const float *v_scale_pages,
    const int32_t *block_table, int64_t max_blocks_per_seq, int64_t num_pages,
    const int32_t *context_lens, float *out, uint32_t *status_word, hipStream_t stream);

/* Token-major values [pages * 16, D] (page-contiguous) -> transposed pages
 * [pages, D, 16]. */
reef_status reef_kv_pack_v_pages(const int8_t *v_tokens, int64_t pages, int64_t head_dim,
                                 int8_t *v_pages, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * KV-cache append: Attention::append_kv_cache (attention.hpp:290-352) on the
 * int8 cache above. The new_tokens fresh key and value rows of every sequence,
 * fp32 [B, Hkv, new_tokens, D] with optional strides (a projection output
 * [new_tokens, Hkv * D] is {0, D, Hkv * D}), are quantized per token exactly as
 * quantize_rows (quant.hpp:112-133) quantizes them and written at positions
 * start_positions[b] .. start_positions[b] + new_tokens - 1 of sequence b, in
 * place. start_positions: [B] int32 on the device.
 *   - REEF_CAPACITY (host) when new_tokens > max_context; a sequence whose
 *     append would pass max_context is not written and sets the CAPACITY bit
 *     (the engine's length_error, attention.hpp:321-327); a negative start sets
 *     BAD_LENGTH; a page number outside [0, num_pages) sets BAD_PAGE and skips
 *     that row.
 *   - Non-finite values set NON_FINITE (the engine throws before writing; here
 *     the rows of such a call are unspecified).
 *   - context_lens (optional, may alias start_positions) receives
 *     start_positions[b] + new_tokens for every sequence that was written.
 */
typedef struct reef_kv_append_params {
    int64_t batch, kv_heads, head_dim; /* head_dim 64 or 128 */
    int64_t new_tokens;                /* tokens appended to every sequence */
    int64_t max_context;               /* capacity per sequence, a multiple of 16 */
} reef_kv_append_params;

reef_status reef_kv_append_int8(const reef_kv_append_params *p, const float *k_new,
                                const reef_strides *k_strides, const float *v_new,
                                const reef_strides *v_strides, const int32_t *start_positions,
                                int8_t *k_cache, int8_t *v_cache, float *k_scales,
                                float *v_scales, int32_t *context_lens, uint32_t *status_word,
                                hipStream_t stream);

/* The same into the paged layout; max_context <= max_blocks_per_seq * 16. */
reef_status reef_kv_append_int8_paged(const reef_kv_append_params *p, const float *k_new,
                                      const reef_strides *k_strides, const float *v_new,
                                      const reef_strides *v_strides,
                                      const int32_t *start_positions, const int32_t *block_table,
                                      int64_t max_blocks_per_seq, int64_t num_pages,
                                      int8_t *k_pages, int8_t *v_pages, float *k_scale_pages,
                                      float *v_scale_pages, int32_t *context_lens,
                                      uint32_t *status_word, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Prefill over the int8 cache (chunked and multi-turn prompts): Attention::forward
 * with query_len > 1 on a cache that already holds the chunk's keys and values
 * (the engine appends first, then runs context() over every cached key with
 * query_start = key_len - query_len, attention.hpp:354-372 and :415). The cache is
 * the decode format above: contiguous when block_table is NULL (k_cache
 * [B, Hkv, max_context, D], v_cache [B, Hkv, max_context/16, D, 16], scales
 * [B, Hkv, max_context]), paged otherwise (k_cache [P, Hkv, 16, D], v_cache
 * [P, Hkv, D, 16], scales [P, Hkv, 16], block_table [B, max_blocks_per_seq],
 * P = num_pages; max_context is not used). p->kv_len is the number of cached
 * tokens of every sequence (the chunk's included), p->q_len the chunk length,
 * p->query_start normally kv_len - q_len; p->kv_granularity must be
 * REEF_SCALE_PER_TOKEN (the cache's scales). q, q_scales, out and out_strides are
 * as for reef_attention_prefill_int8. The call gathers the kv_len cached tokens of
 * every (sequence, kv head) into token-major rows in the workspace (at least
 * reef_attention_prefill_cache_workspace_bytes(p) bytes, 256-byte aligned; its
 * first part is the prefill's balanced-schedule workspace, so it must be
 * zero-filled before its first use, and every call leaves it ready for the next)
 * and runs the prefill attention over them. A page number outside [0, num_pages)
 * sets BAD_PAGE in status_word (optional) and reads as zero codes. */
size_t reef_attention_prefill_cache_workspace_bytes(const reef_attention_params *p);

reef_status reef_attention_prefill_int8_cache(
    const reef_attention_params *p, const int8_t *q, const reef_strides *q_strides,
    const float *q_scales, const int8_t *k_cache, const int8_t *v_cache, const float *k_scales,
    const float *v_scales, int64_t max_context, const int32_t *block_table,
    int64_t max_blocks_per_seq, int64_t num_pages, float *out, const reef_strides *out_strides,
    void *workspace, size_t workspace_bytes, uint32_t *status_word, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* REEF_HIP_ATTENTION_H */
