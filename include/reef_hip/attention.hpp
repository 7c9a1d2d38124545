// C++ face of the reef_hip C ABI for the Reef engine.
//
// The engine's operators report errors by throwing (quant.hpp:72-74,115;
// operator/attention.hpp:293-327; operator/activation.hpp:178-181,204-207).
// The C entry points return a reef_status instead; check() turns a status
// back into the engine's exception type and message, so host code written
// against the engine keeps its error handling when it calls the device path.
//
// Header-only; needs only attention.h and the HIP runtime headers.
#ifndef REEF_HIP_ATTENTION_HPP
#define REEF_HIP_ATTENTION_HPP

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "reef_hip/attention.h"

namespace reef_hip {

// REEF_HIP_ERROR: a HIP runtime call failed (the engine has no device, so no
// engine type corresponds).
struct hip_error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// REEF_UNSUPPORTED: a well-formed request that the kernels do not implement
// (head_dim other than 64 or 128, sizes past the 32-bit launch limits). An
// invalid_argument, as the engine would have had no reason to reject it.
struct unsupported : std::invalid_argument {
    using std::invalid_argument::invalid_argument;
};

// Throws the engine's exception for a status. `what` names the operation; the
// engine's own message is used where the engine has one for that condition.
inline void check(reef_status status, const char *what) {
    switch (status) {
    case REEF_OK:
        return;
    case REEF_INVALID_ARGUMENT:
        throw std::invalid_argument(std::string(what) + ": invalid argument");
    case REEF_NON_FINITE_INPUT:
        // quant.hpp:73
        throw std::invalid_argument("quantize_int8 requires finite values");
    case REEF_CAPACITY:
        // operator/attention.hpp:326
        throw std::length_error("KV cache capacity exceeded");
    case REEF_UNSUPPORTED:
        throw unsupported(std::string(what) + ": not supported by the device kernels");
    case REEF_OVERFLOW:
        // util.hpp:117-123
        throw std::overflow_error("safe_multiply product overflow");
    case REEF_HIP_ERROR:
    default:
        throw hip_error(std::string(what) + ": HIP runtime error");
    }
}

// Waits for `stream`, then throws for any condition the kernels flagged in the
// status word (non-finite input, a page number or length out of range, a full
// cache), clearing the word first so that the next call starts clean.
inline void check_status_word(uint32_t *status_word, hipStream_t stream, const char *what) {
    check(reef_read_status_word(status_word, 1, stream), what);
}

// --- quantization (quant.hpp) ------------------------------------------------------------

// quantize_rows (quant.hpp:112-133): per-row scales of a [rows, width] matrix.
// Throws like the engine once the stream reaches this call: invalid_argument
// for an invalid matrix (checked on the host, before launch) or for non-finite
// values (flagged by the kernel).
inline void quantize_rows(const float *x, int64_t rows, int64_t width, int64_t row_stride,
                          int8_t *q, float *scales, uint32_t *status_word, hipStream_t stream) {
    const reef_status s =
        reef_quantize_int8_per_token(x, rows, width, row_stride, q, scales, status_word, stream);
    if (s == REEF_INVALID_ARGUMENT) throw std::invalid_argument("quantize_rows requires a valid matrix");
    check(s, "quantize_rows");
    if (status_word) check_status_word(status_word, stream, "quantize_rows");
}

inline void quantize_per_tensor(const float *x, int64_t n, int8_t *q, float *scale,
                                uint32_t *status_word, hipStream_t stream) {
    check(reef_quantize_int8_per_tensor(x, n, q, scale, status_word, stream), "quantize_int8");
    if (status_word) check_status_word(status_word, stream, "quantize_int8");
}

inline void quantize_per_head(const float *x, int64_t batch, int64_t heads, int64_t tokens,
                              int64_t head_dim, const reef_strides *x_strides, int8_t *q,
                              float *scales, uint32_t *status_word, hipStream_t stream) {
    check(reef_quantize_int8_per_head(x, batch, heads, tokens, head_dim, x_strides, q, scales,
                                      status_word, stream),
          "quantize_int8");
    if (status_word) check_status_word(status_word, stream, "quantize_int8");
}

// --- attention (operator/attention.hpp) ----------------------------------------------------

// Attention::context (attention.hpp:374-432) for all batches and heads in one
// launch: the engine's query_start is kv_len - q_len (attention.hpp:415) and
// its window is LocalAttention's (attention.hpp:223-261), 0 for GlobalAttention.
// softmax_scale 1 reproduces the engine's unscaled scores (attention.hpp:104).
// The optional workspace (prefill_workspace_bytes(p) bytes, zero-filled once
// before first use) balances launches with few query tiles per compute unit.
inline size_t prefill_workspace_bytes(const reef_attention_params &p) {
    return reef_attention_prefill_workspace_bytes(&p);
}

inline void context(const reef_attention_params &p, const int8_t *q, const reef_strides *q_strides,
                    const int8_t *k, const reef_strides *k_strides, const int8_t *v,
                    const reef_strides *v_strides, const float *q_scales, const float *k_scales,
                    const float *v_scales, float *out, const reef_strides *out_strides,
                    hipStream_t stream, void *workspace = nullptr, size_t workspace_bytes = 0) {
    check(reef_attention_prefill_int8(&p, q, q_strides, k, k_strides, v, v_strides, q_scales,
                                      k_scales, v_scales, out, out_strides, workspace,
                                      workspace_bytes, stream),
          "attention context");
}

// Attention::forward with query_len > 1 on a non-empty cache (attention.hpp:354-372):
// the chunk's keys are already in the int8 cache (append_kv_cache); the chunk's
// queries attend over all p.kv_len cached keys. block_table nullptr: contiguous
// cache of max_context tokens per sequence; otherwise paged. The caller owns the
// workspace (prefill_cache_workspace_bytes(p) bytes).
inline size_t prefill_cache_workspace_bytes(const reef_attention_params &p) {
    return reef_attention_prefill_cache_workspace_bytes(&p);
}

inline void context_cache(const reef_attention_params &p, const int8_t *q,
                          const reef_strides *q_strides, const float *q_scales,
                          const int8_t *k_cache, const int8_t *v_cache, const float *k_scales,
                          const float *v_scales, int64_t max_context, const int32_t *block_table,
                          int64_t max_blocks_per_seq, int64_t num_pages, float *out,
                          const reef_strides *out_strides, void *workspace,
                          size_t workspace_bytes, uint32_t *status_word, hipStream_t stream) {
    check(reef_attention_prefill_int8_cache(&p, q, q_strides, q_scales, k_cache, v_cache,
                                            k_scales, v_scales, max_context, block_table,
                                            max_blocks_per_seq, num_pages, out, out_strides,
                                            workspace, workspace_bytes, status_word, stream),
          "attention context over the cache");
}

// One decode step over a contiguous int8 cache. The caller owns the workspace
// (decode_workspace_bytes(p) bytes); see attention.h for the cache layout.
inline size_t decode_workspace_bytes(const reef_decode_params &p) {
    return reef_attention_decode_workspace_bytes(&p);
}

inline void decode(const reef_decode_params &p, const int8_t *q, const float *q_scales,
                   const int8_t *k_cache, const int8_t *v_cache, const float *k_scales,
                   const float *v_scales, const int32_t *context_lens, float *out,
                   void *workspace, size_t workspace_bytes, uint32_t *status_word,
                   hipStream_t stream) {
    check(reef_attention_decode_int8(&p, q, q_scales, k_cache, v_cache, k_scales, v_scales,
                                     context_lens, out, workspace, workspace_bytes, status_word,
                                     stream),
          "attention decode");
}

inline void decode_paged(const reef_decode_params &p, const int8_t *q, const float *q_scales,
                         const int8_t *k_pages, const int8_t *v_pages, const float *k_scale_pages,
                         const float *v_scale_pages, const int32_t *block_table,
                         int64_t max_blocks_per_seq, int64_t num_pages,
                         const int32_t *context_lens, float *out, void *workspace,
                         size_t workspace_bytes, uint32_t *status_word, hipStream_t stream) {
    check(reef_attention_decode_int8_paged(&p, q, q_scales, k_pages, v_pages, k_scale_pages,
                                           v_scale_pages, block_table, max_blocks_per_seq,
                                           num_pages, context_lens, out, workspace,
                                           workspace_bytes, status_word, stream),
          "attention decode");
}

// Attention::append_kv_cache (attention.hpp:290-352) on the int8 cache, in place;
// a full cache throws std::length_error like the engine once the status word is
// checked.
inline void append_kv_cache(const reef_kv_append_params &p, const float *k_new,
                            const reef_strides *k_strides, const float *v_new,
                            const reef_strides *v_strides, const int32_t *start_positions,
                            int8_t *k_cache, int8_t *v_cache, float *k_scales, float *v_scales,
                            int32_t *context_lens, uint32_t *status_word, hipStream_t stream) {
    check(reef_kv_append_int8(&p, k_new, k_strides, v_new, v_strides, start_positions, k_cache,
                              v_cache, k_scales, v_scales, context_lens, status_word, stream),
          "append_kv_cache");
}

// attend_head_int8 (int8.hpp:250-279) for every (batch, head), bit-identical.
inline void attend_int8_integer(const reef_attention_params &p, const int8_t *q,
                                const reef_strides *q_strides, const int8_t *k,
                                const reef_strides *k_strides, const int8_t *v,
                                const reef_strides *v_strides, unsigned score_shift,
                                const uint16_t *table, unsigned out_shift, int8_t *out,
                                const reef_strides *out_strides, hipStream_t stream) {
    check(reef_attention_int8_integer(&p, q, q_strides, k, k_strides, v, v_strides, score_shift,
                                      table, out_shift, out, out_strides, stream),
          "attend_head_int8");
}

// linear() with a QuantizedWeight (operator/linear.hpp:106-132), bit-identical.
inline void linear_w8a8(const float *x, int64_t rows, int64_t in_features, int64_t x_row_stride,
                        const int8_t *weight, const float *w_scales, const float *bias,
                        int64_t out_features, float *y, int64_t y_row_stride, void *workspace,
                        size_t workspace_bytes, uint32_t *status_word, hipStream_t stream) {
    check(reef_linear_w8a8(x, rows, in_features, x_row_stride, weight, w_scales, bias,
                           out_features, y, y_row_stride, workspace, workspace_bytes, status_word,
                           stream),
          "linear");
}

}  // namespace reef_hip

#endif  // REEF_HIP_ATTENTION_HPP
