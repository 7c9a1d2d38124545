// C entry points over the Reef engine's own header-only functions, so the
// tests can compare the oracle restatement (reef_oracle.c) with the engine
// itself on the same inputs, and bench.py can time the engine's CPU path.
//
// TEST INFRASTRUCTURE ONLY. oracle/Makefile compiles this file against the
// engine headers where they lie in the reference checkout
// (inference-engine/reference/cpp/include) into oracle/_ref/libref.so; the
// headers are never copied. Every wrapper turns the engine's exceptions into
// a nonzero status.
#include "inference_engine/int8.hpp"
#include "inference_engine/math.hpp"
#include "inference_engine/operator/activation.hpp"
#include "inference_engine/operator/attention.hpp"
#include "inference_engine/quant.hpp"
#include "inference_engine/tensor.hpp"

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <exception>
#include <optional>
#include <vector>

namespace ie = inference_engine;

namespace {

template <typename T>
ie::Tensor<T> matrix(const T* data, std::size_t rows, std::size_t cols) {
    return ie::Tensor<T>{{rows, cols}, std::vector<T>(data, data + rows * cols)};
}

std::optional<std::size_t> window_of(std::int64_t window) {
    return window > 0 ? std::optional<std::size_t>(static_cast<std::size_t>(window))
                      : std::nullopt;
}

template <typename F> int guarded(F&& body) {
    try {
        body();
        return 0;
    } catch (const std::invalid_argument&) {
        return 1;
    } catch (const std::exception&) {
        return 3;
    }
}

} // namespace

extern "C" {

float ref_int8_scale(float max_magnitude) { return ie::int8_scale(max_magnitude); }

int ref_quantize_int8(float value, float scale, std::int8_t* out) {
    return guarded([&] { *out = ie::quantize_int8(value, scale); });
}

int ref_quantize_rows(const float* x, std::size_t rows, std::size_t width, std::int8_t* q,
                      float* scales) {
    return guarded([&] {
        const ie::QuantizedWeight<float> r = ie::quantize_rows(matrix(x, rows, width));
        std::memcpy(q, r.values.values.data(), rows * width);
        std::memcpy(scales, r.scales.data(), rows * sizeof(float));
    });
}

float ref_exp_nonpositive(float x) { return ie::exp_nonpositive(x); }

int ref_causal_visibility(std::size_t queries, std::size_t keys, std::size_t query_start,
                          std::int64_t window, std::uint8_t* out) {
    return guarded([&] {
        const ie::Tensor<bool> v =
            ie::causal_visibility(queries, keys, query_start, window_of(window));
        for (std::size_t i = 0; i < v.values.size(); ++i) {
            out[i] = v.values[i] ? 1 : 0;
        }
    });
}

// matmul<int8, int32>(q, transpose(k)): the engine's integer score product.
int ref_qk_i32(const std::int8_t* q, const std::int8_t* k, std::size_t sq, std::size_t sk,
               std::size_t d, std::int32_t* acc) {
    return guarded([&] {
        const ie::Tensor<std::int32_t> s = ie::matmul<std::int8_t, std::int32_t>(
            matrix(q, sq, d), ie::transpose(matrix(k, sk, d), 0, 1));
        std::memcpy(acc, s.values.data(), sq * sk * sizeof(std::int32_t));
    });
}

int ref_masked_softmax(const float* scores, std::size_t rows, std::size_t keys,
                       const std::uint8_t* visible, float* out) {
    return guarded([&] {
        ie::Tensor<bool> mask{{rows, keys}, std::vector<bool>(rows * keys)};
        for (std::size_t i = 0; i < rows * keys; ++i) {
            mask.values[i] = visible[i] != 0;
        }
        const ie::Tensor<float> p = ie::masked_softmax(matrix(scores, rows, keys), mask);
        std::memcpy(out, p.values.data(), rows * keys * sizeof(float));
    });
}

int ref_attend_head(const float* q, const float* k, const float* v, std::size_t sq,
                    std::size_t sk, std::size_t d, std::size_t query_start, std::int64_t window,
                    float* out) {
    return guarded([&] {
        const ie::Tensor<float> y =
            ie::attend_head(matrix(q, sq, d), matrix(k, sk, d), matrix(v, sk, d),
                            ie::causal_visibility(sq, sk, query_start, window_of(window)));
        std::memcpy(out, y.values.data(), sq * d * sizeof(float));
    });
}

void ref_exp_table(std::uint16_t* out) {
    const ie::ExpTable t = ie::exp_table();
    std::memcpy(out, t.data(), sizeof(t));
}

int ref_attend_head_int8(const std::int8_t* q, const std::int8_t* k, const std::int8_t* v,
                         std::size_t sq, std::size_t sk, std::size_t d, std::size_t query_start,
                         std::int64_t window, unsigned score_shift, unsigned out_shift,
                         std::int8_t* out) {
    return guarded([&] {
        const ie::Tensor<std::int8_t> y = ie::attend_head_int8(
            matrix(q, sq, d), matrix(k, sk, d), matrix(v, sk, d),
            ie::causal_visibility(sq, sk, query_start, window_of(window)), score_shift,
            ie::exp_table(), out_shift);
        std::memcpy(out, y.values.data(), sq * d);
    });
}

// One head of int8 attention with a float softmax, composed only of engine
// calls: matmul<int8, int32> scores, float(acc) * (s_q * s_k) dequantization
// (the order of operator/linear.hpp:125-127) times softmax_scale,
// masked_softmax, and the float matmul with the dequantized values. Scales:
// q_scales [sq], k_scales and v_scales [sk] (a per-tensor or per-head scale is
// repeated). This is the engine's CPU path for the path's golden.
int ref_attention_int8_head(const std::int8_t* q, const std::int8_t* k, const std::int8_t* v,
                            const float* q_scales, const float* k_scales, const float* v_scales,
                            std::size_t sq, std::size_t sk, std::size_t d,
                            std::size_t query_start, std::int64_t window, float softmax_scale,
                            float* out) {
    return guarded([&] {
        const ie::Tensor<std::int32_t> acc = ie::matmul<std::int8_t, std::int32_t>(
            matrix(q, sq, d), ie::transpose(matrix(k, sk, d), 0, 1));
        ie::Tensor<float> scores{{sq, sk}, std::vector<float>(sq * sk)};
        for (std::size_t i = 0; i < sq; ++i) {
            for (std::size_t j = 0; j < sk; ++j) {
                scores.values[i * sk + j] =
                    (static_cast<float>(acc.values[i * sk + j]) * (q_scales[i] * k_scales[j])) *
                    softmax_scale;
            }
        }
        ie::Tensor<float> values{{sk, d}, std::vector<float>(sk * d)};
        for (std::size_t j = 0; j < sk; ++j) {
            for (std::size_t c = 0; c < d; ++c) {
                values.values[j * d + c] = static_cast<float>(v[j * d + c]) * v_scales[j];
            }
        }
        const ie::Tensor<float> y = ie::matmul(
            ie::masked_softmax(scores,
                               ie::causal_visibility(sq, sk, query_start, window_of(window))),
            values);
        std::memcpy(out, y.values.data(), sq * d * sizeof(float));
    });
}

} // extern "C"
