// GPT-Neo drop-in (test infrastructure): the Reef engine's own model, compiled
// from its headers, with the attention of every layer answered by the reef_hip
// device path from inside the engine's call stack:
//
//   GPTNeo::forward (model.hpp:86-112) -> Block::forward (operator/block.hpp:97-108)
//     -> Attention::forward (operator/attention.hpp:354-372): the engine projects
//        q, k and v and appends k and v to its own float cache, then calls
//        Attention::context (:374-432), which for the device model is the
//        specialization below: the new key and value rows go into a device int8
//        cache (reef_hip::append_kv_cache), and a prompt is attended with
//        reef_hip::context (int8 prefill kernel), a later chunk of a prompt with
//        reef_hip::context_cache (the prefill over the cache) or one token with
//        reef_hip::decode (int8 decode kernel over the cache). Layer kind
//        (GlobalAttention or LocalAttention and its window) comes from the
//        engine's own visibility policy.
//
// The device model is GPTNeo<double> over the float weights of random_gpt_neo
// (weights.hpp:407) widened to double: the engine's float model (GPTNeo<float>)
// runs in the same program untouched. Checks:
//   1. every attention call of the device model (prefill and decode, global and
//      local layers, every position) against the engine's own int8 attention
//      composition on the same call's q and cache (quantize_rows per token,
//      matmul<int8, int32>, float(acc) * (s_q * s_k), masked_softmax, times the
//      dequantized values): max |diff| <= kCallTol, the path's tolerance;
//   2. prefill == decode, as test_gpt_neo.cpp:50-61 and :97-107 check for the
//      engine (there bitwise): for every prompt length, the logits of the whole
//      prompt in one call against those of the same tokens one call at a time,
//      max |diff| <= kPrefillDecodeTol. Both kernels agree with the int8
//      composition to about 1e-6, so the int8 codes of later layers agree too; a
//      difference of one code step anywhere would show as about 1e-2 here;
//   3. the device model's prompt logits against the engine's float model: int8 q,
//      k and v per token, compounded over the layers and amplified by GPT-Neo's
//      unscaled scores (attention.hpp:104); the bound is the engine's own for its
//      W8A8 model (test_gpt_neo.cpp:167-187), under kModelFrac of the largest
//      logit.
//   4. a prompt fed in chunks: the later chunks attend over the earlier chunks'
//      cached keys through reef_hip::context_cache (the prefill over the device
//      cache); the logits after every chunk against those of one token at a time,
//      max |diff| <= kPrefillDecodeTol;
//   5. greedy generation of kGenerate tokens, reported.
// Exit status 0 when checks 1-4 pass. Built by `make -C oracle gpt_neo` into
// oracle/_ref/ (it needs the engine headers); run on a machine with a GPU.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <map>
#include <memory>
#include <stdexcept>
#include <vector>

#include "inference_engine/model.hpp"
#include "inference_engine/quant.hpp"
#include "inference_engine/weights.hpp"
#include "reef_hip/attention.hpp"

namespace ie = inference_engine;

namespace {

constexpr double kCallTol = 1e-3;
constexpr double kPrefillDecodeTol = 1e-3;
constexpr double kModelFrac = 0.05;
constexpr std::size_t kGenerate = 8;

void hip_ok(hipError_t e, const char *what) {
    if (e != hipSuccess) throw reef_hip::hip_error(what);
}

template <typename T>
T *dev_alloc(size_t count) {
    void *p = nullptr;
    hip_ok(hipMalloc(&p, std::max<size_t>(count * sizeof(T), 256)), "hipMalloc");
    return static_cast<T *>(p);
}

// Device state of one attention layer: the int8 cache (codes, transposed value
// pages, per-token scales) of up to `cap` positions, and the buffers of one call.
struct DeviceLayer {
    int64_t heads = 0, dim = 0, cap = 0;
    int8_t *k = nullptr, *v = nullptr;  // [1, H, cap, D], [1, H, cap / 16, D, 16]
    float *ks = nullptr, *vs = nullptr;  // [1, H, cap]
    int32_t *start = nullptr, *lens = nullptr;
    float *qf = nullptr, *kf = nullptr, *vf = nullptr, *out = nullptr;  // [H, cap, D]
    int8_t *q8 = nullptr, *k8 = nullptr, *v8 = nullptr;                 // [H * cap, D]
    float *qs = nullptr, *ks8 = nullptr, *vs8 = nullptr;                // [H * cap]
    void *pws = nullptr, *dws = nullptr, *cws = nullptr;
    size_t pws_bytes = 0, dws_bytes = 0, cws_bytes = 0;
    uint32_t *status = nullptr;
};

hipStream_t g_stream = nullptr;
int64_t g_capacity = 0;
std::map<const void *, std::unique_ptr<DeviceLayer>> g_layers;
long g_prefill_calls = 0, g_decode_calls = 0, g_chunk_calls = 0;
// Largest |device - engine int8 composition| of an attention call, per call kind
// (0 prefill, 1 decode) and layer kind (0 global, 1 local).
double g_att_err[3][2] = {{0, 0}, {0, 0}, {0, 0}};  // [prompt, decode, chunk][global, local]

DeviceLayer &layer_for(const void *attention, int64_t heads, int64_t dim) {
    auto &slot = g_layers[attention];
    if (!slot) {
        auto L = std::make_unique<DeviceLayer>();
        L->heads = heads;
        L->dim = dim;
        L->cap = g_capacity;
        const size_t hcd = (size_t)heads * g_capacity * dim, hc = (size_t)heads * g_capacity;
        L->k = dev_alloc<int8_t>(hcd);
        L->v = dev_alloc<int8_t>(hcd);
        L->ks = dev_alloc<float>(hc);
        L->vs = dev_alloc<float>(hc);
        L->start = dev_alloc<int32_t>(1);
        L->lens = dev_alloc<int32_t>(1);
        L->qf = dev_alloc<float>(hcd);
        L->kf = dev_alloc<float>(hcd);
        L->vf = dev_alloc<float>(hcd);
        L->out = dev_alloc<float>(hcd);
        L->q8 = dev_alloc<int8_t>(hcd);
        L->k8 = dev_alloc<int8_t>(hcd);
        L->v8 = dev_alloc<int8_t>(hcd);
        L->qs = dev_alloc<float>(hc);
        L->ks8 = dev_alloc<float>(hc);
        L->vs8 = dev_alloc<float>(hc);
        L->status = dev_alloc<uint32_t>(1);
        hip_ok(hipMemset(L->status, 0, 4), "hipMemset");
        reef_attention_params pp{1, heads, heads, g_capacity, g_capacity, dim, 0, 0, 1.0f,
                                 REEF_SCALE_PER_TOKEN, REEF_SCALE_PER_TOKEN, 0};
        L->pws_bytes = reef_hip::prefill_workspace_bytes(pp);
        if (L->pws_bytes) {
            L->pws = dev_alloc<uint8_t>(L->pws_bytes);
            hip_ok(hipMemset(L->pws, 0, L->pws_bytes), "hipMemset");
        }
        L->cws_bytes = reef_hip::prefill_cache_workspace_bytes(pp);
        L->cws = dev_alloc<uint8_t>(L->cws_bytes);
        hip_ok(hipMemset(L->cws, 0, L->cws_bytes), "hipMemset");
        reef_decode_params dp{1, heads, heads, dim, g_capacity, 0, 1.0f, REEF_SCALE_PER_TOKEN, 0, 0};
        L->dws_bytes = reef_hip::decode_workspace_bytes(dp);
        L->dws = dev_alloc<uint8_t>(L->dws_bytes);
        hip_ok(hipMemset(L->dws, 0, L->dws_bytes), "hipMemset");
        slot = std::move(L);
    }
    return *slot;
}

// [1, H, rows, D] double -> fp32 [H, rows, D] on the device.
void put_rows(const ie::Tensor<double> &t, float *dst) {
    std::vector<float> h(t.values.size());
    for (size_t i = 0; i < h.size(); ++i) h[i] = (float)t.values[i];
    hip_ok(hipMemcpy(dst, h.data(), h.size() * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
}

}  // namespace

namespace inference_engine {

// Attention::context of the device model: the engine has projected this call's
// q, k and v and appended k and v to its float cache (attention.hpp:354-360); the
// same k and v rows go into the device int8 cache at the same positions, and the
// queries are attended on the device.
template <>
Tensor<double> Attention<double>::context(const Qkv<double> &qkv) const {
    const int64_t H = (int64_t)qkv.query.shape[1], q_len = (int64_t)qkv.query.shape[2],
                  D = (int64_t)qkv.query.shape[3];
    const int64_t key_len = (int64_t)cache_.key.shape[2];
    const int64_t start = key_len - q_len;  // attention.hpp:415
    // The layer's window from its own visibility policy: the last query sees
    // min(window, key_len) keys.
    const Tensor<bool> last = visibility(1, (size_t)key_len, (size_t)key_len - 1);
    const int64_t seen = std::count(last.values.begin(), last.values.end(), true);
    const int64_t window = seen < key_len ? seen : 0;
    if (key_len > g_capacity) throw std::length_error("KV cache capacity exceeded");

    DeviceLayer &L = layer_for(this, H, D);
    hipStream_t s = g_stream;
    put_rows(qkv.query, L.qf);
    put_rows(qkv.key, L.kf);
    put_rows(qkv.value, L.vf);
    const int32_t start32 = (int32_t)start;
    hip_ok(hipMemcpy(L.start, &start32, 4, hipMemcpyHostToDevice), "hipMemcpy");
    const reef_kv_append_params ap{1, H, D, q_len, L.cap};
    reef_hip::append_kv_cache(ap, L.kf, nullptr, L.vf, nullptr, L.start, L.k, L.v, L.ks, L.vs,
                              L.lens, L.status, s);
    reef_hip::check_status_word(L.status, s, "append_kv_cache");
    reef_hip::quantize_rows(L.qf, H * q_len, D, D, L.q8, L.qs, L.status, s);
    if (q_len == 1) {
        // One token: decode over the device cache of key_len positions.
        const reef_decode_params dp{1, H, H, D, L.cap, window, 1.0f, REEF_SCALE_PER_TOKEN, 0, 0};
        reef_hip::decode(dp, L.q8, L.qs, L.k, L.v, L.ks, L.vs, L.lens, L.out, L.dws, L.dws_bytes,
                         L.status, s);
        reef_hip::check_status_word(L.status, s, "decode");
        ++g_decode_calls;
    } else if (start > 0) {
        // A later chunk of a prompt (or a multi-token turn): its queries attend over
        // every cached position, read from the device cache.
        const reef_attention_params p{1, H, H, q_len, key_len, D, start, window, 1.0f,
                                      REEF_SCALE_PER_TOKEN, REEF_SCALE_PER_TOKEN, 0};
        reef_hip::context_cache(p, L.q8, nullptr, L.qs, L.k, L.v, L.ks, L.vs, L.cap, nullptr, 0,
                                0, L.out, nullptr, L.cws, L.cws_bytes, L.status, s);
        reef_hip::check_status_word(L.status, s, "context_cache");
        ++g_chunk_calls;
    } else {
        // A prompt: the prefill kernel attends it from its own int8 rows (token-major
        // values), the same codes the cache holds.
        reef_hip::quantize_rows(L.kf, H * q_len, D, D, L.k8, L.ks8, L.status, s);
        reef_hip::quantize_rows(L.vf, H * q_len, D, D, L.v8, L.vs8, L.status, s);
        const reef_attention_params p{1, H, H, q_len, q_len, D, 0, window, 1.0f,
                                      REEF_SCALE_PER_TOKEN, REEF_SCALE_PER_TOKEN, 0};
        reef_hip::context(p, L.q8, nullptr, L.k8, nullptr, L.v8, nullptr, L.qs, L.ks8, L.vs8, L.out,
                          nullptr, s, L.pws, L.pws_bytes);
        ++g_prefill_calls;
    }
    std::vector<float> o((size_t)(H * q_len * D));
    hip_ok(hipStreamSynchronize(s), "hipStreamSynchronize");
    hip_ok(hipMemcpy(o.data(), L.out, o.size() * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy");
    Tensor<double> mixed{{1, (size_t)H, (size_t)q_len, (size_t)D}, std::vector<double>(o.size())};
    for (size_t i = 0; i < o.size(); ++i) mixed.values[i] = o[i];
    // The engine's int8 attention composition of the same call (check 1): the
    // call's queries and the whole cache, quantized per row as float.
    const Tensor<bool> visible = visibility((size_t)q_len, (size_t)key_len, (size_t)start);
    auto head_f32 = [](const Tensor<double> &t, int64_t h) {
        const size_t rows = t.shape[2], cols = t.shape[3];
        Tensor<float> m{{rows, cols}, std::vector<float>(rows * cols)};
        for (size_t i = 0; i < rows * cols; ++i) m.values[i] = (float)t.values[h * rows * cols + i];
        return m;
    };
    double err = 0.0;
    for (int64_t h = 0; h < H; ++h) {
        const QuantizedWeight<float> q8 = quantize_rows(head_f32(qkv.query, h));
        const QuantizedWeight<float> k8 = quantize_rows(head_f32(cache_.key, h));
        const QuantizedWeight<float> v8 = quantize_rows(head_f32(cache_.value, h));
        const Tensor<std::int32_t> acc =
            matmul<std::int8_t, std::int32_t>(q8.values, transpose(k8.values, 0, 1));
        Tensor<float> scores{{(size_t)q_len, (size_t)key_len},
                             std::vector<float>((size_t)(q_len * key_len))};
        for (int64_t i = 0; i < q_len; ++i)
            for (int64_t j = 0; j < key_len; ++j)
                scores.values[i * key_len + j] =
                    static_cast<float>(acc.values[i * key_len + j]) * (q8.scales[i] * k8.scales[j]);
        Tensor<float> values{{(size_t)key_len, (size_t)D}, std::vector<float>((size_t)(key_len * D))};
        for (int64_t j = 0; j < key_len; ++j)
            for (int64_t c = 0; c < D; ++c)
                values.values[j * D + c] =
                    static_cast<float>(v8.values.values[j * D + c]) * v8.scales[j];
        const Tensor<float> ref = matmul(masked_softmax(scores, visible), values);
        for (size_t i = 0; i < ref.values.size(); ++i)
            err = std::max(err, std::fabs((double)ref.values[i] -
                                          mixed.values[h * ref.values.size() + i]));
    }
    double &slot = g_att_err[q_len == 1 ? 1 : start > 0 ? 2 : 0][window > 0 ? 1 : 0];
    slot = std::max(slot, err);
    return mixed;
}

}  // namespace inference_engine

namespace {

ie::Tensor<double> widen(const ie::Tensor<float> &t) {
    return ie::Tensor<double>{t.shape, std::vector<double>(t.values.begin(), t.values.end())};
}

ie::ModelWeights<double> widen(const ie::ModelWeights<float> &w) {
    ie::ModelWeights<double> d;
    d.config = w.config;
    d.wte = widen(w.wte);
    d.wpe = widen(w.wpe);
    for (const auto &l : w.layers) {
        ie::LayerWeights<double> x{};
        x.ln_1_weight = widen(l.ln_1_weight);
        x.ln_1_bias = widen(l.ln_1_bias);
        x.attention.num_heads = l.attention.num_heads;
        x.attention.query_weights = widen(l.attention.query_weights);
        x.attention.key_weights = widen(l.attention.key_weights);
        x.attention.value_weights = widen(l.attention.value_weights);
        x.attention.output_weights = widen(l.attention.output_weights);
        x.attention.output_bias = widen(l.attention.output_bias);
        x.ln_2_weight = widen(l.ln_2_weight);
        x.ln_2_bias = widen(l.ln_2_bias);
        x.mlp.input_size = l.mlp.input_size;
        x.mlp.inner_size = l.mlp.inner_size;
        x.mlp.c_fc_weight = widen(l.mlp.c_fc_weight);
        x.mlp.c_fc_bias = widen(l.mlp.c_fc_bias);
        x.mlp.c_proj_weight = widen(l.mlp.c_proj_weight);
        x.mlp.c_proj_bias = widen(l.mlp.c_proj_bias);
        d.layers.push_back(std::move(x));
    }
    d.ln_f_weight = widen(w.ln_f_weight);
    d.ln_f_bias = widen(w.ln_f_bias);
    return d;
}

template <typename A, typename B>
double max_diff(const ie::Tensor<A> &a, const ie::Tensor<B> &b) {
    if (a.values.size() != b.values.size()) return INFINITY;
    double m = 0.0;
    for (size_t i = 0; i < a.values.size(); ++i)
        m = std::max(m, std::fabs((double)a.values[i] - (double)b.values[i]));
    return m;
}

}  // namespace

int main() {
    try {
        // Four heads of 64 (the device kernels take head_dim 64 or 128), four layers
        // alternating global and local attention (window 24), 96 positions.
        ie::GptNeoConfig cfg;
        cfg.vocab_size = 512;
        cfg.max_positions = 96;
        cfg.hidden_size = 256;
        cfg.num_layers = 4;
        cfg.num_heads = 4;
        cfg.inner_size = 1024;
        cfg.window_size = 24;
        g_capacity = 96;  // a multiple of 16 holding every position
        hip_ok(hipStreamCreate(&g_stream), "hipStreamCreate");
        const ie::ModelWeights<float> wf = ie::random_gpt_neo(cfg, 20240611u);
        const ie::ModelWeights<double> wd = widen(wf);
        std::vector<std::uint32_t> prompt;
        for (std::uint32_t i = 0; i < 40; ++i) prompt.push_back((i * 73u + 11u) % 512u);

        // 1. prefill == decode on the device model, every prompt length.
        ie::GPTNeo<double> stepper(wd);
        std::vector<ie::Tensor<double>> stepped;
        for (std::uint32_t t : prompt) stepped.push_back(stepper.forward({t}));
        double pd = 0.0;
        for (size_t len = 1; len <= prompt.size(); ++len) {
            ie::GPTNeo<double> m(wd);
            const ie::Tensor<double> pre =
                m.forward(ie::TokenIds(prompt.begin(), prompt.begin() + (std::ptrdiff_t)len));
            pd = std::max(pd, max_diff(pre, stepped[len - 1]));
        }
        // 1b. a prompt fed in chunks (the later chunks attend over the cached keys of
        // the earlier ones, from the device cache) == the whole prompt == one token at
        // a time, after every chunk.
        const std::vector<std::vector<size_t>> schedules = {
            {17, 13, 10}, {1, 39}, {39, 1}, {20, 20}, {2, 3, 5, 7, 11, 12}, {25, 1, 14}};
        double pc = 0.0;
        for (const auto &chunks : schedules) {
            ie::GPTNeo<double> m(wd);
            size_t at = 0;
            for (size_t n : chunks) {
                const ie::Tensor<double> out = m.forward(ie::TokenIds(
                    prompt.begin() + (std::ptrdiff_t)at, prompt.begin() + (std::ptrdiff_t)(at + n)));
                at += n;
                pc = std::max(pc, max_diff(out, stepped[at - 1]));
            }
        }
        // 2. the device model against the engine's float model, prompt logits.
        ie::GPTNeo<float> engine(wf);
        ie::GPTNeo<double> device(wd);
        const ie::Tensor<float> le = engine.forward(prompt);
        const ie::Tensor<double> ld = device.forward(prompt);
        const double de = max_diff(ld, le);
        double scale = 0.0;
        for (float x : le.values) scale = std::max(scale, (double)std::fabs(x));
        // 3. greedy generation.
        const ie::TokenIds ge = engine.generate(prompt, kGenerate);
        const ie::TokenIds gd = device.generate(prompt, kGenerate);
        size_t same = 0;
        while (same < kGenerate && ge[same] == gd[same]) ++same;

        double call_err = 0.0;
        for (const auto &row : g_att_err) call_err = std::max(call_err, std::max(row[0], row[1]));
        const bool ok1 = call_err <= kCallTol, ok2 = pd <= kPrefillDecodeTol,
                   ok3 = de <= kModelFrac * scale, ok4 = pc <= kPrefillDecodeTol;
        std::printf("%s every attention call vs the engine's int8 composition, max |diff| %.3e "
                    "(bound %.0e): prompt global %.3e local %.3e, decode global %.3e local %.3e, "
                    "later chunk global %.3e local %.3e\n",
                    ok1 ? "ok  " : "FAIL", call_err, kCallTol, g_att_err[0][0], g_att_err[0][1],
                    g_att_err[1][0], g_att_err[1][1], g_att_err[2][0], g_att_err[2][1]);
        std::printf("%s prefill == decode (40 prompt lengths), max |dlogit| %.3e (bound %.0e)\n",
                    ok2 ? "ok  " : "FAIL", pd, kPrefillDecodeTol);
        std::printf("%s chunked prompt == one token at a time (%zu chunk schedules), max |dlogit| "
                    "%.3e (bound %.0e)\n", ok4 ? "ok  " : "FAIL", schedules.size(), pc,
                    kPrefillDecodeTol);
        std::printf("%s device vs engine float model, max |dlogit| %.3e (bound %.3e)\n",
                    ok3 ? "ok  " : "FAIL", de, kModelFrac * scale);
        std::printf("info greedy %zu tokens: first %zu identical to the engine's\n", kGenerate,
                    same);
        std::printf("info device calls: %ld prefill, %ld decode, %ld later-chunk\n",
                    g_prefill_calls, g_decode_calls, g_chunk_calls);
        std::printf("{\"call_max_diff\": %.6e, \"prefill_decode_max_diff\": %.6e, "
                    "\"chunked_max_diff\": %.6e, "
                    "\"engine_max_diff\": %.6e, \"max_logit\": %.6e, \"greedy_same_prefix\": %zu, "
                    "\"prefill_calls\": %ld, \"decode_calls\": %ld, \"chunk_calls\": %ld}\n",
                    call_err, pd, pc, de, scale, same, g_prefill_calls, g_decode_calls,
                    g_chunk_calls);
        return ok1 && ok2 && ok3 && ok4 && g_prefill_calls > 0 && g_decode_calls > 0 &&
                       g_chunk_calls > 0
                   ? 0
                   : 1;
    } catch (const std::exception &e) {
        std::printf("FAIL exception: %s\n", e.what());
        return 2;
    }
}
