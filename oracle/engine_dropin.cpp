// Drop-in check (test infrastructure): the Reef engine's own operators, compiled
// from its headers, beside the reef_hip device path called through
// include/reef_hip/attention.hpp, on the same inputs.
//
//   1. Attention::context (operator/attention.hpp:374-432), GlobalAttention and
//      LocalAttention: per head, the engine's int8 attention composition
//      (quantize_rows per token, matmul<int8, int32>, float(acc) * (s_q * s_k),
//      masked_softmax with causal_visibility, times the dequantized values)
//      against reef_hip::context with per-token scales: max |diff| <= 1e-3.
//   2. The same prompt appended to the device int8 cache with
//      reef_hip::append_kv_cache and its last query decoded with reef_hip::decode
//      (prefill == decode): against the engine's last row.
//   3. attend_head_int8 (int8.hpp:250-279) against reef_hip::attend_int8_integer:
//      bit-identical.
//   4. linear() with a QuantizedWeight (operator/linear.hpp:106-132) against
//      reef_hip::linear_w8a8: bit-identical.
//
// Exit status 0 when every check passes. Built by `make -C oracle dropin` into
// oracle/_ref/ (it needs the engine headers); run on a machine with a GPU.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "inference_engine/int8.hpp"
#include "inference_engine/operator/attention.hpp"
#include "inference_engine/operator/linear.hpp"
#include "inference_engine/quant.hpp"
#include "reef_hip/attention.hpp"

namespace ie = inference_engine;

namespace {

int failures = 0;

void report(const char *name, bool ok, double err) {
    std::printf("%s %-52s max|diff| %.3e\n", ok ? "ok  " : "FAIL", name, err);
    if (!ok) ++failures;
}

template <typename T>
struct Dev {
    T *p = nullptr;
    size_t n = 0;
    explicit Dev(size_t count) : n(count) {
        if (hipMalloc(&p, count * sizeof(T) + 16) != hipSuccess) throw std::runtime_error("hipMalloc");
    }
    Dev(const std::vector<T> &h) : Dev(h.size()) { put(h); }
    ~Dev() { (void)hipFree(p); }
    void put(const std::vector<T> &h) {
        if (hipMemcpy(p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice) != hipSuccess)
            throw std::runtime_error("hipMemcpy");
    }
    std::vector<T> get() const {
        std::vector<T> h(n);
        if (hipMemcpy(h.data(), p, n * sizeof(T), hipMemcpyDeviceToHost) != hipSuccess)
            throw std::runtime_error("hipMemcpy");
        return h;
    }
};

std::vector<float> normals(std::mt19937 &g, size_t n, float scale) {
    std::normal_distribution<float> d(0.0f, 1.0f);
    std::vector<float> v(n);
    for (auto &x : v) x = d(g) * scale;
    return v;
}

ie::Tensor<float> rows_of(const std::vector<float> &v, size_t head, size_t len, size_t dim) {
    return ie::Tensor<float>{{len, dim},
                             std::vector<float>(v.begin() + head * len * dim,
                                                v.begin() + (head + 1) * len * dim)};
}

// The engine's int8 attention for one head (the composition a device call replaces).
std::vector<float> engine_head(const ie::QuantizedWeight<float> &q, const ie::QuantizedWeight<float> &k,
                               const ie::QuantizedWeight<float> &v, size_t start,
                               std::optional<std::size_t> window) {
    const size_t sq = q.values.shape[0], sk = k.values.shape[0], d = q.values.shape[1];
    const ie::Tensor<std::int32_t> acc =
        ie::matmul<std::int8_t, std::int32_t>(q.values, ie::transpose(k.values, 0, 1));
    ie::Tensor<float> scores{{sq, sk}, std::vector<float>(sq * sk)};
    for (size_t i = 0; i < sq; ++i)
        for (size_t j = 0; j < sk; ++j)
            scores.values[i * sk + j] =
                static_cast<float>(acc.values[i * sk + j]) * (q.scales[i] * k.scales[j]);
    ie::Tensor<float> values{{sk, d}, std::vector<float>(sk * d)};
    for (size_t j = 0; j < sk; ++j)
        for (size_t c = 0; c < d; ++c)
            values.values[j * d + c] = static_cast<float>(v.values.values[j * d + c]) * v.scales[j];
    return ie::matmul(ie::masked_softmax(scores, ie::causal_visibility(sq, sk, start, window)),
                      values)
        .values;
}

void check_context_and_decode(std::mt19937 &g, int64_t window) {
    const size_t H = 4, S = 300, D = 64, L = 320;  // cache capacity: a multiple of 16
    // Unscaled scores as the engine's attend_head (attention.hpp:104): keep them moderate.
    const std::vector<float> qf = normals(g, H * S * D, 0.1f), kf = normals(g, H * S * D, 0.1f),
                             vf = normals(g, H * S * D, 1.0f);
    std::vector<std::int8_t> q8(H * S * D), k8(H * S * D), v8(H * S * D);
    std::vector<float> qs(H * S), ks(H * S), vs(H * S), gold(H * S * D);
    const std::optional<std::size_t> win =
        window > 0 ? std::optional<std::size_t>(static_cast<size_t>(window)) : std::nullopt;
    for (size_t h = 0; h < H; ++h) {
        const auto q = ie::quantize_rows(rows_of(qf, h, S, D));
        const auto k = ie::quantize_rows(rows_of(kf, h, S, D));
        const auto v = ie::quantize_rows(rows_of(vf, h, S, D));
        std::memcpy(&q8[h * S * D], q.values.values.data(), S * D);
        std::memcpy(&k8[h * S * D], k.values.values.data(), S * D);
        std::memcpy(&v8[h * S * D], v.values.values.data(), S * D);
        std::memcpy(&qs[h * S], q.scales.data(), S * 4);
        std::memcpy(&ks[h * S], k.scales.data(), S * 4);
        std::memcpy(&vs[h * S], v.scales.data(), S * 4);
        const std::vector<float> y = engine_head(q, k, v, 0, win);
        std::memcpy(&gold[h * S * D], y.data(), S * D * 4);
    }
    Dev<std::int8_t> dq(q8), dk(k8), dv(v8);
    Dev<float> dqs(qs), dks(ks), dvs(vs), dout(H * S * D);
    reef_attention_params p{};
    p.batch = 1;
    p.q_heads = H;
    p.kv_heads = H;
    p.q_len = S;
    p.kv_len = S;
    p.head_dim = D;
    p.query_start = 0;  // kv_len - q_len (attention.hpp:415)
    p.window = window;
    p.softmax_scale = 1.0f;
    p.q_granularity = REEF_SCALE_PER_TOKEN;
    p.kv_granularity = REEF_SCALE_PER_TOKEN;
    reef_hip::context(p, dq.p, nullptr, dk.p, nullptr, dv.p, nullptr, dqs.p, dks.p, dvs.p, dout.p,
                      nullptr, nullptr);
    const std::vector<float> out = dout.get();
    double err = 0.0;
    for (size_t i = 0; i < out.size(); ++i) err = std::max(err, (double)std::fabs(out[i] - gold[i]));
    report(window ? "context, LocalAttention window 64" : "context, GlobalAttention", err <= 1e-3,
           err);

    // Prefill == decode: append the prompt's fp32 K/V to an empty int8 cache, then
    // decode the last query over it.
    Dev<float> dkf(kf), dvf(vf);
    Dev<std::int8_t> kc(H * L * D), vc(H * L * D);
    Dev<float> kcs(H * L), vcs(H * L);
    Dev<std::int32_t> lens(std::vector<std::int32_t>{0});
    Dev<std::uint32_t> status(std::vector<std::uint32_t>{0});
    reef_kv_append_params ap{1, (int64_t)H, (int64_t)D, (int64_t)S, (int64_t)L};
    reef_hip::append_kv_cache(ap, dkf.p, nullptr, dvf.p, nullptr, lens.p, kc.p, vc.p, kcs.p, vcs.p,
                              lens.p, status.p, nullptr);
    reef_hip::check_status_word(status.p, nullptr, "append");
    std::vector<std::int8_t> qlast(H * D);
    std::vector<float> qlast_s(H);
    for (size_t h = 0; h < H; ++h) {
        std::memcpy(&qlast[h * D], &q8[(h * S + S - 1) * D], D);
        qlast_s[h] = qs[h * S + S - 1];
    }
    Dev<std::int8_t> dql(qlast);
    Dev<float> dqls(qlast_s), dlast(H * D);
    reef_decode_params dp{1, (int64_t)H, (int64_t)H, (int64_t)D, (int64_t)L, window, 1.0f,
                          REEF_SCALE_PER_TOKEN, 0, 0};
    Dev<std::uint8_t> ws(reef_hip::decode_workspace_bytes(dp));
    if (hipMemset(ws.p, 0, ws.n) != hipSuccess) throw std::runtime_error("hipMemset");  // once
    reef_hip::decode(dp, dql.p, dqls.p, kc.p, vc.p, kcs.p, vcs.p, lens.p, dlast.p, ws.p, ws.n,
                     status.p, nullptr);
    reef_hip::check_status_word(status.p, nullptr, "decode");
    const std::vector<float> last = dlast.get();
    err = 0.0;
    for (size_t h = 0; h < H; ++h)
        for (size_t c = 0; c < D; ++c)
            err = std::max(err, (double)std::fabs(last[h * D + c] - gold[(h * S + S - 1) * D + c]));
    report(window ? "append + decode == last row, window 64" : "append + decode == last row",
           err <= 1e-3, err);
}

void check_integer_head(std::mt19937 &g) {
    const size_t S = 200, D = 64;
    std::uniform_int_distribution<int> u(-127, 127);
    std::vector<std::int8_t> q(S * D), k(S * D), v(S * D);
    for (auto *a : {&q, &k, &v})
        for (auto &x : *a) x = (std::int8_t)u(g);
    const ie::ExpTable table = ie::exp_table();
    const auto y = ie::attend_head_int8(ie::Tensor<std::int8_t>{{S, D}, q},
                                        ie::Tensor<std::int8_t>{{S, D}, k},
                                        ie::Tensor<std::int8_t>{{S, D}, v},
                                        ie::causal_visibility(S, S, 0), 10, table, 8);
    Dev<std::int8_t> dq(q), dk(k), dv(v), dout(S * D);
    Dev<std::uint16_t> dt(std::vector<std::uint16_t>(table.begin(), table.end()));
    reef_attention_params p{};
    p.batch = 1;
    p.q_heads = 1;
    p.kv_heads = 1;
    p.q_len = S;
    p.kv_len = S;
    p.head_dim = D;
    reef_hip::attend_int8_integer(p, dq.p, nullptr, dk.p, nullptr, dv.p, nullptr, 10, dt.p, 8,
                                  dout.p, nullptr, nullptr);
    const std::vector<std::int8_t> out = dout.get();
    size_t diff = 0;
    for (size_t i = 0; i < out.size(); ++i) diff += out[i] != y.values[i];
    report("attend_head_int8 bit-identical", diff == 0, (double)diff);
}

void check_linear(std::mt19937 &g) {
    const size_t rows = 33, in = 256, out = 96;
    const std::vector<float> x = normals(g, rows * in, 1.0f), wf = normals(g, out * in, 0.05f),
                             bias = normals(g, out, 0.1f);
    const auto w = ie::quantize_rows(ie::Tensor<float>{{out, in}, wf});
    const ie::Tensor<float> bt{{out}, bias};
    const ie::Tensor<float> y = ie::linear<float>(ie::Tensor<float>{{rows, in}, x}, w, std::cref(bt));
    Dev<float> dx(x), dws(w.scales), db(bias), dy(rows * out);
    Dev<std::int8_t> dw(w.values.values);
    Dev<std::uint8_t> ws(reef_linear_w8a8_workspace_bytes(rows, in));
    Dev<std::uint32_t> status(std::vector<std::uint32_t>{0});
    reef_hip::linear_w8a8(dx.p, rows, in, in, dw.p, dws.p, db.p, out, dy.p, out, ws.p, ws.n,
                          status.p, nullptr);
    reef_hip::check_status_word(status.p, nullptr, "linear");
    const std::vector<float> got = dy.get();
    size_t diff = 0;
    for (size_t i = 0; i < got.size(); ++i)
        diff += std::memcmp(&got[i], &y.values[i], 4) != 0;
    report("linear (W8A8) bit-identical", diff == 0, (double)diff);
}

}  // namespace

int main() {
    std::mt19937 g(20261201);
    try {
        check_context_and_decode(g, 0);
        check_context_and_decode(g, 64);
        check_integer_head(g);
        check_linear(g);
    } catch (const std::exception &e) {
        std::printf("FAIL exception: %s\n", e.what());
        return 2;
    }
    std::printf("%d failures\n", failures);
    return failures == 0 ? 0 : 1;
}
