// Host-only check of include/reef_hip/attention.hpp: statuses become the engine's
// exception types and messages. Every call here fails host validation, so no
// device is touched.
#include <cstdio>
#include <cstring>
#include <stdexcept>

#include "reef_hip/attention.hpp"

static int failures = 0;

template <typename E, typename F>
static void expect(const char *name, F f, const char *message = nullptr) {
    try {
        f();
    } catch (const E &e) {
        if (message && std::strcmp(e.what(), message) != 0) {
            std::printf("FAIL %s: message '%s'\n", name, e.what());
            ++failures;
        } else {
            std::printf("ok   %s: %s\n", name, e.what());
        }
        return;
    } catch (const std::exception &e) {
        std::printf("FAIL %s: wrong exception '%s'\n", name, e.what());
        ++failures;
        return;
    }
    std::printf("FAIL %s: no exception\n", name);
    ++failures;
}

int main() {
    // Non-null, aligned host addresses: validation never dereferences them.
    auto *i8 = reinterpret_cast<int8_t *>(0x10000);
    auto *f32 = reinterpret_cast<float *>(0x20000);
    reef_attention_params p{};
    p.batch = 1;
    p.q_heads = 4;
    p.kv_heads = 2;
    p.q_len = 8;
    p.kv_len = 8;
    p.head_dim = 128;
    p.softmax_scale = 0.1f;
    p.q_granularity = REEF_SCALE_PER_HEAD;
    p.kv_granularity = REEF_SCALE_PER_HEAD;
    reef_attention_params rows_past_keys = p;
    rows_past_keys.query_start = 1;
    expect<std::invalid_argument>("context rows past the keys", [&] {
        reef_hip::context(rows_past_keys, i8, nullptr, i8, nullptr, i8, nullptr, f32, f32, f32,
                          f32, nullptr, nullptr);
    });
    reef_attention_params odd_dim = p;
    odd_dim.head_dim = 96;
    expect<reef_hip::unsupported>("context head_dim 96", [&] {
        reef_hip::context(odd_dim, i8, nullptr, i8, nullptr, i8, nullptr, f32, f32, f32, f32,
                          nullptr, nullptr);
    });
    expect<std::invalid_argument>("quantize_rows invalid matrix", [&] {
        reef_hip::quantize_rows(f32, 4, 8, 7, i8, f32, nullptr, nullptr);
    }, "quantize_rows requires a valid matrix");
    expect<std::invalid_argument>("non-finite status", [&] {
        reef_hip::check(REEF_NON_FINITE_INPUT, "x");
    }, "quantize_int8 requires finite values");
    reef_kv_append_params ap{1, 1, 64, 40, 32};
    expect<std::length_error>("append longer than the cache", [&] {
        reef_hip::check(reef_kv_append_int8(&ap, f32, nullptr, f32, nullptr,
                                            reinterpret_cast<int32_t *>(0x30000), i8, i8, f32,
                                            f32, nullptr, nullptr, nullptr),
                        "kv append");
    }, "KV cache capacity exceeded");
    // the prefill over the cache: the cache's per-token scales are required, and a
    // contiguous cache shorter than kv_len is refused
    reef_attention_params chunk = p;
    chunk.kv_len = 40;
    chunk.query_start = 32;
    expect<std::invalid_argument>("context_cache without per-token K/V scales", [&] {
        reef_hip::context_cache(chunk, i8, nullptr, f32, i8, i8, f32, f32, 64, nullptr, 0, 0, f32,
                                nullptr, i8, 1 << 30, nullptr, nullptr);
    });
    chunk.kv_granularity = REEF_SCALE_PER_TOKEN;
    expect<std::invalid_argument>("context_cache on a cache shorter than kv_len", [&] {
        reef_hip::context_cache(chunk, i8, nullptr, f32, i8, i8, f32, f32, 32, nullptr, 0, 0, f32,
                                nullptr, i8, 1 << 30, nullptr, nullptr);
    });
    expect<reef_hip::hip_error>("hip error status", [&] { reef_hip::check(REEF_HIP_ERROR, "x"); });
    std::printf("%d failures\n", failures);
    return failures == 0 ? 0 : 1;
}
