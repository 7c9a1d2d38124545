// Integer-only int8 attention for gfx950: the engine's attend_head_int8
// (int8.hpp:250-279) for every (batch, head) in one launch, bit-exact.
//
// Per query row (int8.hpp:180-232): int32 scores s = q . k over the visible keys,
// d = (max - s) >> score_shift, weight w = table[min(d, 255)], reciprocal
// r = (255 << 16) / sum(w), probability p = min(round_half_up(w * r / 2^16), 255),
// then out = saturate_int8(rounding_shift(sum_k p * v, out_shift)) (:43-60).
//
// The weights depend on the row's final maximum and the probabilities on the
// final sum, so the keys are visited three times (maximum, sum, output), each
// time recomputing the exact int32 scores on v_mfma_i32_32x32x32_i8 rather than
// storing them. Each pass stages the key tiles in LDS once per workgroup (double
// buffered, the next tile's loads in flight); tiles that every row of a wave sees
// skip the per-key mask. p * v runs on v_mfma_f32_32x32x16_f16 with the value
// tile staged as fp16 in channel-major rows (one 16-byte LDS read per operand):
// p <= 255 and v are exact
// in fp16, and every partial sum is an integer below 2^24 (at most 510 keys can
// carry p > 0 beyond the ~255 the probabilities sum to, so |sum| <= 128 * 510),
// so the fp32 accumulation is exact and the result is the engine's integer.
#include <algorithm>

#include "reef_common.hpp"

namespace reef {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kIntThreads = 256;  // 4 waves x 32 query rows
constexpr int kIntRows = 128;
constexpr int kIntKeys = 64;  // keys per tile
// Most keys a row may see: 65536 x 65535 (the largest table weight) < 2^32, so
// no row's weight sum wraps.
constexpr int64_t kMaxIntKeys = 65536;

struct IntHeadArgs {
    const int8_t *q, *k, *v;
    const uint16_t *table;
    int8_t *out;
    int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st, o_sb, o_sh, o_st;
    int32_t batch, q_heads, kv_heads, q_len, kv_len, query_start, window;
    int32_t score_shift, out_shift, q_tiles;
};

// Row m of a 32-key score block holds key 16 ((m >> 2) & 1) + 4 (m >> 3) + (m & 3),
// so that output register r of lane group g is key 16 g + r. The K tile sits in
// LDS in that row order: key kk of a block is stored at row
// (kk & 3) | ((kk >> 4) & 1) << 2 | ((kk >> 2) & 3) << 3, the inverse map.
__device__ __forceinline__ int int_row_of_key(int kk) {
    return (kk & 3) | (((kk >> 4) & 1) << 2) | (((kk >> 2) & 3) << 3);
}

// a * b + c for a, b < 2^24 (low 32 bits), one full-rate instruction; the compiler
// otherwise picks a 64-bit multiply-add for this form.
__device__ __forceinline__ uint32_t mad_u24(uint32_t a, uint32_t b, uint32_t c) {
    uint32_t r;
    asm("v_mad_u32_u24 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

__device__ __forceinline__ int32_t rounding_shift_dev(int32_t value, int shift) {
    return shift == 0 ? value : (value >> shift) + ((value >> (shift - 1)) & 1);
}

// LDS tiles, each double-buffered (tile j in buffer j & 1, one barrier per tile):
// - K: rows of D bytes padded by 16, in the score blocks' row order, so that lane
//   c's 16-byte operand read is row c and 8 consecutive lanes hit distinct banks;
// - V (output pass only): fp16, channel-major (row c holds the tile's 64 keys of
//   channel c), rows padded to 72 halves for the same reason.
template <int D>
struct IntLds {
    static constexpr int K_ROW = D + 16;
    static constexpr int K_BYTES = kIntKeys * K_ROW;
    static constexpr int V_ROW = kIntKeys + 8;
    static constexpr int V_BYTES = D * V_ROW * 2;
    static constexpr int K_CHUNKS = kIntKeys * D / 16;  // 16-byte chunks per K tile
    static constexpr int K_PER_THREAD = (K_CHUNKS + kIntThreads - 1) / kIntThreads;
};

template <int D>
__global__ __launch_bounds__(kIntThreads, 2) void int_head_kernel(IntHeadArgs a) {
    using L = IntLds<D>;
    constexpr int DB = D / 32;
    __shared__ uint16_t sTable[256];
    __shared__ __attribute__((aligned(16))) int8_t sK[2][L::K_BYTES];
    __shared__ __attribute__((aligned(16))) _Float16 sV[2][D * L::V_ROW];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31, grp = lane >> 5;
    sTable[tid] = a.table[tid];  // 256 threads, 256 entries

    const int pairs = a.batch * a.q_heads;
    const int tile = a.q_tiles - 1 - (int)blockIdx.x / pairs;  // heaviest first
    const int bh = (int)blockIdx.x % pairs;
    const int b = bh / a.q_heads, h = bh % a.q_heads;
    const int kvh = h / (a.q_heads / a.kv_heads);
    const int q0 = tile * kIntRows;
    const int row = q0 + wave * 32 + col;
    const bool row_ok = row < a.q_len;

    i32x4 qop[DB];
    const int8_t *qrow = a.q + b * a.q_sb + h * a.q_sh + (int64_t)(row_ok ? row : 0) * a.q_st;
#pragma unroll
    for (int t = 0; t < DB; ++t)
        qop[t] = row_ok ? *reinterpret_cast<const i32x4 *>(qrow + 32 * t + 16 * grp)
                        : i32x4{0, 0, 0, 0};

    // Visible keys: of this lane's row [lo, hi], of the wave, of the workgroup.
    const int pos = a.query_start + row;
    const int lo = a.window > 0 ? max(0, pos + 1 - a.window) : 0;
    const int hi = min(pos, a.kv_len - 1);
    const int w_first = q0 + wave * 32;
    const int w_last = min(w_first + 31, a.q_len - 1);
    const bool wave_active = w_first < a.q_len;
    const int wk_lo = a.window > 0 ? max(0, a.query_start + w_first + 1 - a.window) : 0;
    const int wk_hi = min(a.query_start + w_last, a.kv_len - 1);
    // Keys every valid row of the wave sees: [full_lo, full_hi].
    const int full_lo = a.window > 0 ? max(0, a.query_start + w_last + 1 - a.window) : 0;
    const int full_hi = min(a.query_start + w_first, a.kv_len - 1);
    const int r_last = min(q0 + kIntRows, a.q_len) - 1;
    const int key_lo = a.window > 0 ? max(0, a.query_start + q0 + 1 - a.window) : 0;
    const int key_hi = min(a.query_start + r_last, a.kv_len - 1);
    const int kt0 = key_lo / kIntKeys * kIntKeys;
    // The wave's tiles: [wt0, wt1] (empty when the wave holds no row).
    const int wt0 = wk_lo / kIntKeys * kIntKeys;
    const int wt1 = wave_active ? wk_hi / kIntKeys * kIntKeys : wt0 - kIntKeys;

    const int8_t *kbase = a.k + b * a.k_sb + kvh * a.k_sh;
    const int8_t *vbase = a.v + b * a.v_sb + kvh * a.v_sh;

    // lo <= key <= hi as one unsigned compare (a select, not a branch)
    auto visible = [&](int key) { return (uint32_t)(key - lo) <= (uint32_t)(hi - lo); };
    // Every valid row of the wave sees every key of tile kt: no per-key mask.
    auto tile_full = [&](int kt) { return kt >= full_lo && kt + kIntKeys - 1 <= full_hi; };

    // K staging: chunk i = tid + 256 j is key i / (D / 16), bytes 16 (i % (D / 16)).
    i32x4 kr[L::K_PER_THREAD];
    auto load_k = [&](int kt) {
#pragma unroll
        for (int j = 0; j < L::K_PER_THREAD; ++j) {
            const int i = tid + kIntThreads * j;
            const int key = kt + i / (D / 16);
            kr[j] = i < L::K_CHUNKS && key < a.kv_len
                        ? *reinterpret_cast<const i32x4 *>(kbase + (int64_t)key * a.k_st +
                                                           16 * (i % (D / 16)))
                        : i32x4{0, 0, 0, 0};
        }
    };
    auto store_k = [&](int buf) {
#pragma unroll
        for (int j = 0; j < L::K_PER_THREAD; ++j) {
            const int i = tid + kIntThreads * j;
            const int kk = i / (D / 16);
            if (i < L::K_CHUNKS)
                *reinterpret_cast<i32x4 *>(
                    &sK[buf][((kk & ~31) | int_row_of_key(kk & 31)) * L::K_ROW + 16 * (i % (D / 16))]) =
                    kr[j];
        }
    };
    // Scores of 32-key block u of the staged tile for this lane's query: register r
    // of lane group g is key 32 u + 16 g + r (each lane reads the K row of its
    // output column).
    auto scores = [&](int buf, int u) {
        const int8_t *krow = &sK[buf][(32 * u + col) * L::K_ROW + 16 * grp];
        i32x16 s = {};
#pragma unroll
        for (int t = 0; t < DB; ++t)
            s = mfma_32x32x32_i8(*reinterpret_cast<const i32x4 *>(krow + 32 * t), qop[t], s);
        return s;
    };
    // Walk the workgroup's tiles: tile kt is staged in LDS (the next one's global
    // loads in flight meanwhile), then f(kt, buf) runs for the wave's own tiles.
    // extra_load(kt) / extra_store(buf) stage more per-tile data the same way.
    auto walk = [&](auto f, auto extra_load, auto extra_store) {
        load_k(kt0);
        extra_load(kt0);
        int buf = 0;
        for (int kt = kt0; kt <= key_hi; kt += kIntKeys, buf ^= 1) {
            store_k(buf);
            extra_store(buf);
            if (kt + kIntKeys <= key_hi) {
                load_k(kt + kIntKeys);
                extra_load(kt + kIntKeys);
            }
            // the stores are visible; every wave has finished reading this buffer's
            // previous tile (it did so before the last barrier)
            __syncthreads();
            if (kt >= wt0 && kt <= wt1) f(kt, buf);
        }
        __syncthreads();  // the next walk's first stores reuse the buffers
    };
    auto no_load = [](int) {};
    auto no_store = [](int) {};

    // The per-key work below is branch-free: a tile is either seen whole by every
    // row of the wave (wave-uniform test, no mask) or masked with selects.
    // Pass 1: the row maximum over visible keys (int8.hpp:197-203).
    int32_t mx = INT32_MIN;
    walk([&](int kt, int buf) {
        const i32x16 s[2] = {scores(buf, 0), scores(buf, 1)};
        if (tile_full(kt)) {
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int r = 0; r < 16; ++r) mx = max(mx, s[u][r]);
        } else {
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    mx = max(mx, visible(kt + 32 * u + 16 * grp + r) ? s[u][r] : INT32_MIN);
        }
    }, no_load, no_store);
    {
        const auto sw = __builtin_amdgcn_permlane32_swap((uint32_t)mx, (uint32_t)mx, false, false);
        mx = max((int32_t)sw[0], (int32_t)sw[1]);
    }

    // Pass 2: the sum of table weights (:208-217).
    uint32_t sum = 0;
    auto weight = [&](int32_t sc) {
        const uint32_t d = (uint32_t)((mx - sc) >> a.score_shift);
        return (uint32_t)sTable[d < 255u ? d : 255u];
    };
    walk([&](int kt, int buf) {
        const i32x16 s[2] = {scores(buf, 0), scores(buf, 1)};
        if (tile_full(kt)) {
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int r = 0; r < 16; ++r) sum += weight(s[u][r]);
        } else {
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t w = weight(s[u][r]);  // any d indexes the table
                    sum += visible(kt + 32 * u + 16 * grp + r) ? w : 0u;
                }
        }
    }, no_load, no_store);
    {
        const auto sw = __builtin_amdgcn_permlane32_swap(sum, sum, false, false);
        sum = sw[0] + sw[1];
    }
    // The maximum's weight is the table's first entry, so sum > 0 on a row that
    // sees a key; rows outside the tensor never store.
    const uint32_t recip = sum > 0 ? (255u << 16) / sum : 0u;
    const uint32_t recip24 = recip & 0xFFFFFFu;  // the same value (< 2^24)
    const uint32_t half16 = 32768u;

    // Pass 3: probabilities and P.V (:218-227, 268-276). Thread i < 2 D also stages
    // keys 2 (i % 32) and 2 (i % 32) + 1, channels 16 (i / 32) .. + 15 of each
    // value tile, converted exactly to fp16 and stored as key pairs into the
    // channel-major tile. Each lane then reads its 8 keys of one channel as one
    // 16-byte operand.
    const bool stager = tid < 2 * D;
    const int vkp = tid % 32, vc16 = tid / 32;
    i32x4 vr[2];
    auto load_v = [&](int kt) {
        if (!stager) return;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int key = kt + 2 * vkp + j;
            vr[j] = key < a.kv_len
                        ? *reinterpret_cast<const i32x4 *>(vbase + (int64_t)key * a.v_st + 16 * vc16)
                        : i32x4{0, 0, 0, 0};
        }
    };
    auto store_v = [&](int buf) {
        if (!stager) return;
        const int8_t *b0 = reinterpret_cast<const int8_t *>(&vr[0]);
        const int8_t *b1 = reinterpret_cast<const int8_t *>(&vr[1]);
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
            const f16x2 pr = {(_Float16)(int16_t)b0[c], (_Float16)(int16_t)b1[c]};
            *reinterpret_cast<f16x2 *>(&sV[buf][(16 * vc16 + c) * L::V_ROW + 2 * vkp]) = pr;
        }
    };
    f32x16 acc[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) acc[d] = f32x16{};
    walk([&](int kt, int buf) {
        const bool full = tile_full(kt);
        const i32x16 s[2] = {scores(buf, 0), scores(buf, 1)};
        // (scaled >> 16) + ((scaled >> 15) & 1) == (scaled + 2^15) >> 16. A visible
        // key's w is one of the summed weights, so scaled = w * recip <= 255 << 16:
        // a 24-bit product (v_mad_u32_u24), and p <= 255 (the engine's clamp never
        // binds). Masked keys' products are discarded.
        uint32_t pv[2][16];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int r = 0; r < 16; ++r) pv[u][r] = mad_u24(weight(s[u][r]), recip24, half16) >> 16;
        if (!full) {  // one uniform branch around all of the tile's selects
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    pv[u][r] = visible(kt + 32 * u + 16 * grp + r) ? pv[u][r] : 0u;
        }
        // p <= 255 to fp16, two at a time: 0x6400 | p is the fp16 bit pattern of
        // 1024 + p, and one packed subtraction of 1024 leaves p exactly.
        f16x8 pop[2][2];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                u32x4 bits;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    bits[e] = pv[u][8 * hf + 2 * e] | (pv[u][8 * hf + 2 * e + 1] << 16) | 0x64006400u;
                pop[u][hf] = __builtin_bit_cast(f16x8, bits) - (f16x8)(_Float16)1024.0f;
            }
        const _Float16 *vt = &sV[buf][col * L::V_ROW];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int s8 = 0; s8 < 2; ++s8) {
                const int k0 = 32 * u + 16 * grp + 8 * s8;  // this lane's 8 keys in the tile
#pragma unroll
                for (int d = 0; d < DB; ++d) {
                    const f16x8 vop = *reinterpret_cast<const f16x8 *>(vt + 32 * d * L::V_ROW + k0);
                    acc[d] = mfma_32x32x16_f16(vop, pop[u][s8], acc[d]);
                }
            }
    }, load_v, store_v);

    if (!row_ok) return;
    // acc[d][4j + i] is channel 32 d + 8 j + 4 grp + i of this lane's row.
    int8_t *orow = a.out + b * a.o_sb + h * a.o_sh + (int64_t)row * a.o_st;
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            char4 c4;
            int8_t *cp = reinterpret_cast<int8_t *>(&c4);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int32_t sum_pv = (int32_t)acc[d][4 * j + i];
                const int32_t sh = rounding_shift_dev(sum_pv, a.out_shift);
                cp[i] = (int8_t)(sh < -128 ? -128 : (sh > 127 ? 127 : sh));
            }
            *reinterpret_cast<char4 *>(orow + 32 * d + 8 * j + 4 * grp) = c4;
        }
}

bool int8_strides_ok(const reef_strides *s, const void *base) {
    if (!aligned(base, 16)) return false;
    if (!s) return true;
    return s->batch >= 0 && s->head >= 0 && s->token >= 0 && s->batch % 16 == 0 &&
           s->head % 16 == 0 && s->token % 16 == 0;
}

}  // namespace
}  // namespace reef

using namespace reef;

extern "C" reef_status reef_attention_int8_integer(
    const reef_attention_params *p, const int8_t *q, const reef_strides *q_strides,
    const int8_t *k, const reef_strides *k_strides, const int8_t *v,
    const reef_strides *v_strides, uint32_t score_shift, const uint16_t *table,
    uint32_t out_shift, int8_t *out, const reef_strides *out_strides, hipStream_t stream) {
    if (!p || !q || !k || !v || !table || !out) return REEF_INVALID_ARGUMENT;
    const int64_t D = p->head_dim;
    if (p->batch <= 0 || p->q_heads <= 0 || p->kv_heads <= 0 || p->q_len <= 0 ||
        p->kv_len <= 0 || D <= 0 || p->q_heads % p->kv_heads != 0 || p->query_start < 0 ||
        p->window < 0 || p->query_start + p->q_len > p->kv_len || score_shift > 31 ||
        out_shift > 31)
        return REEF_INVALID_ARGUMENT;
    if (D != 32 && D != 64 && D != 128) return REEF_UNSUPPORTED;
    if (p->kv_len >= (int64_t(1) << 30) || p->window >= (int64_t(1) << 30)) return REEF_UNSUPPORTED;
    // A row's weight sum is a uint32 of at most (visible keys) x 65535. Beyond 65536
    // visible keys the engine's sum could wrap, and the kernel's shortcuts (24-bit
    // multiply-adds, one rounding step, no clamp) hold only while it does not.
    const int64_t visible = p->window > 0 ? std::min<int64_t>(p->window, p->kv_len) : p->kv_len;
    if (visible > kMaxIntKeys) return REEF_UNSUPPORTED;
    if (!int8_strides_ok(q_strides, q) || !int8_strides_ok(k_strides, k) ||
        !int8_strides_ok(v_strides, v) || !aligned(out, 4))
        return REEF_INVALID_ARGUMENT;
    if (out_strides && (out_strides->batch % 4 || out_strides->head % 4 || out_strides->token % 4 ||
                        out_strides->batch < 0 || out_strides->head < 0 || out_strides->token < 0))
        return REEF_INVALID_ARGUMENT;
    IntHeadArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.table = table;
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
    a.score_shift = (int32_t)score_shift;
    a.out_shift = (int32_t)out_shift;
    a.q_tiles = (int32_t)ceil_div(Sq, kIntRows);
    const int64_t items = a.q_tiles * Hq * p->batch;
    if (items >= (int64_t(1) << 31)) return REEF_UNSUPPORTED;
    const dim3 grid((unsigned)items);
    if (D == 128)
        hipLaunchKernelGGL(int_head_kernel<128>, grid, dim3(kIntThreads), 0, stream, a);
    else if (D == 64)
        hipLaunchKernelGGL(int_head_kernel<64>, grid, dim3(kIntThreads), 0, stream, a);
    else
        hipLaunchKernelGGL(int_head_kernel<32>, grid, dim3(kIntThreads), 0, stream, a);
    return launch_status();
}
