// Prefill attention over a packed value image (gfx950, head_dim 128, per-tensor or
// per-head K/V scales).
//
// The same computation as prefill.hip (Attention::context, attention.hpp:374-432:
// attend_head :117-123 per (batch, head), causal_visibility :82-100 or a window),
// arranged so that a key tile reaches the matrix instructions with no vector-ALU
// work on the way:
//
//   * vt_pack_kernel writes, once per call, an fp16 image of V: per (batch, kv head)
//     and 64-key tile, 128 channel rows of 64 keys (16 KB), the 16-byte chunks of
//     each row in the bank-swizzled order the P.V operand reads use. Every int8 code
//     is an fp16 integer, so the image is exact. Beside it, per tile, the largest
//     |code| in each 32-channel block.
//   * The attention kernel copies K (the caller's int8 rows) and the V image into
//     LDS with direct-to-LDS buffer loads: three stages, one barrier per tile, the
//     loads of tile j + 2 in flight while tile j computes.
//   * A workgroup is 8 waves x 32 query rows. Per 64-key tile a wave computes
//     S^T = K . Q^T on v_mfma_i32_32x32x32_i8 (K rows permuted so that each lane's
//     scores are the P operand of the next step), an fp32 online softmax in base 2
//     with a lazy rescale, and O^T = V^T . P^T on v_mfma_f32_32x32x16_f16.
//   * Precision of P: for a value block whose dequantized magnitudes reach above
//     kPreciseAbove, P is split into fp16 hi + lo parts (two products, 22 bits);
//     below it, P is one fp16 (11 bits). The rounding of P moves an output by about
//     2^-12 |v_j - out| per dominant key, which at |v| <= 6 stays under 5e-4; the
//     activation-outlier channels of int8 LLM attention (|v| ~ 30) need the split.
//     Each block keeps the row sum of exactly the P values its product uses.
//   * Schedule: persistent workgroups; a causal head's query tiles t and T-1-t form
//     one item with the same work as any other pair. Items are numbered head-major
//     and dealt out so that the workgroups of one XCD hold consecutive items, i.e.
//     a few heads at a time, whose K and V stay in that XCD's L2. The light tile
//     runs first: its keys are a prefix of the heavy one's.
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "reef_common.hpp"

namespace reef {

// Host side, used by prefill.hip's entry point.
int64_t packed_image_bytes(int64_t batch, int64_t kv_heads, int64_t kv_len);
reef_status prefill_packed_launch(const reef_attention_params *p, const int8_t *q,
                                  const int64_t (&qst)[3], const int8_t *k,
                                  const int64_t (&kst)[3], const int8_t *v,
                                  const int64_t (&vst)[3], const float *q_scales,
                                  const float *k_scales, const float *v_scales, float *out,
                                  const int64_t (&ost)[3], void *image, hipStream_t stream);

namespace {

constexpr int kPK = 64;                    // keys per tile
constexpr int kPD = 128;                   // head_dim of this path
constexpr int kKTile = kPK * kPD;          // int8 K bytes per tile
constexpr int kVTile = kPK * kPD * 2;      // fp16 V image bytes per tile
constexpr int kStage = kKTile + kVTile;    // 24 KB
constexpr int kStages = 3;
constexpr int kBlocks1K = kStage / 1024;   // 1 KB direct-load blocks per tile (8 K + 16 V)
constexpr int kXcdCount = 8;               // workgroup i of a launch runs on XCD i % 8
#ifndef REEF_PACKED_WAVES
#define REEF_PACKED_WAVES 4                // waves (of 32 query rows) per workgroup: 4 or 8
#endif

// Position of 16-byte chunk c in a 128-byte LDS row r: the 16 lanes that read
// chunk c of 16 consecutive rows land in 16 distinct bank groups.
__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r >> 1) & 7); }

// Row m of a 32-row score block holds key 16 ((m >> 2) & 1) + 4 (m >> 3) + (m & 3),
// so that output register r = 4j + i of lane group g is key 16g + r.
__device__ __forceinline__ int key_of_row32(int m) {
    return 16 * ((m >> 2) & 1) + 4 * (m >> 3) + (m & 3);
}

struct PackArgs {
    const int8_t *v;
    int64_t v_sb, v_sh, v_st;
    int32_t kv_heads, kv_len, tiles;
    int8_t *img;      // [B * Hkv][tiles][kVTile]
    uint32_t *bmax;   // [B * Hkv][tiles]: byte i = max |code| of channels 32i .. 32i + 31
};

// One workgroup per (tile, batch x kv head).
__global__ __launch_bounds__(256) void vt_pack_kernel(PackArgs a) {
    constexpr int kRow = kPD + 4;  // LDS bytes per key row: column reads 8 rows apart
                                   // fall in 8 distinct banks
    __shared__ __attribute__((aligned(16))) int8_t sV[kPK * kRow];
    __shared__ uint32_t sMax[4][4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tile = blockIdx.x, bkv = blockIdx.y;
    const int b = bkv / a.kv_heads, h = bkv % a.kv_heads;
    const int kt = tile * kPK;
    const int8_t *src = a.v + b * a.v_sb + h * a.v_sh;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int chunk = tid + 256 * i, key = chunk >> 3, part = chunk & 7;
        i32x4 x = {0, 0, 0, 0};
        if (kt + key < a.kv_len)
            x = *reinterpret_cast<const i32x4 *>(src + (int64_t)(kt + key) * a.v_st + 16 * part);
        int32_t *d = reinterpret_cast<int32_t *>(sV + key * kRow + 16 * part);
        d[0] = x[0];
        d[1] = x[1];
        d[2] = x[2];
        d[3] = x[3];
    }
    __syncthreads();
    int8_t *dst = a.img + ((int64_t)bkv * a.tiles + tile) * kVTile;
    uint32_t mx[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // image chunk s: channel m, position s % 8 holding keys 8c .. 8c + 7
        const int s = tid + 256 * i, m = s >> 3, c = swz(m, s & 7);
        f16x8 o;
        int big = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int code = sV[(8 * c + e) * kRow + m];
            o[e] = (_Float16)code;
            big = max(big, code < 0 ? -code : code);
        }
        *reinterpret_cast<f16x8 *>(dst + 16 * s) = o;
        mx[i] = wave_max_u32((uint32_t)big);  // chunk i of every thread is channel block i
    }
    if (lane == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) sMax[wave][i] = mx[i];
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t m = max(max(sMax[0][i], sMax[1][i]), max(sMax[2][i], sMax[3][i]));
            word |= m << (8 * i);
        }
        a.bmax[(int64_t)bkv * a.tiles + tile] = word;
    }
}

struct PackedArgs {
    const int8_t *q, *k, *img;
    const uint32_t *bmax;
    const float *qs, *ks, *vs;
    float *out;
    int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_st, o_sb, o_sh, o_st;
    int32_t batch, q_heads, kv_heads, q_len, kv_len, query_start, window;
    float score_scale;  // softmax_scale * log2(e)
    int32_t q_gran, kv_gran;
    int32_t kv_tiles;   // 64-key tiles per (batch, kv head) in the image
    int32_t q_tiles;    // query tiles per (batch, head)
    int32_t per_head;   // items per (batch, head): ceil(q_tiles / 2)
    int32_t items;      // batch * q_heads * per_head
    int32_t all_precise;
};

// Two probabilities (p0, p1) rounded to fp16 (the packed P operand) and the fp16
// residuals p - fp16(p) of both (the lo operand). Each residual is exact in fp32
// (fewer than 14 significant bits), one v_fma_mix_f32 reading the fp16 half.
__device__ __forceinline__ uint32_t pack_f16(float p0, float p1) {
    const f16x2 h = __builtin_convertvector((float __attribute__((ext_vector_type(2)))){p0, p1},
                                            f16x2);
    return __builtin_bit_cast(uint32_t, h);
}
__device__ __forceinline__ uint32_t residual_f16(uint32_t hi, float p0, float p1) {
    float r0, r1;
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r0) : "v"(hi), "v"(p0));
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
        : "=v"(r1)
        : "v"(hi), "v"(p1));
    return pack_f16(r0, r1);
}

__device__ __forceinline__ float scale_at(const float *s, int gran, int b, int h, int t, int heads,
                                          int tokens) {
    if (gran == REEF_SCALE_PER_TENSOR) return s[0];
    if (gran == REEF_SCALE_PER_HEAD) return s[h];
    return s[((int64_t)b * heads + h) * tokens + t];
}

template <int WAVES>
struct PackedShape {
    static constexpr int BM = 32 * WAVES;                 // query rows per tile
    static constexpr int PER_WAVE = kBlocks1K / WAVES;    // direct loads per wave and tile
    static constexpr int K_LOADS = (kKTile / 1024) / WAVES;  // of which K blocks
    static_assert(kBlocks1K % WAVES == 0 && (kKTile / 1024) % WAVES == 0, "loads split evenly");
};

// One query tile of one (batch, head). LO: some value block splits P into hi + lo
// (pmask bit d: channels 32d .. 32d + 31).
template <int WAVES, bool LO>
__device__ __forceinline__ void packed_tile(const PackedArgs &a, int b, int h, int tile,
                                            int8_t *smem, uint32_t pmask) {
    using S = PackedShape<WAVES>;
    constexpr int BM = S::BM;
    constexpr int DB = kPD / 32;
    constexpr float kLazy = 8.0f;  // the running max moves when a row max grows by > 2^8
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31, grp = lane >> 5;
    const int kvh = h / (a.q_heads / a.kv_heads);
    const int q0 = tile * BM;
    const int row = q0 + wave * 32 + col;
    const bool row_ok = row < a.q_len;

    // Visible keys of this lane's row [lo, hi], of the workgroup and of the wave.
    const int pos = a.query_start + row;
    const int lo = a.window > 0 ? max(0, pos + 1 - a.window) : 0;
    const int hi = min(pos, a.kv_len - 1);
    const int r_last = min(q0 + BM, a.q_len) - 1;
    const int key_lo = a.window > 0 ? max(0, a.query_start + q0 + 1 - a.window) : 0;
    const int key_hi = min(a.query_start + r_last, a.kv_len - 1);
    const int w_first = q0 + wave * 32;
    const int w_last = min(w_first + 31, a.q_len - 1);
    const bool wave_active = w_first < a.q_len;
    const int wk_lo = a.window > 0 ? max(0, a.query_start + w_first + 1 - a.window) : 0;
    const int wk_hi = min(a.query_start + w_last, a.kv_len - 1);
    const int full_lo = a.window > 0 ? a.query_start + w_last + 1 - a.window : 0;
    const int full_hi = min(a.query_start + w_first, a.kv_len - 1);
    const int kt0 = key_lo / kPK * kPK;
    const int n_tiles = (key_hi - kt0) / kPK + 1;

    // Query operand and scales (independent loads, issued before the tile loads).
    i32x4 qop[kPD / 32];
    {
        const int8_t *qrow = a.q + b * a.q_sb + h * a.q_sh + (int64_t)(row_ok ? row : 0) * a.q_st;
#pragma unroll
        for (int t = 0; t < kPD / 32; ++t)
            qop[t] = row_ok ? *reinterpret_cast<const i32x4 *>(qrow + 32 * t + 16 * grp)
                            : i32x4{0, 0, 0, 0};
    }
    const float cq = row_ok ? scale_at(a.qs, a.q_gran, b, h, row, a.q_heads, a.q_len) : 0.0f;
    const float ck = scale_at(a.ks, a.kv_gran, b, kvh, 0, a.kv_heads, a.kv_len);
    const float cv = scale_at(a.vs, a.kv_gran, b, kvh, 0, a.kv_heads, a.kv_len);
    const float c = cq * ck * a.score_scale;  // log2-domain score per unit of int32 sum

    // Direct loads: wave w fills 1 KB blocks w, w + WAVES, ... of a stage (blocks
    // 0-7 are K, 8-23 the V image). Lane L of K block kb writes LDS row
    // 8 kb + L / 8 at position L % 8, which holds chunk swz(row, L % 8) of the key
    // that the row stands for.
    uint32_t loff[S::PER_WAVE];
#pragma unroll
    for (int i = 0; i < S::PER_WAVE; ++i) {
        const int blk = wave + WAVES * i;
        if (i < S::K_LOADS) {
            const int r = 8 * blk + lane / 8;
            const int key = 32 * (r >> 5) + key_of_row32(r & 31);
            loff[i] = (uint32_t)(key * a.k_st + 16 * swz(r, lane & 7));
        } else {
            loff[i] = (uint32_t)(16 * (64 * (blk - kKTile / 1024) + lane));
        }
    }
    const int8_t *kbase = a.k + b * a.k_sb + kvh * a.k_sh;
    const int8_t *ibase = a.img + ((int64_t)(b * a.kv_heads + kvh) * a.kv_tiles) * kVTile;
    auto issue = [&](int j) {  // tile j into stage j % kStages
        const int kt = kt0 + kPK * j;
        int8_t *st = smem + (j % kStages) * kStage;
        // The tile's K rows as their own buffer range: rows past kv_len read zeros.
        const __amdgpu_buffer_rsrc_t kr = buffer_rsrc(
            kbase + (int64_t)kt * a.k_st, (uint32_t)((int64_t)(a.kv_len - 1 - kt) * a.k_st + kPD));
        const __amdgpu_buffer_rsrc_t vr = buffer_rsrc(ibase + (int64_t)(kt / kPK) * kVTile, kVTile);
#pragma unroll
        for (int i = 0; i < S::PER_WAVE; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                i < S::K_LOADS ? kr : vr,
                (__attribute__((address_space(3))) void *)(st + 1024 * (wave + WAVES * i)), 16,
                loff[i], 0, 0, 0);
    };

    // LDS operand positions: K row 32u + col, chunk 2t + grp; V row 32d + col, chunk
    // 4u + 2 grp + s (keys 32u + 16 grp + 8s .. + 8, the P operand's keys).
    int kpos[kPD / 32], vpos[2][2];
#pragma unroll
    for (int t = 0; t < kPD / 32; ++t) kpos[t] = col * kPD + 16 * swz(col, 2 * t + grp);
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int s = 0; s < 2; ++s) vpos[u][s] = col * 128 + 16 * swz(col, 4 * u + 2 * grp + s);

    float m_run = -INFINITY, l_hi = 0.0f, l_lo = 0.0f;
    f32x16 acc[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) acc[d] = f32x16{};

    auto tile_math = [&](const int kt, const int8_t *sK, auto mask_tag) {
        constexpr bool need_mask = decltype(mask_tag)::value;
        const int8_t *sV = sK + kKTile;
        i32x16 sc[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            sc[u] = i32x16{};
#pragma unroll
            for (int t = 0; t < kPD / 32; ++t)
                sc[u] = mfma_32x32x32_i8(*reinterpret_cast<const i32x4 *>(sK + 4096 * u + kpos[t]),
                                         qop[t], sc[u]);
        }
        if constexpr (need_mask) {
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kt + 32 * u + 16 * grp + r;
                    if (key < lo || key > hi) sc[u][r] = INT32_MIN;
                }
        }
        int mi = sc[0][0];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int r = (u == 0 ? 1 : 0); r < 16; ++r) mi = max(mi, sc[u][r]);
        // c > 0, so the largest float score is c times the largest integer.
        float mt = mi == INT32_MIN ? -INFINITY : (float)mi * c;
        mt = xor32_max(mt);
        if (__any(mt > m_run + kLazy)) {  // wave-uniform
            const float m_new = fmaxf(m_run, mt);
            const float alpha = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
            m_run = m_new;
            l_hi *= alpha;
            if (LO) l_lo *= alpha;
#pragma unroll
            for (int d = 0; d < DB; ++d) acc[d] *= alpha;
        }
        // P in fp16 pairs (4 words per 8 keys) and, with LO, the fp16 residuals.
        uint32_t phi[2][2][4], plo[2][2][4];
        const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    float p[2];
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        const int r = 8 * s + e + i;
                        p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf((float)sc[u][r], c, -m_run));
                        if constexpr (need_mask) {
                            if (sc[u][r] == INT32_MIN) p[i] = 0.0f;
                        }
                    }
                    const uint32_t h = pack_f16(p[0], p[1]);
                    phi[u][s][e / 2] = h;
                    // Row sums of exactly the fp16 values the products use, fp32 accumulation.
                    l_hi = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, h), one, l_hi, false);
                    if (LO) {
                        const uint32_t r = residual_f16(h, p[0], p[1]);
                        plo[u][s][e / 2] = r;
                        l_lo = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, r), one, l_lo, false);
                    }
                }
        auto operand = [](const uint32_t (&w)[4]) {
            return __builtin_bit_cast(f16x8, i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]});
        };
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
                for (int d = 0; d < DB; ++d)
                    acc[d] = mfma_32x32x16_f16(
                        *reinterpret_cast<const f16x8 *>(sV + 4096 * d + vpos[u][s]),
                        operand(phi[u][s]), acc[d]);
        if (LO) {
            // The residual products of the value blocks that need them (uniform).
#pragma unroll
            for (int d = 0; d < DB; ++d) {
                if ((pmask >> d) & 1) {
#pragma unroll
                    for (int u = 0; u < 2; ++u)
#pragma unroll
                        for (int s = 0; s < 2; ++s)
                            acc[d] = mfma_32x32x16_f16(
                                *reinterpret_cast<const f16x8 *>(sV + 4096 * d + vpos[u][s]),
                                operand(plo[u][s]), acc[d]);
                }
            }
        }
    };

    // Each wave has issued PER_WAVE loads per tile; the next tile's may still be in
    // flight when this tile's must have landed (vmcnt in bits 3:0 and 15:14 of the
    // s_waitcnt immediate; 0xf70 leaves expcnt and lgkmcnt unconstrained).
    constexpr int kNext = S::PER_WAVE;
    static_assert(kNext < 16, "vmcnt fits the low field");
    issue(0);
    if (n_tiles > 1) issue(1);
    // Steps [it_a, it_b): tiles every row of the workgroup sees whole.
    const int wg_full_lo = a.window > 0 ? a.query_start + r_last + 1 - a.window : 0;
    const int wg_full_hi = min(a.query_start + q0, a.kv_len - 1);
    const int it_a = max(0, wg_full_lo - kt0 + kPK - 1) / kPK;
    const int span = wg_full_hi + 1 - kt0;
    const int it_b = max(it_a, min(n_tiles, span > 0 ? span / kPK : 0));
    auto step = [&](const int j, auto every_row_tag) {
        constexpr bool every_row = decltype(every_row_tag)::value;
        if (j + 1 < n_tiles) __builtin_amdgcn_s_waitcnt(0xf70 | kNext);
        else __builtin_amdgcn_s_waitcnt(0xf70);
        // Every wave's loads of tile j are in LDS and every wave is done with tile
        // j - 1, whose stage tile j + 2 now fills. A bare barrier (no wait for the
        // loads still in flight).
        __builtin_amdgcn_s_barrier();
        if (j + 2 < n_tiles) issue(j + 2);
        const int kt = kt0 + kPK * j;
        const int8_t *sK = smem + (j % kStages) * kStage;
        if constexpr (every_row) {
            tile_math(kt, sK, std::false_type{});
        } else if (wave_active && kt <= wk_hi && kt + kPK - 1 >= wk_lo) {  // wave-uniform
            if (kt + kPK - 1 <= full_hi && kt >= full_lo)
                tile_math(kt, sK, std::false_type{});
            else
                tile_math(kt, sK, std::true_type{});
        }
    };
    int j = 0;
    for (; j < it_a; ++j) step(j, std::false_type{});
    for (; j < it_b; ++j) step(j, std::true_type{});
    for (; j < n_tiles; ++j) step(j, std::false_type{});

    if (row_ok) {
        const float lh = xor32_sum(l_hi);
        const float ll = LO ? xor32_sum(l_lo) : 0.0f;
        float *orow = a.out + b * a.o_sb + h * a.o_sh + (int64_t)row * a.o_st;
#pragma unroll
        for (int d = 0; d < DB; ++d) {
            const float norm = cv / (LO && ((pmask >> d) & 1) ? lh + ll : lh);
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                f32x4 o;
#pragma unroll
                for (int i = 0; i < 4; ++i) o[i] = acc[d][4 * jj + i] * norm;
                *reinterpret_cast<f32x4 *>(orow + 32 * d + 8 * jj + 4 * grp) = o;
            }
        }
    }
    // The next tile of this workgroup reuses the stages.
    __syncthreads();
}

// Blocks of (batch, kv head) whose dequantized values reach above kPreciseAbove:
// the largest |code| of each 32-channel block over the head's tiles, times the
// value scale. Uniform over the workgroup.
template <int WAVES>
__device__ __forceinline__ uint32_t precise_blocks(const PackedArgs &a, int b, int kvh,
                                                   uint32_t *sRed) {
    if (a.all_precise) return 0xFu;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t *bm = a.bmax + (int64_t)(b * a.kv_heads + kvh) * a.kv_tiles;
    uint32_t m[4] = {0, 0, 0, 0};
    for (int t = tid; t < a.kv_tiles; t += 64 * WAVES) {
        const uint32_t w = bm[t];
#pragma unroll
        for (int i = 0; i < 4; ++i) m[i] = max(m[i], (w >> (8 * i)) & 0xffu);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) m[i] = wave_max_u32(m[i]);
    if (lane == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) sRed[wave * 4 + i] = m[i];
    }
    __syncthreads();
    uint32_t top[4] = {0, 0, 0, 0};
    for (int w = 0; w < WAVES; ++w)
#pragma unroll
        for (int i = 0; i < 4; ++i) top[i] = max(top[i], sRed[w * 4 + i]);
    __syncthreads();  // sRed is reused by the next item
    const float cv = scale_at(a.vs, a.kv_gran, b, kvh, 0, a.kv_heads, a.kv_len);
    uint32_t mask = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if ((float)top[i] * cv > kPreciseAbove) mask |= 1u << i;
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)mask);
}

// Workgroups resident per compute unit: 4-wave workgroups run two at a time (2 x 72 KB
// of LDS), so the two waves on each SIMD belong to different workgroups and drift
// apart (one computes scores while the other runs its softmax).
template <int WAVES>
constexpr int kPackedPerCu = WAVES == 4 ? 2 : 1;

template <int WAVES>
__global__ __launch_bounds__(64 * WAVES, kPackedPerCu<WAVES>) void prefill_packed_kernel(PackedArgs a) {
    __shared__ __attribute__((aligned(1024))) int8_t smem[kStages * kStage];
    __shared__ uint32_t sRed[4 * WAVES];
    const int G = gridDim.x, g = blockIdx.x;
    const int x = g % kXcdCount, per = G / kXcdCount, rem = G % kXcdCount;
    const int L = x * per + min(x, rem) + g / kXcdCount;  // XCD-contiguous logical index
    for (int it = L; it < a.items; it += G) {
        const int bh = it / a.per_head, i = it % a.per_head;
        const int b = bh / a.q_heads, h = bh % a.q_heads;
        const int kvh = h / (a.q_heads / a.kv_heads);
        const uint32_t pmask = precise_blocks<WAVES>(a, b, kvh, sRed);
        const int light = i, heavy = a.q_tiles - 1 - i;
        if (pmask) {
            packed_tile<WAVES, true>(a, b, h, light, smem, pmask);
            if (heavy != light) packed_tile<WAVES, true>(a, b, h, heavy, smem, pmask);
        } else {
            packed_tile<WAVES, false>(a, b, h, light, smem, 0);
            if (heavy != light) packed_tile<WAVES, false>(a, b, h, heavy, smem, 0);
        }
    }
}

}  // namespace

int64_t packed_image_bytes(int64_t batch, int64_t kv_heads, int64_t kv_len) {
    const int64_t tiles = ceil_div(kv_len, kPK);
    const int64_t img = batch * kv_heads * tiles * kVTile;
    return img + ceil_div(batch * kv_heads * tiles * 4, 256) * 256;
}

reef_status prefill_packed_launch(const reef_attention_params *p, const int8_t *q,
                                  const int64_t (&qst)[3], const int8_t *k,
                                  const int64_t (&kst)[3], const int8_t *v,
                                  const int64_t (&vst)[3], const float *q_scales,
                                  const float *k_scales, const float *v_scales, float *out,
                                  const int64_t (&ost)[3], void *image, hipStream_t stream) {
    constexpr int WAVES = REEF_PACKED_WAVES;
    const int64_t tiles = ceil_div(p->kv_len, kPK);
    const int64_t bkv = p->batch * p->kv_heads;
    if (tiles > 65535 || bkv > 65535) return REEF_UNSUPPORTED;
    PackArgs pa;
    pa.v = v;
    pa.v_sb = vst[0];
    pa.v_sh = vst[1];
    pa.v_st = vst[2];
    pa.kv_heads = (int32_t)p->kv_heads;
    pa.kv_len = (int32_t)p->kv_len;
    pa.tiles = (int32_t)tiles;
    pa.img = static_cast<int8_t *>(image);
    pa.bmax = reinterpret_cast<uint32_t *>(static_cast<int8_t *>(image) + bkv * tiles * kVTile);
    hipLaunchKernelGGL(vt_pack_kernel, dim3((unsigned)tiles, (unsigned)bkv), dim3(256), 0, stream,
                       pa);
    if (hipGetLastError() != hipSuccess) return REEF_HIP_ERROR;

    PackedArgs a;
    a.q = q;
    a.k = k;
    a.img = pa.img;
    a.bmax = pa.bmax;
    a.qs = q_scales;
    a.ks = k_scales;
    a.vs = v_scales;
    a.out = out;
    a.q_sb = qst[0];
    a.q_sh = qst[1];
    a.q_st = qst[2];
    a.k_sb = kst[0];
    a.k_sh = kst[1];
    a.k_st = kst[2];
    a.o_sb = ost[0];
    a.o_sh = ost[1];
    a.o_st = ost[2];
    a.batch = (int32_t)p->batch;
    a.q_heads = (int32_t)p->q_heads;
    a.kv_heads = (int32_t)p->kv_heads;
    a.q_len = (int32_t)p->q_len;
    a.kv_len = (int32_t)p->kv_len;
    a.query_start = (int32_t)p->query_start;
    a.window = (int32_t)p->window;
    a.score_scale = p->softmax_scale * kLog2e;
    a.q_gran = p->q_granularity;
    a.kv_gran = p->kv_granularity;
    a.kv_tiles = (int32_t)tiles;
    a.q_tiles = (int32_t)ceil_div(p->q_len, PackedShape<WAVES>::BM);
    a.per_head = (a.q_tiles + 1) / 2;
    const int64_t items = (int64_t)a.per_head * p->batch * p->q_heads;
    if (items >= (int64_t(1) << 31)) return REEF_UNSUPPORTED;
    a.items = (int32_t)items;
    a.all_precise = (p->flags & REEF_ATTN_PRECISE_PV) != 0;
    const int64_t grid = std::min<int64_t>(items, kPackedPerCu<WAVES> * compute_units());
    hipLaunchKernelGGL(prefill_packed_kernel<WAVES>, dim3((unsigned)grid), dim3(64 * WAVES), 0,
                       stream, a);
    return launch_status();
}

}  // namespace reef
