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
//     is an fp16 integer, so the image is exact.
//   * The attention kernel copies K (the caller's int8 rows) and the V image into
//     LDS with direct-to-LDS buffer loads: a ring of three K slots and one of three
//     V slots, one barrier per tile, two tiles in flight beyond the one computed.
//   * A workgroup is 4 waves x 32 query rows, two workgroups per compute unit. Per
//     64-key tile a wave computes S^T = K . Q^T on v_mfma_i32_32x32x32_i8 (K rows
//     permuted so that each lane's scores are the P operand of the next step), an
//     fp32 online softmax in base 2 with a lazy rescale, and O^T = V^T . P^T on
//     v_mfma_f32_32x32x16_f16. The scores of tile j + 1 are issued before tile j's
//     softmax so the matrix cores and the vector ALU work side by side.
//   * Precision of P: when a head's value scale allows dequantized values above
//     kHiOnlyMax (127 s_v > 1), P is split into fp16 hi + lo parts (two products, 22
//     bits) in every block; otherwise one fp16 P, each off by at most 2^-11 of
//     itself, moves an output by at most 2^-11 max|v_j - out| < 1e-3. The
//     probabilities carry an exponent offset (kShift) that keeps them out of the fp16
//     subnormals, and the row sums are of exactly the P parts the products use.
//   * Schedule: persistent workgroups; a causal head's query tiles t and T-1-t form
//     one unit with the same number of key tiles as any other pair. Each XCD owns
//     an eighth of the heads (a few at a time, whose K and V stay in that XCD's L2)
//     in a queue its workgroups take from as they finish, then the other XCDs'
//     queues; the last heads of a share come as single tiles, heaviest first. The
//     light tile of a pair runs first: its keys are a prefix of the heavy one's.
//     Grids with fewer pairs than compute units take the balanced form instead:
//     equal runs of (query tile, key tile) steps per workgroup, cut tiles merged.
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "prefill_packed.hpp"

namespace reef {

namespace {

constexpr int kPK = 64;                    // keys per tile
constexpr int kPD = 128;                   // head_dim of this path
constexpr int kKTile = kPK * kPD;          // int8 K bytes per tile
constexpr int kVTile = kPK * kPD * 2;      // fp16 V image bytes per tile
constexpr int kWaves = 4;                  // waves (32 query rows each) per workgroup
constexpr int kBM = 32 * kWaves;           // query rows per tile
// LDS: a ring of 3 K slots and a ring of 3 V slots. Tile j's values are read while
// tile j + 1's keys are read (the scores of the next tile are computed one tile
// ahead), and both rings keep two more tiles in flight.
constexpr int kSlots = 3;
constexpr int kKRing = kSlots * kKTile, kVRing = kSlots * kVTile;  // 24 KB + 48 KB
constexpr int kKBlocks = kKTile / 1024 / kWaves;  // 1 KB direct loads per wave: K tile
constexpr int kVBlocks = kVTile / 1024 / kWaves;  //                             V tile
constexpr int kXcdCount = 8;               // workgroup i of a launch runs on XCD i % 8
constexpr int kPerCu = 2;                  // resident workgroups per compute unit (2 x 72 KB)
constexpr int kQueueWords = kXcdCount + 1;
// The part a tile call computes, written to LDS by the kernel before the call (read
// there rather than passed: extra arguments of the called tile function cost it the
// address space of its LDS pointers or a save of its registers): key tiles [c0, c1)
// of the query tile, and the part slot its unnormalized result goes to (-1: the
// whole tile, normalized into the output).
struct PartInfo {
    int32_t c0, c1, slot, pad;
};
constexpr int kSmem = kKRing + kVRing + 2 * (int)sizeof(PartInfo);  // part, queue state
// A part slot (8-byte words): per wave and lane, the 64 accumulators in register
// order, then (running maximum, row sum); word e of wave w, lane l at [(w E + e) 64 + l].
constexpr int kSlotWords = kWaves * 33 * 64;
static_assert(2 * kSlotWords == kPartSlotFloats, "a part slot of the balanced schedule");

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
};

// One workgroup per (tile, batch x kv head).
__global__ __launch_bounds__(256) void vt_pack_kernel(PackArgs a) {
    constexpr int kRow = kPD + 4;  // LDS bytes per key row: column reads 8 rows apart
                                   // fall in 8 distinct banks
    __shared__ __attribute__((aligned(16))) int8_t sV[kPK * kRow];
    const int tid = threadIdx.x;
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
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // image chunk s: channel m, position s % 8 holding keys 8c .. 8c + 7
        const int s = tid + 256 * i, m = s >> 3, c = swz(m, s & 7);
        f16x8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (_Float16)sV[(8 * c + e) * kRow + m];
        *reinterpret_cast<f16x8 *>(dst + 16 * s) = o;
    }
}

struct PackedArgs {
    const int8_t *q, *k, *img;
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
    uint32_t *queue;    // kQueueWords zero-filled words: next item per XCD, then done count
    int32_t *tap;       // test hook: the exact int32 score of every visible pair, or null
    uint64_t *slots;    // balanced: part slots (kSlotWords words each)
};

// Two probabilities rounded to fp16 (a packed P operand), and the fp16 of their
// residuals p - fp16(p) (the lo operand). Each residual is exact in fp32 (one
// v_fma_mix_f32 reading the fp16 half), so hi + lo carries 22 bits of p.
__device__ __forceinline__ uint32_t pack_f16(float p0, float p1) {
    const f16x2 h = __builtin_convertvector((float __attribute__((ext_vector_type(2)))){p0, p1},
                                            f16x2);
    return __builtin_bit_cast(uint32_t, h);
}
__device__ __forceinline__ uint32_t residual_f16(uint32_t hi, float p0, float p1) {
    // Two fp32 residuals and one conversion: v_fma_mixlo/mixhi_f16 would take one
    // instruction less but read their own destination, and beside matrix instructions
    // they measured several times slower than this form.
    float r0, r1;
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r0) : "v"(hi), "v"(p0));
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
        : "=v"(r1)
        : "v"(hi), "v"(p1));
    return pack_f16(r0, r1);
}

// Row sums of the hi parts on the matrix core: v_mfma_f32_16x16x32_f16 with A = a 0/1
// pattern and B = the 32 x 16 P operand, whose lane 16g + n holds row n (g = 0, 2) or
// row 16 + n (g = 1, 3) of the score block. A row 0 sums the groups of rows 0-15, A
// row 1 those of rows 16-31: lane n (< 16) accumulates row n in register 0 and row
// 16 + n in register 1 (the other lanes' registers stay zero).
__device__ __forceinline__ f16x8 row_sum_pattern(int lane) {
    const int m = lane & 15, g = lane >> 4;
    const bool one = (m == 0 && (g & 1) == 0) || (m == 1 && (g & 1) == 1);
    const _Float16 v = one ? (_Float16)1.0f : (_Float16)0.0f;
    return f16x8{v, v, v, v, v, v, v, v};
}
// The row sum of this lane's row (lane % 32) from the accumulator above.
__device__ __forceinline__ float row_sum_of_lane(const f32x4 &rs, int lane) {
    const int col = lane & 31;
    const float r0 = __shfl(rs[0], col & 15), r1 = __shfl(rs[1], col & 15);
    return col < 16 ? r0 : r1;
}
// Scale the row sums by this lane's row factor (lanes 0-15 hold rows n and 16 + n).
__device__ __forceinline__ void scale_row_sums(f32x4 &rs, float alpha, int lane) {
    const float upper = __shfl(alpha, (lane & 15) | 16);
    rs[0] *= alpha;
    rs[1] *= upper;
}

__device__ __forceinline__ float scale_at(const float *s, int gran, int b, int h, int t, int heads,
                                          int tokens) {
    if (gran == REEF_SCALE_PER_TENSOR) return s[0];
    if (gran == REEF_SCALE_PER_HEAD) return s[h];
    return s[((int64_t)b * heads + h) * tokens + t];
}
// The same for a uniform (b, h) and token 0, as a scalar load (the scales are
// read-only during a launch).
__device__ __forceinline__ float scale_uni(const float *s, int gran, int b, int h, int heads,
                                           int tokens) {
    const int64_t i = gran == REEF_SCALE_PER_TENSOR ? 0
                      : gran == REEF_SCALE_PER_HEAD ? h
                                                    : ((int64_t)b * heads + h) * tokens;
    return *(const __attribute__((address_space(4))) float *)(s + i);
}

// Scores relative to the row's running maximum s_run, read as floats without a
// conversion: the integer product accumulates from the bit pattern 0x4B400000 - s_run,
// so the int32 result is the bit pattern of the float 12582912 + (s - s_run) for
// |s - s_run| <= 2^22 (|q.k| <= 128 * 128 * 128 = 2^21). The probability
// p = exp2((s - s_run) c + kShift) is then one FMA and an exp2: exp2(sf c - kc) with
// the per-row constant kc = 12582912 c - kShift, whose single rounding (within 1/4
// when c <= 1/2) is a factor common to the row that the row sum cancels. With a
// larger c the exact difference sf - 12582912 comes first (FAST = false).
//
// The running maximum moves when a row's largest score exceeds it by more than kLazy
// (log2 units). Then every p lies below 2^(kLazy + kShift + 1/4) < 2^16, inside the
// fp16 range, and the row's leading key has p >= 2^(kShift - 1/4): a key of weight
// 2^-22 of it still has a normal fp16 p (hi and lo keep 11 bits each), and below
// that every p is off by at most 2^-25, under 2^-33 of the row sum per key.
constexpr int32_t kScoreBias = 0x4B400000;
constexpr float kBiasF = 12582912.0f;
constexpr float kLazy = 6.0f;
constexpr float kShift = 9.0f;
constexpr float kFastCMax = 0.5f;
constexpr int32_t kMasked = 0;  // below every biased score (>= 0x4B000000)

__device__ __forceinline__ int32_t imax3(int32_t a, int32_t b, int32_t c) {
    return max(max(a, b), c);
}

// One query tile (128 rows) of one (batch, head), one wave per 32 rows. LO: P is
// hi + lo in every value block. FAST: see kScoreBias.
//
// Per 64-key tile j a wave issues 40 matrix instructions: the 8 score products of
// tile j + 1 (K rows permuted so that each lane's scores are the P operand of the
// value products), then for each of the four 16-key chunks of tile j its 4 hi and 4
// lo value products (one per 32-channel block). The vector work of tile j (exp2 of
// the scores, fp16 hi and lo, the row sum) runs one chunk ahead of the products
// that use it, between the matrix instructions: chunk 0 beside the score products,
// chunk c + 1 beside chunk c's products, and the row maximum of tile j + 1 beside
// chunk 3's. Scheduling barriers pin that interleave, so that the matrix core and
// the vector ALU of a SIMD work side by side within one wave as well as across the
// two waves of the SIMD.
//
// Not inlined: each variant's loop has the whole scalar register file (inlined
// into the item loop, the variants' scalars spilled). Arguments of a called
// function arrive in vector registers; the tile function moves every launch-wide
// value back to scalar registers so that buffer descriptors and LDS destinations
// stay scalar (no per-lane loops).
__device__ __forceinline__ int32_t uni(int32_t x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ float uni(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int32_t, x)));
}
__device__ __forceinline__ int64_t uni(int64_t x) {
    const uint64_t u = (uint64_t)x;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int32_t)(uint32_t)u);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int32_t)(uint32_t)(u >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}
template <class T>
__device__ __forceinline__ T *uni(T *p) {
    return reinterpret_cast<T *>(uni((int64_t)reinterpret_cast<uintptr_t>(p)));
}

__device__ __forceinline__ PackedArgs uniform_args(const PackedArgs &x) {
    PackedArgs a;
    a.q = uni(x.q); a.k = uni(x.k); a.img = uni(x.img);
    a.qs = uni(x.qs); a.ks = uni(x.ks); a.vs = uni(x.vs); a.out = uni(x.out);
    a.q_sb = uni(x.q_sb); a.q_sh = uni(x.q_sh); a.q_st = uni(x.q_st);
    a.k_sb = uni(x.k_sb); a.k_sh = uni(x.k_sh); a.k_st = uni(x.k_st);
    a.o_sb = uni(x.o_sb); a.o_sh = uni(x.o_sh); a.o_st = uni(x.o_st);
    a.batch = uni(x.batch); a.q_heads = uni(x.q_heads); a.kv_heads = uni(x.kv_heads);
    a.q_len = uni(x.q_len); a.kv_len = uni(x.kv_len); a.query_start = uni(x.query_start);
    a.window = uni(x.window); a.score_scale = uni(x.score_scale);
    a.q_gran = uni(x.q_gran); a.kv_gran = uni(x.kv_gran); a.kv_tiles = uni(x.kv_tiles);
    a.q_tiles = uni(x.q_tiles); a.per_head = uni(x.per_head); a.items = uni(x.items);
    a.all_precise = uni(x.all_precise);
    a.queue = uni(x.queue);
    a.tap = uni(x.tap);
    a.slots = uni(x.slots);
    return a;
}

// LDS views of the tile function's ring pointers: written as such, every operand read
// is a ds_read whatever the compiler infers across the calls.
typedef __attribute__((address_space(3))) int8_t lds_i8;
typedef __attribute__((address_space(3))) i32x4 lds_i32x4;
typedef __attribute__((address_space(3))) f16x8 lds_f16x8;

#define REEF_SLOT() __builtin_amdgcn_sched_barrier(0)
// Empty asm statements that hold a vector value in place: pin() makes the value
// appear at this point (work that reads it cannot move above), keep() makes it
// needed at this point (work that computes it cannot move below). Together with the
// scheduling barriers they keep each slot's vector work in its slot. Only values of
// vector instructions (or long-finished matrix results) pass through them.
template <class T>
__device__ __forceinline__ void pin(T &x) {
    asm volatile("" : "+v"(x));
}
template <class T>
__device__ __forceinline__ void keep(const T &x) {
    asm volatile("" ::"v"(x));
}

template <bool LO, bool FAST, bool TAP>
__device__ __forceinline__ void tile_body(const PackedArgs &a, const int b, const int h,
                                          const int tile, lds_i8 *const smem) {
    constexpr int DB = kPD / 32;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31, grp = lane >> 5;
    const int kvh = h / (a.q_heads / a.kv_heads);
    const int q0 = tile * kBM;
    const int row = q0 + wave * 32 + col;
    const bool row_ok = row < a.q_len;

    // Visible keys of this lane's row [lo, hi]; keys every row of the wave sees.
    const int pos = a.query_start + row;
    const int lo = a.window > 0 ? max(0, pos + 1 - a.window) : 0;
    const int hi = min(pos, a.kv_len - 1);
    const int w_first = q0 + wave * 32, w_last = min(w_first + 31, a.q_len - 1);
    const int full_lo = a.window > 0 ? a.query_start + w_last + 1 - a.window : 0;
    const int full_hi = w_first < a.q_len ? min(a.query_start + w_first, a.kv_len - 1) : -1;
    const int r_last = min(q0 + kBM, a.q_len) - 1;
    const int key_lo = a.window > 0 ? max(0, a.query_start + q0 + 1 - a.window) : 0;
    const int key_hi = min(a.query_start + r_last, a.kv_len - 1);
    const int kt0 = key_lo / kPK * kPK;
    // This call's key tiles [j_lo, n_tiles) of the query tile's, and its part slot.
    const __attribute__((address_space(3))) PartInfo *part =
        (const __attribute__((address_space(3))) PartInfo *)(smem + kKRing + kVRing);
    const int n_tiles = min(uni(part->c1), (key_hi - kt0) / kPK + 1);
    const int j_lo = uni(part->c0);
    const int slot = uni(part->slot);

    // Query operand and scales (independent loads, issued before the tile loads).
    i32x4 qop[kPD / 32];
    {
        const int8_t *qrow = a.q + b * a.q_sb + h * a.q_sh + (int64_t)(row_ok ? row : 0) * a.q_st;
#pragma unroll
        for (int t = 0; t < kPD / 32; ++t)
            qop[t] = row_ok ? *reinterpret_cast<const i32x4 *>(qrow + 32 * t + 16 * grp)
                            : i32x4{0, 0, 0, 0};
    }
    const float ck = scale_uni(a.ks, a.kv_gran, b, kvh, a.kv_heads, a.kv_len);
    const float cv = scale_uni(a.vs, a.kv_gran, b, kvh, a.kv_heads, a.kv_len);
    const float cq = row_ok ? scale_at(a.qs, a.q_gran, b, h, row, a.q_heads, a.q_len) : 0.0f;
    const float c = cq * ck * a.score_scale;  // log2-domain score per unit of int32 sum
    const float kc = __builtin_fmaf(kBiasF, c, -kShift);
    // Largest integer growth of a row maximum that stays within kLazy.
    const int32_t lazy_i = (int32_t)fminf(kLazy / c, 8388608.0f);

    // Direct loads: wave w fills 1 KB blocks w, w + 4, ... of a K tile and of a V
    // tile. Lane L of K block kb writes LDS row 8 kb + L / 8 at position L % 8,
    // which holds chunk swz(row, L % 8) of the key that the row stands for.
    uint32_t koff[kKBlocks], voff[kVBlocks];
#pragma unroll
    for (int i = 0; i < kKBlocks; ++i) {
        const int r = 8 * (wave + kWaves * i) + lane / 8;
        const int key = 32 * (r >> 5) + key_of_row32(r & 31);
        koff[i] = (uint32_t)(key * a.k_st + 16 * swz(r, lane & 7));
    }
#pragma unroll
    for (int i = 0; i < kVBlocks; ++i) voff[i] = (uint32_t)(16 * (64 * (wave + kWaves * i) + lane));
    const int8_t *kbase = a.k + b * a.k_sb + kvh * a.k_sh;
    const int8_t *ibase = a.img + ((int64_t)(b * a.kv_heads + kvh) * a.kv_tiles) * kVTile;
    lds_i8 *kring = smem, *vring = smem + kKRing;
    auto issue_k = [&](int j) {  // K of tile j into K slot j % 3; rows past kv_len read zeros
        const int kt = kt0 + kPK * j;
        const __amdgpu_buffer_rsrc_t kr = buffer_rsrc(
            kbase + (int64_t)kt * a.k_st, (uint32_t)((int64_t)(a.kv_len - 1 - kt) * a.k_st + kPD));
        lds_i8 *st = kring + (j % kSlots) * kKTile;
#pragma unroll
        for (int i = 0; i < kKBlocks; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                kr, (__attribute__((address_space(3))) void *)(st + 1024 * (wave + kWaves * i)), 16,
                koff[i], 0, 0, 0);
    };
    auto issue_v = [&](int j) {  // V image of tile j into V slot j % 3
        const __amdgpu_buffer_rsrc_t vr =
            buffer_rsrc(ibase + (int64_t)(kt0 / kPK + j) * kVTile, kVTile);
        lds_i8 *st = vring + (j % kSlots) * kVTile;
#pragma unroll
        for (int i = 0; i < kVBlocks; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                vr, (__attribute__((address_space(3))) void *)(st + 1024 * (wave + kWaves * i)), 16,
                voff[i], 0, 0, 0);
    };

    // LDS operand positions: K row 32u + col, chunk 2t + grp; V row 32d + col, chunk
    // 4u + 2 grp + s (keys 32u + 16 grp + 8s .. + 8, the P operand's keys).
    int kpos[kPD / 32], vpos[4];
#pragma unroll
    for (int t = 0; t < kPD / 32; ++t) kpos[t] = col * kPD + 16 * swz(col, 2 * t + grp);
#pragma unroll
    for (int cc = 0; cc < 4; ++cc)
        vpos[cc] = col * 128 + 16 * swz(col, 4 * (cc >> 1) + 2 * grp + (cc & 1));

    int32_t s_run = -(1 << 21);  // the row's running maximum of integer scores
    i32x16 bias;                 // kScoreBias - s_run in every element
#pragma unroll
    for (int r = 0; r < 16; ++r) bias[r] = kScoreBias - s_run;
    // Row sums of exactly the P parts the products use: the hi parts on the matrix core
    // (rs), the lo parts in packed fp16 per tile (lsum; a tile's lo parts sum below
    // 2^10, so its rounding is under 2^-11 of a term that is itself 2^-11 of the row
    // sum) added into this lane's fp32 share (l_lo).
    const f16x8 ones = row_sum_pattern(lane);
    f32x4 rs = {};
    float l_lo = 0.0f;
    f32x16 acc[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) acc[d] = f32x16{};
    auto operand = [](const uint32_t (&w)[4]) {
        return __builtin_bit_cast(f16x8, i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]});
    };

    struct Scores {
        i32x16 u[2];  // keys 32u .. 32u + 31 of a tile: register r of lane group g is key 16g + r
    };
    // The lane's largest score of a tile, then the row's (both lane groups).
    auto lane_max = [](const Scores &sc) {
        int32_t t[11];
#pragma unroll
        for (int i = 0; i < 10; ++i) {
            const int k0 = 3 * i, k1 = 3 * i + 1, k2 = 3 * i + 2;
            t[i] = imax3(sc.u[k0 >> 4][k0 & 15], sc.u[k1 >> 4][k1 & 15], sc.u[k2 >> 4][k2 & 15]);
        }
        t[10] = max(sc.u[1][14], sc.u[1][15]);
        const int32_t a0 = imax3(t[0], t[1], t[2]), a1 = imax3(t[3], t[4], t[5]);
        const int32_t a2 = imax3(t[6], t[7], t[8]), a3 = max(t[9], t[10]);
        return max(imax3(a0, a1, a2), a3);
    };
    auto row_max = [](int32_t m) {
        const auto r = __builtin_amdgcn_permlane32_swap(m, m, false, false);
        return max((int32_t)r[0], (int32_t)r[1]);
    };
    auto mask_scores = [&](Scores &sc, int j) {  // keys outside [lo, hi] of tile j
        const int kt = kt0 + kPK * j;
        if (!(kt + kPK - 1 <= full_hi && kt >= full_lo)) {  // uniform
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kt + 32 * u + 16 * grp + r;
                    if (key < lo || key > hi) sc.u[u][r] = kMasked;
                }
            return true;
        }
        return false;
    };
    // The lazy rescale before tile j's probabilities, from this lane's maximum mx of
    // the tile: when some score exceeds s_run by more than lazy_i, each row moves s_run
    // to its maximum, and the scores already computed against the old s_run move with
    // it.
    auto rescale = [&](Scores &sc, int32_t mx) {
        if (__any(mx - kScoreBias > lazy_i)) {  // wave-uniform
            // The row's maximum over both lane groups (a cross-lane swap, which waits
            // for the matrix instructions in flight: only here, on the rare rescale).
            const int32_t d = row_max(mx) - kScoreBias;
            const int32_t delta = d > 0 ? d : 0;
            s_run += delta;
            const float alpha = __builtin_amdgcn_exp2f(-(float)delta * c);
            scale_row_sums(rs, alpha, lane);
            l_lo *= alpha;
#pragma unroll
            for (int dd = 0; dd < DB; ++dd) acc[dd] *= alpha;
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int r = 0; r < 16; ++r) sc.u[u][r] -= delta;
#pragma unroll
            for (int r = 0; r < 16; ++r) bias[r] = kScoreBias - s_run;
        }
    };
    // Keys 8s + e .. 8s + e + 3 of chunk cc = 2u + s in two stages, placed a matrix
    // instruction apart so that the exp2 latency is covered: expo() the probabilities
    // p in fp32, pack() their fp16 hi and lo parts and the lo parts' sum. A masked key
    // (or, after a rescale, a masked key moved below zero) has p = 0.
    auto expo = [&](const Scores &sc, int cc, int e, float (&p)[4], auto masked_tag) {
        constexpr bool MASKED = decltype(masked_tag)::value;
        int32_t x[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[i] = sc.u[cc >> 1][8 * (cc & 1) + e + i];
            pin(x[i]);
        }
        float arg[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float sf = __int_as_float(x[i]);
            arg[i] = FAST ? __builtin_fmaf(sf, c, -kc) : __builtin_fmaf(sf - kBiasF, c, kShift);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            p[i] = __builtin_amdgcn_exp2f(arg[i]);
            if (MASKED) p[i] = x[i] <= kMasked ? 0.0f : p[i];
            keep(p[i]);
        }
    };
    auto pack = [&](int e, const float (&p)[4], uint32_t (&ph)[4], uint32_t (&pl)[4],
                    f16x2 &lsum) {
        float q[4] = {p[0], p[1], p[2], p[3]};
#pragma unroll
        for (int i = 0; i < 4; ++i) pin(q[i]);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const uint32_t hw = pack_f16(q[2 * k], q[2 * k + 1]);
            ph[e / 2 + k] = hw;
            keep(hw);
        }
        if (LO) {
            uint32_t lw[2];
#pragma unroll
            for (int k = 0; k < 2; ++k) lw[k] = residual_f16(ph[e / 2 + k], q[2 * k], q[2 * k + 1]);
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                pl[e / 2 + k] = lw[k];
                keep(lw[k]);
            }
            lsum += __builtin_bit_cast(f16x2, lw[0]) + __builtin_bit_cast(f16x2, lw[1]);
            keep(lsum);
        }
    };

    // Loads: K of tile 0, then per iteration g the group {K(g + 1), V(g)}, issued two
    // iterations ahead. Iteration j waits for its own group (the next group may be
    // in flight; counts are this wave's loads, vmcnt in bits 3:0 of the s_waitcnt
    // immediate, 0xf70 leaving expcnt and lgkmcnt unconstrained) and a barrier makes
    // every wave's loads visible and frees the slots of tiles j - 1 (values) and j
    // (keys, read in iteration j - 1).
    auto group_loads = [&](int g) {
        return (g + 1 < n_tiles ? kKBlocks : 0) + (g < n_tiles ? kVBlocks : 0);
    };
    auto issue_group = [&](int g) {
        if (g + 1 < n_tiles) issue_k(g + 1);
        if (g < n_tiles) issue_v(g);
    };
    auto wait_loads = [](int n) {  // at most n of this wave's loads still in flight
        switch (n) {
        case 0: __builtin_amdgcn_s_waitcnt(0xf70); break;
        case kKBlocks: __builtin_amdgcn_s_waitcnt(0xf70 | kKBlocks); break;
        case kVBlocks: __builtin_amdgcn_s_waitcnt(0xf70 | kVBlocks); break;
        default: __builtin_amdgcn_s_waitcnt(0xf70 | (kKBlocks + kVBlocks)); break;
        }
    };
    static_assert(kKBlocks + kVBlocks < 16, "vmcnt fits the low field");

    struct Tile {
        Scores s;
        int32_t mx;  // this lane's maximum of s
    };
    // Scores of tile j_lo (the prologue; later tiles' scores come from step()).
    auto first_scores = [&]() {
        Tile t;
        const lds_i8 *sK = kring + (j_lo % kSlots) * kKTile;
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int tt = 0; tt < kPD / 32; ++tt) {
                const i32x4 kop = *reinterpret_cast<const lds_i32x4 *>(sK + 4096 * u + kpos[tt]);
                t.s.u[u] = mfma_32x32x32_i8(kop, qop[tt], tt == 0 ? bias : t.s.u[u]);
            }
        mask_scores(t.s, j_lo);
        t.mx = lane_max(t.s);
        return t;
    };

    // Tile j: wait for its loads, rescale, then the interleaved products and vector
    // work described above; returns tile j + 1's scores and row maximum. Past the last
    // tile the scores are computed from a stale K slot (no slot is being written at
    // that point) and discarded.
    auto step = [&](const int j, auto masked_tag, auto mask_next_tag, Tile &cur) {
        constexpr bool MASK_NEXT = decltype(mask_next_tag)::value;
        wait_loads(group_loads(j + 1));
        __builtin_amdgcn_s_barrier();
        issue_group(j + 2);
        rescale(cur.s, cur.mx);
        if constexpr (TAP) {
            // Test hook: tile j's integer scores, read back from the accumulators
            // relative to s_run, for every key the row sees.
            int32_t *trow = a.tap + ((int64_t)(b * a.q_heads + h) * a.q_len + row) * a.kv_len;
            const int kt = kt0 + kPK * j;
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kt + 32 * u + 16 * grp + r;
                    if (row_ok && key >= lo && key <= hi)
                        trow[key] = cur.s.u[u][r] - kScoreBias + s_run;
                }
        }
        const lds_i8 *sK = kring + ((j + 1) % kSlots) * kKTile;
        const lds_i8 *sV = vring + (j % kSlots) * kVTile;
        i32x4 kop[2][kPD / 32];
        f16x8 vop[4][DB];
        uint32_t ph[4][4], pl[4][4];
        Tile nx;
        auto kread = [&](int u, int t) {
            kop[u][t] = *reinterpret_cast<const lds_i32x4 *>(sK + 4096 * u + kpos[t]);
        };
        auto vread = [&](int cc) {
#pragma unroll
            for (int d = 0; d < DB; ++d)
                vop[cc][d] = *reinterpret_cast<const lds_f16x8 *>(sV + 4096 * d + vpos[cc]);
        };
        auto qk = [&](int u, int t) {
            nx.s.u[u] = mfma_32x32x32_i8(kop[u][t], qop[t], t == 0 ? bias : nx.s.u[u]);
        };
        auto pv = [&](int cc, int d, bool lo_part) {
            acc[d] = mfma_32x32x16_f16(vop[cc][d], operand(lo_part ? pl[cc] : ph[cc]), acc[d]);
        };
        f16x2 lsum = {};
        float pe[4][2][4];  // fp32 p of chunk cc, keys 4h .. 4h + 3, between the two stages
        auto ex = [&](int cc, int hh) { expo(cur.s, cc, 4 * hh, pe[cc][hh], masked_tag); };
        auto pk = [&](int cc, int hh) { pack(4 * hh, pe[cc][hh], ph[cc], pl[cc], lsum); };
        // This tile's hi row sums on their own, added to the running sums once per tile.
        f32x4 rs_tile = {};
        auto rsum = [&](int cc) { rs_tile = mfma_16x16x32_f16(ones, operand(ph[cc]), rs_tile); };

        kread(0, 0);
        kread(1, 0);
        kread(0, 1);
        kread(1, 1);
        vread(0);
        REEF_SLOT();
        // Score products of tile j + 1 beside chunk 0's probabilities and chunk 1's
        // exponentials.
        ex(0, 0);
        qk(0, 0);
        REEF_SLOT();
        ex(0, 1);
        qk(1, 0);
        REEF_SLOT();
        kread(0, 2);
        kread(1, 2);
        kread(0, 3);
        kread(1, 3);
        pk(0, 0);
        qk(0, 1);
        REEF_SLOT();
        pk(0, 1);
        qk(1, 1);
        REEF_SLOT();
        ex(1, 0);
        qk(0, 2);
        REEF_SLOT();
        ex(1, 1);
        qk(1, 2);
        REEF_SLOT();
        qk(0, 3);
        REEF_SLOT();
        qk(1, 3);
        REEF_SLOT();
        // Chunk cc's row sum and value products beside chunk cc + 1's packing and chunk
        // cc + 2's exponentials (for the last chunks, beside tile j + 1's row maximum).
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            if (cc < 3) vread(cc + 1);
            rsum(cc);
            REEF_SLOT();
#pragma unroll
            for (int d = 0; d < DB; ++d) {
                if (cc < 3 && d < 2) pk(cc + 1, d);
                if (cc < 2 && d >= 2) ex(cc + 2, d - 2);
                if (cc == 2 && d == 2) {
                    pin(nx.s.u[0]);
                    pin(nx.s.u[1]);
                    nx.mx = lane_max(nx.s);
                    keep(nx.mx);
                }
                pv(cc, d, false);
                REEF_SLOT();
            }
            if (LO) {
#pragma unroll
                for (int d = 0; d < DB; ++d) {
                    pv(cc, d, true);
                    REEF_SLOT();
                }
            }
        }
        if (LO) l_lo += (float)lsum[0] + (float)lsum[1];
        rs[0] += rs_tile[0];
        rs[1] += rs_tile[1];
        if (MASK_NEXT && mask_scores(nx.s, j + 1)) nx.mx = lane_max(nx.s);
        return nx;
    };

    issue_k(j_lo);
    issue_group(j_lo);
    issue_group(j_lo + 1);
    wait_loads(group_loads(j_lo) + group_loads(j_lo + 1));
    __builtin_amdgcn_s_barrier();
    Tile tl = first_scores();
    // Tiles [it_a, it_b) are whole for every row of the workgroup: no masks (segment
    // ends clamped to this call's tiles).
    const int wg_full_lo = a.window > 0 ? a.query_start + r_last + 1 - a.window : 0;
    const int wg_full_hi = min(a.query_start + q0, a.kv_len - 1);
    const int span = wg_full_hi + 1 - kt0;
    const int it_a = max(j_lo, min(n_tiles, max(0, wg_full_lo - kt0 + kPK - 1) / kPK));
    const int it_b = max(it_a, min(n_tiles, span > 0 ? span / kPK : 0));
    // Two tiles per iteration: the loop-carried scores come back in the registers
    // they left, with no copies.
    // Tile j + 1 needs its scores masked only when it lies outside [it_a, it_b).
    int j = j_lo;
    auto run = [&](const int end, auto masked_tag, auto mask_next_tag) {
        for (; j + 1 < end; j += 2) {
            Tile mid = step(j, masked_tag, mask_next_tag, tl);
            tl = step(j + 1, masked_tag, mask_next_tag, mid);
        }
        if (j < end) {
            tl = step(j, masked_tag, mask_next_tag, tl);
            ++j;
        }
    };
    run(it_a, std::true_type{}, std::true_type{});
    run(it_b - 1, std::false_type{}, std::false_type{});
    run(it_b, std::false_type{}, std::true_type{});
    run(n_tiles, std::true_type{}, std::true_type{});

    const float l_row = row_sum_of_lane(rs, lane) + (LO ? xor32_sum(l_lo) : 0.0f);
    if (slot >= 0) {
        // A part of the query tile: its unnormalized accumulators and (s_run, row sum),
        // every lane (rows past q_len hold finite values), with device-coherent stores
        // (written through beneath the per-XCD L2s) that complete before the barrier
        // below. The merge reads them the same way.
        uint64_t *so = a.slots + (int64_t)slot * kSlotWords;
        auto put = [&](int e, uint64_t v) { part_store(so + (wave * 33 + e) * 64 + lane, v); };
        auto pack2 = [](float x, float y) {
            return (uint64_t)__float_as_uint(x) | ((uint64_t)__float_as_uint(y) << 32);
        };
#pragma unroll
        for (int d = 0; d < DB; ++d)
#pragma unroll
            for (int e = 0; e < 8; ++e) put(8 * d + e, pack2(acc[d][2 * e], acc[d][2 * e + 1]));
        put(32, (uint64_t)(uint32_t)s_run | ((uint64_t)__float_as_uint(l_row) << 32));
        part_stores_done();
    } else if (row_ok) {
        float *orow = a.out + b * a.o_sb + h * a.o_sh + (int64_t)row * a.o_st;
        const float norm = cv / l_row;
#pragma unroll
        for (int d = 0; d < DB; ++d) {
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                f32x4 o;
#pragma unroll
                for (int i = 0; i < 4; ++i) o[i] = acc[d][4 * jj + i] * norm;
                *reinterpret_cast<f32x4 *>(orow + 32 * d + 8 * jj + 4 * grp) = o;
            }
        }
    }
    // The next tile of this workgroup reuses the rings.
    __syncthreads();
}

template <bool LO, bool FAST>
__device__ __attribute__((noinline)) void packed_tile(const PackedArgs &args, int b_in, int h_in,
                                                      int tile_in, int8_t *smem_in) {
    tile_body<LO, FAST, false>(uniform_args(args), uni(b_in), uni(h_in), uni(tile_in),
                               (lds_i8 *)uni(smem_in));
}

// Whether P needs hi + lo parts for (batch, kv head): its value scale allows
// dequantized magnitudes above kHiOnlyMax (the same rule as the other prefill
// schedules: 127 s_v, the largest magnitude the engine's quantize_int8 produces).
__device__ __forceinline__ bool needs_lo(const PackedArgs &a, int b, int kvh) {
    if (a.all_precise) return true;
    return 127.0f * scale_uni(a.vs, a.kv_gran, b, kvh, a.kv_heads, a.kv_len) > kHiOnlyMax;
}

// XCD y's share of the work: the (batch, head) pairs [bh0, bh0 + nh), an eighth of
// them (a few consecutive heads, whose K and V stay in the XCD's L2). Its units: the
// query-tile pairs of the first nh - tail heads, then the single query tiles of the
// last `tail` heads, heaviest first, so that the last units of a launch are short.
struct Share {
    int bh0, nh, tail, pairs, units;
};
__device__ __forceinline__ Share share_of(const PackedArgs &a, int y) {
    const int64_t bh_total = (int64_t)a.batch * a.q_heads;
    const int wgs = max(1, (int)gridDim.x / kXcdCount);
    Share s;
    s.bh0 = (int)(bh_total * y / kXcdCount);
    s.nh = (int)(bh_total * (y + 1) / kXcdCount) - s.bh0;
    s.tail = min(s.nh, (4 * wgs + a.q_tiles - 1) / a.q_tiles);  // about four tiles per workgroup
    s.pairs = (s.nh - s.tail) * a.per_head;
    s.units = s.pairs + s.tail * a.q_tiles;
    return s;
}

// The queue state of a workgroup, in LDS after the part record: the unit taken last
// (its XCD share and index, or unit -1 when every queue is empty) and the number of
// queues found empty so far (the own XCD's first).
struct QueueState {
    int32_t share, unit, tried, pad;
};
constexpr int kQueueOff = kKRing + kVRing + (int)sizeof(PartInfo);
static_assert(kQueueOff + (int)sizeof(QueueState) <= kSmem, "queue state in LDS");

// Thread 0: takes the next unit into q (unit -1 when every queue is empty). The caller
// places a barrier before the unit is read.
__device__ __forceinline__ void take_unit(const PackedArgs &a,
                                          __attribute__((address_space(3))) QueueState *q) {
    const int x = blockIdx.x % kXcdCount;
    int tried = q->tried;
    int unit = -1, share = 0;
    while (tried < kXcdCount) {
        share = (x + tried) % kXcdCount;
        const uint32_t n = __hip_atomic_fetch_add(a.queue + share, 1u, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
        if ((int64_t)n < share_of(a, share).units) {
            unit = (int)n;
            break;
        }
        ++tried;
    }
    q->tried = tried;
    q->share = share;
    q->unit = unit;
}

// (batch x head, light tile, heavy tile or -1) of unit u of XCD share y.
struct Unit {
    int bh, first, second;
};
__device__ __forceinline__ Unit unit_tiles(const PackedArgs &a, int y, int u) {
    const Share s = share_of(a, y);
    Unit r;
    r.second = -1;
    if (u < s.pairs) {
        r.bh = s.bh0 + u / a.per_head;
        r.first = u % a.per_head;                  // the light tile, whose keys are a prefix
        if (a.q_tiles - 1 - r.first != r.first) r.second = a.q_tiles - 1 - r.first;  // of the heavy's
    } else {
        const int v = u - s.pairs;
        r.bh = s.bh0 + (s.nh - s.tail) + v % s.tail;
        r.first = a.q_tiles - 1 - v / s.tail;
    }
    return r;
}

// The tile-function variant of (batch, head): bit 0 hi + lo P, bit 1 one FMA per
// probability (the score factor c small enough that 12582912 c rounds within 1/4;
// not with per-token q scales, where c varies by row).
__device__ __forceinline__ int head_variant(const PackedArgs &a, int b, int h) {
    const int kvh = h / (a.q_heads / a.kv_heads);
    const float c = a.q_gran == REEF_SCALE_PER_TOKEN
                        ? INFINITY
                        : scale_uni(a.qs, a.q_gran, b, h, a.q_heads, a.q_len) *
                              scale_uni(a.ks, a.kv_gran, b, kvh, a.kv_heads, a.kv_len) *
                              a.score_scale;
    return (needs_lo(a, b, kvh) ? 1 : 0) | (c <= kFastCMax ? 2 : 0);
}

// Units of one variant, from the unit in the queue state on: computes each unit's
// tiles and takes the next unit, until every queue is empty (returns -1) or the next
// unit needs another variant (returns that variant; the unit stays in the queue state
// for the next call). One call per workgroup and variant: the launch arguments,
// scales and registers of a call are set up once, not per tile.
template <bool LO, bool FAST, bool TAP>
__device__ __attribute__((noinline)) int packed_units(const PackedArgs &args, int8_t *smem_in) {
    const PackedArgs a = uniform_args(args);
    lds_i8 *const smem = (lds_i8 *)uni(smem_in);
    auto *q = (__attribute__((address_space(3))) QueueState *)(smem + kQueueOff);
    constexpr int kMine = (LO ? 1 : 0) | (FAST ? 2 : 0);
    for (;;) {
        const int y = uni(q->share), u = uni(q->unit);
        if (u < 0) return -1;
        const Unit t = unit_tiles(a, y, u);
        const int b = t.bh / a.q_heads, h = t.bh % a.q_heads;
        if (!TAP) {
            const int var = head_variant(a, b, h);
            if (var != kMine) return var;
        }
        tile_body<LO, FAST, TAP>(a, b, h, t.first, smem);
        if (t.second >= 0) tile_body<LO, FAST, TAP>(a, b, h, t.second, smem);
        // The tile body ended with a barrier: every thread has read the queue state.
        if (threadIdx.x == 0) take_unit(a, q);
        __syncthreads();
    }
}

// Two workgroups per compute unit: the two waves on each SIMD belong to different
// workgroups and fill each other's waits. Units are taken from a queue per XCD (its
// share above, in order, as the workgroups finish the previous one), then from the
// other XCDs' queues. Units differ in cost (the single tiles; heads with hi + lo P):
// with pairs dealt out in a fixed order the last workgroups ended 15 % after the mean
// (4x32x8192x128: 2.30 ms dealt out, 2.18-2.19 ms from the queues of pairs, whose
// last workgroups still ended 7 % after the mean; with the single tiles last 3 %, 1 %
// faster; with four single tiles per workgroup instead of two, 2173 against 2213 us
// over six runs on one box, and no run slower than 2.2 ms). The last workgroup to
// finish resets the queue to zero for the next call.
__global__ __launch_bounds__(64 * kWaves, kPerCu) void prefill_packed_kernel(PackedArgs a) {
    __shared__ __attribute__((aligned(1024))) int8_t smem[kSmem];
    auto *q = reinterpret_cast<QueueState *>(smem + kQueueOff);
    if (threadIdx.x == 0) {
        // Every call computes a whole query tile.
        *reinterpret_cast<PartInfo *>(smem + kKRing + kVRing) = PartInfo{0, INT32_MAX, -1, 0};
        q->tried = 0;
        take_unit(a, (__attribute__((address_space(3))) QueueState *)q);
    }
    __syncthreads();
    for (;;) {
        const int u = __builtin_amdgcn_readfirstlane(q->unit);
        if (u < 0) break;
        int var;
        if (a.tap) {  // the score hook's launch: one fp16 P, small c (see the entry point)
            var = packed_units<false, true, true>(a, smem);
        } else {
            const Unit t = unit_tiles(a, __builtin_amdgcn_readfirstlane(q->share), u);
            switch (head_variant(a, t.bh / a.q_heads, t.bh % a.q_heads)) {
            case 0: var = packed_units<false, false, false>(a, smem); break;
            case 1: var = packed_units<true, false, false>(a, smem); break;
            case 2: var = packed_units<false, true, false>(a, smem); break;
            default: var = packed_units<true, true, false>(a, smem); break;
            }
        }
        if (__builtin_amdgcn_readfirstlane(var) < 0) break;
    }
    // Every take of this workgroup has returned; the last workgroup to count itself
    // here is the last to use the queue.
    if (threadIdx.x == 0 &&
        __hip_atomic_fetch_add(a.queue + kXcdCount, 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1) {
        for (int y = 0; y < kQueueWords; ++y)
            __hip_atomic_store(a.queue + y, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Steps of the balanced form: a step is (query tile, 64-key tile). Key tiles of query
// tile `tile`, and their sum over the tiles before T (each of them 128 rows; a window
// drops a prefix of keys), in closed form.
__host__ __device__ inline int64_t floor_div64(int64_t x, int64_t y) {  // y > 0
    return x >= 0 ? x / y : -((-x + y - 1) / y);
}
__host__ __device__ inline int64_t tile_key_tiles(int64_t q_len, int64_t kv_len, int64_t qstart,
                                                  int64_t window, int64_t tile) {
    const int64_t q0 = tile * kBM;
    const int64_t r_last = (q0 + kBM < q_len ? q0 + kBM : q_len) - 1;
    int64_t key_lo = window > 0 ? qstart + q0 + 1 - window : 0;
    if (key_lo < 0) key_lo = 0;
    const int64_t key_hi = (qstart + r_last < kv_len - 1 ? qstart + r_last : kv_len - 1);
    return (key_hi - key_lo / kPK * kPK) / kPK + 1;
}
__host__ __device__ inline int64_t key_tiles_before(int64_t qstart, int64_t window, int64_t T) {
    // Without a window tile t has 2t + 1 + floor((qstart + 127) / 64) key tiles.
    int64_t s = T + T * (T - 1) + ((qstart + 127) / kPK) * T;
    if (window > 0) {
        int64_t t0 = floor_div64(window - qstart - 1, kBM) + 1;
        if (t0 < 0) t0 = 0;
        if (T > t0) s -= (T - t0) * (T + t0 - 1) + floor_div64(qstart + 1 - window, kPK) * (T - t0);
    }
    return s;
}

struct BalArgs {
    int64_t units;       // steps of all query tiles
    int64_t per_head;    // steps of one (batch, head)
    uint32_t *counters;  // one per query tile, zero between launches
};

// The last part of a cut query tile: every part's accumulators and (s_run, row sum)
// from its slot (this part's too), folded in part order, so the output does not
// depend on which part finished last.
__device__ void merge_parts(const PackedArgs &a, int b, int h, int tile, int parts, int first_wg,
                            int64_t item_u0, int64_t units) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, grp = lane >> 5;
    const int kvh = h / (a.q_heads / a.kv_heads);
    const int row = tile * kBM + wave * 32 + col;
    const bool row_ok = row < a.q_len;
    const int G = gridDim.x;
    const float ck = scale_uni(a.ks, a.kv_gran, b, kvh, a.kv_heads, a.kv_len);
    const float cv = scale_uni(a.vs, a.kv_gran, b, kvh, a.kv_heads, a.kv_len);
    const float cq = row_ok ? scale_at(a.qs, a.q_gran, b, h, row, a.q_heads, a.q_len) : 0.0f;
    const float c = cq * ck * a.score_scale;
    auto get = [](const uint64_t *p) { return part_load(p); };
    // Part p is logical workgroup first_wg + p; the first part sits in that
    // workgroup's second slot when its range began before this tile.
    auto slot_of = [&](int p) {
        const int lp = first_wg + p;
        const bool second = p == 0 && (int64_t)lp * units / G < item_u0;
        return a.slots + (int64_t)(2 * lp + (second ? 1 : 0)) * kSlotWords + wave * 33 * 64 + lane;
    };
    // One pass: a running maximum of the parts' s_run with explicit fused
    // multiply-adds, the next part's loads in flight while this one is folded.
    uint64_t cur[33], nxt[33];
    auto fetch = [&](uint64_t(&v)[33], int p) {
        const uint64_t *sl = slot_of(p);
#pragma unroll
        for (int e = 0; e < 33; ++e) v[e] = get(sl + e * 64);
    };
    auto lo32 = [](uint64_t w) { return __uint_as_float((uint32_t)w); };
    auto hi32 = [](uint64_t w) { return __uint_as_float((uint32_t)(w >> 32)); };
    fetch(cur, 0);
    int32_t m = 0;
    float l = 0.0f;
    f32x16 tot[kPD / 32];
#pragma unroll
    for (int d = 0; d < kPD / 32; ++d) tot[d] = f32x16{};
    for (int p = 0; p < parts; ++p) {
        if (p + 1 < parts) fetch(nxt, p + 1);
        const int32_t sp = (int32_t)(uint32_t)cur[32];
        const int32_t mn = p == 0 ? sp : max(m, sp);
        const float er = p == 0 ? 0.0f : __builtin_amdgcn_exp2f((float)(m - mn) * c);
        const float ep = __builtin_amdgcn_exp2f((float)(sp - mn) * c);
        l = __builtin_fmaf(ep, hi32(cur[32]), l * er);
#pragma unroll
        for (int e = 0; e < 32; ++e) {
            const int d = e / 8, i = 2 * (e % 8);
            tot[d][i] = __builtin_fmaf(ep, lo32(cur[e]), tot[d][i] * er);
            tot[d][i + 1] = __builtin_fmaf(ep, hi32(cur[e]), tot[d][i + 1] * er);
        }
        m = mn;
#pragma unroll
        for (int e = 0; e < 33; ++e) cur[e] = nxt[e];
    }
    if (!row_ok) return;
    float *orow = a.out + b * a.o_sb + h * a.o_sh + (int64_t)row * a.o_st;
    const float norm = cv / l;
#pragma unroll
    for (int d = 0; d < kPD / 32; ++d) {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            f32x4 o;
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = tot[d][4 * jj + i] * norm;
            *reinterpret_cast<f32x4 *>(orow + 32 * d + 8 * jj + 4 * grp) = o;
        }
    }
}

// Balanced form for grids with fewer query-tile pairs than compute units: the steps
// of all query tiles ((batch, head), then tile, then key tile) are cut into G equal
// runs, one per workgroup, logical workgroup L holding [L units / G, (L + 1) units /
// G); the G / 8 workgroups of one XCD (hardware workgroup g runs on XCD g % 8) hold
// consecutive L, so an XCD's L2 sees a few heads. A query tile that a run boundary
// cuts is computed in parts: each part leaves its unnormalized result in a slot, and
// the part that counts in last (a counter per query tile) merges them. The counting
// protocol is the balanced prefill's and the decode merge's: slot stores are
// device-coherent and complete before the barrier that precedes the relaxed
// agent-scope increment; the merging part reads the slots after its increment
// returned.
__global__ __launch_bounds__(64 * kWaves, kPerCu) void prefill_packed_bal_kernel(PackedArgs a,
                                                                                 BalArgs ba) {
    __shared__ __attribute__((aligned(1024))) int8_t smem[kSmem];
    __shared__ uint32_t sTicket;
    PartInfo *sPart = reinterpret_cast<PartInfo *>(smem + kKRing + kVRing);
    const int G = gridDim.x, g = blockIdx.x;
    const int x = g % kXcdCount, per = G / kXcdCount, rem = G % kXcdCount;
    const int L = x * per + min(x, rem) + g / kXcdCount;
    int64_t u = (int64_t)L * ba.units / G;
    const int64_t u_end = (int64_t)(L + 1) * ba.units / G;
    // The first step: (batch, head), then the query tile by bisection over the
    // closed-form prefix sums (the grid has at most one workgroup per step).
    int bh = (int)(u / ba.per_head);
    const int64_t r0 = u - (int64_t)bh * ba.per_head;
    int lo = 0, hi = a.q_tiles - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (key_tiles_before(a.query_start, a.window, mid) <= r0) lo = mid;
        else hi = mid - 1;
    }
    int tile = lo;
    int c0 = (int)(r0 - key_tiles_before(a.query_start, a.window, tile));
    auto wg_of = [&](int64_t unit) { return (int)(((unit + 1) * G - 1) / ba.units); };
    bool first = true;
    while (u < u_end) {
        const int n = (int)tile_key_tiles(a.q_len, a.kv_len, a.query_start, a.window, tile);
        const int c1 = (int)(c0 + (u_end - u) < n ? c0 + (u_end - u) : n);
        const int64_t item_u0 = u - c0;
        const int first_wg = wg_of(item_u0);
        const int parts = wg_of(item_u0 + n - 1) - first_wg + 1;
        const int b = bh / a.q_heads, h = bh % a.q_heads;
        if (threadIdx.x == 0)
            *sPart = PartInfo{c0, c1, parts > 1 ? 2 * L + (first ? 0 : 1) : -1, 0};
        __syncthreads();
        switch (head_variant(a, b, h)) {
        case 0: packed_tile<false, false>(a, b, h, tile, smem); break;
        case 1: packed_tile<true, false>(a, b, h, tile, smem); break;
        case 2: packed_tile<false, true>(a, b, h, tile, smem); break;
        default: packed_tile<true, true>(a, b, h, tile, smem); break;
        }
        if (parts > 1) {
            // The tile call ended with a barrier after every slot store completed.
            uint32_t *counter = ba.counters + (int64_t)bh * a.q_tiles + tile;
            if (threadIdx.x == 0) sTicket = part_count(counter);
            __syncthreads();
            if (sTicket == (uint32_t)(parts - 1)) {
                part_claimed();
                if (threadIdx.x == 0) part_reset(counter);  // ready for the next launch
                merge_parts(a, b, h, tile, parts, first_wg, item_u0, ba.units);
            }
        }
        u += c1 - c0;
        c0 = 0;
        first = false;
        if (++tile == a.q_tiles) {
            tile = 0;
            ++bh;
        }
        __syncthreads();  // sPart and sTicket are written again for the next tile
    }
}

}  // namespace

int64_t packed_image_bytes(int64_t batch, int64_t kv_heads, int64_t kv_len) {
    return batch * kv_heads * ceil_div(kv_len, kPK) * kVTile;
}

namespace {
reef_status packed_launch(const reef_attention_params *p, const int8_t *q, const int64_t (&qst)[3],
                          const int8_t *k, const int64_t (&kst)[3], const int8_t *v,
                          const int64_t (&vst)[3], const float *q_scales, const float *k_scales,
                          const float *v_scales, float *out, const int64_t (&ost)[3], void *image,
                          const PackedWork &work, int32_t *tap, hipStream_t stream) {
    if (!packed_fits(*p)) return REEF_UNSUPPORTED;
    const int64_t tiles = ceil_div(p->kv_len, kPK);
    const int64_t bkv = p->batch * p->kv_heads;
    PackArgs pa;
    pa.v = v;
    pa.v_sb = vst[0];
    pa.v_sh = vst[1];
    pa.v_st = vst[2];
    pa.kv_heads = (int32_t)p->kv_heads;
    pa.kv_len = (int32_t)p->kv_len;
    pa.tiles = (int32_t)tiles;
    pa.img = static_cast<int8_t *>(image);
    hipLaunchKernelGGL(vt_pack_kernel, dim3((unsigned)tiles, (unsigned)bkv), dim3(256), 0, stream,
                       pa);
    if (hipGetLastError() != hipSuccess) return REEF_HIP_ERROR;

    PackedArgs a;
    a.q = q;
    a.k = k;
    a.img = pa.img;
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
    a.q_tiles = (int32_t)ceil_div(p->q_len, kBM);
    a.per_head = (a.q_tiles + 1) / 2;
    const int64_t items = (int64_t)a.per_head * p->batch * p->q_heads;
    a.items = (int32_t)items;
    a.all_precise = (p->flags & REEF_ATTN_PRECISE_PV) != 0;
    a.queue = work.queue;
    a.tap = tap;
    a.slots = reinterpret_cast<uint64_t *>(work.slots);
    if (work.balanced && !tap) {
        BalArgs ba;
        ba.per_head = key_tiles_before(p->query_start, p->window, a.q_tiles - 1) +
                      tile_key_tiles(p->q_len, p->kv_len, p->query_start, p->window, a.q_tiles - 1);
        ba.units = ba.per_head * p->batch * p->q_heads;
        ba.counters = work.counters;
        // At most one workgroup per step, so that every run holds a step.
        const int64_t grid = std::min<int64_t>(ba.units, kPerCu * compute_units());
        hipLaunchKernelGGL(prefill_packed_bal_kernel, dim3((unsigned)grid), dim3(64 * kWaves), 0,
                           stream, a, ba);
        return launch_status();
    }
    const int64_t grid = std::min<int64_t>(items, kPerCu * compute_units());
    hipLaunchKernelGGL(prefill_packed_kernel, dim3((unsigned)grid), dim3(64 * kWaves), 0, stream,
                       a);
    return launch_status();
}

__global__ void tap_scales_kernel(float *s) {
    s[0] = 1.0f;          // q and k: per tensor, unit scale
    s[1] = 1.0f / 254.0f;  // v: values within 1/2, one fp16 P
}

// Workspace of the score hook: queue words, the V image, the attention output, scales.
struct TapLayout {
    int64_t image, out, scales, total;
};
TapLayout tap_layout(int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t q_len,
                     int64_t kv_len) {
    TapLayout t;
    t.image = 256;
    t.out = t.image + ceil_div(packed_image_bytes(batch, kv_heads, kv_len), 256) * 256;
    t.scales = t.out + ceil_div(batch * q_heads * q_len * kPD * 4, 256) * 256;
    t.total = t.scales + 256;
    return t;
}
}  // namespace

reef_status prefill_packed_launch(const reef_attention_params *p, const int8_t *q,
                                  const int64_t (&qst)[3], const int8_t *k,
                                  const int64_t (&kst)[3], const int8_t *v,
                                  const int64_t (&vst)[3], const float *q_scales,
                                  const float *k_scales, const float *v_scales, float *out,
                                  const int64_t (&ost)[3], void *image, const PackedWork &work,
                                  hipStream_t stream) {
    return packed_launch(p, q, qst, k, kst, v, vst, q_scales, k_scales, v_scales, out, ost, image,
                         work, nullptr, stream);
}

bool packed_fits(const reef_attention_params &p) {
    const int64_t tiles = ceil_div(p.kv_len, kPK);
    const int64_t items = (ceil_div(p.q_len, kBM) + 1) / 2 * p.batch * p.q_heads;
    return tiles <= 65535 && p.batch * p.kv_heads <= 65535 && items < (int64_t(1) << 31);
}

}  // namespace reef

// Test hook of the packed schedule (head_dim 128): the packed kernel runs one
// attention over (q, k, v = k) with every row seeing every key (query_start =
// kv_len - 1), unit q and k scales and a softmax scale small enough for its one-FMA
// probabilities, and stores the score accumulators of every (query, key) pair as it
// reads them, relative to its running maximum, back into plain int32 sums.
extern "C" size_t reef_qk_scores_i32_packed_workspace_bytes(int64_t batch, int64_t q_heads,
                                                            int64_t kv_heads, int64_t q_len,
                                                            int64_t kv_len) {
    if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || q_len <= 0 || kv_len <= 0) return 0;
    return (size_t)reef::tap_layout(batch, q_heads, kv_heads, q_len, kv_len).total;
}

extern "C" reef_status reef_qk_scores_i32_packed(const int8_t *q, const int8_t *k, int64_t batch,
                                                 int64_t q_heads, int64_t kv_heads, int64_t q_len,
                                                 int64_t kv_len, int32_t *acc, void *workspace,
                                                 size_t workspace_bytes, hipStream_t stream) {
    using namespace reef;
    if (!q || !k || !acc || !workspace || batch <= 0 || q_heads <= 0 || kv_heads <= 0 ||
        q_len <= 0 || kv_len <= 0 || q_heads % kv_heads != 0 || !aligned(q, 16) ||
        !aligned(k, 16) || !aligned(workspace, 256))
        return REEF_INVALID_ARGUMENT;
    if (q_len >= (int64_t(1) << 30) || kv_len >= (int64_t(1) << 30)) return REEF_UNSUPPORTED;
    const TapLayout t = tap_layout(batch, q_heads, kv_heads, q_len, kv_len);
    if ((int64_t)workspace_bytes < t.total) return REEF_INVALID_ARGUMENT;
    char *ws = static_cast<char *>(workspace);
    float *scales = reinterpret_cast<float *>(ws + t.scales);
    hipLaunchKernelGGL(tap_scales_kernel, dim3(1), dim3(1), 0, stream, scales);
    if (hipGetLastError() != hipSuccess) return REEF_HIP_ERROR;
    reef_attention_params p{};
    p.batch = batch;
    p.q_heads = q_heads;
    p.kv_heads = kv_heads;
    p.q_len = q_len;
    p.kv_len = kv_len;
    p.head_dim = kPD;
    p.query_start = kv_len - 1;
    p.window = 0;
    p.softmax_scale = 1e-3f;
    p.q_granularity = REEF_SCALE_PER_TENSOR;
    p.kv_granularity = REEF_SCALE_PER_TENSOR;
    p.flags = 0;
    const int64_t qst[3] = {q_heads * q_len * kPD, q_len * kPD, kPD};
    const int64_t kst[3] = {kv_heads * kv_len * kPD, kv_len * kPD, kPD};
    const int64_t ost[3] = {q_heads * q_len * kPD, q_len * kPD, kPD};
    return packed_launch(&p, q, qst, k, kst, k, kst, scales, scales, scales + 1,
                         reinterpret_cast<float *>(ws + t.out), ost, ws + t.image,
                         PackedWork{false, reinterpret_cast<uint32_t *>(ws), nullptr, nullptr}, acc,
                         stream);
}
