// Shared device and host helpers for the reef_hip kernels (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "reef_hip/attention.h"

namespace reef {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;
constexpr float kLog2e = 1.44269504088896341f;
// P.V precision of the packed prefill: where a head's dequantized values reach above
// this magnitude, P is split into fp16 hi + lo parts (22 bits). Below it one fp16 P,
// each off by at most 2^-11 of itself, moves an output by at most
// 2^-11 max|v_j - out| <= 2^-11 * 2 = 9.8e-4, inside the 1e-3 attention tolerance for
// every input (REEF_ATTN_PRECISE_PV splits every head whatever the values; the other
// prefill kernels and decode always split).
constexpr float kHiOnlyMax = 1.0f;

// --- matrix instructions ---------------------------------------------------------------
// Output layout of the 32x32 instructions: lane l holds column l % 32 and, in
// register 4j + i, row 8j + 4(l / 32) + i. Of the 16x16 instructions: lane l
// holds column l % 16 and, in register i, row 4(l / 16) + i. In both operands,
// lane group l / 32 (l / 16) supplies the same slice of the reduction index, so
// any consistent assignment of reduction indices to (group, element) is valid.

__device__ __forceinline__ i32x16 mfma_32x32x32_i8(i32x4 a, i32x4 b, i32x16 c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ i32x4 mfma_16x16x64_i8(i32x4 a, i32x4 b, i32x4 c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma_32x32x16_f16(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_16x16x32_f16(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// --- small device helpers -----------------------------------------------------------------

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint32_t w = (uint32_t)__shfl_xor((int)v, o);
        v = v > w ? v : w;
    }
    return v;
}

// max / sum of x over lanes l and l ^ 32, in one VALU op (v_permlane32_swap).
__device__ __forceinline__ float xor32_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                   false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                   false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// A raw buffer resource over [base, base + bytes): loads through it take a
// per-lane VGPR offset and a uniform SGPR offset, and read zeros past the end.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                             0x00020000);
}

// Scale of quant.hpp:51-57 from a largest magnitude: max / 127 (IEEE
// division), or 1 when every value was zero.
__device__ __forceinline__ float int8_scale(float max_magnitude) {
    return max_magnitude > 0.0f ? max_magnitude / 127.0f : 1.0f;
}

// quantize_int8 of quant.hpp:68-81 for a finite value: nearbyint(x / scale),
// ties to even (v_rndne_f32), clamped to +-127.
__device__ __forceinline__ int8_t quantize_int8(float x, float scale) {
    float r = __builtin_rintf(x / scale);
    r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
    return (int8_t)(int)r;
}

__device__ __forceinline__ void flag_status(uint32_t *word, uint32_t bits) {
    if (word) atomicOr(word, bits);
}

// --- cross-workgroup parts (decode and prefill merges) -----------------------------------
//
// A result cut across workgroups is merged by the part that counts in last:
//   publish: every thread stores its part with part_store, then part_stores_done();
//   a barrier; one thread counts the part in with part_count (the old count);
//   claim: the part whose count was parts - 1 reads every part with part_load (after
//   its count returned) and resets the counter with part_reset.
// The ordering rests on the gfx950 memory model as LLVM implements it (AMDGPUUsage,
// "Memory Model GFX942", which gfx950 follows), not on release/acquire: monotonic
// atomic loads, stores and read-modify-writes at agent scope compile to global or flat
// accesses with sc1 set, which bypass the per-XCD L2 and are coherent at the memory
// side; s_waitcnt vmcnt(0) returns only when every earlier store has completed there;
// the signal fences keep the compiler from moving memory accesses across that wait.
// A release/acquire pair would order the same accesses under the language model,
// but compiles to an L2 write-back (buffer_wbl2) and invalidate (buffer_inv) of the
// whole XCD on every cut item, which the other workgroups then pay in misses.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "the cross-workgroup part protocol is written for gfx950"
#endif

__device__ __forceinline__ void part_store(uint64_t *p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t part_load(const uint64_t *p) {
    return __hip_atomic_load(const_cast<uint64_t *>(p), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
// Every part_store of this thread has completed before any later access is issued.
__device__ __forceinline__ void part_stores_done() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// Counts a part in; the previous count (parts - 1: this part merges). The caller
// places part_claimed() after reading the result, before its first part_load.
__device__ __forceinline__ uint32_t part_count(uint32_t *counter) {
    return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void part_claimed() { __atomic_signal_fence(__ATOMIC_SEQ_CST); }
// Leaves the counter at zero for the next launch (after the last count of this item).
__device__ __forceinline__ void part_reset(uint32_t *counter) {
    __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// --- host helpers -----------------------------------------------------------------------

inline bool aligned(const void *p, size_t bytes) {
    return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}

// Compute units of the current device (256 on MI355X; also the answer without one).
inline int64_t compute_units() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
        return 256;
    return n;
}

inline reef_status launch_status() {
    return hipGetLastError() == hipSuccess ? REEF_OK : REEF_HIP_ERROR;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace reef
