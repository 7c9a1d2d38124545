// The packed prefill schedule (prefill_packed.hip), as the prefill entry point
// (prefill.hip) calls it.
#pragma once

#include "reef_common.hpp"

namespace reef {

// Where the packed schedule's work comes from: per-XCD queues of whole query tiles
// (large grids), or equal runs of (query tile, key tile) steps with cut tiles merged
// through the balanced schedule's counters and part slots (small grids).
struct PackedWork {
    bool balanced;
    uint32_t *queue;     // 9 zero-filled words (queue mode)
    uint32_t *counters;  // one zero-filled counter per query tile (balanced)
    float *slots;        // two part slots of kPartSlotFloats floats per workgroup (balanced)
};
// One part slot of the balanced schedules: a 128-row query tile's accumulators at
// head_dim 128 and two words per row (both schedules' layouts fit it exactly).
constexpr int kPartSlotFloats = 16896;

// Workspace bytes of the V image.
int64_t packed_image_bytes(int64_t batch, int64_t kv_heads, int64_t kv_len);

// The packed schedule's limits: its grids address (batch x kv head, key tile) in
// 16-bit launch dimensions.
bool packed_fits(const reef_attention_params &p);

reef_status prefill_packed_launch(const reef_attention_params *p, const int8_t *q,
                                  const int64_t (&qst)[3], const int8_t *k,
                                  const int64_t (&kst)[3], const int8_t *v,
                                  const int64_t (&vst)[3], const float *q_scales,
                                  const float *k_scales, const float *v_scales, float *out,
                                  const int64_t (&ost)[3], void *image, const PackedWork &work,
                                  hipStream_t stream);

}  // namespace reef
