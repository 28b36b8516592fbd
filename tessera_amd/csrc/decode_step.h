// The persistent decode step (decode_step.hip): every layer of a Qwen3-shaped
// decoder, the tied lm_head and the greedy pick for `steps` tokens in one launch.
#pragma once

#include <stdint.h>

namespace ts {

constexpr uint32_t kStepMaxLayers = 32;

struct DecodeStepArgs {
    // Per-layer weights (row-major [N, K] bf16; gains f32) and kept rows.
    const uint16_t *qkv[kStepMaxLayers], *o[kStepMaxLayers], *gate_up[kStepMaxLayers], *down[kStepMaxLayers];
    const float *ln1[kStepMaxLayers], *ln2[kStepMaxLayers], *q_norm[kStepMaxLayers], *k_norm[kStepMaxLayers];
    uint16_t *k_cache[kStepMaxLayers], *v_cache[kStepMaxLayers];
    const uint16_t *embed;  // [V, H]; also the lm_head
    const float *norm;      // [H]
    const float *rope;      // [positions][64] (cos, sin)
    const uint32_t *table;  // the slot's page table, [kept_pages]
    uint32_t *tok, *pos, *hist;
    float *logits;          // [V], the last step's
    uint64_t *hand;         // tagged hand-off words (value, epoch), zeroed at open
    uint32_t *error;        // nonzero after a timed-out wait
    uint64_t *marks;        // optional: [groups][layers + 1][10] clock stamps of the first step
    uint32_t H, L, Hq, Hkv, F, V, NG, kept_pages, page_shift, steps, epoch;
    float eps, scale;
};

// Hand-off words the step needs (uint64 each) for NG groups.
size_t decode_step_hand_words(uint32_t H, uint32_t L, uint32_t Hq, uint32_t Hkv, uint32_t F, uint32_t NG);

// TS_OK, or 1 when the shape is outside what the kernel supports (the caller then
// uses the graph of kernels), or an error.
int decode_step_supported(uint32_t H, uint32_t L, uint32_t Hq, uint32_t Hkv, uint32_t D, uint32_t F,
                          uint32_t kept_pages);
int decode_step_groups(uint32_t *groups);
int decode_step_launch(const DecodeStepArgs *a, void *stream);

}  // namespace ts
