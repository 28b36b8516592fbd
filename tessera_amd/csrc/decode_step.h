// The persistent decode step (decode_step.hip): every layer of a Qwen3-shaped
// decoder, the tied lm_head and the greedy pick for `steps` tokens in one launch.
#pragma once

#include <stdint.h>

namespace ts {

constexpr uint32_t kStepMaxLayers = 32;
constexpr uint32_t kStepMaxGroups = 448;  // groups the step supports (one per CU)

struct DecodeStepArgs {
    // Per-layer gains (f32) and kept rows; the product weights come packed (below).
    const float *ln1[kStepMaxLayers], *ln2[kStepMaxLayers], *q_norm[kStepMaxLayers], *k_norm[kStepMaxLayers];
    uint16_t *k_cache[kStepMaxLayers], *v_cache[kStepMaxLayers];
    const uint16_t *embed;  // [V, H]: the token's embedding row
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
    // Groups of each role (qkv, o, gate/up, down, attention), set by decode_step_launch.
    uint32_t role_first[5], role_count[5];
    // The weights as decode_step_pack laid them out: per layer and product role
    // (qkv, o, gate/up, down), and the lm_head rows.
    const uint16_t *packed[kStepMaxLayers][4];
    const uint16_t *lm_packed;
};

// Elements (bf16) of the packed copy of product role r (0 qkv, 1 o, 2 gate/up, 3 down;
// 4: the lm_head) for one layer, for NG groups.
size_t decode_step_packed_elems(uint32_t H, uint32_t Hq, uint32_t Hkv, uint32_t F, uint32_t V, uint32_t NG,
                                uint32_t role);
// Lays W (row-major [N, K] bf16: the role's matrix, or the embedding table for the
// lm_head) out for the persistent step: each group's rows as 16-row tiles, each tile
// as 32-deep k-steps of 64 lanes x 16 bytes in the matrix unit's A-operand order
// (rows past a group's share are zeros), so that every load instruction of the step
// reads 1 KB contiguous.
int decode_step_pack(const uint16_t *W, uint16_t *dst, uint32_t H, uint32_t Hq, uint32_t Hkv, uint32_t F, uint32_t V,
                     uint32_t NG, uint32_t role, void *stream);

// Hand-off words the step needs (uint64 each) for NG groups.
size_t decode_step_hand_words(uint32_t H, uint32_t L, uint32_t Hq, uint32_t Hkv, uint32_t F, uint32_t NG);

// TS_OK, or 1 when the shape is outside what the kernel supports (the caller then
// uses the graph of kernels), or an error.
int decode_step_supported(uint32_t H, uint32_t L, uint32_t Hq, uint32_t Hkv, uint32_t D, uint32_t F, uint32_t V,
                          uint32_t kept_pages);
int decode_step_groups(uint32_t *groups);
int decode_step_launch(const DecodeStepArgs *a, void *stream);

}  // namespace ts
