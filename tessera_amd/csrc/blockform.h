// The seven block forms of the reference (engine/ir/mem/src/block.rs:251-291) as
// compile-time descriptions, and their exact decode on the device.
//
// A packed tensor is an optional 4-byte f32 head, then blocks in element order; each
// block is one narrow scale followed by B codes (block.rs:118-131). A [n, k] weight
// matrix is one tensor, so row r's blocks start at head + r (k / B) block bytes.
#pragma once

#include "after.h"

namespace ts {

enum { kScaleF16, kScaleE8M0, kScaleE4M3 };
enum { kCodeI8, kCodeE4M3, kCodeNibble, kCodeE2M1 };

// F: the form's index from TS_Q8_0 (0 q8_0, 1 mxfp8, 2 int4_g32, 3 q4_0, 4 nvfp4,
// 5 mxfp4, 6 int4_g128).
template <int F>
struct BlockForm {
    static constexpr int SCALE = (F == 1 || F == 5) ? kScaleE8M0 : F == 4 ? kScaleE4M3 : kScaleF16;
    static constexpr int CODE = F == 0 ? kCodeI8 : F == 1 ? kCodeE4M3 : (F == 4 || F == 5) ? kCodeE2M1 : kCodeNibble;
    static constexpr int B = F == 4 ? 16 : F == 6 ? 128 : 32;  // codes a block
    static constexpr bool HALVES = F == 3;                      // q4_0 pairs element j with j + B/2
    static constexpr int HEAD = F == 4 ? 4 : 0;                 // nvfp4's f32 tensor scale
    static constexpr int SB = SCALE == kScaleF16 ? 2 : 1;       // scale bytes
    static constexpr int BITS = CODE == kCodeI8 || CODE == kCodeE4M3 ? 8 : 4;
    static constexpr int BB = SB + B * BITS / 8;                // block bytes
};

// f16 scale, little-endian (exact widening, subnormals included).
TS_DEV float f16_value(uint32_t lo, uint32_t hi) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(lo | (hi << 8)));
}

// e8m0 scale: 2^(e - 127); 0xFF is NaN (engine/ir/graph/src/scalar.rs:154-161).
TS_DEV float e8m0_value(uint32_t e) {
    if (e == 0xFF) return __uint_as_float(0x7fc00000u);
    return e == 0 ? __uint_as_float(0x00400000u) : __uint_as_float(e << 23);
}

// e2m1 code (sign bit 3): 0, 0.5, 1, 1.5, 2, 3, 4, 6 by magnitude (scalar.rs:132-135).
// Magnitudes from 1 up are 2^(e - 1) (1 + m / 2) for the two exponent bits e and the
// mantissa bit m: an f32 with exponent 126 + e and mantissa bit 22 set to m.
TS_DEV float e2m1_value(uint32_t c) {
    const uint32_t m = c & 7u;
    const float v = m < 2 ? 0.5f * (float)m : __uint_as_float(((126u + (m >> 1)) << 23) | ((m & 1u) << 22));
    return (c & 8u) ? -v : v;
}

// The block's scale, widened exactly.
template <int F>
TS_DEV float block_scale(const uint8_t *blk) {
    using BF = BlockForm<F>;
    if (BF::SCALE == kScaleE8M0) return e8m0_value(blk[0]);
    if (BF::SCALE == kScaleE4M3) return e4m3_float(blk[0]);
    return f16_value(blk[0], blk[1]);
}

// Code j of the block (before its scale), exactly: place (block.rs:131-137) then
// decode (I8, E4M3, Nibble = code - 8, E2M1).
template <int F>
TS_DEV float block_code(const uint8_t *codes, int j) {
    using BF = BlockForm<F>;
    if (BF::BITS == 8) {
        const uint32_t c = codes[j];
        return BF::CODE == kCodeI8 ? (float)(int8_t)c : e4m3_float(c);
    }
    const uint32_t byte = BF::HALVES ? codes[j % (BF::B / 2)] : codes[j / 2];
    const uint32_t c = (BF::HALVES ? j / (BF::B / 2) : j % 2) ? byte >> 4 : byte & 15u;
    return BF::CODE == kCodeNibble ? (float)c - 8.0f : e2m1_value(c);
}

// Codes q P .. q P + P - 1 of the block into wv (exact, before the scale). e2m1 pairs
// convert two at a time on gfx950's fp4 conversion (scale 1: exact).
template <int F, int P>
TS_DEV void block_codes(const uint8_t *codes, int q, float *wv) {
    using BF = BlockForm<F>;
    if (BF::CODE == kCodeE2M1 && !BF::HALVES) {
        typedef float f32x2_t __attribute__((ext_vector_type(2)));
#pragma unroll
        for (int b = 0; b < P / 2; b++) {
            const f32x2_t v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4((uint32_t)codes[(q * P) / 2 + b], 1.0f, 0);
            wv[2 * b] = v.x;
            wv[2 * b + 1] = v.y;
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < P; j++) wv[j] = block_code<F>(codes, q * P + j);
}

}  // namespace ts
