// Block-scaled weight forms on the decode product (m <= 4 rows): q8_0, mxfp8,
// int4_g32 and q4_0, each 32 codes under one narrow scale.
//
// Replaces the decode of a block form inside the few-row product: the reference's
// Block::dot (engine/ir/mem/src/block.rs:202-219) with the forms Q8_0 (f16 scale,
// signed bytes), MXFP8 (e8m0 scale, e4m3 codes) and INT4_G32 (f16 scale, nibbles
// 8 below their value, adjacent pairs per byte) and Q4_0 (the same nibbles paired
// by halves: element j in byte j % 16, high nibble for j >= 16), block.rs:258-286, as the lanes
// rule reads them through a form's load (engine/plan/codegen/src/form.rs:10-93).
//
// gfx950 design. One wave per 4 weight rows. A row is K/32 blocks of 33, 34 or 18
// bytes, so blocks are not 16-byte aligned: the wave streams its rows' bytes with
// coalesced 4-byte loads (all four rows in flight together) into its own LDS
// slices, 64 blocks at a time, and lane l then decodes block l of each row. Each lane forms its block's part in the
// reference's order (x_j times the decoded code, summed from 0.0 in j order, no
// contraction), times the block scale; lane (row, m) then adds the contributions of
// activation row m in block order. Every rounding step is the reference's, so the
// product is bit-identical to Block::dot for the same f32 activations.
#include "common.h"

namespace ts {

namespace {

constexpr int kWaves = 4;
constexpr int kChunk = 64;  // blocks per LDS slice: one per lane
constexpr int kRows = 4;    // weight rows per wave, their loads overlapped

struct BlockParams {
    const void *x;
    const uint8_t *w;
    const float *a0;
    void *out;
    uint32_t m, n, k;
    uint32_t stages;
    int out_bf16;
};

// FORM: 0 q8_0, 1 mxfp8, 2 int4_g32, 3 q4_0.
template <int FORM>
struct Form {
    static constexpr int kScaleBytes = FORM == 1 ? 1 : 2;
    static constexpr int kBytes = kScaleBytes + (FORM >= 2 ? 16 : 32);
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

// Waits for this wave's LDS traffic so the other lanes' writes are visible.
TS_DEV void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt not waited on
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

template <int FORM, int M, bool XF32>
__global__ __launch_bounds__(kWaves * 64) void block_gemv_kernel(BlockParams p) {
#pragma clang fp contract(off)
    constexpr int SB = Form<FORM>::kScaleBytes, BB = Form<FORM>::kBytes;
    constexpr int kSlice = kChunk * BB / 4;                 // words of one row's slice
    constexpr int kWords = (kSlice + 63) / 64;              // of them per lane (at most 9)
    __shared__ __attribute__((aligned(16))) uint32_t stage[kWaves][kRows][kSlice];
    __shared__ __attribute__((aligned(16))) float contrib[kWaves][kRows * M][kChunk];

    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t r0 = (blockIdx.x * kWaves + wave) * kRows;  // this wave's kRows rows
    if (r0 >= p.n) return;  // waves are independent: no group barrier below
    const uint32_t K = p.k, N = p.n, Mr = p.m, nb = K / 32;
    const uint32_t nrows = min((uint32_t)kRows, N - r0);

    float run = 0.0f;  // lane rr * M + m: the running sum of output (m, r0 + rr)
    for (uint32_t c0 = 0; c0 < nb; c0 += kChunk) {
        const uint32_t cnt = min((uint32_t)kChunk, nb - c0), words = cnt * BB / 4;
        // Every word of the rows' slices in flight before any is written.
        uint32_t wt[kRows][kWords];
#pragma unroll
        for (int rr = 0; rr < kRows; rr++) {
            const uint32_t *src = (const uint32_t *)(p.w + (size_t)(r0 + min((uint32_t)rr, nrows - 1)) * nb * BB) +
                                  (size_t)c0 * BB / 4;
#pragma unroll
            for (int q = 0; q < kWords; q++) {
                const uint32_t i = lane + 64 * q;
                wt[rr][q] = i < words ? __builtin_nontemporal_load(src + i) : 0u;
            }
        }
#pragma unroll
        for (int rr = 0; rr < kRows; rr++)
#pragma unroll
            for (int q = 0; q < kWords; q++)
                if (lane + 64 * q < words) stage[wave][rr][lane + 64 * q] = wt[rr][q];
        wave_lds_sync();
        if (lane < cnt) {
            const uint32_t k0 = (c0 + lane) * 32;
#pragma unroll
            for (int m = 0; m < M; m++) {
                if ((uint32_t)m >= Mr) break;
                float xv[32];
                if (XF32) {
                    const float4 *xs = (const float4 *)((const float *)p.x + (size_t)m * K + k0);
#pragma unroll
                    for (int q = 0; q < 8; q++) {
                        const float4 t = xs[q];
                        xv[4 * q] = t.x; xv[4 * q + 1] = t.y; xv[4 * q + 2] = t.z; xv[4 * q + 3] = t.w;
                    }
                } else {
                    const u32x4 *xs = (const u32x4 *)((const uint16_t *)p.x + (size_t)m * K + k0);
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const u32x4 t = xs[q];
                        const uint32_t u[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            xv[8 * q + 2 * e] = lo_bf16(u[e]);
                            xv[8 * q + 2 * e + 1] = hi_bf16(u[e]);
                        }
                    }
                }
#pragma unroll
                for (int rr = 0; rr < kRows; rr++) {
                    const uint8_t *blk = (const uint8_t *)stage[wave][rr] + lane * BB;
                    const float scale = FORM == 1 ? e8m0_value(blk[0]) : f16_value(blk[0], blk[1]);
                    float wv[32];
                    if (FORM == 0) {
#pragma unroll
                        for (int j = 0; j < 32; j++) wv[j] = (float)(int8_t)blk[SB + j];
                    } else if (FORM == 1) {
#pragma unroll
                        for (int q = 0; q < 8; q++) {
                            const uint32_t c = blk[SB + 4 * q] | (blk[SB + 4 * q + 1] << 8) |
                                               (blk[SB + 4 * q + 2] << 16) | ((uint32_t)blk[SB + 4 * q + 3] << 24);
                            e4m3x4_to_f32(c, wv + 4 * q);
                        }
                    } else if (FORM == 2) {  // adjacent pairs: element 2q low, 2q + 1 high
#pragma unroll
                        for (int q = 0; q < 16; q++) {
                            const uint32_t b = blk[SB + q];
                            wv[2 * q] = (float)(b & 15u) - 8.0f;
                            wv[2 * q + 1] = (float)(b >> 4) - 8.0f;
                        }
                    } else {  // halves: element q low, q + 16 high
#pragma unroll
                        for (int q = 0; q < 16; q++) {
                            const uint32_t b = blk[SB + q];
                            wv[q] = (float)(b & 15u) - 8.0f;
                            wv[q + 16] = (float)(b >> 4) - 8.0f;
                        }
                    }
                    float part = 0.0f;
#pragma unroll
                    for (int j = 0; j < 32; j++) part = part + xv[j] * wv[j];
                    contrib[wave][rr * M + m][lane] = scale * part;
                }
            }
        }
        wave_lds_sync();
        if (lane < kRows * M) {  // all 64 contributions read first, then added in block order
            const float4 *cv = (const float4 *)contrib[wave][lane];
            float4 t[kChunk / 4];
#pragma unroll
            for (int q = 0; q < kChunk / 4; q++) t[q] = cv[q];
#pragma unroll
            for (int q = 0; q < kChunk / 4; q++)
                if ((uint32_t)(4 * q) < cnt) {  // cnt is a multiple of 4
                    run = run + t[q].x;
                    run = run + t[q].y;
                    run = run + t[q].z;
                    run = run + t[q].w;
                }
        }
        wave_lds_sync();  // the next slice overwrites stage and contrib
    }
    const uint32_t rr = lane / M, m = lane % M;
    if (lane >= kRows * M || rr >= nrows || m >= Mr) return;
    float v = 1.0f * run;  // Block::dot's head: 1.0 for these forms
    const size_t at = (size_t)m * N + r0 + rr;
    if (p.stages & TS_AFTER_ADD) v += p.a0[at];
    if (p.out_bf16) ((uint16_t *)p.out)[at] = bf16_bits(v);
    else ((float *)p.out)[at] = v;
}

using Kern = void (*)(BlockParams);

template <int FORM, bool XF32>
Kern pick_m(uint32_t m) {
    return m == 1 ? block_gemv_kernel<FORM, 1, XF32>
         : m == 2 ? block_gemv_kernel<FORM, 2, XF32> : block_gemv_kernel<FORM, 4, XF32>;
}

template <int FORM>
Kern pick_x(uint32_t m, bool xf) {
    return xf ? pick_m<FORM, true>(m) : pick_m<FORM, false>(m);
}

}  // namespace

bool block_form(int32_t dtype) {
    return dtype == TS_Q8_0 || dtype == TS_MXFP8 || dtype == TS_INT4_G32 || dtype == TS_Q4_0;
}

size_t block_row_bytes(int32_t dtype, uint32_t k) {
    const size_t bb = dtype == TS_Q8_0 ? Form<0>::kBytes : dtype == TS_MXFP8 ? Form<1>::kBytes : Form<2>::kBytes;  // q4_0: 18 as int4_g32
    return (size_t)(k / 32) * bb;
}

int block_gemv_launch(const ts_linear_args *a, void *stream) {
    TS_REQUIRE(a && a->x && a->w && a->out, "lanes (block form): null pointer");
    TS_REQUIRE(a->m >= 1 && a->m <= 4, "lanes (block form): m=%u outside 1..4 (block forms decode rows only)",
               a->m);
    TS_REQUIRE(a->n >= 1 && a->k >= 128 && a->k % 128 == 0, "lanes (block form): k=%u must be a multiple of 128",
               a->k);
    TS_REQUIRE(a->x_dtype == TS_F32 || a->x_dtype == TS_BF16, "lanes (block form): x dtype %d", a->x_dtype);
    TS_REQUIRE(a->out_dtype == TS_F32 || a->out_dtype == TS_BF16, "lanes (block form): out dtype %d", a->out_dtype);
    TS_REQUIRE((a->stages & ~TS_AFTER_ADD) == 0, "lanes (block form): stages %#x (only TS_AFTER_ADD)", a->stages);
    TS_REQUIRE(!(a->stages & TS_AFTER_ADD) || a->a0, "lanes (block form): TS_AFTER_ADD needs a0");
    TS_REQUIRE(aligned(a->x, 16) && aligned(a->w, 4), "lanes (block form): x 16-byte and w 4-byte aligned");
    BlockParams p;
    p.x = a->x; p.w = (const uint8_t *)a->w; p.a0 = a->a0; p.out = a->out;
    p.m = a->m; p.n = a->n; p.k = a->k; p.stages = a->stages; p.out_bf16 = a->out_dtype == TS_BF16;
    const bool xf = a->x_dtype == TS_F32;
    Kern k = a->w_dtype == TS_Q8_0    ? pick_x<0>(a->m, xf)
           : a->w_dtype == TS_MXFP8   ? pick_x<1>(a->m, xf)
           : a->w_dtype == TS_INT4_G32 ? pick_x<2>(a->m, xf) : pick_x<3>(a->m, xf);
    hipLaunchKernelGGL(k, dim3((a->n + kWaves * kRows - 1) / (kWaves * kRows)), dim3(kWaves * 64), 0, (hipStream_t)stream, p);
    TS_CHECK_LAUNCH("lanes (block form) launch");
    return TS_OK;
}

}  // namespace ts
