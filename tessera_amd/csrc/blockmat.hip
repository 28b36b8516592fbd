// Block-form weights on the matrix unit: the product of many rows (m > 4) against
// any of the seven block forms.
//
// Replaces the reference's tiled and lanes rules reading a block form through its
// load (engine/rules/linear/src/tiled.rs:297-316, every form of
// engine/plan/codegen/src/form.rs:10-93 and block.rs:251-291), checked as
// tiled_test.rs:58-121 does: against the CPU product over the form's decoded weights,
// within an error bound derived from the unit's summation.
//
// gfx950 design:
//  * 64 x 64 output tiles (weight rows; 32 output columns of gate/up pairs), 256
//    threads as 2 x 2 waves of 32 x 32, k in steps of 128 (256 for 128-code blocks)
//    so each row's step is a whole number of blocks and 4-byte words.
//  * A step's packed bytes stream in with coalesced 4-byte loads into an LDS staging
//    area; each thread then decodes whole blocks: codes to bf16 (every I8, nibble,
//    e4m3 and e2m1 code is exact in bf16) into the B tile, the block's scale to an LDS
//    table. nvfp4 folds its e4m3 scale into the codes instead (e2m1 times e4m3 has at
//    most 6 significant bits: still exact in bf16).
//  * v_mfma_f32_16x16x32_bf16 sums one 32-code stretch of a block per instruction from
//    zero; at the block's end the lane multiplies the block sum by the scale of its
//    four weight rows and adds it to the accumulator, as Block::dot scales each block's
//    part (block.rs:202-217). f32 rows enter as two exact bf16 parts.
//  * The next step's loads are issued before the current step's matrix work.
#include "blockform.h"

namespace ts {

namespace {

constexpr int kTM = 64, kTN = 64, kThreads = 256;

struct MatParams {
    const void *x;
    const uint8_t *w;  // the packed tensor (head included)
    const float *a0;
    void *out;
    uint32_t m, n, k;
    uint32_t stages;
    int out_bf16;
    ts_after after;  // stage chain (count 0: none)
};

template <int F>
struct Step {
    using BF = BlockForm<F>;
    static constexpr int KC = BF::B == 128 ? 256 : 128;       // k per step
    static constexpr int NBLK = KC / BF::B;                   // blocks per row per step
    static constexpr int WPR = NBLK * BF::BB / 4;             // words per row per step
    static constexpr int RAW = (kTN * WPR + kThreads - 1) / kThreads;  // raw words per thread
    static constexpr int CPR = KC / 8;                        // 16-byte chunks per tile row
    static constexpr int XCH = kTM * CPR / kThreads;          // x chunks (8 elements) per thread
    static constexpr int UNITS = kTN * NBLK;                  // blocks to decode per step
    static constexpr int TILE = kTM * KC * 2;                 // bytes of one bf16 tile
    static_assert(NBLK * BF::BB % 4 == 0, "a step is whole words");
};

// Byte offset of 16-byte chunk c of row r in a tile of CPR chunks a row: chunk c ^ (r &
// 15), so the 16 rows of a fragment read (one chunk each) land on distinct banks.
template <int CPR>
TS_DEV uint32_t tile_at(uint32_t r, uint32_t c) {
    return r * CPR * 16 + ((c ^ (r & 15)) << 4);
}

template <int F, bool XF32, bool SILU>
__global__ __launch_bounds__(kThreads) void block_tiled_kernel(MatParams p) {
    using BF = BlockForm<F>;
    using S = Step<F>;
    constexpr int KC = S::KC, CPR = S::CPR, B = BF::B, BB = BF::BB;
    constexpr bool FOLD = F == 4;  // nvfp4: the scale rides in the decoded codes
    constexpr int CPB = B >= 32 ? B / 32 : 1;  // 32-code stretches per block
    __shared__ __attribute__((aligned(16))) char a_hi[S::TILE];
    __shared__ __attribute__((aligned(16))) char a_lo[XF32 ? S::TILE : 16];
    __shared__ __attribute__((aligned(16))) char b_tile[S::TILE];
    __shared__ __attribute__((aligned(16))) uint32_t raw[kTN * S::WPR];
    __shared__ float scales[kTN][S::NBLK];

    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1, col = lane & 15, grp = lane >> 4;
    const uint32_t N = p.n, K = p.k;
    const uint32_t n0 = blockIdx.x * (SILU ? kTN / 2 : kTN), m0 = blockIdx.y * kTM;
    const size_t row_bytes = (size_t)(K / B) * BB;
    const uint8_t *rows = p.w + BF::HEAD;

    // The tensor row behind B-tile row br (rows past the end read the last one; their
    // outputs are never stored). SILU: each wave's 32 rows are 16 gate rows, then the
    // up rows of the same columns.
    auto wrow = [&](uint32_t br) -> uint32_t {
        if (!SILU) return min(n0 + br, N - 1);
        const uint32_t half = br / 32, within = br % 32;
        const uint32_t c = min(n0 + half * 16 + within % 16, N - 1);
        return within < 16 ? c : N + c;
    };

    uint32_t rw[S::RAW];
    u32x4 xr[XF32 ? 2 * S::XCH : S::XCH];
    auto load = [&](uint32_t s) {
#pragma unroll
        for (int i = 0; i < S::RAW; i++) {
            const uint32_t f = t + i * kThreads, br = f / S::WPR, wd = f % S::WPR;
            rw[i] = br < kTN ? *((const uint32_t *)(rows + (size_t)wrow(br) * row_bytes + (size_t)s * S::WPR * 4) + wd)
                             : 0u;
        }
#pragma unroll
        for (int i = 0; i < S::XCH; i++) {
            const uint32_t f = t + i * kThreads, r = f / CPR, c = f % CPR;
            const size_t at = (size_t)min(m0 + r, p.m - 1) * K + (size_t)s * KC + c * 8;
            if (XF32) {
                xr[2 * i] = *(const u32x4 *)((const float *)p.x + at);
                xr[2 * i + 1] = *(const u32x4 *)((const float *)p.x + at + 4);
            } else {
                xr[i] = *(const u32x4 *)((const uint16_t *)p.x + at);
            }
        }
    };

    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f32x4{0, 0, 0, 0};

    const uint32_t steps = K / KC;
    load(0);
    for (uint32_t s = 0; s < steps; s++) {
        // Registers to LDS: the packed words as they lie, x as bf16 (f32: hi and lo).
#pragma unroll
        for (int i = 0; i < S::RAW; i++)
            if (t + i * kThreads < (uint32_t)(kTN * S::WPR)) raw[t + i * kThreads] = rw[i];
#pragma unroll
        for (int i = 0; i < S::XCH; i++) {
            const uint32_t f = t + i * kThreads, r = f / CPR, c = f % CPR;
            if (XF32) {
                const float v[8] = {__uint_as_float(xr[2 * i].x),     __uint_as_float(xr[2 * i].y),
                                    __uint_as_float(xr[2 * i].z),     __uint_as_float(xr[2 * i].w),
                                    __uint_as_float(xr[2 * i + 1].x), __uint_as_float(xr[2 * i + 1].y),
                                    __uint_as_float(xr[2 * i + 1].z), __uint_as_float(xr[2 * i + 1].w)};
                uint32_t h[4], l[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float h0 = bf16_round(v[2 * e]), h1 = bf16_round(v[2 * e + 1]);
                    h[e] = pack_bf16x2(h0, h1);
                    l[e] = pack_bf16x2(v[2 * e] - h0, v[2 * e + 1] - h1);
                }
                *(u32x4 *)(a_hi + tile_at<CPR>(r, c)) = u32x4{h[0], h[1], h[2], h[3]};
                *(u32x4 *)(a_lo + tile_at<CPR>(r, c)) = u32x4{l[0], l[1], l[2], l[3]};
            } else {
                *(u32x4 *)(a_hi + tile_at<CPR>(r, c)) = xr[i];
            }
        }
        __syncthreads();
        // Decode whole blocks: B-tile row u / NBLK, block u % NBLK of the step.
        for (uint32_t u = t; u < (uint32_t)S::UNITS; u += kThreads) {
            const uint32_t br = u / S::NBLK, bi = u % S::NBLK;
            const uint8_t *blk = (const uint8_t *)raw + br * S::WPR * 4 + bi * BB;
            const float sc = block_scale<F>(blk);
            if (!FOLD) scales[br][bi] = sc;
#pragma unroll
            for (int g = 0; g < B / 8; g++) {
                float cv[8];
                block_codes<F, 8>(blk + BF::SB, g, cv);
                uint32_t pk[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float c0 = cv[2 * e], c1 = cv[2 * e + 1];
                    if (FOLD) {
                        c0 *= sc;
                        c1 *= sc;
                    }
                    pk[e] = pack_bf16x2(c0, c1);
                }
                *(u32x4 *)(b_tile + tile_at<CPR>(br, (bi * B) / 8 + g)) = u32x4{pk[0], pk[1], pk[2], pk[3]};
            }
        }
        __syncthreads();
        if (s + 1 < steps) load(s + 1);
        // Matrix work: per 32-code stretch kc, fragments of A (x rows) and B (weight rows).
        f32x4 d[2][2];
#pragma unroll
        for (int kc = 0; kc < KC / 32; kc++) {
            const uint32_t chunk = kc * 4 + grp;
            bf16x8 af[2], al[2], bfr[2];
#pragma unroll
            for (int i = 0; i < 2; i++) {
                af[i] = as_bf16x8(*(const u32x4 *)(a_hi + tile_at<CPR>(wm * 32 + i * 16 + col, chunk)));
                if (XF32) al[i] = as_bf16x8(*(const u32x4 *)(a_lo + tile_at<CPR>(wm * 32 + i * 16 + col, chunk)));
                bfr[i] = as_bf16x8(*(const u32x4 *)(b_tile + tile_at<CPR>(wn * 32 + i * 16 + col, chunk)));
            }
            if (FOLD) {
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        acc[i][j] = mfma16(bfr[j], af[i], acc[i][j]);
                        if (XF32) acc[i][j] = mfma16(bfr[j], al[i], acc[i][j]);
                    }
                continue;
            }
            if (kc % CPB == 0) {
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++) d[i][j] = f32x4{0, 0, 0, 0};
            }
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    d[i][j] = mfma16(bfr[j], af[i], d[i][j]);
                    if (XF32) d[i][j] = mfma16(bfr[j], al[i], d[i][j]);
                }
            if (kc % CPB == CPB - 1) {
                // The block's sum for weight rows wn 32 + 16 j + 4 grp + r, times their scales.
                const uint32_t bi = kc / CPB;
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    float sc[4];
#pragma unroll
                    for (int r = 0; r < 4; r++) sc[r] = scales[wn * 32 + j * 16 + 4 * grp + r][bi];
#pragma unroll
                    for (int i = 0; i < 2; i++)
#pragma unroll
                        for (int r = 0; r < 4; r++) acc[i][j][r] += sc[r] * d[i][j][r];
                }
            }
        }
        __syncthreads();  // the next step overwrites the tiles, the staging and the scales
    }

    // Epilogue: lane (col, grp) holds x row m0 + wm 32 + 16 i + col and weight rows
    // wn 32 + 16 j + 4 grp .. + 3 (SILU: gate j = 0, up j = 1, output columns
    // n0 + wn 16 + 4 grp .. + 3). nvfp4's head multiplies the sum (Block::dot).
    const float head = BF::HEAD ? *(const float *)p.w : 1.0f;
    constexpr int JO = SILU ? 1 : 2;
    // Value e = (i JO + j) 4 + r: row m0 + wm 32 + 16 i + col, column col_of(e).
    auto row_of = [&](int e) { return m0 + wm * 32 + (uint32_t)(e / (4 * JO)) * 16 + col; };
    auto col_of = [&](int e) {
        return n0 + (SILU ? wn * 16 : wn * 32 + (uint32_t)(e / 4 % JO) * 16) + 4 * grp + (uint32_t)(e % 4);
    };
    float val[2 * JO * 4];
#pragma unroll
    for (int e = 0; e < 2 * JO * 4; e++) {
        const int i = e / (4 * JO), j = e / 4 % JO, r = e % 4;
        if (SILU) {
            const float g = head * acc[i][0][r], u = head * acc[i][1][r];
            val[e] = g / (1.0f + expf(-g)) * u;
        } else {
            val[e] = head * acc[i][j][r];
        }
    }
    if (p.after.count)
        after_values<2 * JO * 4, false>(p.after, val, [&](int e) { return (size_t)row_of(e) * N + col_of(e); },
                                        [&](int e) { return row_of(e) < p.m && col_of(e) < N; });
#pragma unroll
    for (int e = 0; e < 2 * JO * 4; e++) {
        const uint32_t m = row_of(e), n = col_of(e);
        if (m >= p.m || n >= N) continue;
        float v = val[e];
        const size_t at = (size_t)m * N + n;
        if (p.stages & TS_AFTER_ADD) v += p.a0[at];
        if (p.out_bf16) ((uint16_t *)p.out)[at] = bf16_bits(v);
        else ((float *)p.out)[at] = v;
    }
}

using Kern = void (*)(MatParams);

template <int F>
Kern pick(bool xf, bool silu) {
    return xf ? (silu ? block_tiled_kernel<F, true, true> : block_tiled_kernel<F, true, false>)
              : (silu ? block_tiled_kernel<F, false, true> : block_tiled_kernel<F, false, false>);
}

}  // namespace

int block_tiled_launch(const ts_linear_args *a, void *stream) {
    const int bad = block_check(a, "tiled");
    if (bad) return bad;
    TS_REQUIRE(a->m >= 1, "tiled (block form): m=0");
    TS_REQUIRE((a->stages & ~(TS_AFTER_ADD | TS_AFTER_SILU_MUL)) == 0,
               "tiled (block form): stages %#x (TS_AFTER_ADD, TS_AFTER_SILU_MUL)", a->stages);
    const bool silu = a->stages & TS_AFTER_SILU_MUL, xf = a->x_dtype == TS_F32;
    const uint32_t kc = block_shape(a->w_dtype).block == 128 ? 256 : 128;
    TS_REQUIRE(a->k % kc == 0, "tiled (block form): k=%u must be a multiple of %u", a->k, kc);
    const uint32_t gy = (a->m + kTM - 1) / kTM;
    TS_REQUIRE(gy <= 65535, "tiled (block form): m=%u too large for one launch", a->m);
    MatParams p;
    p.x = a->x; p.w = (const uint8_t *)a->w; p.a0 = a->a0; p.out = a->out;
    p.m = a->m; p.n = a->n; p.k = a->k; p.stages = a->stages; p.out_bf16 = a->out_dtype == TS_BF16;
    const int rc = linear_after(a, "tiled (block form)", &p.after);
    if (rc) return rc;
    Kern k;
    switch (a->w_dtype) {
    case TS_Q8_0: k = pick<0>(xf, silu); break;
    case TS_MXFP8: k = pick<1>(xf, silu); break;
    case TS_INT4_G32: k = pick<2>(xf, silu); break;
    case TS_Q4_0: k = pick<3>(xf, silu); break;
    case TS_NVFP4: k = pick<4>(xf, silu); break;
    case TS_MXFP4: k = pick<5>(xf, silu); break;
    default: k = pick<6>(xf, silu); break;
    }
    const uint32_t cols = silu ? kTN / 2 : kTN;
    hipLaunchKernelGGL(k, dim3((a->n + cols - 1) / cols, gy), dim3(kThreads), 0, (hipStream_t)stream, p);
    TS_CHECK_LAUNCH("tiled (block form) launch");
    return TS_OK;
}

}  // namespace ts
