// "tiled" for large products with bf16 rows and weights: 256x256 output tiles.
//
// Same product as tiled.hip (the reference's tiled rule, engine/rules/linear/
// src/tiled.rs:281-345), used when both operands are bf16 and there are enough
// 256x256 tiles to cover the chip.
//
// gfx950 design:
//  * 512 threads = 8 waves in a 2 x 4 grid, each wave 128 x 64 = 8 x 4 tiles of
//    v_mfma_f32_16x16x32_bf16 (32 accumulators): per 32-deep k step a wave reads
//    12 operand fragments from LDS for 32 MFMAs, half the LDS traffic per MFMA of
//    a 64 x 64 wave tile.
//  * k advances 64 at a time through two LDS stages of 64 KiB each (A 256 x 64 and
//    B 256 x 64 bf16, 128-byte rows with 16-byte chunks XOR-swizzled by row). The
//    stages fill with global_load_lds_dwordx4, straight from HBM to LDS (no staging
//    registers), and the next stage's loads overlap the current stage's MFMAs.
//  * Scheduling groups pin the order: one substep's fragment reads, then its MFMAs
//    interleaved with the other substep's reads and the next stage's loads.
//  * 128 KiB of dynamic LDS per group (gfx950 has 160 KiB per CU): one group per CU.
#include "common.h"

namespace ts {

namespace {

constexpr int BM = 256, BN = 256, BK = 64, kThreads = 512;
constexpr int kStage = BM * BK * 2;  // bytes of one operand stage (A or B)
constexpr int kLds = 2 * 2 * kStage;  // two stages of A and B

struct BigParams {
    const uint16_t *x;
    const uint16_t *w;
    const float *a0;
    void *out;
    uint32_t m, n, k;
    uint32_t stages;
    int out_bf16;
    uint32_t mtiles;
};

TS_DEV uint32_t swz(uint32_t row, uint32_t chunk) { return row * 128 + ((chunk ^ (row & 7)) << 4); }

typedef __attribute__((address_space(3))) void lds_void;

// One stage: A and B tiles straight from global memory into LDS with
// global_load_lds_dwordx4 (lane i of an instruction lands at M0 + 16 i). Wave w's
// instruction i fills the 1 KiB holding rows 8b..8b+7, b = 4w + i; lane l fetches
// the logical chunk that the swizzle places at physical chunk l % 8 of row l / 8.
TS_DEV void fetch_stage(const BigParams &p, char *stage, uint32_t m0, uint32_t n0, uint32_t k0, uint32_t wave,
                        uint32_t lane) {
    const uint32_t rl = lane >> 3, lc = (lane & 7) ^ rl;  // row within the 8, logical chunk
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t b = wave * 4 + i, row = 8 * b + rl;
        const uint32_t m = min(m0 + row, p.m - 1), n = min(n0 + row, p.n - 1);  // rows past the end are never stored
        const uint16_t *ga = p.x + (size_t)m * p.k + k0 + lc * 8;
        const uint16_t *gb = p.w + (size_t)n * p.k + k0 + lc * 8;
        __builtin_amdgcn_global_load_lds((const void *)ga, (lds_void *)(stage + b * 1024), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((const void *)gb, (lds_void *)(stage + kStage + b * 1024), 16, 0, 0);
    }
}

// s_waitcnt immediate for vmcnt(0) expcnt(7) lgkmcnt(0) (gfx9 packs vmcnt's high
// bits at 15:14; they stay zero).
constexpr int kWaitAll = 0x0070;

// One 64-deep step over stage s & 1: 2 x 12 fragment reads, 64 MFMAs and, when
// FETCH, the 8 loads that fill the other stage for step s + 1. The order is pinned
// with scheduling groups: the first substep's reads, then its MFMAs interleaved
// with the second substep's reads and the next stage's loads, then the second
// substep's MFMAs, so LDS and HBM latency hide under matrix work.
template <bool FETCH>
TS_DEV void mfma_step(const BigParams &p, char *lds, uint32_t s, f32x4 (&acc)[8][4], uint32_t m0, uint32_t n0,
                      uint32_t wave, uint32_t lane, uint32_t wm, uint32_t wn, uint32_t col, uint32_t grp) {
    const char *sa = lds + (s & 1) * 2 * kStage, *sb = sa + kStage;
    bf16x8 af[2][8], bfr[2][4];
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
        const uint32_t c = ks * 4 + grp;
#pragma unroll
        for (int j = 0; j < 4; j++) bfr[ks][j] = as_bf16x8(*(const u32x4 *)(sb + swz(wn * 64 + j * 16 + col, c)));
#pragma unroll
        for (int i = 0; i < 8; i++) af[ks][i] = as_bf16x8(*(const u32x4 *)(sa + swz(wm * 128 + i * 16 + col, c)));
    }
    if (FETCH) fetch_stage(p, lds + ((s + 1) & 1) * 2 * kStage, m0, n0, (s + 1) * BK, wave, lane);
#pragma unroll
    for (int ks = 0; ks < 2; ks++)
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] = mfma16(bfr[ks][j], af[ks][i], acc[i][j]);
    // Masks: 0x008 MFMA, 0x020 VMEM read, 0x100 DS read.
    __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);
#pragma unroll
    for (int i = 0; i < 12; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    if (FETCH) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 44, 0);
    } else {
        __builtin_amdgcn_sched_group_barrier(0x008, 52, 0);
    }
    __builtin_amdgcn_sched_barrier(0);  // nothing moves past here (the wait and barrier follow)
}

__global__ __launch_bounds__(kThreads, 1) void tiled_big_kernel(BigParams p) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t wm = wave >> 2, wn = wave & 3;
    const uint32_t col = lane & 15, grp = lane >> 4;
    // XCD-aware order: groups are dispatched round-robin over the 8 XCDs, so group
    // b runs on XCD b % 8. Each XCD walks its own column tiles (n tile = x mod 8) and
    // runs all row tiles of one column tile back to back: the 256 x K weight tile
    // is fetched into that XCD's L2 once and shared by every row tile.
    const uint32_t b = blockIdx.x, x = b & 7, j = b >> 3;
    const uint32_t mt = j % p.mtiles, nt = (j / p.mtiles) * 8 + x;
    if (nt * BN >= p.n) return;
    const uint32_t m0 = mt * BM, n0 = nt * BN;

    f32x4 acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f32x4{0, 0, 0, 0};

    const uint32_t steps = p.k / BK;
    fetch_stage(p, lds, m0, n0, 0, wave, lane);
    __builtin_amdgcn_s_waitcnt(kWaitAll);  // this wave's stage loads are in LDS
    __syncthreads();
    for (uint32_t s = 0; s + 1 < steps; s++) {
        // The other stage was last read before the previous barrier: refill it now.
        mfma_step<true>(p, lds, s, acc, m0, n0, wave, lane, wm, wn, col, grp);
        __builtin_amdgcn_s_waitcnt(kWaitAll);  // the next stage's loads have landed
        __syncthreads();
    }
    mfma_step<false>(p, lds, steps - 1, acc, m0, n0, wave, lane, wm, wn, col, grp);

    const uint32_t N = p.n, M = p.m;
    if (p.out_bf16 && !(p.stages & TS_AFTER_ADD)) {
        // bf16 output with no added operand: the tile goes through LDS (the stages
        // are free once every wave has read the last one) as 256 rows of 512 B,
        // 16-byte chunks XOR-swizzled by row, and leaves as whole rows: two rows of
        // 512 contiguous bytes per store instruction instead of 16 rows x 32 B.
        lds_barrier();
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t r = wm * 128 + i * 16 + col;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t c = wn * 64 + j * 16 + 4 * grp;  // first of 4 columns (8 B)
                const f32x4 v = acc[i][j];
                *(u32x2 *)(lds + r * 512 + ((((c >> 3) ^ (r & 31))) << 4) + (c & 7) * 2) =
                    u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
            }
        }
        lds_barrier();
        const bool rows16 = (N & 7) == 0;  // every row starts 16-byte aligned
#pragma unroll 4
        for (int it = 0; it < 16; it++) {
            const uint32_t f = it * kThreads + t, r = f >> 5, c = f & 31;
            const uint32_t m = m0 + r, n = n0 + c * 8;
            if (m >= M || n >= N) continue;
            const u32x4 v = *(const u32x4 *)(lds + r * 512 + ((c ^ (r & 31)) << 4));
            uint16_t *o = (uint16_t *)p.out + (size_t)m * N + n;
            if (rows16 && n + 8 <= N) {
                *(u32x4 *)o = v;
            } else {
                for (uint32_t e = 0; e < 8 && n + e < N; e++) o[e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
            }
        }
        return;
    }
    // Epilogue with f32 output or an added operand. The MFMA operands are swapped
    // (weights first), so lane l holds row col of each 16x16 tile and its four
    // adjacent columns 4 grp .. + 3: one 8-byte (bf16) or 16-byte (f32) store per
    // lane and tile instead of four 2-byte ones.
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t m = m0 + wm * 128 + i * 16 + col;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t n = n0 + wn * 64 + j * 16 + 4 * grp;
            if (n >= N) continue;
            const size_t e = (size_t)m * N + n;
            f32x4 v = acc[i][j];
            const bool whole = n + 3 < N && (e & 3) == 0;
            if (p.stages & TS_AFTER_ADD) {
                if (whole) {
                    v += *(const f32x4 *)(p.a0 + e);
                } else {
                    for (uint32_t r = 0; r < 4 && n + r < N; r++) v[r] += p.a0[e + r];
                }
            }
            if (p.out_bf16) {
                uint16_t *o = (uint16_t *)p.out + e;
                if (whole) {
                    *(u32x2 *)o = u32x2{(uint32_t)bf16_bits(v[0]) | ((uint32_t)bf16_bits(v[1]) << 16),
                                        (uint32_t)bf16_bits(v[2]) | ((uint32_t)bf16_bits(v[3]) << 16)};
                } else {
                    for (uint32_t r = 0; r < 4 && n + r < N; r++) o[r] = bf16_bits(v[r]);
                }
            } else {
                float *o = (float *)p.out + e;
                if (whole) {
                    *(f32x4 *)o = v;
                } else {
                    for (uint32_t r = 0; r < 4 && n + r < N; r++) o[r] = v[r];
                }
            }
        }
    }
}

}  // namespace

// Launches the 256x256 kernel when it applies (bf16 x and w, no SiLU pair, at
// least ~one tile per CU); returns 1 when it did not apply.
int tiled_big_launch(const ts_linear_args *a, void *stream) {
    if (a->x_dtype != TS_BF16 || a->w_dtype != TS_BF16 || (a->stages & TS_AFTER_SILU_MUL)) return 1;
    // A stage chain takes the 128x128 kernel: its values per lane (128 here) would need
    // a second 128 registers for the chain's sums.
    if (a->after) return 1;
    if (a->k % BK != 0) return 1;  // whole 64-deep steps: loads go straight to LDS, no zero fill
    const uint32_t gx = (a->n + BN - 1) / BN, gy = (a->m + BM - 1) / BM;
    if ((uint64_t)gx * gy < 240 || gy > 65535) return 1;
    // 128 KiB of dynamic LDS needs the function attribute raised once per process.
    static const hipError_t attr =
        hipFuncSetAttribute((const void *)tiled_big_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
    if (attr != hipSuccess) return hip_status(attr, "tiled (256x256) LDS attribute");
    BigParams p;
    p.x = (const uint16_t *)a->x; p.w = (const uint16_t *)a->w; p.a0 = a->a0; p.out = a->out;
    p.m = a->m; p.n = a->n; p.k = a->k; p.stages = a->stages; p.out_bf16 = a->out_dtype == TS_BF16;
    p.mtiles = gy;
    const uint64_t groups = (uint64_t)gy * ((gx + 7) / 8 * 8);
    if (groups > 0x7fffffffu) return 1;
    hipLaunchKernelGGL(tiled_big_kernel, dim3((uint32_t)groups), dim3(kThreads), kLds, (hipStream_t)stream, p);
    TS_CHECK_LAUNCH("tiled (256x256) launch");
    return TS_OK;
}

}  // namespace ts
