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
#include <algorithm>

#include "common.h"

namespace ts {

namespace {

constexpr int BM = 256, BN = 256, BK = 64, kThreads = 512;
constexpr int kStage = BM * BK * 2;  // bytes of one operand stage (A or B)
constexpr int kStages = 2 * 2 * kStage;  // two stages of A and B
constexpr int kLds = kStages + 64 * 512;  // and a 64-row bf16 output chunk (160 KiB in all)

struct BigParams {
    const uint16_t *x;
    const uint16_t *w;
    const float *a0;
    void *out;
    uint32_t m, n, k;
    uint32_t stages;
    int out_bf16;
    uint32_t mtiles;
    uint32_t slots;  // dispatch slots: row tiles x column tiles rounded up to 8
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
                      uint32_t wave, uint32_t lane, uint32_t wm, uint32_t wn, uint32_t col, uint32_t grp,
                      uint32_t k_next) {
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
    if (FETCH) fetch_stage(p, lds + ((s + 1) & 1) * 2 * kStage, m0, n0, k_next, wave, lane);
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

// The tile of dispatch slot b (XCD-aware order: slot b runs on XCD b % 8, each XCD
// walks its own column tiles, n tile = x mod 8, and all row tiles of one column tile
// back to back, so the 256 x K weight tile is fetched into that XCD's L2 once and
// shared by every row tile). False for slots past the last column tile.
TS_DEV bool tile_of(const BigParams &p, uint32_t b, uint32_t &m0, uint32_t &n0) {
    const uint32_t x = b & 7, j = b >> 3;
    const uint32_t mt = j % p.mtiles, nt = (j / p.mtiles) * 8 + x;
    m0 = mt * BM;
    n0 = nt * BN;
    return n0 < p.n;
}

#ifndef TS_BIG_MIN_TILES
#define TS_BIG_MIN_TILES 240
#endif
#ifndef TS_BIG_STAGGER
#define TS_BIG_STAGGER 5
#endif
// The k step a tile starts from: row tiles of one column tile run at once on one XCD,
// and starting them at different k spreads their requests for the same weight lines.
TS_DEV uint32_t k_rot(uint32_t m0, uint32_t steps) { return (m0 / BM * TS_BIG_STAGGER) % steps; }

// Persistent: gridDim.x groups (a multiple of 8, one per CU) walk the dispatch slots
// b = blockIdx.x, + gridDim.x, ... (same XCD for every slot of a group). After a
// tile's last MFMAs the group issues the next tile's first stage, then writes this
// tile's output; the stores drain while the next tile computes, and no group waits
// on a dispatch or an exposed first stage.
__global__ __launch_bounds__(kThreads, 1) void tiled_big_kernel(BigParams p) {
    extern __shared__ __attribute__((aligned(16))) char lds[];  // two stages, then the output chunk
    char *outc = lds + kStages;
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t wm = wave >> 2, wn = wave & 3;
    const uint32_t col = lane & 15, grp = lane >> 4;
    const uint32_t N = p.n, M = p.m, total = p.slots;
    uint32_t b = blockIdx.x, m0 = 0, n0 = 0;
    while (b < total && !tile_of(p, b, m0, n0)) b += gridDim.x;
    if (b >= total) return;
    const uint32_t steps = p.k / BK;
    fetch_stage(p, lds, m0, n0, k_rot(m0, steps) * BK, wave, lane);
    bool stores_pending = false;  // the previous tile's 16 stores a thread may still be in flight
    const bool rows16 = (N & 7) == 0;  // every row starts 16-byte aligned
    while (true) {
        f32x4 acc[8][4];
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] = f32x4{0, 0, 0, 0};
        // Stage 0 has landed once at most the previous tile's stores are outstanding
        // (they were issued after it: the counter retires in order).
        if (stores_pending) asm volatile("s_waitcnt vmcnt(16) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const uint32_t rot = k_rot(m0, steps);
        for (uint32_t s = 0; s + 1 < steps; s++) {
            // The other stage was last read before the previous barrier: refill it now.
            const uint32_t kn = s + 1 + rot < steps ? s + 1 + rot : s + 1 + rot - steps;
            mfma_step<true>(p, lds, s, acc, m0, n0, wave, lane, wm, wn, col, grp, kn * BK);
            // the next stage's loads have landed (in every wave, after the barrier)
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        }
        mfma_step<false>(p, lds, steps - 1, acc, m0, n0, wave, lane, wm, wn, col, grp, 0);

        // The next tile's first stage, issued before this tile's stores.
        uint32_t b2 = b + gridDim.x, m1 = 0, n1 = 0;
        while (b2 < total && !tile_of(p, b2, m1, n1)) b2 += gridDim.x;
        lds_barrier();  // every wave is done reading both stages
        if (b2 < total) fetch_stage(p, lds, m1, n1, k_rot(m1, steps) * BK, wave, lane);
        __builtin_amdgcn_sched_barrier(0);

        const bool whole_tile = rows16 && m0 + BM <= M && n0 + BN <= N;
        if (p.out_bf16 && !(p.stages & TS_AFTER_ADD)) {
            // bf16 output with no added operand: the tile goes through the 32 KiB
            // output chunk 64 rows at a time and leaves as whole rows (two rows of 512
            // contiguous bytes per store instruction). Chunk c holds the 16-row slabs i
            // = 2c and 2c + 1 of both wave rows, so every wave writes its accumulators
            // acc[2c], acc[2c + 1] and they are free after it (512-byte rows, 16-byte
            // chunks XOR-swizzled by row). Local row 16 (2 wm + i - 2c) + col is tile
            // row 128 wm + 16 i + col.
#pragma unroll
            for (int c = 0; c < 4; c++) {
#pragma unroll
                for (int ii = 0; ii < 2; ii++) {
                    const int i = 2 * c + ii;
                    const uint32_t r = (2 * wm + ii) * 16 + col;  // row within the chunk
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const uint32_t cc = wn * 64 + j * 16 + 4 * grp;  // first of 4 columns (8 B)
                        const f32x4 v = acc[i][j];
                        *(u32x2 *)(outc + r * 512 + ((((cc >> 3) ^ (r & 31))) << 4) + (cc & 7) * 2) =
                            u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
                    }
                }
                lds_barrier();
#pragma unroll
                for (int it = 0; it < 4; it++) {
                    const uint32_t f = it * kThreads + t, r = f >> 5, cc = f & 31;
                    const uint32_t sl = r >> 4, tr = (sl >> 1) * 128 + (2 * c + (sl & 1)) * 16 + (r & 15);
                    const uint32_t m = m0 + tr, n = n0 + cc * 8;
                    const u32x4 v = *(const u32x4 *)(outc + r * 512 + ((cc ^ (r & 31)) << 4));
                    uint16_t *o = (uint16_t *)p.out + (size_t)m * N + n;
                    if (whole_tile) {
                        *(u32x4 *)o = v;
                    } else if (m < M && n < N) {
                        if (rows16 && n + 8 <= N) {
                            *(u32x4 *)o = v;
                        } else {
                            for (uint32_t e = 0; e < 8 && n + e < N; e++)
                                o[e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
                        }
                    }
                }
                lds_barrier();  // the chunk is read before the next one overwrites it
            }
            stores_pending = whole_tile;
        } else {
            // f32 output or an added operand, straight from the accumulators. The MFMA
            // operands are swapped (weights first), so lane l holds row col of each
            // 16x16 tile and its four adjacent columns 4 grp .. + 3: one 8-byte (bf16)
            // or 16-byte (f32) store per lane and tile instead of four 2-byte ones.
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
            stores_pending = false;  // the a0 loads and the stores: wait for all of them
        }
        if (b2 >= total) break;
        b = b2; m0 = m1; n0 = n1;
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
    if ((uint64_t)gx * gy < TS_BIG_MIN_TILES || gy > 65535) return 1;
    // 128 KiB of dynamic LDS needs the function attribute raised once per process.
    static const hipError_t attr =
        hipFuncSetAttribute((const void *)tiled_big_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
    if (attr != hipSuccess) return hip_status(attr, "tiled (256x256) LDS attribute");
    BigParams p;
    p.x = (const uint16_t *)a->x; p.w = (const uint16_t *)a->w; p.a0 = a->a0; p.out = a->out;
    p.m = a->m; p.n = a->n; p.k = a->k; p.stages = a->stages; p.out_bf16 = a->out_dtype == TS_BF16;
    p.mtiles = gy;
    const uint64_t slots = (uint64_t)gy * ((gx + 7) / 8 * 8);
    if (slots > 0x7fffffffu) return 1;
    p.slots = (uint32_t)slots;
    // One persistent group per CU (a multiple of 8: each group stays on one XCD).
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return hip_status(e, "tiled (256x256): device attributes");
    const uint32_t groups = (uint32_t)std::min<uint64_t>(slots, (uint64_t)std::max(8, cus / 8 * 8));
    hipLaunchKernelGGL(tiled_big_kernel, dim3(groups), dim3(kThreads), kLds, (hipStream_t)stream, p);
    TS_CHECK_LAUNCH("tiled (256x256) launch");
    return TS_OK;
}

}  // namespace ts
