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
//  * k advances 64 at a time. The rows of x sit in two 32 KiB LDS stages and the weight
//    rows in three, all of a CU's 160 KiB (256 x 64 bf16 each, 128-byte rows with
//    16-byte chunks XOR-swizzled by row), filled with global_load_lds_dwordx4 straight
//    from memory (no staging registers): the weight tile's loads run two steps ahead of
//    the matrix work (its first row tile misses L2), the rows' one step (they stay in L2).
//  * Scheduling groups pin the order: one substep's fragment reads, then its MFMAs
//    interleaved with the other substep's reads and the loads.
//  * The row tiles of one weight column tile run on one XCD at once; each starts at its
//    own k step so they do not ask for the same weight lines together.
#include <algorithm>

#include "common.h"

namespace ts {

namespace {

constexpr int BM = 256, BN = 256, BK = 64, kThreads = 512;
constexpr int kStage = BM * BK * 2;  // bytes of one operand stage (A or B)
constexpr int kLds = 5 * kStage;  // two stages of A, three of B: 160 KiB, all of a CU's LDS

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

constexpr uint32_t kStagger = 5;  // k steps between consecutive row tiles' starts
// The k step a tile starts from: row tiles of one column tile run at once on one XCD,
// and starting them at different k spreads their requests for the same weight lines.
TS_DEV uint32_t k_rot(uint32_t m0, uint32_t steps) { return (m0 / BM * kStagger) % steps; }

// ---------------------------------------------------------------------------
// The three-stage weight form: A (rows of x) in two 32 KiB stages, B (weight rows) in
// three, 160 KiB in all, so the weight tile's loads run two steps ahead of the matrix
// work and the rows' one step (a weight column tile's first row tile misses L2; x
// stays there). One tile per group; the output leaves through the stage area.
// ---------------------------------------------------------------------------
// Per-lane element offsets of the four rows a lane fetches in a 256-row tile (rows
// past the end repeat the last; never stored): 32 bits, the launcher checks the
// operands fit.
TS_DEV void half_offsets(uint32_t rows, uint32_t r0, uint32_t K, uint32_t wave, uint32_t lane, uint32_t (&off)[4]) {
    const uint32_t rl = lane >> 3, lc = (lane & 7) ^ rl;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t row = 8 * (wave * 4 + i) + rl;
        off[i] = min(r0 + row, rows - 1) * K + lc * 8;
    }
}

TS_DEV void fetch_half(const uint16_t *src, const uint32_t (&off)[4], char *stage, uint32_t k0, uint32_t wave) {
    const uint16_t *base = src + k0;
#pragma unroll
    for (int i = 0; i < 4; i++)
        __builtin_amdgcn_global_load_lds((const void *)(base + off[i]), (lds_void *)(stage + (wave * 4 + i) * 1024),
                                         16, 0, 0);
}

template <bool FA, bool FB>
TS_DEV void mfma_step(const BigParams &p, char *lds, uint32_t s, f32x4 (&acc)[8][4], const uint32_t (&oa)[4],
                       const uint32_t (&ob)[4], uint32_t wave, uint32_t wm, uint32_t wn, uint32_t col, uint32_t grp,
                       uint32_t ka, uint32_t kb) {
    const char *sa = lds + (s & 1) * kStage, *sb = lds + 2 * kStage + (s % 3) * kStage;
    bf16x8 af[2][8], bfr[2][4];
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
        const uint32_t c = ks * 4 + grp;
#pragma unroll
        for (int j = 0; j < 4; j++) bfr[ks][j] = as_bf16x8(*(const u32x4 *)(sb + swz(wn * 64 + j * 16 + col, c)));
#pragma unroll
        for (int i = 0; i < 8; i++) af[ks][i] = as_bf16x8(*(const u32x4 *)(sa + swz(wm * 128 + i * 16 + col, c)));
    }
    if (FA) fetch_half(p.x, oa, lds + ((s + 1) & 1) * kStage, ka, wave);
    if (FB) fetch_half(p.w, ob, lds + 2 * kStage + ((s + 2) % 3) * kStage, kb, wave);
#pragma unroll
    for (int ks = 0; ks < 2; ks++)
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] = mfma16(bfr[ks][j], af[ks][i], acc[i][j]);
    // Masks: 0x008 MFMA, 0x020 VMEM read, 0x100 DS read. The first substep's reads,
    // then its MFMAs interleaved with the second substep's reads and the loads, then
    // the remaining MFMAs: LDS and load latency hide under matrix work.
    constexpr int NV = (FA ? 4 : 0) + (FB ? 4 : 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);
#pragma unroll
    for (int i = 0; i < 12; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
#pragma unroll
    for (int i = 0; i < NV; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 52 - NV, 0);
    __builtin_amdgcn_sched_barrier(0);
}

__global__ __launch_bounds__(kThreads, 1) void tiled_big_kernel(BigParams p) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t wm = wave >> 2, wn = wave & 3;
    const uint32_t col = lane & 15, grp = lane >> 4;
    uint32_t m0, n0;
    if (!tile_of(p, blockIdx.x, m0, n0)) return;
    const uint32_t N = p.n, M = p.m, steps = p.k / BK, rot = k_rot(m0, steps);
    auto kof = [&](uint32_t s) { return (s + rot < steps ? s + rot : s + rot - steps) * BK; };
    f32x4 acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f32x4{0, 0, 0, 0};
    uint32_t oa[4], ob[4];
    half_offsets(M, m0, p.k, wave, lane, oa);
    half_offsets(N, n0, p.k, wave, lane, ob);
    fetch_half(p.x, oa, lds, kof(0), wave);
    fetch_half(p.w, ob, lds + 2 * kStage, kof(0), wave);
    if (steps > 1) {
        fetch_half(p.w, ob, lds + 3 * kStage, kof(1), wave);
        asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");  // A 0 and B 0 landed
    } else {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    for (uint32_t s = 0; s + 1 < steps; s++) {
        // Buffers refilled here were last read before the previous barrier. The
        // second-to-last step refills the free weight buffer with step 0's k again (one
        // loop body: no second copy of the step's registers), drained below.
        mfma_step<true, true>(p, lds, s, acc, oa, ob, wave, wm, wn, col, grp, kof(s + 1),
                               kof(s + 2 < steps ? s + 2 : 0));
        // A s+1 (issued before B s+2) and B s+1 (a step earlier) have landed.
        asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    mfma_step<false, false>(p, lds, steps - 1, acc, oa, ob, wave, wm, wn, col, grp, 0, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no load lands in the stage area from here on

    if (p.out_bf16 && !(p.stages & TS_AFTER_ADD)) {
        // bf16 rows through the stage area (free once every wave has read the last
        // stage): 256 rows of 512 B, 16-byte chunks XOR-swizzled by row, leaving as
        // whole rows (two rows of 512 contiguous bytes per store instruction).
        lds_barrier();
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t r = wm * 128 + i * 16 + col;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t c = wn * 64 + j * 16 + 4 * grp;
                const f32x4 v = acc[i][j];
                *(u32x2 *)(lds + r * 512 + ((((c >> 3) ^ (r & 31))) << 4) + (c & 7) * 2) =
                    u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
            }
        }
        lds_barrier();
        const bool rows16 = (N & 7) == 0;
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
                if (whole) v += *(const f32x4 *)(p.a0 + e);
                else
                    for (uint32_t r = 0; r < 4 && n + r < N; r++) v[r] += p.a0[e + r];
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
                if (whole) *(f32x4 *)o = v;
                else
                    for (uint32_t r = 0; r < 4 && n + r < N; r++) o[r] = v[r];
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
    // Lanes address their rows with 32-bit element offsets.
    if ((uint64_t)a->m * a->k >= (1ull << 32) || (uint64_t)a->n * a->k >= (1ull << 32)) return 1;
    // 160 KiB of dynamic LDS needs the function attribute raised once per process.
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
    hipLaunchKernelGGL(tiled_big_kernel, dim3(p.slots), dim3(kThreads), kLds, (hipStream_t)stream, p);
    TS_CHECK_LAUNCH("tiled (256x256) launch");
    return TS_OK;
}

}  // namespace ts
