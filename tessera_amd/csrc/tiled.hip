// "tiled": out[m, n] = after(sum_k x[m, k] w[n, k]) for many rows.
//
// Replaces the reference's matrix-unit matmul rule (engine/rules/linear/src/
// tiled.rs:281-345 tiled, :186-278 tiled_parts, :441-453, :611-672 propose),
// which on gfx950 is refused today (no tile row for gfx9_5). Same product and
// fused stages (engine/plan/lower/src/kernels/map.rs:155-185).
//
// gfx950 design (bf16 rows and weights take the pipelined kernel further down, which
// shares the tile order, swizzle and epilogue described here):
//  * 128x128 output tile per 256-thread group (4 waves in 2x2, each 64x64 =
//    4x4 v_mfma_f32_16x16x32_bf16 tiles), k in 64-deep steps; 64x64 tiles (waves of
//    32x32) when 128x128 would give fewer than 2 groups per CU, since each group is a
//    latency chain (load, LDS, barrier, store) rather than MFMA-bound.
//  * The MFMA computes the transposed tile (weights as the first operand), so a lane
//    holds 4 consecutive output columns of one row: one 8-byte (bf16) or 16-byte (f32)
//    store per 4 outputs instead of four 2- or 4-byte ones.
//  * Both operands are k-contiguous ([m,k] and [n,k]), which is the matrix
//    unit's native operand order: a lane's 8 k values are one 16-byte LDS read.
//  * LDS holds two stages (A and B, 16 KiB each per stage, plus a second A
//    stage for the low part of f32 rows); the next k-step is fetched from HBM
//    into registers while the current one multiplies, then stored to the other
//    stage: one barrier per k-step.
//  * LDS rows are 128 bytes (8 chunks of 16B); chunk c of row r sits at chunk
//    c ^ (r & 7), so the 16 rows one MFMA operand read touches spread over all
//    banks instead of hitting one.
//  * f32 rows are split into two exact bf16 parts (as tiled_parts does with
//    three), e4m3 weights decode to bf16 on the way into LDS with the per-row
//    scale applied to the finished sum; SiLU-gate pairs are laid out so a lane
//    holds gate and up of the same column.
#include "after.h"

namespace {

#ifndef TS_PIPE_WIDE
#define TS_PIPE_WIDE 1
#endif
constexpr int BM = 128, BN = 128, BK = 64;  // the default tile; BT = 64 for products with few tiles
constexpr int kThreads = 256;

struct TiledParams {
    const void *x;
    const void *w;
    const uint16_t *w_scale;
    const float *a0;
    void *out;
    uint32_t m, n, k;
    uint32_t stages;
    int out_bf16;
    // Picked products (PICK): rows sorted by matrix. perm[pos] is the row at sorted
    // position pos; matrix e owns positions [row_start[e], row_start[e + 1]) and
    // row tiles [tile_start[e], tile_start[e + 1]). Row r reads x row r / repeat;
    // matrix e's rows start at w + (e * stride + offset) * k (scales likewise).
    const uint32_t *perm, *row_start, *tile_start;
    uint32_t matrices, repeat, stride, offset;
    ts_after after;  // stage chain (count 0: none)
    int pair_sum;    // TS_F32_PARTS: the second row block is the low parts; the output sums the pair
    uint32_t pick_cols;  // PICK on the pipelined tiles: column tiles (0: a 2-D grid of them)
};

// Byte offset of (row, chunk) in a swizzled [rows][8 chunks of 16B] tile.
TS_DEV uint32_t swz(uint32_t row, uint32_t chunk) { return row * 128 + ((chunk ^ (row & 7)) << 4); }

template <int BT, bool XF32, bool W8, bool SILU>
struct Loader {
    static constexpr int RPT = BT / 32;  // rows per thread per operand
    static constexpr int WT = BT / 2;    // a wave's share of the tile's columns
    // Per thread per stage: A: RPT chunks (rows t/8 + 32i, chunk t%8), B: RPT chunks.
    u32x4 a_hi[RPT], a_lo[RPT], b[RPT];
    // x row of each of this thread's A rows, or -1 for a zero row.
    int64_t src[RPT];
    // The weights of this tile's matrix (the whole w outside picked products).
    const void *w;
    const uint16_t *w_scale;

    // Weight row of B-tile row `br` for this output tile. SILU: each wave's WT rows are
    // WT/2 gate rows then the WT/2 up rows of the same output columns.
    TS_DEV static uint32_t wrow(uint32_t br, uint32_t n0, uint32_t N) {
        if (!SILU) return n0 + br;
        const uint32_t half = br / WT, within = br % WT;
        return within < WT / 2 ? n0 + half * (WT / 2) + within : N + n0 + half * (WT / 2) + (within - WT / 2);
    }

    TS_DEV void fetch(const TiledParams &p, uint32_t m0, uint32_t n0, uint32_t k0) {
        const uint32_t t = threadIdx.x, chunk = t & 7;
        const uint32_t kk = k0 + chunk * 8;
        const bool kin = kk < p.k;
#pragma unroll
        for (int i = 0; i < RPT; i++) {
            const uint32_t r = (t >> 3) + 32 * i;
            const bool ain = src[i] >= 0 && kin;
            if (XF32) {
                float v[8];
                if (ain) {
                    const float4 *src4 = (const float4 *)((const float *)p.x + (size_t)src[i] * p.k + kk);
                    float4 u0 = src4[0], u1 = src4[1];
                    v[0] = u0.x; v[1] = u0.y; v[2] = u0.z; v[3] = u0.w;
                    v[4] = u1.x; v[5] = u1.y; v[6] = u1.z; v[7] = u1.w;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; e++) v[e] = 0.0f;
                }
                uint32_t h[4], l[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float x0 = v[2 * e], x1 = v[2 * e + 1];
                    float h0 = bf16_round(x0), h1 = bf16_round(x1);
                    h[e] = pack_bf16x2(h0, h1);
                    l[e] = pack_bf16x2(x0 - h0, x1 - h1);
                }
                a_hi[i] = u32x4{h[0], h[1], h[2], h[3]};
                a_lo[i] = u32x4{l[0], l[1], l[2], l[3]};
            } else {
                a_hi[i] = ain ? *(const u32x4 *)((const uint16_t *)p.x + (size_t)src[i] * p.k + kk) : u32x4{0, 0, 0, 0};
            }
            const uint32_t nr = wrow(r, n0, p.n);
            const uint32_t nrows = SILU ? 2 * p.n : p.n;
            const bool nin = (SILU ? (n0 + (r / WT) * (WT / 2) + (r % (WT / 2))) < p.n : nr < nrows) && kin;
            if (W8) {
                if (nin) {
                    const u32x2 c = *(const u32x2 *)((const uint8_t *)w + (size_t)nr * p.k + kk);
                    u32x2 lo = e4m3x4_to_bf16x4(c.x), hi = e4m3x4_to_bf16x4(c.y);
                    b[i] = u32x4{lo.x, lo.y, hi.x, hi.y};
                } else {
                    b[i] = u32x4{0, 0, 0, 0};
                }
            } else {
                b[i] = nin ? *(const u32x4 *)((const uint16_t *)w + (size_t)nr * p.k + kk) : u32x4{0, 0, 0, 0};
            }
        }
    }

    TS_DEV void store(char *sa, char *sa_lo, char *sb) {
        const uint32_t t = threadIdx.x, chunk = t & 7;
#pragma unroll
        for (int i = 0; i < RPT; i++) {
            const uint32_t r = (t >> 3) + 32 * i;
            *(u32x4 *)(sa + swz(r, chunk)) = a_hi[i];
            if (XF32) *(u32x4 *)(sa_lo + swz(r, chunk)) = a_lo[i];
            *(u32x4 *)(sb + swz(r, chunk)) = b[i];
        }
    }
};

template <int BT, bool XF32, bool W8, bool SILU, bool PICK, bool CHAIN>
__global__ __launch_bounds__(kThreads) void tiled_kernel(TiledParams p) {
    constexpr int TILE = BT * BK * 2;         // bytes of one operand stage
    constexpr int WT = BT / 2, FT = WT / 16;  // wave tile, 16x16 fragments per wave side
    constexpr int RPT = BT / 32;
    __shared__ __attribute__((aligned(16))) char lds[2][XF32 ? 3 : 2][TILE];
    __shared__ uint32_t rows_out[PICK ? BT : 1];  // output row of each tile row (PICK)

    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1;
    const uint32_t col = lane & 15, grp = lane >> 4;
    const uint32_t n0 = blockIdx.x * (SILU ? BT / 2 : BT);  // SILU: BT / 2 output columns per tile

    Loader<BT, XF32, W8, SILU> ld;
    uint32_t m0 = blockIdx.y * BT, mend = p.m;  // tile rows [m0, min(m0 + BT, mend))
    ld.w = p.w;
    ld.w_scale = p.w_scale;
    if (PICK) {
        // Row tile blockIdx.y belongs to the matrix e with tile_start[e] <= y < tile_start[e + 1].
        const uint32_t y = blockIdx.y;
        if (y >= p.tile_start[p.matrices]) return;
        uint32_t lo = 0, hi = p.matrices;  // invariant: tile_start[lo] <= y < tile_start[hi]
        while (hi - lo > 1) {
            const uint32_t mid = (lo + hi) / 2;
            if (p.tile_start[mid] <= y) lo = mid;
            else hi = mid;
        }
        const uint32_t e = lo;
        m0 = p.row_start[e] + (y - p.tile_start[e]) * BT;
        mend = p.row_start[e + 1];
        const size_t first_row = (size_t)e * p.stride + p.offset;
        ld.w = (const char *)p.w + first_row * p.k * (W8 ? 1 : 2);
        if (W8) ld.w_scale = p.w_scale + first_row;
        for (uint32_t r = threadIdx.x; r < BT; r += kThreads)
            rows_out[r] = m0 + r < mend ? p.perm[m0 + r] : 0xffffffffu;
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < RPT; i++) {
        const uint32_t r = (threadIdx.x >> 3) + 32 * i;
        if (PICK) ld.src[i] = rows_out[r] != 0xffffffffu ? (int64_t)(rows_out[r] / p.repeat) : -1;
        else ld.src[i] = m0 + r < p.m ? (int64_t)(m0 + r) : -1;
    }

    f32x4 acc[FT][FT];
#pragma unroll
    for (int i = 0; i < FT; i++)
#pragma unroll
        for (int j = 0; j < FT; j++) acc[i][j] = f32x4{0, 0, 0, 0};

    const uint32_t steps = (p.k + BK - 1) / BK;
    ld.fetch(p, m0, n0, 0);
    ld.store(lds[0][0], lds[0][XF32 ? 2 : 0], lds[0][1]);
    __syncthreads();

    for (uint32_t s = 0; s < steps; s++) {
        const int cur = s & 1;
        if (s + 1 < steps) ld.fetch(p, m0, n0, (s + 1) * BK);
        const char *sa = lds[cur][0], *sb = lds[cur][1], *sl = lds[cur][XF32 ? 2 : 0];
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            const uint32_t chunk = ks * 4 + grp;
            bf16x8 af[FT], al[FT], bfr[FT];
#pragma unroll
            for (int i = 0; i < FT; i++) {
                const uint32_t ra = wm * WT + i * 16 + col;
                af[i] = as_bf16x8(*(const u32x4 *)(sa + swz(ra, chunk)));
                if (XF32) al[i] = as_bf16x8(*(const u32x4 *)(sl + swz(ra, chunk)));
                const uint32_t rb = wn * WT + i * 16 + col;
                bfr[i] = as_bf16x8(*(const u32x4 *)(sb + swz(rb, chunk)));
            }
#pragma unroll
            for (int i = 0; i < FT; i++)
#pragma unroll
                for (int j = 0; j < FT; j++) {
                    acc[i][j] = mfma16(bfr[j], af[i], acc[i][j]);
                    if (XF32) acc[i][j] = mfma16(bfr[j], al[i], acc[i][j]);
                }
        }
        if (s + 1 < steps) {
            const int nxt = cur ^ 1;
            ld.store(lds[nxt][0], lds[nxt][XF32 ? 2 : 0], lds[nxt][1]);
        }
        __syncthreads();
    }

    // Epilogue. acc[i][j] is the transposed 16x16 tile: lane (col, grp) holds row
    // m = wm WT + 16 i + col and columns n = wn WT + 16 j + 4 grp + 0..3 (SILU: gate in
    // j < FT/2, up in j + FT/2, columns wn WT/2 + 16 j + 4 grp + 0..3).
    const uint32_t N = p.n;
    const uint16_t *scale = ld.w_scale;
    const bool vec = (N & 3) == 0;
    constexpr int JO = SILU ? FT / 2 : FT;
    float val[FT][JO][4];
#pragma unroll
    for (int i = 0; i < FT; i++)
#pragma unroll
        for (int j = 0; j < JO; j++) {
            const uint32_t n = n0 + (SILU ? wn * (WT / 2) : wn * WT) + j * 16 + 4 * grp;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float g = acc[i][j][r];
                if (SILU) {
                    float u = acc[i][j + FT / 2][r];
                    if (W8) {
                        g *= bf16_float(scale[min(n + r, N - 1)]);
                        u *= bf16_float(scale[N + min(n + r, N - 1)]);
                    }
                    val[i][j][r] = p.pair_sum ? g + u : g / (1.0f + expf(-g)) * u;
                } else {
                    if (W8) g *= bf16_float(scale[min(n + r, N - 1)]);
                    val[i][j][r] = g;
                }
            }
        }
    if (CHAIN) {  // the chain's variant: its values and sums need more registers
        // Value e = (i JO + j) 4 + r: row tile i, column tile j, column 4 grp + r.
        auto row_of = [&](int e) {
            const uint32_t tr = wm * WT + (e / (4 * JO)) * 16 + col;
            return m0 + tr < mend ? (PICK ? rows_out[tr] : m0 + tr) : ~0u;
        };
        auto col_of = [&](int e) {
            return n0 + (SILU ? wn * (WT / 2) : wn * WT) + (e / 4 % JO) * 16 + 4 * grp + e % 4;
        };
        ts::after_values<FT * JO * 4, false>(
            p.after, *(float(*)[FT * JO * 4])val, [&](int e) { return (size_t)row_of(e) * N + col_of(e); },
            [&](int e) { return row_of(e) != ~0u && col_of(e) < N; });
    }
#pragma unroll
    for (int i = 0; i < FT; i++) {
        const uint32_t tr = wm * WT + i * 16 + col;
        if (m0 + tr >= mend) continue;
        const uint32_t m = PICK ? rows_out[tr] : m0 + tr;
#pragma unroll
        for (int j = 0; j < JO; j++) {
            const uint32_t n = n0 + (SILU ? wn * (WT / 2) : wn * WT) + j * 16 + 4 * grp;
            if (n >= N) continue;
            float *v = val[i][j];
            const size_t at = (size_t)m * N + n;
            if (vec && n + 3 < N) {
                if (p.stages & TS_AFTER_ADD) {
                    const float4 a = *(const float4 *)(p.a0 + at);
                    v[0] += a.x; v[1] += a.y; v[2] += a.z; v[3] += a.w;
                }
                if (p.out_bf16) *(u32x2 *)((uint16_t *)p.out + at) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
                else *(float4 *)((float *)p.out + at) = float4{v[0], v[1], v[2], v[3]};
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    if (n + r >= N) break;
                    float u = v[r];
                    if (p.stages & TS_AFTER_ADD) u += p.a0[at + r];
                    if (p.out_bf16) ((uint16_t *)p.out)[at + r] = bf16_bits(u);
                    else ((float *)p.out)[at + r] = u;
                }
            }
        }
    }
}


// ---------------------------------------------------------------------------
// The pipelined form for bf16 rows and weights (k a multiple of 64): TM x TN tiles,
// 4 waves in 2 x 2 (each (TM/2) x (TN/2)), and NS LDS stages KD deep filled straight
// from memory with global_load_lds_dwordx4 (no staging registers, no LDS stores),
// NS - 1 of them in flight ahead of the MFMAs, groups in an XCD-aware order, and
// each configuration sized so two groups share a CU: one group's loads, barriers and
// epilogue overlap the other's matrix work. bf16 results leave through LDS as whole
// rows. The register-staged form above still serves f32 rows and e4m3 weights.
// ---------------------------------------------------------------------------
template <int TM, int TN, int KD, int NS>
struct Pipe {
    static constexpr int RB = KD * 2;          // bytes of one LDS row (KD bf16)
    static constexpr int CPR = KD / 8;         // 16-byte chunks per row
    static constexpr int RPI = 1024 / RB;      // rows one load instruction fills
    static constexpr int NA = TM / RPI / 4;    // A load instructions per wave per stage
    static constexpr int NB = TN / RPI / 4;    // B load instructions per wave per stage
    static constexpr int A_BYTES = TM * RB, STAGE = (TM + TN) * RB, LDS = NS * STAGE;
    static constexpr int WM = TM / 2, WN = TN / 2, FI = WM / 16, FJ = WN / 16;
    static_assert(NA >= 1 && NB >= 1 && (KD == 32 || KD == 64), "pipe shape");

    // Byte offset of logical chunk c of row r. 128-byte rows: chunk c ^ (r & 7) of row
    // r. 64-byte rows: rows pair up in 128-byte lines L = r / 2, and 16-byte unit
    // u = 4 (r & 1) + c of a line sits at u ^ (L & 7). Either way the 16 rows one
    // fragment read touches (one chunk each) spread over all banks (measured: no
    // conflicts; a per-row XOR of 64-byte rows conflicts).
    TS_DEV static uint32_t at(uint32_t r, uint32_t c) {
        if (CPR == 8) return r * 128 + ((c ^ (r & 7)) << 4);
        const uint32_t L = r >> 1, u = (r & 1) * 4 + c;
        return L * 128 + ((u ^ (L & 7)) << 4);
    }
    // The row (within the RPI rows an instruction fills) and logical chunk that lane l
    // of a load instruction brings: the lane lands at byte 16 l of the instruction's KiB.
    TS_DEV static void source(uint32_t l, uint32_t &row, uint32_t &chunk) {
        const uint32_t line = l >> 3, u = (l & 7) ^ line;  // line & 7 == line: 8 lines per KiB
        if (CPR == 8) {
            row = line;
            chunk = u;
        } else {
            row = 2 * line + (u >> 2);
            chunk = u & 3;
        }
    }
};

constexpr uint32_t kBand = 8;  // tile rows per band of the XCD-aware order

typedef __attribute__((address_space(3))) void lds_void;

// Waits until at most N of this wave's loads are outstanding, then meets the group's
// other waves (no fence: the LDS reads of the previous k-step completed before their
// MFMAs, and the loads waited for here wrote LDS directly).
template <int N>
TS_DEV void pipe_wait() {
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

// The wait for a stage with `ahead` later stages (L loads each) still allowed in flight.
template <int L, int A>
TS_DEV void pipe_wait_ahead(uint32_t ahead) {
    if constexpr (A == 0) {
        pipe_wait<0>();
    } else {
        if (ahead >= A) pipe_wait<L * A>();
        else pipe_wait_ahead<L, A - 1>(ahead);
    }
}

TS_DEV const char *uniform_ptr(const void *ptr) {
    const uint64_t v = (uint64_t)ptr;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const char *)(((uint64_t)hi << 32) | lo);
}

template <int TM, int TN, int KD, int NS, bool SILU, bool PICK, bool CHAIN>
__global__ __launch_bounds__(kThreads, 2) void tiled_pipe_kernel(TiledParams p) {
    using P = Pipe<TM, TN, KD, NS>;
    extern __shared__ __attribute__((aligned(16))) char lds[];  // the only LDS: two groups share a CU
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1;
    const uint32_t col = lane & 15, grp = lane >> 4;
    constexpr uint32_t OC = SILU ? TN / 2 : TN;  // output columns per tile
    uint32_t tx = blockIdx.x, ty = blockIdx.y;
    if (!PICK) {
        // XCD-aware order (one-dimensional grid): group b runs on XCD b % 8, and XCD x
        // takes the x-th eighth of the tiles, walked in bands of kBand tile rows column
        // by column, so the groups an XCD runs at once share rows and weight columns
        // in its L2.
        const uint32_t gx = p.stride, gy = p.offset, tiles = gx * gy, per = (tiles + 7) / 8;
        const uint32_t t = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
        if (t >= tiles) return;
        const uint32_t band = t / (kBand * gx), rows = min(kBand, gy - band * kBand);
        const uint32_t within = t - band * kBand * gx;
        ty = band * kBand + within % rows;
        tx = within / rows;
    }
    uint32_t n0 = tx * OC;
    uint32_t m0 = ty * TM, mend = p.m;
    const uint16_t *w = (const uint16_t *)p.w;
    if (PICK) {
        uint32_t y = blockIdx.y;
        if (p.pick_cols) {
            // XCD-aware order (one-dimensional grid, group b on XCD b % 8): XCD x takes
            // the sorted row tiles [x Y / 8, (x + 1) Y / 8) and walks them matrix by
            // matrix, each matrix's column tiles in turn over its row tiles, so the
            // gathered rows and the weight tile both stay in that XCD's L2.
            const uint32_t Y = p.tile_start[p.matrices], gx = p.pick_cols;
            const uint32_t xcd = blockIdx.x & 7, j = blockIdx.x >> 3;
            const uint32_t y0 = (uint32_t)((uint64_t)xcd * Y / 8), y1 = (uint32_t)((uint64_t)(xcd + 1) * Y / 8);
            if (j >= gx * (y1 - y0)) return;
            uint32_t lo = 0, hi = p.matrices;  // the matrix holding row tile y0
            while (hi - lo > 1) {
                const uint32_t mid = (lo + hi) / 2;
                if (p.tile_start[mid] <= y0) lo = mid;
                else hi = mid;
            }
            uint32_t e = lo, ys = y0, rem = j;
            for (;;) {  // ends: j < gx (y1 - y0), and every row tile in range belongs to a matrix
                const uint32_t ye = min(p.tile_start[e + 1], y1), ne = ye - ys;
                if (rem < gx * ne) {
                    tx = rem / ne;
                    n0 = tx * OC;
                    y = ys + rem % ne;
                    break;
                }
                rem -= gx * ne;
                ys = ye;
                e++;
            }
        }
        if (y >= p.tile_start[p.matrices]) return;
        uint32_t lo = 0, hi = p.matrices;  // invariant: tile_start[lo] <= y < tile_start[hi]
        while (hi - lo > 1) {
            const uint32_t mid = (lo + hi) / 2;
            if (p.tile_start[mid] <= y) lo = mid;
            else hi = mid;
        }
        const uint32_t e = lo;
        m0 = p.row_start[e] + (y - p.tile_start[e]) * TM;
        mend = p.row_start[e + 1];
        w += ((size_t)e * p.stride + p.offset) * p.k;
    }
    // PICK: the output row of tile row tr (~0u past the matrix's rows), read where needed
    // (no LDS copy, so two groups' stages fill a CU's LDS).
    auto row_out = [&](uint32_t tr) { return m0 + tr < mend ? p.perm[m0 + tr] : 0xffffffffu; };
    // Element offsets (at k = 0) of the row each of this lane's loads reads, and the
    // logical chunk it fetches: instruction i of the wave fills rows RPI b .. RPI b +
    // RPI - 1, b = NA wave + i (A) or NB wave + i (B). Rows past the end read a row
    // that exists (never stored).
    uint32_t rl, lc;
    P::source(lane, rl, lc);
    uint32_t aoff[P::NA], boff[P::NB];
#pragma unroll
    for (int i = 0; i < P::NA; i++) {
        const uint32_t r = P::RPI * (wave * P::NA + i) + rl;
        uint32_t xr;
        if (PICK) {
            const uint32_t o = row_out(r);
            xr = (o != 0xffffffffu ? o : p.perm[m0]) / p.repeat;
        } else {
            xr = min(m0 + r, p.m - 1);
        }
        aoff[i] = xr * p.k + lc * 8;
    }
#pragma unroll
    for (int i = 0; i < P::NB; i++) {
        const uint32_t r = P::RPI * (wave * P::NB + i) + rl;
        uint32_t nr;
        if (SILU) {
            // Each wave's WN weight rows: WN/2 gate rows, then the up rows of the same columns.
            const uint32_t half = r / P::WN, within = r % P::WN;
            const uint32_t c = min(n0 + half * (P::WN / 2) + within % (P::WN / 2), p.n - 1);
            nr = within < P::WN / 2 ? c : p.n + c;
        } else {
            nr = min(n0 + r, p.n - 1);
        }
        boff[i] = nr * p.k + lc * 8;
    }
    const uint16_t *xs = (const uint16_t *)p.x;

    auto fetch = [&](uint32_t slot, uint32_t k0) {
        char *stage = lds + slot * P::STAGE;
        const char *xb = uniform_ptr(xs + k0), *wb = uniform_ptr(w + k0);
#pragma unroll
        for (int i = 0; i < P::NA; i++)
            __builtin_amdgcn_global_load_lds((const void *)(xb + (size_t)aoff[i] * 2),
                                             (lds_void *)(stage + (wave * P::NA + i) * 1024), 16, 0, 0);
#pragma unroll
        for (int i = 0; i < P::NB; i++)
            __builtin_amdgcn_global_load_lds((const void *)(wb + (size_t)boff[i] * 2),
                                             (lds_void *)(stage + P::A_BYTES + (wave * P::NB + i) * 1024), 16, 0, 0);
    };

    f32x4 acc[P::FI][P::FJ];
#pragma unroll
    for (int i = 0; i < P::FI; i++)
#pragma unroll
        for (int j = 0; j < P::FJ; j++) acc[i][j] = f32x4{0, 0, 0, 0};

    const uint32_t steps = p.k / KD;
    // 16-row fragments of this wave that hold a row of the tile (wave-uniform).
    const uint32_t wrow0 = m0 + wm * P::WM;
    const uint32_t live_frags = mend > wrow0 ? min((mend - wrow0 + 15) / 16, (uint32_t)P::FI) : 0u;
#pragma unroll
    for (int s = 0; s < NS - 1; s++)
        if ((uint32_t)s < steps) fetch(s, s * KD);
    for (uint32_t s = 0; s < steps; s++) {
        // Stage s has landed once no more than the later stages' loads are
        // outstanding; the barrier also ends every wave's reads of the stage refilled next.
        pipe_wait_ahead<P::NA + P::NB, NS - 2>(min(steps - 1 - s, (uint32_t)NS - 2));
        if (s + NS - 1 < steps) fetch((s + NS - 1) % NS, (s + NS - 1) * KD);
        const char *sa = lds + (s % NS) * P::STAGE, *sb = sa + P::A_BYTES;
        // PICK mode: row fragments wholly past the matrix's last row (its partial last
        // tile) skip their MFMAs; their loads and the barriers stay, so every wave keeps
        // the same pipeline.
        auto step = [&](const bool all) {
#pragma unroll
            for (int ks = 0; ks < KD / 32; ks++) {
                const uint32_t chunk = ks * 4 + grp;
                bf16x8 af[P::FI], bfr[P::FJ];
#pragma unroll
                for (int i = 0; i < P::FI; i++)
                    if (all || (uint32_t)i < live_frags)
                        af[i] = as_bf16x8(*(const u32x4 *)(sa + P::at(wm * P::WM + i * 16 + col, chunk)));
#pragma unroll
                for (int j = 0; j < P::FJ; j++) bfr[j] = as_bf16x8(*(const u32x4 *)(sb + P::at(wn * P::WN + j * 16 + col, chunk)));
#pragma unroll
                for (int i = 0; i < P::FI; i++)
                    if (all || (uint32_t)i < live_frags)
#pragma unroll
                        for (int j = 0; j < P::FJ; j++) acc[i][j] = mfma16(bfr[j], af[i], acc[i][j]);
            }
        };
        if (!PICK || live_frags >= (uint32_t)P::FI) step(true);
        else step(false);
    }

    // Epilogue. acc[i][j] is the transposed 16x16 tile: lane (col, grp) holds tile row
    // wm WM + 16 i + col and columns wn WN + 16 j + 4 grp .. + 3 (SILU: gate in j < FJ/2,
    // up in j + FJ/2, output columns wn WN/2 + 16 j + 4 grp .. + 3).
    const uint32_t N = p.n;
    auto value = [&](int i, int j, int r) {
        const float g = acc[i][j][r];
        const float u = SILU ? acc[i][j + P::FJ / 2][r] : 0.0f;
        return SILU ? (p.pair_sum ? g + u : g / (1.0f + expf(-g)) * u) : g;
    };
    constexpr int JO = SILU ? P::FJ / 2 : P::FJ;
    constexpr uint32_t WO = SILU ? P::WN / 2 : P::WN;
    if (!PICK && p.out_bf16 && !(p.stages & TS_AFTER_ADD) && !p.after.count) {
        // bf16 rows through LDS: the tile as TM rows of OC bf16 (16-byte chunks
        // XOR-swizzled by row), then whole 16-byte chunks of rows to memory.
        constexpr uint32_t CH = OC / 8;  // chunks per output row
        static_assert(TM * OC * 2 <= P::LDS, "pipe epilogue fits the stages");
        // Chunk c of row r: XOR by the row when CH is a power of two, else rotated by
        // the row (an XOR could leave the row).
        auto slot = [](uint32_t r, uint32_t c) {
            return (CH & (CH - 1)) == 0 ? c ^ (r % CH) : (c + r) % CH;
        };
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
        for (int i = 0; i < P::FI; i++) {
            const uint32_t r = wm * P::WM + i * 16 + col;
#pragma unroll
            for (int j = 0; j < JO; j++) {
                const uint32_t c = wn * WO + j * 16 + 4 * grp;
                *(u32x2 *)(lds + r * OC * 2 + (slot(r, c >> 3) << 4) + (c & 7) * 2) =
                    u32x2{pack_bf16x2(value(i, j, 0), value(i, j, 1)), pack_bf16x2(value(i, j, 2), value(i, j, 3))};
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const bool rows16 = (N & 7) == 0;
#pragma unroll 4
        for (uint32_t f = threadIdx.x; f < TM * CH; f += kThreads) {
            const uint32_t r = f / CH, c = f % CH;
            const uint32_t m = m0 + r, n = n0 + c * 8;
            if (m >= p.m || n >= N) continue;
            const u32x4 v = *(const u32x4 *)(lds + r * OC * 2 + (slot(r, c) << 4));
            uint16_t *o = (uint16_t *)p.out + (size_t)m * N + n;
            if (rows16 && n + 8 <= N) {
                *(u32x4 *)o = v;
            } else {
                for (uint32_t e = 0; e < 8 && n + e < N; e++) o[e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
            }
        }
        return;
    }
    const bool vec = (N & 3) == 0;
    float val[P::FI][JO][4];
#pragma unroll
    for (int i = 0; i < P::FI; i++)
#pragma unroll
        for (int j = 0; j < JO; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) val[i][j][r] = value(i, j, r);
    if (CHAIN) {  // the chain's variant: its values and sums need more registers
        // Value e = (i JO + j) 4 + r: row fragment i, column fragment j, column 4 grp + r.
        auto row_of = [&](int e) {
            const uint32_t tr = wm * P::WM + (e / (4 * JO)) * 16 + col;
            return m0 + tr < mend ? (PICK ? row_out(tr) : m0 + tr) : ~0u;
        };
        auto col_of = [&](int e) { return n0 + wn * WO + (e / 4 % JO) * 16 + 4 * grp + e % 4; };
        ts::after_values<P::FI * JO * 4, false>(
            p.after, *(float(*)[P::FI * JO * 4])val, [&](int e) { return (size_t)row_of(e) * N + col_of(e); },
            [&](int e) { return row_of(e) != ~0u && col_of(e) < N; });
    }
#pragma unroll
    for (int i = 0; i < P::FI; i++) {
        const uint32_t tr = wm * P::WM + i * 16 + col;
        if (m0 + tr >= mend) continue;
        const uint32_t m = PICK ? row_out(tr) : m0 + tr;
#pragma unroll
        for (int j = 0; j < JO; j++) {
            const uint32_t n = n0 + wn * WO + j * 16 + 4 * grp;
            if (n >= N) continue;
            float *v = val[i][j];
            const size_t at = (size_t)m * N + n;
            if (vec && n + 3 < N) {
                if (p.stages & TS_AFTER_ADD) {
                    const float4 a = *(const float4 *)(p.a0 + at);
                    v[0] += a.x; v[1] += a.y; v[2] += a.z; v[3] += a.w;
                }
                if (p.out_bf16) *(u32x2 *)((uint16_t *)p.out + at) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
                else *(float4 *)((float *)p.out + at) = float4{v[0], v[1], v[2], v[3]};
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    if (n + r >= N) break;
                    float u = v[r];
                    if (p.stages & TS_AFTER_ADD) u += p.a0[at + r];
                    if (p.out_bf16) ((uint16_t *)p.out)[at + r] = bf16_bits(u);
                    else ((float *)p.out)[at + r] = u;
                }
            }
        }
    }
}

template <int TM, int TN, int KD, int NS, bool PICK>
int pipe_launch(TiledParams p, bool silu, void *stream) {
    constexpr int lds = Pipe<TM, TN, KD, NS>::LDS;
    const void *kerns[4] = {(const void *)tiled_pipe_kernel<TM, TN, KD, NS, false, PICK, false>,
                            (const void *)tiled_pipe_kernel<TM, TN, KD, NS, true, PICK, false>,
                            (const void *)tiled_pipe_kernel<TM, TN, KD, NS, false, PICK, true>,
                            (const void *)tiled_pipe_kernel<TM, TN, KD, NS, true, PICK, true>};
    // The dynamic LDS size is raised once per kernel (thread-safe static initialisation).
    static const hipError_t attr[4] = {
        hipFuncSetAttribute(kerns[0], hipFuncAttributeMaxDynamicSharedMemorySize, lds),
        hipFuncSetAttribute(kerns[1], hipFuncAttributeMaxDynamicSharedMemorySize, lds),
        hipFuncSetAttribute(kerns[2], hipFuncAttributeMaxDynamicSharedMemorySize, lds),
        hipFuncSetAttribute(kerns[3], hipFuncAttributeMaxDynamicSharedMemorySize, lds)};
    const int which = (silu ? 1 : 0) + (p.after.count ? 2 : 0);
    if (attr[which]) return ts::hip_status(attr[which], "tiled (pipelined): LDS attribute");
    const void *k = kerns[which];
    const uint32_t oc = silu ? TN / 2 : TN;
    const uint32_t gx = (p.n + oc - 1) / oc;
    dim3 grid;
    if (PICK) {
        // Row tiles: at most one partial tile per matrix beyond rows / TM full ones.
        const uint32_t gy = (p.m + TM - 1) / TM + p.matrices;
        // XCD-aware (C5 gate/up 1214 -> 1189 us, layer 2.48-2.53 -> 2.44 ms) where the
        // one-dimensional grid fits.
        if ((uint64_t)8 * gx * ((gy + 7) / 8) < (1ull << 31)) {
            p.pick_cols = gx;
            grid = dim3(8 * gx * ((gy + 7) / 8));
        } else {
            grid = dim3(gx, gy);
        }
    } else {
        // A one-dimensional grid of 8 x ceil(tiles / 8) groups; stride and offset,
        // unused outside picked products, carry the tile grid's width and height.
        const uint32_t gy = (p.m + TM - 1) / TM;
        p.stride = gx;
        p.offset = gy;
        grid = dim3(8 * (uint32_t)(((uint64_t)gx * gy + 7) / 8));
    }
    void *args[] = {(void *)&p};
    const hipError_t e = hipLaunchKernel(k, grid, dim3(kThreads), args, lds, (hipStream_t)stream);
    if (e != hipSuccess) return ts::hip_status(e, "tiled (pipelined): launch");
    return TS_OK;
}

// The pipelined kernels take bf16 operands, whole 64-deep k steps and element offsets
// of rows (x rows, and the rows of one weight matrix) that fit 32 bits.
bool pipe_fits(int x_dtype, int w_dtype, uint32_t x_rows, uint32_t k, uint32_t w_rows) {
    return x_dtype == TS_BF16 && w_dtype == TS_BF16 && k % 64 == 0 && (uint64_t)x_rows * k < (1ull << 32) &&
           (uint64_t)w_rows * k < (1ull << 32);
}

using Kern = void (*)(TiledParams);

template <int BT, bool XF32, bool W8, bool PICK>
Kern pick_silu(bool silu, bool chain) {
    if (chain) return silu ? tiled_kernel<BT, XF32, W8, true, PICK, true> : tiled_kernel<BT, XF32, W8, false, PICK, true>;
    return silu ? tiled_kernel<BT, XF32, W8, true, PICK, false> : tiled_kernel<BT, XF32, W8, false, PICK, false>;
}

template <int BT, bool PICK>
Kern pick_kernel(bool xf, bool w8, bool silu, bool chain) {
    return xf ? (w8 ? pick_silu<BT, true, true, PICK>(silu, chain) : pick_silu<BT, true, false, PICK>(silu, chain))
              : (w8 ? pick_silu<BT, false, true, PICK>(silu, chain) : pick_silu<BT, false, false, PICK>(silu, chain));
}

}  // namespace

extern "C" int tessera_hip_tiled(const ts_linear_args *a, void *stream) {
    if (a && ts::block_form(a->w_dtype)) return ts::block_tiled_launch(a, stream);
    TS_REQUIRE(a && a->x && a->w && a->out, "tiled: null pointer");
    TS_REQUIRE(a->m >= 1 && a->n >= 1 && a->k >= 1, "tiled: empty product m=%u n=%u k=%u", a->m, a->n, a->k);
    TS_REQUIRE(a->k % 8 == 0, "tiled: k=%u must be a multiple of 8", a->k);
    TS_REQUIRE(a->x_dtype == TS_F32 || a->x_dtype == TS_BF16, "tiled: x dtype %d", a->x_dtype);
    TS_REQUIRE(a->w_dtype == TS_BF16 || a->w_dtype == TS_E4M3 || a->w_dtype == TS_F32_PARTS,
               "tiled: w dtype %d (f32 weights: pack them with tessera_hip_pack_f32, TS_F32_PARTS)", a->w_dtype);
    TS_REQUIRE(a->w_dtype != TS_F32_PARTS || !(a->stages & TS_AFTER_SILU_MUL),
               "tiled: TS_F32_PARTS weights with TS_AFTER_SILU_MUL");
    TS_REQUIRE(a->out_dtype == TS_F32 || a->out_dtype == TS_BF16, "tiled: out dtype %d", a->out_dtype);
    TS_REQUIRE(a->w_dtype != TS_E4M3 || a->w_scale, "tiled: e4m3 weights need w_scale");
    TS_REQUIRE(!(a->stages & TS_AFTER_ADD) || a->a0, "tiled: TS_AFTER_ADD needs a0");
    TS_REQUIRE(!(a->stages & TS_BEFORE_RMS_NORM), "tiled: RmsNorm prologue is fused only for m <= 16");
    TS_REQUIRE((a->stages & ~(TS_AFTER_ADD | TS_AFTER_SILU_MUL)) == 0, "tiled: unknown stage bits %#x",
               a->stages);
    TS_REQUIRE(ts::aligned(a->x, 16) && ts::aligned(a->w, 16), "tiled: x and w must be 16-byte aligned");
    TiledParams p;
    p.pick_cols = 0;
    int rc = ts::linear_after(a, "tiled", &p.after);
    if (rc) return rc;
    const int big = ts::tiled_big_launch(a, stream);
    if (big != 1) return big;
    // f32 weights as two bf16 parts run as a pair of row blocks, summed at the store.
    const bool parts = a->w_dtype == TS_F32_PARTS;
    const bool silu = (a->stages & TS_AFTER_SILU_MUL) || parts;
    const int32_t w_dtype = parts ? TS_BF16 : a->w_dtype;
    p.pair_sum = parts;
    p.x = a->x; p.w = a->w; p.w_scale = (const uint16_t *)a->w_scale; p.a0 = a->a0; p.out = a->out;
    p.m = a->m; p.n = a->n; p.k = a->k; p.stages = a->stages; p.out_bf16 = a->out_dtype == TS_BF16;
    // 64x64 tiles when 128x128 would give fewer than 2 groups per CU: more groups to
    // hide each one's load/store latency chain (measured: MFMA time is not the limit).
    const uint64_t big_tiles = (uint64_t)((a->n + (silu ? BN / 2 : BN) - 1) / (silu ? BN / 2 : BN)) *
                               ((a->m + BM - 1) / BM);
    const int bt = big_tiles < 512 ? 64 : 128;
    const uint32_t cols = silu ? bt / 2 : bt;
    const uint32_t gx = (a->n + cols - 1) / cols, gy = (a->m + bt - 1) / bt;
    TS_REQUIRE(gy <= 65535, "tiled: m=%u too large for one launch", a->m);
    p.perm = p.row_start = p.tile_start = nullptr;
    p.matrices = 0; p.repeat = 1; p.stride = 0; p.offset = 0;
    if (pipe_fits(a->x_dtype, w_dtype, a->m, a->k, silu ? 2 * a->n : a->n)) {
        // 128 x 128 tiles from one tile per CU up (fewer, larger tiles read less per
        // flop), 64 x 64 below that (measured on the 2048-row projections: q with 256
        // tiles of 128 runs 1.15x faster than with 1024 of 64; o, kv and down with 128
        // tiles of 128 run 1.4-1.5x slower than with 512 of 64).
        const uint64_t oc = silu ? 64 : 128;
        const uint64_t tiles = (a->n + oc - 1) / oc * ((a->m + 127) / 128);
        // 128 x 192 when that fills the 512 group slots (two groups a CU) in fewer
        // rounds of equal work than 128 x 128 does (the C2 gate_up: 768 tiles of 128,
        // a round and a half, against 512 of 192).
        const uint64_t tiles192 = (a->n + oc * 3 / 2 - 1) / (oc * 3 / 2) * ((a->m + 127) / 128);
        const bool wide = ((tiles192 + 511) / 512) * 3 < ((tiles + 511) / 512) * 2;
        // A stage chain takes 64 x 64 tiles: at 128 x 128 its values and sums spill.
        if (tiles >= 256 && !p.after.count) {
            if (wide && TS_PIPE_WIDE) return pipe_launch<128, 192, 64, 2, false>(p, silu, stream);
            return pipe_launch<128, 128, 64, 2, false>(p, silu, stream);
        }
        return pipe_launch<64, 64, 64, 4, false>(p, silu, stream);
    }
    const bool chain = p.after.count;
    Kern k = bt == 64 ? pick_kernel<64, false>(a->x_dtype == TS_F32, w_dtype == TS_E4M3, silu, chain)
                      : pick_kernel<128, false>(a->x_dtype == TS_F32, w_dtype == TS_E4M3, silu, chain);
    hipLaunchKernelGGL(k, dim3(gx, gy), dim3(kThreads), 0, (hipStream_t)stream, p);
    TS_CHECK_LAUNCH("tiled launch");
    return TS_OK;
}

static int picked_check(const ts_picked_args *a) {
    TS_REQUIRE(a && a->x && a->w && a->ids && a->out, "picked: null pointer");
    TS_REQUIRE(a->n >= 1 && a->k >= 1, "picked: empty product n=%u k=%u", a->n, a->k);
    TS_REQUIRE(a->k % 8 == 0, "picked: k=%u must be a multiple of 8", a->k);
    TS_REQUIRE(a->count >= 1 && a->count <= 16384, "picked: count=%u (1..16384 matrices)", a->count);
    TS_REQUIRE(a->repeat >= 1, "picked: repeat 0");
    const uint32_t used = (a->stages & TS_AFTER_SILU_MUL) ? 2 * a->n : a->n;
    TS_REQUIRE((uint64_t)a->offset + used <= a->stride, "picked: rows %u..%u outside a matrix of %u rows", a->offset,
               a->offset + used, a->stride);
    TS_REQUIRE(a->x_dtype == TS_F32 || a->x_dtype == TS_BF16, "picked: x dtype %d", a->x_dtype);
    TS_REQUIRE(a->w_dtype == TS_BF16 || a->w_dtype == TS_E4M3, "picked: w dtype %d", a->w_dtype);
    TS_REQUIRE(a->out_dtype == TS_F32 || a->out_dtype == TS_BF16, "picked: out dtype %d", a->out_dtype);
    TS_REQUIRE(a->w_dtype != TS_E4M3 || a->w_scale, "picked: e4m3 weights need w_scale");
    TS_REQUIRE((a->stages & ~TS_AFTER_SILU_MUL) == 0, "picked: stage bits %#x (only TS_AFTER_SILU_MUL)", a->stages);
    TS_REQUIRE(ts::aligned(a->x, 16) && ts::aligned(a->w, 16), "picked: x and w must be 16-byte aligned");
    TS_REQUIRE((uint64_t)a->rows / BM + a->count <= 65535, "picked: %u rows and %u matrices in one launch", a->rows,
               a->count);
    ts_after c;
    return ts::after_check(a->after, true, "picked", &c);
}

extern "C" size_t tessera_hip_picked_workspace(const ts_picked_args *a) {
    if (!a) return 0;
    return ts::route_words(a->rows, a->count) * sizeof(uint32_t);
}

extern "C" int tessera_hip_picked(const ts_picked_args *a, void *stream) {
    const int bad = picked_check(a);
    if (bad) return bad;
    if (a->rows == 0) return TS_OK;
    const size_t need = tessera_hip_picked_workspace(a);
    if (!a->workspace || a->workspace_bytes < need)
        return ts::fail(TS_ERR_WORKSPACE, "picked: workspace %zu bytes, need %zu", a->workspace_bytes, need);
    TS_REQUIRE(ts::aligned(a->workspace, 4), "picked: workspace must be 4-byte aligned");
    ts::Route route;
    int rc = ts::route_launch(a->ids, a->rows, a->first, a->count, BM, a->workspace, &route, stream);
    if (rc) return rc;
    const bool silu = a->stages & TS_AFTER_SILU_MUL;
    TiledParams p;
    p.pick_cols = 0;
    p.pair_sum = 0;
    ts::after_check(a->after, true, "picked", &p.after);
    rc = ts::zero_absent_launch(route, a->count, a->out, a->n, a->out_dtype == TS_BF16, p.after, stream);
    if (rc) return rc;
    p.x = a->x; p.w = a->w; p.w_scale = (const uint16_t *)a->w_scale; p.a0 = nullptr; p.out = a->out;
    p.m = a->rows; p.n = a->n; p.k = a->k; p.stages = a->stages; p.out_bf16 = a->out_dtype == TS_BF16;
    p.perm = route.perm; p.row_start = route.row_start; p.tile_start = route.tile_start;
    p.matrices = a->count; p.repeat = a->repeat; p.stride = a->stride; p.offset = a->offset;
    const uint32_t cols = silu ? BN / 2 : BN;
    // Row tiles: at most one partial tile per matrix beyond rows / BM full ones.
    const uint32_t gx = (a->n + cols - 1) / cols, gy = (a->rows + BM - 1) / BM + a->count;
    // A stage chain takes the register-staged kernel (the pipelined one's chain variant spills).
    // 128 x 192 tiles where the columns divide evenly (fewer re-reads of the gathered
    // rows per weight byte: C5 gate/up 1249 -> 1202 us), else 128 x 128.
    if (pipe_fits(a->x_dtype, a->w_dtype, a->rows, a->k, a->stride) && !p.after.count) {
        if ((silu ? a->n % 96 : a->n % 192) == 0) return pipe_launch<128, 192, 64, 2, true>(p, silu, stream);
        return pipe_launch<128, 128, 64, 2, true>(p, silu, stream);
    }
    Kern k = pick_kernel<BM, true>(a->x_dtype == TS_F32, a->w_dtype == TS_E4M3, silu, p.after.count != 0);
    hipLaunchKernelGGL(k, dim3(gx, gy), dim3(kThreads), 0, (hipStream_t)stream, p);
    TS_CHECK_LAUNCH("picked launch");
    return TS_OK;
}

extern "C" size_t tessera_hip_linear_workspace(const ts_linear_args *a) {
    if (!a) return 0;
    return a->m <= 64 ? tessera_hip_lanes_workspace(a) : 0;
}

extern "C" int tessera_hip_linear(const ts_linear_args *a, void *stream) {
    TS_REQUIRE(a, "linear: null args");
    return a->m <= 64 ? tessera_hip_lanes(a, stream) : tessera_hip_tiled(a, stream);
}
