// "lanes": out[m, n] = after(sum_k x[m, k] w[n, k]) for m <= 64 rows.
// Rows 1..4 go to the vector-ALU kernel in gemv.hip; 5..64 run here.
//
// Replaces the reference's few-row matmul rules: lanes (a 32-lane group per
// column, engine/rules/linear/src/lanes.rs:17-143) and thin (a thread per
// column, thin.rs:11-104). Same product, same fused stages (map.rs:155-185).
//
// gfx950 design. Few-row products are HBM-bound: every weight byte is read once
// and the chip must be covered. A wave owns 16 output columns; a group of 4 waves
// (64 columns) shares each 128-deep chunk of x, staged once in LDS (double-
// buffered) as MFMA A fragments for up to 4 row tiles of 16. Each lane streams 64
// bytes of its column's weight row per chunk (16B vector loads; the 4 lanes of a row
// read contiguous runs), a ring of chunks ahead, and feeds them to
// v_mfma_f32_16x16x32_bf16 straight from registers (no LDS for the weights). The x
// fragments use the same k permutation, so the product is unchanged. When the
// column groups alone do not give ~512 groups, k is split across groups: raw sums
// go to the caller's workspace and a second kernel adds the splits in split order
// (deterministic) before the epilogue (a single launch whose last-arriving group adds
// a column tile's splits measured slower: that group's serial tail of atomic count,
// cache invalidate and partial reads outlasts the second launch). f32 activations are
// split into two exact bf16 parts (hi = bf16(x), lo = bf16(x - hi)), so f32 rows
// times bf16 weights stay close to the f32 oracle. e4m3 weights decode to bf16 in
// registers; the per-row scale multiplies the finished sum.
#include "after.h"

#include <algorithm>

namespace {

constexpr int kWaves = 4;
constexpr int kChunk = 128;  // k per chunk: 4 MFMA steps of 32

struct LanesParams {
    const void *x;
    const void *w;
    const uint16_t *w_scale;
    const float *gain;
    const float *a0;
    void *out;
    uint32_t m, n, k;
    uint32_t stages;
    float eps;
    int out_bf16;
    ts_after after;  // stage chain (count 0: none)
    int pair_sum;    // TS_F32_PARTS: rows n.. are the low parts; the output sums the pair
};

// Raw weight bytes of one lane (row `row`, lane group g) for the 128-deep chunk at
// k0, laid out so the 4 lanes of a row read contiguous runs: bf16 b[j] = k [32j + 8g,
// +8) (each load instruction covers 64 contiguous bytes per row); e4m3 b[h] = k [64h +
// 16g, +16) (h = 0, 1). Decoded at use by w_frag, so the loads stay in flight.
// `full` (uniform per chunk): the chunk lies inside K and rows are 16-byte aligned;
// otherwise element loads zero-fill past K.
template <bool W8>
TS_DEV void load_w(const void *w, uint32_t row, uint32_t k0, uint32_t g, uint32_t K, bool full, u32x4 (&b)[4]) {
    if (!W8) {
        const uint16_t *p = (const uint16_t *)w + (size_t)row * K;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t k = k0 + 32 * j + 8 * g;
            if (full) {
                b[j] = __builtin_nontemporal_load((const u32x4 *)(p + k));
            } else {
                uint32_t v[4];
#pragma unroll
                for (int e = 0; e < 4; e++)
                    v[e] = (k + 2 * e < K ? (uint32_t)p[k + 2 * e] : 0u) | ((k + 2 * e + 1 < K ? (uint32_t)p[k + 2 * e + 1] : 0u) << 16);
                b[j] = u32x4{v[0], v[1], v[2], v[3]};
            }
        }
    } else {
        const uint8_t *p = (const uint8_t *)w + (size_t)row * K;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t k = k0 + 64 * h + 16 * g;
            if (full) {
                b[h] = __builtin_nontemporal_load((const u32x4 *)(p + k));
            } else {
                uint32_t c[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    uint32_t v = 0;
#pragma unroll
                    for (int e = 0; e < 4; e++) v |= (k + 4 * i + e < K ? (uint32_t)p[k + 4 * i + e] : 0u) << (8 * e);
                    c[i] = v;
                }
                b[h] = u32x4{c[0], c[1], c[2], c[3]};
            }
        }
    }
}

// MFMA B fragment j of a raw chunk: 8 k values of this lane.
template <bool W8>
TS_DEV bf16x8 w_frag(const u32x4 (&b)[4], int j) {
    if (!W8) return as_bf16x8(b[j]);
    const u32x4 q = b[j >> 1];
    const uint32_t lo = (j & 1) ? q.z : q.x, hi = (j & 1) ? q.w : q.y;
    const u32x2 a = e4m3x4_to_bf16x4(lo), d = e4m3x4_to_bf16x4(hi);
    return as_bf16x8(u32x4{a.x, a.y, d.x, d.y});
}

// The 16-byte piece (8 k values) of an x row chunk that pairs with w_frag j of lane
// group g: bf16 weights k [32j + 8g, +8); e4m3 k [64 (j/2) + 16g + 8 (j%2), +8).
template <bool W8>
TS_DEV uint32_t x_piece(int j, uint32_t g) {
    return W8 ? 8 * (j >> 1) + 2 * g + (j & 1) : 4 * j + g;
}

TS_DEV float silu(float v) { return v / (1.0f + expf(-v)); }

// The split sums leave the kernel as agent-scope (write-through) stores: lanes_finish
// reads them from memory anyway, and lines left dirty in the XCDs' L2s cost a write-
// back at the kernel's end (plain stores measured 15.1 against 12.9 us on 4096 x 4096
// e4m3 at m 64).
TS_DEV void put_part(float *p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// One 128-deep chunk of x rows [0, M) in flight: thread t holds pieces i = t + 256 j
// (piece = 8 k values of one row; 16 pieces per row). Loaded early into registers,
// written to LDS later (store_x), so the load latency hides under the MFMAs.
template <int MT, bool XF32>
struct XRegs {
    static constexpr uint32_t kPieces = 16 * MT * (kChunk / 8), kPer = kPieces / (kWaves * 64);
    float4 f[XF32 ? 2 * kPer : 1];
    u32x4 b[XF32 ? 1 : kPer];
};

// Rows past M repeat row M - 1 (their products are never stored). `full` (uniform):
// the chunk lies inside K and rows are 16-byte aligned.
template <int MT, bool XF32>
TS_DEV void load_x(const LanesParams &p, uint32_t k0, bool full, XRegs<MT, XF32> &r) {
    const uint32_t M = p.m, K = p.k;
#pragma unroll
    for (uint32_t j = 0; j < XRegs<MT, XF32>::kPer; j++) {
        const uint32_t i = threadIdx.x + j * kWaves * 64, k = k0 + 8 * (i % (kChunk / 8));
        const uint32_t m = min(i / (kChunk / 8), M - 1);
        if (XF32) {
            if (full) {
                const float4 *q = (const float4 *)((const float *)p.x + (size_t)m * K + k);
                r.f[2 * j] = q[0];
                r.f[2 * j + 1] = q[1];
            } else {
                float v[8];
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = k + e < K ? ((const float *)p.x)[(size_t)m * K + k + e] : 0.0f;
                r.f[2 * j] = float4{v[0], v[1], v[2], v[3]};
                r.f[2 * j + 1] = float4{v[4], v[5], v[6], v[7]};
            }
        } else {
            u32x4 v;
            if (full) {
                v = *(const u32x4 *)((const uint16_t *)p.x + (size_t)m * K + k);
            } else {
                uint32_t w[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const uint16_t *q = (const uint16_t *)p.x + (size_t)m * K + k + 2 * e;
                    w[e] = (k + 2 * e < K ? (uint32_t)q[0] : 0u) | ((k + 2 * e + 1 < K ? (uint32_t)q[1] : 0u) << 16);
                }
                v = u32x4{w[0], w[1], w[2], w[3]};
            }
            r.b[j] = v;
        }
    }
}

// The chunk into LDS as bf16 (hi, and lo for f32 rows: hi = bf16(x), lo = bf16(x -
// hi)), rows of 256 bytes with 16-byte pieces XOR-swizzled by row. NORM scales f32
// rows by inv[m] * gain[k].
template <int MT, bool XF32, bool NORM>
TS_DEV void store_x(const LanesParams &p, const float *inv, uint32_t k0, const XRegs<MT, XF32> &r, char *hi,
                    char *lo) {
#pragma unroll
    for (uint32_t j = 0; j < XRegs<MT, XF32>::kPer; j++) {
        const uint32_t i = threadIdx.x + j * kWaves * 64, m = i / (kChunk / 8), c = i % (kChunk / 8);
        const uint32_t at = m * 256 + ((c ^ (m & 15)) << 4);
        if (XF32) {
            const float4 u0 = r.f[2 * j], u1 = r.f[2 * j + 1];
            float v[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
            if (NORM && m < p.m) {
                const uint32_t k = k0 + 8 * c;
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] *= inv[m] * (k + e < p.k ? p.gain[k + e] : 0.0f);
            }
            uint32_t h[4], l[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float a = v[2 * e], b = v[2 * e + 1], ha = bf16_round(a), hb = bf16_round(b);
                h[e] = pack_bf16x2(ha, hb);
                l[e] = pack_bf16x2(a - ha, b - hb);
            }
            *(u32x4 *)(hi + at) = u32x4{h[0], h[1], h[2], h[3]};
            *(u32x4 *)(lo + at) = u32x4{l[0], l[1], l[2], l[3]};
        } else {
            *(u32x4 *)(hi + at) = r.b[j];
        }
    }
}

// Few rows (m <= 64): wave w of group (tile group gx, split s) owns output columns
// [16 (4 gx + w), +16) over the chunks of split s. Each 128-deep chunk of x is staged
// in LDS once per group (double-buffered; its global loads are issued a chunk early)
// and read as MFMA A fragments. Each lane streams 64 bytes of its column's weight row
// per chunk (the 4 lanes of a row read contiguous runs, see load_w) into a register
// ring D chunks deep, so D chunks of weights are in flight per wave. splits == 1: the epilogue runs here;
// otherwise the raw sums go to part[s][SILU ? 2 : 1][m][n] for lanes_finish.
template <int MT, bool XF32, bool W8, bool SILU, bool NORM, bool CHAIN>
__global__ __launch_bounds__(kWaves * 64) void lanes_kernel(LanesParams p, float *part) {
    constexpr int D = (SILU && !W8) ? 2 : 4;     // weight chunks in flight per wave
    constexpr uint32_t kXBytes = 16 * MT * 256;  // one chunk of x rows, bf16
    __shared__ __attribute__((aligned(16))) char xs[2][XF32 ? 2 : 1][kXBytes];
    __shared__ float inv_s[16 * MT];
    __shared__ float part_s[kWaves][16 * MT];

    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t col = lane & 15, grp = lane >> 4;
    const uint32_t n0 = (blockIdx.x * kWaves + wave) * 16, M = p.m, N = p.n, K = p.k;
    const uint32_t split = blockIdx.y, splits = gridDim.y;

    const uint32_t chunks = (K + kChunk - 1) / kChunk;
    const uint32_t cb = (uint32_t)(((uint64_t)chunks * split) / splits);
    const uint32_t ce = (uint32_t)(((uint64_t)chunks * (split + 1)) / splits);

    // Columns past N read row N - 1 (never stored). A chunk is `full` when it lies
    // inside K and rows are 16-byte aligned (uniform: no per-lane branches).
    const uint32_t wrow = min(n0 + col, N - 1);
    const bool w_aligned = W8 ? (K % 16) == 0 : (K % 8) == 0, x_aligned = XF32 ? (K % 4) == 0 : (K % 8) == 0;
    auto w_full = [&](uint32_t c) { return w_aligned && (c + 1) * kChunk <= K; };
    auto x_full = [&](uint32_t c) { return x_aligned && (c + 1) * kChunk <= K; };

    // Weights first: they are the HBM stream.
    u32x4 wg[D][4], wu[D][4];
#pragma unroll
    for (int d = 0; d < D; d++)
        if (cb + d < ce) {
            load_w<W8>(p.w, wrow, (cb + d) * kChunk, grp, K, w_full(cb + d), wg[d]);
            if (SILU) load_w<W8>(p.w, N + wrow, (cb + d) * kChunk, grp, K, w_full(cb + d), wu[d]);
        }
    XRegs<MT, XF32> xr;
    if (cb < ce) load_x<MT, XF32>(p, cb * kChunk, x_full(cb), xr);

    // Fused RmsNorm prologue (f32 rows): every group computes the same inverse roots
    // in the same order, so all groups agree bit for bit.
    if (NORM) {
        for (uint32_t m = 0; m < M; m++) {
            const float *xrow = (const float *)p.x + (size_t)m * K;
            float s = 0.0f;
            for (uint32_t i = threadIdx.x; i < K; i += blockDim.x) s += xrow[i] * xrow[i];
            s = wave_sum(s);
            if (lane == 0) part_s[wave][m] = s;
        }
        __syncthreads();
        if (threadIdx.x < M) {
            float s = 0.0f;
            for (int w = 0; w < kWaves; w++) s += part_s[w][threadIdx.x];
            inv_s[threadIdx.x] = 1.0f / sqrtf(s / (float)K + p.eps);
        }
        __syncthreads();
    }

    f32x4 acc_g[MT], acc_u[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc_g[t] = acc_u[t] = f32x4{0, 0, 0, 0};
    for (uint32_t c = cb; c < ce; c += D) {
#pragma unroll
        for (int u = 0; u < D; u++) {
            const uint32_t cc = c + u;
            if (cc >= ce) break;
            char *xh = xs[cc & 1][0], *xl = xs[cc & 1][XF32 ? 1 : 0];
            // Buffer cc & 1 was last read before the previous barrier.
            store_x<MT, XF32, NORM>(p, inv_s, cc * kChunk, xr, xh, xl);
            if (cc + 1 < ce) load_x<MT, XF32>(p, (cc + 1) * kChunk, x_full(cc + 1), xr);
            lds_barrier();  // x of chunk cc is in LDS; the weight ring stays in flight
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t xc = x_piece<W8>(j, grp);
#pragma unroll
                for (int t = 0; t < MT; t++) {
                    const uint32_t m = 16 * t + col;
                    const bf16x8 ah = as_bf16x8(*(const u32x4 *)(xh + m * 256 + ((xc ^ (m & 15)) << 4)));
                    acc_g[t] = mfma16(ah, w_frag<W8>(wg[u], j), acc_g[t]);
                    if (SILU) acc_u[t] = mfma16(ah, w_frag<W8>(wu[u], j), acc_u[t]);
                    if (XF32) {
                        const bf16x8 al = as_bf16x8(*(const u32x4 *)(xl + m * 256 + ((xc ^ (m & 15)) << 4)));
                        acc_g[t] = mfma16(al, w_frag<W8>(wg[u], j), acc_g[t]);
                        if (SILU) acc_u[t] = mfma16(al, w_frag<W8>(wu[u], j), acc_u[t]);
                    }
                }
            }
            if (cc + D < ce) {  // refill this ring slot D chunks ahead
                load_w<W8>(p.w, wrow, (cc + D) * kChunk, grp, K, w_full(cc + D), wg[u]);
                if (SILU) load_w<W8>(p.w, N + wrow, (cc + D) * kChunk, grp, K, w_full(cc + D), wu[u]);
            }
        }
    }

    // D lane layout: column col, rows 4 grp + r of each 16-row tile.
    const uint32_t n = n0 + col;
    if (n >= N) return;
    if (splits > 1) {
        float *dst = part + (size_t)split * (SILU ? 2 : 1) * M * N;
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t m = 16 * t + 4 * grp + r;
                if (m >= M) continue;
                put_part(dst + (size_t)m * N + n, acc_g[t][r]);
                if (SILU) put_part(dst + (size_t)M * N + (size_t)m * N + n, acc_u[t][r]);
            }
        return;
    }
    float val[MT * 4];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float g = acc_g[t][r], u = acc_u[t][r];
            if (W8) {
                g *= bf16_float(p.w_scale[n]);
                if (SILU) u *= bf16_float(p.w_scale[N + n]);
            }
            val[4 * t + r] = SILU ? (p.pair_sum ? g + u : silu(g) * u) : g;
        }
    // Value e: row 16 (e / 4) + 4 grp + e % 4.
    auto row_of = [&](int e) { return 16 * (uint32_t)(e / 4) + 4 * grp + (uint32_t)(e % 4); };
    if (CHAIN)  // the chain's variant: its values and sums need more registers
        ts::after_values<MT * 4, false>(p.after, val, [&](int e) { return (size_t)row_of(e) * N + n; },
                                        [&](int e) { return row_of(e) < M; });
#pragma unroll
    for (int e = 0; e < MT * 4; e++) {
        const uint32_t m = row_of(e);
        if (m >= M) continue;
        float v = val[e];
        if (p.stages & TS_AFTER_ADD) v += p.a0[(size_t)m * N + n];
        if (p.out_bf16) ((uint16_t *)p.out)[(size_t)m * N + n] = bf16_bits(v);
        else ((float *)p.out)[(size_t)m * N + n] = v;
    }
}

// Sums the splits' partials in split order, then the epilogue.
template <bool W8, bool SILU>
__global__ __launch_bounds__(256) void lanes_finish(LanesParams p, const float *part, uint32_t splits) {
    const uint64_t i = blockIdx.x * 256ull + threadIdx.x, MN = (uint64_t)p.m * p.n;
    if (i >= MN) return;
    const uint32_t n = (uint32_t)(i % p.n), N = p.n;
    // Eight splits' loads in flight at a time, added in split order (the same sums
    // as one split at a time).
    constexpr uint32_t kB = 8;
    const size_t stride = (size_t)(SILU ? 2 : 1) * MN;
    float g = 0.0f, u = 0.0f;
    for (uint32_t s0 = 0; s0 < splits; s0 += kB) {
        float tg[kB], tu[kB];
#pragma unroll
        for (uint32_t j = 0; j < kB; j++) {
            const uint32_t s = min(s0 + j, splits - 1);  // clamped: read but not added
            tg[j] = part[s * stride + i];
            if (SILU) tu[j] = part[s * stride + MN + i];
        }
#pragma unroll
        for (uint32_t j = 0; j < kB; j++)
            if (s0 + j < splits) {
                g += tg[j];
                if (SILU) u += tu[j];
            }
    }
    if (W8) {
        g *= bf16_float(p.w_scale[n]);
        if (SILU) u *= bf16_float(p.w_scale[N + n]);
    }
    float v = SILU ? (p.pair_sum ? g + u : silu(g) * u) : g;
    if (p.stages & TS_AFTER_ADD) v += p.a0[i];
    if (p.after.count) v = ts::after_apply(p.after, v, i);
    if (p.out_bf16) ((uint16_t *)p.out)[i] = bf16_bits(v);
    else ((float *)p.out)[i] = v;
}

struct Plan {
    uint32_t groups, splits;
};

// Enough groups to cover the chip (~512): the column groups, times a k split when
// they are fewer. Each split keeps at least two 128-deep chunks: one-chunk splits
// measured slower (4096 x 1024 e4m3 at m 8: 7.0 us against 5.9 us with two).
Plan plan(const ts_linear_args *a) {
    Plan pl;
    const uint32_t tiles = (a->n + 15) / 16, chunks = (a->k + kChunk - 1) / kChunk;
    pl.groups = (tiles + kWaves - 1) / kWaves;
    pl.splits = std::max(1u, std::min(chunks / 2, (512u + pl.groups - 1) / pl.groups));
    return pl;
}

using Kern = void (*)(LanesParams, float *);

template <int MT, bool XF32, bool W8, bool CHAIN>
Kern pick4(bool silu, bool norm) {
    if (silu) return norm ? lanes_kernel<MT, XF32, W8, true, true, CHAIN> : lanes_kernel<MT, XF32, W8, true, false, CHAIN>;
    return norm ? lanes_kernel<MT, XF32, W8, false, true, CHAIN> : lanes_kernel<MT, XF32, W8, false, false, CHAIN>;
}

template <int MT, bool XF32, bool W8>
Kern pick3(bool silu, bool norm, bool chain) {
    return chain ? pick4<MT, XF32, W8, true>(silu, norm) : pick4<MT, XF32, W8, false>(silu, norm);
}

template <int MT>
Kern pick2(bool xf, bool w8, bool silu, bool norm, bool chain) {
    return xf ? (w8 ? pick3<MT, true, true>(silu, norm, chain) : pick3<MT, true, false>(silu, norm, chain))
              : (w8 ? pick3<MT, false, true>(silu, norm, chain) : pick3<MT, false, false>(silu, norm, chain));
}

int check(const ts_linear_args *a) {
    TS_REQUIRE(a && a->x && a->w && a->out, "lanes: null pointer");
    TS_REQUIRE(a->m >= 1 && a->m <= 64, "lanes: m=%u outside 1..64", a->m);
    TS_REQUIRE(a->n >= 1 && a->k >= 1, "lanes: empty product n=%u k=%u", a->n, a->k);
    TS_REQUIRE(a->x_dtype == TS_F32 || a->x_dtype == TS_BF16, "lanes: x dtype %d", a->x_dtype);
    TS_REQUIRE(a->w_dtype == TS_BF16 || a->w_dtype == TS_E4M3 || a->w_dtype == TS_F32_PARTS,
               "lanes: w dtype %d (f32 weights: pack them with tessera_hip_pack_f32, TS_F32_PARTS)", a->w_dtype);
    TS_REQUIRE(a->w_dtype != TS_F32_PARTS || !(a->stages & TS_AFTER_SILU_MUL),
               "lanes: TS_F32_PARTS weights with TS_AFTER_SILU_MUL");
    TS_REQUIRE(a->out_dtype == TS_F32 || a->out_dtype == TS_BF16, "lanes: out dtype %d", a->out_dtype);
    TS_REQUIRE(a->w_dtype != TS_E4M3 || a->w_scale, "lanes: e4m3 weights need w_scale");
    TS_REQUIRE(!(a->stages & TS_AFTER_ADD) || a->a0, "lanes: TS_AFTER_ADD needs a0");
    TS_REQUIRE(!(a->stages & TS_BEFORE_RMS_NORM) || (a->gain && a->x_dtype == TS_F32 && a->m <= 16),
               "lanes: TS_BEFORE_RMS_NORM needs gain, f32 x and m <= 16");
    TS_REQUIRE((a->stages & ~(TS_AFTER_ADD | TS_AFTER_SILU_MUL | TS_BEFORE_RMS_NORM | TS_AFTER_ARGMAX)) == 0,
               "lanes: unknown stage bits %#x", a->stages);
    TS_REQUIRE(ts::aligned(a->x, 16) && ts::aligned(a->w, 16), "lanes: x and w must be 16-byte aligned");
    if (a->stages & TS_AFTER_ARGMAX) {
        TS_REQUIRE(a->m <= 4 && a->out_dtype == TS_F32 && !(a->stages & TS_AFTER_SILU_MUL),
                   "lanes: TS_AFTER_ARGMAX needs m <= 4, f32 out and no SiLU pair");
        if (!a->workspace || a->workspace_bytes < (size_t)a->m * 8 || !ts::aligned(a->workspace, 8))
            return ts::fail(TS_ERR_WORKSPACE, "lanes: TS_AFTER_ARGMAX needs %u 8-byte-aligned keys", a->m);
    }
    return TS_OK;
}

}  // namespace

extern "C" size_t tessera_hip_lanes_workspace(const ts_linear_args *a) {
    if (a && (a->stages & TS_AFTER_ARGMAX)) return (size_t)a->m * 8;  // the keys
    if (!a || a->m <= 4 || a->m > 64 || ts::block_form(a->w_dtype)) return 0;
    const Plan pl = plan(a);
    if (pl.splits <= 1) return 0;
    const size_t per = (size_t)a->m * a->n * ((a->stages & TS_AFTER_SILU_MUL) || a->w_dtype == TS_F32_PARTS ? 2 : 1);
    return (size_t)pl.splits * per * sizeof(float);
}

extern "C" int tessera_hip_lanes(const ts_linear_args *a, void *stream) {
    if (a && ts::block_form(a->w_dtype))
        return a->m <= 4 ? ts::block_gemv_launch(a, stream) : ts::block_tiled_launch(a, stream);
    int rc = check(a);
    if (rc) return rc;
    if (a->m <= 4) {
        ts_after c;
        rc = ts::linear_after(a, "lanes", &c);
        return rc ? rc : ts::gemv_launch(a, stream);
    }
    const Plan pl = plan(a);
    const size_t need = tessera_hip_lanes_workspace(a);
    if (need && (!a->workspace || a->workspace_bytes < need))
        return ts::fail(TS_ERR_WORKSPACE, "lanes: workspace %zu bytes, need %zu", a->workspace_bytes, need);
    LanesParams p;
    p.x = a->x; p.w = a->w; p.w_scale = (const uint16_t *)a->w_scale; p.gain = a->gain; p.a0 = a->a0;
    p.out = a->out; p.m = a->m; p.n = a->n; p.k = a->k; p.stages = a->stages; p.eps = a->eps;
    p.out_bf16 = a->out_dtype == TS_BF16;
    rc = ts::linear_after(a, "lanes", &p.after);
    if (rc) return rc;
    const bool parts = a->w_dtype == TS_F32_PARTS;
    const bool silu = (a->stages & TS_AFTER_SILU_MUL) || parts, norm = a->stages & TS_BEFORE_RMS_NORM;
    p.pair_sum = parts;
    const bool xf = a->x_dtype == TS_F32, w8 = a->w_dtype == TS_E4M3;
    const uint32_t mt = (a->m + 15) / 16;
    const bool chain = p.after.count;
    Kern k = mt == 1 ? pick2<1>(xf, w8, silu, norm, chain)
           : mt == 2 ? pick2<2>(xf, w8, silu, norm, chain)
           : mt == 3 ? pick2<3>(xf, w8, silu, norm, chain) : pick2<4>(xf, w8, silu, norm, chain);
    float *part = need ? (float *)a->workspace : nullptr;
    hipLaunchKernelGGL(k, dim3(pl.groups, pl.splits), dim3(kWaves * 64), 0, (hipStream_t)stream, p, part);
    TS_CHECK_LAUNCH("lanes launch");
    if (pl.splits > 1) {
        const uint64_t mn = (uint64_t)a->m * a->n;
        auto fin = w8 ? (silu ? lanes_finish<true, true> : lanes_finish<true, false>)
                      : (silu ? lanes_finish<false, true> : lanes_finish<false, false>);
        hipLaunchKernelGGL(fin, dim3((uint32_t)((mn + 255) / 256)), dim3(256), 0, (hipStream_t)stream, p,
                           (const float *)part, pl.splits);
        TS_CHECK_LAUNCH("lanes finish");
    }
    return TS_OK;
}
