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
// contiguous bytes of its column's weight row per chunk (16B vector loads; lane
// group g holds k [32g, 32g+32)), fetched one chunk ahead, and feeds them to
// v_mfma_f32_16x16x32_bf16 straight from registers (no LDS for the weights). The x
// fragments use the same k assignment, so the product is unchanged. When the
// column groups alone do not give ~512 groups, k is split across groups: raw sums
// go to the caller's workspace and a second kernel adds the splits in split order
// (deterministic) before the epilogue. f32 activations are split into two exact
// bf16 parts (hi = bf16(x), lo = bf16(x - hi)), so f32 rows times bf16 weights stay
// close to the f32 oracle. e4m3 weights decode to bf16 in registers; the per-row
// scale multiplies the finished sum.
#include "common.h"

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
};

// Weight chunk for one lane: 32 consecutive k of one row as bf16 (4 x 16B).
template <bool W8>
TS_DEV void load_w(const void *w, uint32_t row, uint32_t nrows, uint32_t k0, uint32_t K, u32x4 (&b)[4]) {
    if (row >= nrows) {
#pragma unroll
        for (int j = 0; j < 4; j++) b[j] = u32x4{0, 0, 0, 0};
        return;
    }
    if (!W8) {
        const uint16_t *p = (const uint16_t *)w + (size_t)row * K + k0;
        if (k0 + 32 <= K && (K % 8) == 0) {
            const u32x4 *q = (const u32x4 *)p;
#pragma unroll
            for (int j = 0; j < 4; j++) b[j] = __builtin_nontemporal_load(q + j);
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                uint32_t v[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    uint32_t ka = k0 + 8 * j + 2 * e;
                    uint32_t lo = ka < K ? p[8 * j + 2 * e] : 0u;
                    uint32_t hi = ka + 1 < K ? p[8 * j + 2 * e + 1] : 0u;
                    v[e] = lo | (hi << 16);
                }
                b[j] = u32x4{v[0], v[1], v[2], v[3]};
            }
        }
    } else {
        const uint8_t *p = (const uint8_t *)w + (size_t)row * K + k0;
        uint32_t c[8];
        if (k0 + 32 <= K && (K % 16) == 0) {
            const u32x4 *q = (const u32x4 *)p;
            u32x4 c0 = __builtin_nontemporal_load(q), c1 = __builtin_nontemporal_load(q + 1);
            c[0] = c0.x; c[1] = c0.y; c[2] = c0.z; c[3] = c0.w;
            c[4] = c1.x; c[5] = c1.y; c[6] = c1.z; c[7] = c1.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                uint32_t v = 0;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    uint32_t ka = k0 + 4 * i + e;
                    v |= (ka < K ? (uint32_t)p[4 * i + e] : 0u) << (8 * e);
                }
                c[i] = v;
            }
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            u32x2 a = e4m3x4_to_bf16x4(c[2 * j]), d = e4m3x4_to_bf16x4(c[2 * j + 1]);
            b[j] = u32x4{a.x, a.y, d.x, d.y};
        }
    }
}

TS_DEV float silu(float v) { return v / (1.0f + expf(-v)); }

// One 128-deep chunk of x rows [0, M) into LDS as bf16 (hi, and lo for f32 rows:
// hi = bf16(x), lo = bf16(x - hi)), rows of 256 bytes with 16-byte chunks XOR-swizzled
// by row. Rows >= M and k >= K are zero. NORM scales f32 rows by inv[m] * gain[k].
template <int MT, bool XF32, bool NORM>
TS_DEV void stage_x(const LanesParams &p, const float *inv, uint32_t k0, char *hi, char *lo) {
    constexpr uint32_t kRows = 16 * MT, kPieces = kRows * (kChunk / 8);  // 8 k values per piece
    const uint32_t M = p.m, K = p.k;
    for (uint32_t i = threadIdx.x; i < kPieces; i += kWaves * 64) {
        const uint32_t m = i / (kChunk / 8), c = i % (kChunk / 8), k = k0 + 8 * c;
        const uint32_t at = m * 256 + ((c ^ (m & 15)) << 4);
        if (XF32) {
            float v[8];
            if (m < M && k + 8 <= K) {
                const float4 *q = (const float4 *)((const float *)p.x + (size_t)m * K + k);
                const float4 u0 = q[0], u1 = q[1];
                v[0] = u0.x; v[1] = u0.y; v[2] = u0.z; v[3] = u0.w; v[4] = u1.x; v[5] = u1.y; v[6] = u1.z; v[7] = u1.w;
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = (m < M && k + e < K) ? ((const float *)p.x)[(size_t)m * K + k + e] : 0.0f;
            }
            if (NORM && m < M) {
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] *= inv[m] * (k + e < K ? p.gain[k + e] : 0.0f);
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
            u32x4 v = {0, 0, 0, 0};
            if (m < M && k + 8 <= K) {
                v = *(const u32x4 *)((const uint16_t *)p.x + (size_t)m * K + k);
            } else if (m < M) {
                uint32_t w[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const uint16_t *q = (const uint16_t *)p.x + (size_t)m * K + k + 2 * e;
                    w[e] = (k + 2 * e < K ? (uint32_t)q[0] : 0u) | ((k + 2 * e + 1 < K ? (uint32_t)q[1] : 0u) << 16);
                }
                v = u32x4{w[0], w[1], w[2], w[3]};
            }
            *(u32x4 *)(hi + at) = v;
        }
    }
}

// Few rows (m <= 64): wave w of group (tile group gx, split s) owns output columns
// [16 (4 gx + w), +16) over the chunks of split s. Each 128-deep chunk of x is staged
// in LDS once per group (double-buffered) and read as MFMA A fragments; each lane
// streams 64 bytes of its column's weight row per chunk (lane group g: k [32g, 32g +
// 32)), fetched one chunk ahead. splits == 1: the epilogue runs here; otherwise the
// raw sums go to part[s][SILU ? 2 : 1][m][n] for lanes_finish.
template <int MT, bool XF32, bool W8, bool SILU, bool NORM>
__global__ __launch_bounds__(kWaves * 64) void lanes_kernel(LanesParams p, float *part) {
    constexpr uint32_t kXBytes = 16 * MT * 256;  // one chunk of x rows, bf16
    __shared__ __attribute__((aligned(16))) char xs[2][XF32 ? 2 : 1][kXBytes];
    __shared__ float inv_s[16 * MT];
    __shared__ float part_s[kWaves][16 * MT];

    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t col = lane & 15, grp = lane >> 4;
    const uint32_t n0 = (blockIdx.x * kWaves + wave) * 16, M = p.m, N = p.n, K = p.k;
    const uint32_t split = blockIdx.y, splits = gridDim.y;

    // Fused RmsNorm prologue (f32 rows): every group computes the same inverse roots
    // in the same order, so all groups agree bit for bit.
    if (NORM) {
        for (uint32_t m = 0; m < M; m++) {
            const float *xr = (const float *)p.x + (size_t)m * K;
            float s = 0.0f;
            for (uint32_t i = threadIdx.x; i < K; i += blockDim.x) s += xr[i] * xr[i];
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

    const uint32_t chunks = (K + kChunk - 1) / kChunk;
    const uint32_t cb = (uint32_t)(((uint64_t)chunks * split) / splits);
    const uint32_t ce = (uint32_t)(((uint64_t)chunks * (split + 1)) / splits);

    f32x4 acc_g[MT], acc_u[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc_g[t] = acc_u[t] = f32x4{0, 0, 0, 0};
    u32x4 bg[4], bu[4];
    if (cb < ce) {
        stage_x<MT, XF32, NORM>(p, inv_s, cb * kChunk, xs[0][0], xs[0][XF32 ? 1 : 0]);
        load_w<W8>(p.w, n0 + col, N, cb * kChunk + 32 * grp, K, bg);
        if (SILU) load_w<W8>(p.w, N + n0 + col, 2 * N, cb * kChunk + 32 * grp, K, bu);
    }
    __syncthreads();
    for (uint32_t c = cb; c < ce; c++) {
        const uint32_t cur = (c - cb) & 1;
        u32x4 ng[4], nu[4];
        if (c + 1 < ce) {  // next chunk: weights into registers, x into the other buffer
            load_w<W8>(p.w, n0 + col, N, (c + 1) * kChunk + 32 * grp, K, ng);
            if (SILU) load_w<W8>(p.w, N + n0 + col, 2 * N, (c + 1) * kChunk + 32 * grp, K, nu);
            stage_x<MT, XF32, NORM>(p, inv_s, (c + 1) * kChunk, xs[cur ^ 1][0], xs[cur ^ 1][XF32 ? 1 : 0]);
        }
        const char *xh = xs[cur][0], *xl = xs[cur][XF32 ? 1 : 0];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t xc = 4 * grp + j;  // 16-byte piece of the chunk: k 32 grp + 8 j
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const uint32_t m = 16 * t + col;
                const bf16x8 ah = as_bf16x8(*(const u32x4 *)(xh + m * 256 + ((xc ^ (m & 15)) << 4)));
                acc_g[t] = mfma16(ah, as_bf16x8(bg[j]), acc_g[t]);
                if (SILU) acc_u[t] = mfma16(ah, as_bf16x8(bu[j]), acc_u[t]);
                if (XF32) {
                    const bf16x8 al = as_bf16x8(*(const u32x4 *)(xl + m * 256 + ((xc ^ (m & 15)) << 4)));
                    acc_g[t] = mfma16(al, as_bf16x8(bg[j]), acc_g[t]);
                    if (SILU) acc_u[t] = mfma16(al, as_bf16x8(bu[j]), acc_u[t]);
                }
            }
        }
        if (c + 1 < ce) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                bg[j] = ng[j];
                if (SILU) bu[j] = nu[j];
            }
        }
        __syncthreads();
    }

    // D lane layout: column col, rows 4 grp + r of each 16-row tile.
    const uint32_t n = n0 + col;
    if (n >= N) return;
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t m = 16 * t + 4 * grp + r;
            if (m >= M) continue;
            float g = acc_g[t][r], u = acc_u[t][r];
            if (splits > 1) {
                float *dst = part + (size_t)split * (SILU ? 2 : 1) * M * N;
                dst[(size_t)m * N + n] = g;
                if (SILU) dst[(size_t)M * N + (size_t)m * N + n] = u;
                continue;
            }
            if (W8) {
                g *= bf16_float(p.w_scale[n]);
                if (SILU) u *= bf16_float(p.w_scale[N + n]);
            }
            float v = SILU ? silu(g) * u : g;
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
    float g = 0.0f, u = 0.0f;
    for (uint32_t s = 0; s < splits; s++) {
        g += part[(size_t)s * (SILU ? 2 : 1) * MN + i];
        if (SILU) u += part[(size_t)s * 2 * MN + MN + i];
    }
    if (W8) {
        g *= bf16_float(p.w_scale[n]);
        if (SILU) u *= bf16_float(p.w_scale[N + n]);
    }
    float v = SILU ? silu(g) * u : g;
    if (p.stages & TS_AFTER_ADD) v += p.a0[i];
    if (p.out_bf16) ((uint16_t *)p.out)[i] = bf16_bits(v);
    else ((float *)p.out)[i] = v;
}

struct Plan {
    uint32_t groups, splits;
};

// Enough groups to cover the chip (~512): the column groups, times a k split when
// they are fewer (each split keeps at least one 128-deep chunk).
Plan plan(const ts_linear_args *a) {
    Plan pl;
    const uint32_t tiles = (a->n + 15) / 16, chunks = (a->k + kChunk - 1) / kChunk;
    pl.groups = (tiles + kWaves - 1) / kWaves;
    pl.splits = std::max(1u, std::min(chunks, (512u + pl.groups - 1) / pl.groups));
    return pl;
}

using Kern = void (*)(LanesParams, float *);

template <int MT, bool XF32, bool W8>
Kern pick3(bool silu, bool norm) {
    if (silu) return norm ? lanes_kernel<MT, XF32, W8, true, true> : lanes_kernel<MT, XF32, W8, true, false>;
    return norm ? lanes_kernel<MT, XF32, W8, false, true> : lanes_kernel<MT, XF32, W8, false, false>;
}

template <int MT>
Kern pick2(bool xf, bool w8, bool silu, bool norm) {
    return xf ? (w8 ? pick3<MT, true, true>(silu, norm) : pick3<MT, true, false>(silu, norm))
              : (w8 ? pick3<MT, false, true>(silu, norm) : pick3<MT, false, false>(silu, norm));
}

int check(const ts_linear_args *a) {
    TS_REQUIRE(a && a->x && a->w && a->out, "lanes: null pointer");
    TS_REQUIRE(a->m >= 1 && a->m <= 64, "lanes: m=%u outside 1..64", a->m);
    TS_REQUIRE(a->n >= 1 && a->k >= 1, "lanes: empty product n=%u k=%u", a->n, a->k);
    TS_REQUIRE(a->x_dtype == TS_F32 || a->x_dtype == TS_BF16, "lanes: x dtype %d", a->x_dtype);
    TS_REQUIRE(a->w_dtype == TS_BF16 || a->w_dtype == TS_E4M3, "lanes: w dtype %d", a->w_dtype);
    TS_REQUIRE(a->out_dtype == TS_F32 || a->out_dtype == TS_BF16, "lanes: out dtype %d", a->out_dtype);
    TS_REQUIRE(a->w_dtype != TS_E4M3 || a->w_scale, "lanes: e4m3 weights need w_scale");
    TS_REQUIRE(!(a->stages & TS_AFTER_ADD) || a->a0, "lanes: TS_AFTER_ADD needs a0");
    TS_REQUIRE(!(a->stages & TS_BEFORE_RMS_NORM) || (a->gain && a->x_dtype == TS_F32 && a->m <= 16),
               "lanes: TS_BEFORE_RMS_NORM needs gain, f32 x and m <= 16");
    TS_REQUIRE((a->stages & ~(TS_AFTER_ADD | TS_AFTER_SILU_MUL | TS_BEFORE_RMS_NORM)) == 0,
               "lanes: unknown stage bits %#x", a->stages);
    TS_REQUIRE(ts::aligned(a->x, 16) && ts::aligned(a->w, 16), "lanes: x and w must be 16-byte aligned");
    return TS_OK;
}

}  // namespace

extern "C" size_t tessera_hip_lanes_workspace(const ts_linear_args *a) {
    if (!a || a->m <= 4 || a->m > 64) return 0;
    const Plan pl = plan(a);
    if (pl.splits <= 1) return 0;
    const size_t per = (size_t)a->m * a->n * ((a->stages & TS_AFTER_SILU_MUL) ? 2 : 1);
    return (size_t)pl.splits * per * sizeof(float);
}

extern "C" int tessera_hip_lanes(const ts_linear_args *a, void *stream) {
    int rc = check(a);
    if (rc) return rc;
    if (a->m <= 4) return ts::gemv_launch(a, stream);
    const Plan pl = plan(a);
    const size_t need = tessera_hip_lanes_workspace(a);
    if (need && (!a->workspace || a->workspace_bytes < need))
        return ts::fail(TS_ERR_WORKSPACE, "lanes: workspace %zu bytes, need %zu", a->workspace_bytes, need);
    LanesParams p;
    p.x = a->x; p.w = a->w; p.w_scale = (const uint16_t *)a->w_scale; p.gain = a->gain; p.a0 = a->a0;
    p.out = a->out; p.m = a->m; p.n = a->n; p.k = a->k; p.stages = a->stages; p.eps = a->eps;
    p.out_bf16 = a->out_dtype == TS_BF16;
    const bool silu = a->stages & TS_AFTER_SILU_MUL, norm = a->stages & TS_BEFORE_RMS_NORM;
    const bool xf = a->x_dtype == TS_F32, w8 = a->w_dtype == TS_E4M3;
    const uint32_t mt = (a->m + 15) / 16;
    Kern k = mt == 1 ? pick2<1>(xf, w8, silu, norm)
           : mt == 2 ? pick2<2>(xf, w8, silu, norm)
           : mt == 3 ? pick2<3>(xf, w8, silu, norm) : pick2<4>(xf, w8, silu, norm);
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
