// "lanes": out[m, n] = after(sum_k x[m, k] w[n, k]) for m <= 16 rows.
// Rows 1..4 go to the vector-ALU kernel in gemv.hip; 5..16 run here.
//
// Replaces the reference's few-row matmul rules: lanes (a 32-lane group per
// column, engine/rules/linear/src/lanes.rs:17-143) and thin (a thread per
// column, thin.rs:11-104). Same product, same fused stages (map.rs:155-185).
//
// gfx950 design. Decode products are HBM-bound: every weight byte is read
// once and nothing else matters. A wave owns 16 output columns and a slice of
// k. Each lane streams 64 contiguous bytes of one weight row per 128-deep
// chunk (16B vector loads, four per row per chunk), which feeds four
// v_mfma_f32_16x16x32_bf16 steps directly from registers, with no LDS for the
// weights. Inside one chunk lane group g holds k [32g, 32g+32) of its row;
// MFMA step j takes elements [8j, 8j+8) of that run. The x operand uses the
// same k assignment, so the product is unchanged by this ordering. Rows m >= M
// of the 16-row A operand are zero (M=1 wastes matrix-unit work, not bytes).
// f32 activations are split into two exact bf16 parts (hi = bf16(x),
// lo = bf16(x - hi)); hi*w + lo*w carries 16 mantissa bits of x, so f32 rows
// times bf16 weights stay close to the f32 oracle. e4m3 weights decode to bf16
// in registers; the per-row scale multiplies the finished sum.
// k is split across the waves of a group and reduced in LDS; nothing crosses
// groups (a device-wide fence to hand partials between groups costs more than
// the whole product here), so results are deterministic.
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

// x chunk for one lane as bf16 parts: hi (and lo for f32 x). Rows >= M are zero.
template <bool XF32, bool NORM>
TS_DEV void load_x(const void *x, const float *gain, float inv, uint32_t m, uint32_t M, uint32_t k0,
                   uint32_t K, u32x4 (&hi)[4], u32x4 (&lo)[4]) {
    if (m >= M) {
#pragma unroll
        for (int j = 0; j < 4; j++) hi[j] = lo[j] = u32x4{0, 0, 0, 0};
        return;
    }
    if (XF32) {
        const float *p = (const float *)x + (size_t)m * K + k0;
        float v[32];
        if (k0 + 32 <= K && (K % 4) == 0) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float4 t = *((const float4 *)p + i);
                v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
            }
            if (NORM) {
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    float4 g = *((const float4 *)(gain + k0) + i);
                    v[4 * i] *= inv * g.x; v[4 * i + 1] *= inv * g.y;
                    v[4 * i + 2] *= inv * g.z; v[4 * i + 3] *= inv * g.w;
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < 32; i++) {
                v[i] = (k0 + i < K) ? p[i] : 0.0f;
                if (NORM && k0 + i < K) v[i] *= inv * gain[k0 + i];
            }
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            uint32_t h[4], l[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float a = v[8 * j + 2 * e], b = v[8 * j + 2 * e + 1];
                float ha = bf16_round(a), hb = bf16_round(b);
                h[e] = pack_bf16x2(ha, hb);
                l[e] = pack_bf16x2(a - ha, b - hb);
            }
            hi[j] = u32x4{h[0], h[1], h[2], h[3]};
            lo[j] = u32x4{l[0], l[1], l[2], l[3]};
        }
    } else {
        const uint16_t *p = (const uint16_t *)x + (size_t)m * K + k0;
        if (k0 + 32 <= K && (K % 8) == 0) {
#pragma unroll
            for (int j = 0; j < 4; j++) hi[j] = *((const u32x4 *)p + j);
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                uint32_t v[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    uint32_t ka = k0 + 8 * j + 2 * e;
                    uint32_t a = ka < K ? p[8 * j + 2 * e] : 0u;
                    uint32_t b = ka + 1 < K ? p[8 * j + 2 * e + 1] : 0u;
                    v[e] = a | (b << 16);
                }
                hi[j] = u32x4{v[0], v[1], v[2], v[3]};
            }
        }
#pragma unroll
        for (int j = 0; j < 4; j++) lo[j] = u32x4{0, 0, 0, 0};
    }
}

TS_DEV float silu(float v) { return v / (1.0f + expf(-v)); }

template <bool XF32, bool W8, bool SILU, bool NORM>
__global__ __launch_bounds__(kWaves * 64) void lanes_kernel(LanesParams p) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t tile = blockIdx.x, split = 0, splits = 1;
    const uint32_t col = lane & 15, grp = lane >> 4;
    const uint32_t n0 = tile * 16, M = p.m, N = p.n, K = p.k;

    __shared__ float red[kWaves][SILU ? 2 : 1][256];
    __shared__ float inv_s[16];
    __shared__ float part_s[kWaves][16];

    // Fused RmsNorm prologue: every group computes the same inverse roots
    // (fixed reduction order, so all groups agree bit for bit).
    float inv = 1.0f;
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
        if (col < M) inv = inv_s[col];
    }

    // This wave's chunk range.
    const uint32_t chunks = (K + kChunk - 1) / kChunk;
    const uint32_t slice = split * kWaves + wave, nslices = splits * kWaves;
    const uint32_t cb = (uint32_t)(((uint64_t)chunks * slice) / nslices);
    const uint32_t ce = (uint32_t)(((uint64_t)chunks * (slice + 1)) / nslices);

    f32x4 acc_g = {0, 0, 0, 0}, acc_u = {0, 0, 0, 0};
    const uint32_t wrows = SILU ? 2 * N : N;
    for (uint32_t c = cb; c < ce; c++) {
        const uint32_t k0 = c * kChunk + 32 * grp;
        u32x4 bg[4], bu[4], xh[4], xl[4];
        load_w<W8>(p.w, n0 + col, SILU ? N : N, k0, K, bg);
        if (SILU) load_w<W8>(p.w, N + n0 + col, wrows, k0, K, bu);
        load_x<XF32, NORM>(p.x, p.gain, inv, col, M, k0, K, xh, xl);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            acc_g = mfma16(as_bf16x8(xh[j]), as_bf16x8(bg[j]), acc_g);
            if (XF32) acc_g = mfma16(as_bf16x8(xl[j]), as_bf16x8(bg[j]), acc_g);
            if (SILU) {
                acc_u = mfma16(as_bf16x8(xh[j]), as_bf16x8(bu[j]), acc_u);
                if (XF32) acc_u = mfma16(as_bf16x8(xl[j]), as_bf16x8(bu[j]), acc_u);
            }
        }
    }
    // D lane layout: column col, rows 4*grp + r.
#pragma unroll
    for (int r = 0; r < 4; r++) {
        red[wave][0][(4 * grp + r) * 16 + col] = acc_g[r];
        if (SILU) red[wave][SILU ? 1 : 0][(4 * grp + r) * 16 + col] = acc_u[r];
    }
    __syncthreads();

    const uint32_t t = threadIdx.x;  // one tile element per thread: m = t/16, n = t%16
    float g = 0.0f, u = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; w++) {
        g += red[w][0][t];
        if (SILU) u += red[w][SILU ? 1 : 0][t];
    }
    const uint32_t m = t >> 4, n = n0 + (t & 15);
    if (m >= M || n >= N) return;
    if (W8) {
        g *= bf16_float(p.w_scale[n]);
        if (SILU) u *= bf16_float(p.w_scale[N + n]);
    }
    float v = SILU ? silu(g) * u : g;
    if (p.stages & TS_AFTER_ADD) v += p.a0[(size_t)m * N + n];
    if (p.out_bf16) ((uint16_t *)p.out)[(size_t)m * N + n] = bf16_bits(v);
    else ((float *)p.out)[(size_t)m * N + n] = v;
}

struct Plan {
    uint32_t tiles, splits;
};

Plan plan(const ts_linear_args *a) {
    Plan pl;
    pl.tiles = (a->n + 15) / 16;
    pl.splits = 1;
    return pl;
}

using Kern = void (*)(LanesParams);

template <bool XF32, bool W8>
Kern pick2(bool silu, bool norm) {
    if (silu) return norm ? lanes_kernel<XF32, W8, true, true> : lanes_kernel<XF32, W8, true, false>;
    return norm ? lanes_kernel<XF32, W8, false, true> : lanes_kernel<XF32, W8, false, false>;
}

int check(const ts_linear_args *a) {
    TS_REQUIRE(a && a->x && a->w && a->out, "lanes: null pointer");
    TS_REQUIRE(a->m >= 1 && a->m <= 16, "lanes: m=%u outside 1..16", a->m);
    TS_REQUIRE(a->n >= 1 && a->k >= 1, "lanes: empty product n=%u k=%u", a->n, a->k);
    TS_REQUIRE(a->x_dtype == TS_F32 || a->x_dtype == TS_BF16, "lanes: x dtype %d", a->x_dtype);
    TS_REQUIRE(a->w_dtype == TS_BF16 || a->w_dtype == TS_E4M3, "lanes: w dtype %d", a->w_dtype);
    TS_REQUIRE(a->out_dtype == TS_F32 || a->out_dtype == TS_BF16, "lanes: out dtype %d", a->out_dtype);
    TS_REQUIRE(a->w_dtype != TS_E4M3 || a->w_scale, "lanes: e4m3 weights need w_scale");
    TS_REQUIRE(!(a->stages & TS_AFTER_ADD) || a->a0, "lanes: TS_AFTER_ADD needs a0");
    TS_REQUIRE(!(a->stages & TS_BEFORE_RMS_NORM) || (a->gain && a->x_dtype == TS_F32),
               "lanes: TS_BEFORE_RMS_NORM needs gain and f32 x");
    TS_REQUIRE((a->stages & ~(TS_AFTER_ADD | TS_AFTER_SILU_MUL | TS_BEFORE_RMS_NORM)) == 0,
               "lanes: unknown stage bits %#x", a->stages);
    TS_REQUIRE(ts::aligned(a->x, 16) && ts::aligned(a->w, 16), "lanes: x and w must be 16-byte aligned");
    return TS_OK;
}

}  // namespace

extern "C" size_t tessera_hip_lanes_workspace(const ts_linear_args *a) {
    (void)a;
    return 0;  // no entry point of this rule needs scratch
}

extern "C" int tessera_hip_lanes(const ts_linear_args *a, void *stream) {
    int rc = check(a);
    if (rc) return rc;
    Plan pl = plan(a);
    LanesParams p;
    p.x = a->x; p.w = a->w; p.w_scale = (const uint16_t *)a->w_scale; p.gain = a->gain; p.a0 = a->a0;
    p.out = a->out; p.m = a->m; p.n = a->n; p.k = a->k; p.stages = a->stages; p.eps = a->eps;
    p.out_bf16 = a->out_dtype == TS_BF16;
    if (a->m <= 4) return ts::gemv_launch(a, stream);
    const bool silu = a->stages & TS_AFTER_SILU_MUL, norm = a->stages & TS_BEFORE_RMS_NORM;
    const bool xf = a->x_dtype == TS_F32, w8 = a->w_dtype == TS_E4M3;
    Kern k = xf ? (w8 ? pick2<true, true>(silu, norm) : pick2<true, false>(silu, norm))
                : (w8 ? pick2<false, true>(silu, norm) : pick2<false, false>(silu, norm));
    hipLaunchKernelGGL(k, dim3(pl.tiles), dim3(kWaves * 64), 0, (hipStream_t)stream, p);
    TS_CHECK_LAUNCH("lanes launch");
    return TS_OK;
}
