// Decode-shaped products (m <= 4 rows) on the vector ALUs: the lanes rule's
// kernel for batch-1 decode.
//
// Replaces the reference's lanes kernel (a 32-lane group per column, 4-wide
// loads, engine/rules/linear/src/lanes.rs:17-63) and thin (thin.rs:11-55) for
// the rows the decode step has. Products are exact f32 (bf16 and e4m3 weights
// widen exactly), as in tessera-interp (engine/ir/interp/src/cpu.rs:108-138),
// so only the summation order differs from the oracle.
//
// gfx950 design. At m <= 4 these products only stream weights: every byte is
// read once and the rest is latency. So:
//  * a group owns R weight rows (R output columns, or R/2 gate + R/2 up for the
//    SiLU pair) and W waves split k; a lane reads 16 contiguous bytes per row
//    per step (a wave reads 1 KiB of one row per instruction);
//  * every load of a batch (up to 16 x 16 B per lane: R rows x steps) is issued
//    before any is used, together with the x (and gain) slices it needs;
//  * a fused RmsNorm does not rescale x first: inv = 1/sqrt(mean(x^2)+eps) is a
//    scalar per row, so sum_k (x_k inv g_k) w_k = inv * sum_k (x_k g_k) w_k and
//    the sum of squares accumulates in the same pass;
//  * waves reduce with butterflies, groups with one LDS exchange; nothing crosses
//    groups, so there are no fences, atomics or workspace, and results are
//    deterministic.
#include <stdio.h>
#include <stdlib.h>

#include "after.h"

namespace ts {

struct GemvParams {
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
    void *keys;  // TS_AFTER_ARGMAX: [m] uint64
    uint32_t waves;  // waves per group splitting k
    ts_after after;  // stage chain (count 0: none)
    int pair_sum;    // TS_F32_PARTS: rows n.. are the low parts; the output sums the pair
};

namespace {

constexpr int kMaxW = 4;
constexpr int kMaxLoads = 16;  // 16-byte weight loads in flight per lane per batch

template <bool W8>
TS_DEV void widen_w(u32x4 v, float (&f)[W8 ? 16 : 8]) {
    if (!W8) {
        f[0] = lo_bf16(v.x); f[1] = hi_bf16(v.x); f[2] = lo_bf16(v.y); f[3] = hi_bf16(v.y);
        f[4] = lo_bf16(v.z); f[5] = hi_bf16(v.z); f[6] = lo_bf16(v.w); f[7] = hi_bf16(v.w);
    } else {
        e4m3x4_to_f32(v.x, f);
        e4m3x4_to_f32(v.y, f + 4);
        e4m3x4_to_f32(v.z, f + 8);
        e4m3x4_to_f32(v.w, f + 12);
    }
}

template <int M, int R, bool XF32, bool W8>
__global__ __launch_bounds__(kMaxW * 64) void gemv_kernel(GemvParams p) {
    constexpr int E = W8 ? 16 : 8;       // weights per 16-byte load
    constexpr int STEP = 64 * E;         // k covered by one load across the wave
    // Steps per batch: at most 16 weight loads and 64 x values per lane in flight.
    constexpr int B1 = kMaxLoads / R, B2 = 64 / (M * E);
    constexpr int B = (B1 < B2 ? B1 : B2) > 0 ? (B1 < B2 ? B1 : B2) : 1;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, W = p.waves;
    const uint32_t K = p.k, N = p.n, Mr = p.m;
    const bool silu = (p.stages & TS_AFTER_SILU_MUL) || p.pair_sum, norm = p.stages & TS_BEFORE_RMS_NORM;
    const uint32_t outs = silu ? R / 2 : R;
    const uint32_t o0 = blockIdx.x * outs;

    // Rows this group streams.
    uint32_t row[R];
    bool row_ok[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint32_t o = silu ? (r < R / 2 ? r : r - R / 2) : r;
        row_ok[r] = o0 + o < N;
        row[r] = silu && r >= R / 2 ? N + o0 + o : o0 + o;
    }

    // This wave's k slice, whole steps.
    const uint32_t steps_all = (K + STEP - 1) / STEP;
    const uint32_t s_per = (steps_all + W - 1) / W;
    const uint32_t kb = wave * s_per * STEP;
    const uint32_t ke = min(K, kb + s_per * STEP);
    const bool vec = (K % E) == 0;  // 16-byte aligned rows

    // Epilogue operands of the output this lane may finish (wave 0, lane < outs*M),
    // fetched now so their latency hides under the weight stream.
    float pre_a0 = 0.0f, pre_sg = 1.0f, pre_su = 1.0f;
    {
        const uint32_t o = lane / M, m = lane % M, n = o0 + o;
        if (wave == 0 && lane < outs * M && m < Mr && n < N) {
            if (p.stages & TS_AFTER_ADD) pre_a0 = p.a0[(size_t)m * N + n];
            if (W8) {
                pre_sg = bf16_float(p.w_scale[n]);
                if (silu) pre_su = bf16_float(p.w_scale[N + n]);
            }
        }
    }

    float acc[R][M];
    float ssq[M];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int m = 0; m < M; m++) acc[r][m] = 0.0f;
#pragma unroll
    for (int m = 0; m < M; m++) ssq[m] = 0.0f;

    for (uint32_t k0 = kb; k0 < ke; k0 += B * STEP) {
        u32x4 wv[B][R];
        float xv[B][M][E];
        float gv[B][E];
        // Issue every load of the batch first.
#pragma unroll
        for (int b = 0; b < B; b++) {
            const uint32_t kk = k0 + b * STEP + lane * E;
            const bool full = vec && kk + E <= ke;
#pragma unroll
            for (int r = 0; r < R; r++) {
                if (full && row_ok[r]) {
                    const char *base = (const char *)p.w + ((size_t)row[r] * K + kk) * (W8 ? 1 : 2);
                    wv[b][r] = __builtin_nontemporal_load((const u32x4 *)base);
                } else if (row_ok[r] && kk < ke) {
                    uint32_t t[4] = {0, 0, 0, 0};
                    for (int e = 0; e < E && kk + e < ke; e++) {
                        const uint32_t code = W8 ? ((const uint8_t *)p.w)[(size_t)row[r] * K + kk + e]
                                                 : ((const uint16_t *)p.w)[(size_t)row[r] * K + kk + e];
                        t[e / (E / 4)] |= code << ((e % (E / 4)) * (W8 ? 8 : 16));
                    }
                    wv[b][r] = u32x4{t[0], t[1], t[2], t[3]};
                } else {
                    wv[b][r] = u32x4{0, 0, 0, 0};
                }
            }
            if (norm) {
                if (full) {
#pragma unroll
                    for (int q = 0; q < E / 4; q++) {
                        const float4 t = ((const float4 *)(p.gain + kk))[q];
                        gv[b][4 * q] = t.x; gv[b][4 * q + 1] = t.y; gv[b][4 * q + 2] = t.z; gv[b][4 * q + 3] = t.w;
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < E; e++) gv[b][e] = kk + e < ke ? p.gain[kk + e] : 0.0f;
                }
            }
#pragma unroll
            for (int m = 0; m < M; m++) {
                if ((uint32_t)m < Mr && full) {
                    if (XF32) {
                        const float4 *xs = (const float4 *)((const float *)p.x + (size_t)m * K + kk);
#pragma unroll
                        for (int q = 0; q < E / 4; q++) {
                            const float4 t = xs[q];
                            xv[b][m][4 * q] = t.x; xv[b][m][4 * q + 1] = t.y;
                            xv[b][m][4 * q + 2] = t.z; xv[b][m][4 * q + 3] = t.w;
                        }
                    } else {
                        const u32x4 *xs = (const u32x4 *)((const uint16_t *)p.x + (size_t)m * K + kk);
#pragma unroll
                        for (int q = 0; q < E / 8; q++) {
                            const u32x4 t = xs[q];
                            xv[b][m][8 * q] = lo_bf16(t.x); xv[b][m][8 * q + 1] = hi_bf16(t.x);
                            xv[b][m][8 * q + 2] = lo_bf16(t.y); xv[b][m][8 * q + 3] = hi_bf16(t.y);
                            xv[b][m][8 * q + 4] = lo_bf16(t.z); xv[b][m][8 * q + 5] = hi_bf16(t.z);
                            xv[b][m][8 * q + 6] = lo_bf16(t.w); xv[b][m][8 * q + 7] = hi_bf16(t.w);
                        }
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < E; e++) {
                        const uint32_t ke2 = kk + e;
                        float v = 0.0f;
                        if ((uint32_t)m < Mr && ke2 < ke)
                            v = XF32 ? ((const float *)p.x)[(size_t)m * K + ke2]
                                     : bf16_float(((const uint16_t *)p.x)[(size_t)m * K + ke2]);
                        xv[b][m][e] = v;
                    }
                }
            }
        }
        // Then use them: RmsNorm's sum of squares, the gain, the dots.
#pragma unroll
        for (int b = 0; b < B; b++) {
            if (norm) {
#pragma unroll
                for (int m = 0; m < M; m++)
#pragma unroll
                    for (int e = 0; e < E; e++) {
                        ssq[m] += xv[b][m][e] * xv[b][m][e];
                        xv[b][m][e] *= gv[b][e];
                    }
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                float wf[E];
                widen_w<W8>(wv[b][r], wf);
#pragma unroll
                for (int m = 0; m < M; m++)
#pragma unroll
                    for (int e = 0; e < E; e++) acc[r][m] += xv[b][m][e] * wf[e];
            }
        }
    }

    // Wave sums.
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int m = 0; m < M; m++) acc[r][m] = wave_sum(acc[r][m]);
    if (norm) {
#pragma unroll
        for (int m = 0; m < M; m++) ssq[m] = wave_sum(ssq[m]);
    }
    // Group sums (waves split k).
    __shared__ float red[kMaxW][R * M + M];
    if (W > 1) {
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int m = 0; m < M; m++) red[wave][r * M + m] = acc[r][m];
#pragma unroll
            for (int m = 0; m < M; m++) red[wave][R * M + m] = ssq[m];
        }
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int m = 0; m < M; m++) {
                float s = 0.0f;
                for (uint32_t w = 0; w < W; w++) s += red[w][r * M + m];
                acc[r][m] = s;
            }
#pragma unroll
        for (int m = 0; m < M; m++) {
            float s = 0.0f;
            for (uint32_t w = 0; w < W; w++) s += red[w][R * M + m];
            ssq[m] = s;
        }
    }
    // Lane t of wave 0 finishes output (t / M, t % M).
    if (wave != 0) return;
    const uint32_t o = lane / M, m = lane % M;
    const bool live = lane < outs * M && m < Mr && o0 + o < N;
    float g = 0.0f, u = 0.0f, sq = 0.0f;
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int mm = 0; mm < M; mm++) {
            if ((uint32_t)r == o && (uint32_t)mm == m) g = acc[r][mm];
            if (silu && (uint32_t)r == o + R / 2 && (uint32_t)mm == m) u = acc[r][mm];
        }
#pragma unroll
    for (int mm = 0; mm < M; mm++)
        if ((uint32_t)mm == m) sq = ssq[mm];
    const uint32_t n = o0 + o;
    if (norm) {
        const float inv = 1.0f / sqrtf(sq / (float)K + p.eps);
        g *= inv;
        u *= inv;
    }
    if (W8) {
        g *= pre_sg;
        u *= pre_su;
    }
    float v = silu ? (p.pair_sum ? g + u : g / (1.0f + expf(-g)) * u) : g;
    if (p.stages & TS_AFTER_ADD) v += pre_a0;
    if (p.after.count && live) v = after_apply(p.after, v, (size_t)m * N + n);
    if (live) {
        if (p.out_bf16) ((uint16_t *)p.out)[(size_t)m * N + n] = bf16_bits(v);
        else ((float *)p.out)[(size_t)m * N + n] = v;
    }
    if (p.stages & TS_AFTER_ARGMAX) {
        // The group's best entry per row (lanes m, m + M, ... share row m), folded into
        // keys[m] only when it beats what is there: after the first few groups almost
        // none does, so few atomics reach the one address.
        uint64_t key = live ? argmax_key(v, n) : 0;
#pragma unroll
        for (int off = M; off < 64; off *= 2) {
            const uint64_t other = __shfl_xor(key, off);
            key = other > key ? other : key;
        }
        uint64_t *keys = (uint64_t *)p.keys;
        if (lane < M && m < Mr && key > __hip_atomic_load(keys + m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
            __hip_atomic_fetch_max(keys + m, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

using Kern = void (*)(GemvParams);

template <int M, bool XF32, bool W8>
Kern pick_r(int r) {
    switch (r) {
    case 2: return gemv_kernel<M, 2, XF32, W8>;
    case 4: return gemv_kernel<M, 4, XF32, W8>;
    default: return gemv_kernel<M, 8, XF32, W8>;
    }
}

template <bool XF32, bool W8>
Kern pick_m(uint32_t m, int r) {
    if (m == 1) return pick_r<1, XF32, W8>(r);
    if (m == 2) return pick_r<2, XF32, W8>(r);
    return pick_r<4, XF32, W8>(r);
}

}  // namespace

// Rows per group and waves per group for a product shape: enough waves to
// cover the chip (~2048), whole k steps per wave.
void gemv_plan(uint32_t n, uint32_t k, bool silu, bool w8, int *rows, uint32_t *waves, uint32_t *groups) {
    // Measured on MI355X (graph-replayed, cold weights): for bf16 weights one wave
    // per group is fastest at every decode shape (an LDS exchange costs more than it
    // saves), and rows per wave grow with the row count: 8 for >= 3072 rows of 1024,
    // 4 for ~1024 rows of 2048, 2 for ~1024 rows of 3072.
    const uint32_t total = silu ? 2 * n : n;
    int r;
    uint32_t w = 1;
    if (w8) {
        // e4m3 rows (16 weights per 16-byte load): measured on the C4 shapes. Rows much
        // longer than the row count leave too few waves with one wave per group, so four
        // waves split k there (4096 x 14336: 20.3 -> 12.8 us at m = 1).
        if (k >= 3 * total && total >= 4096) { r = 8; w = 4; }
        else if (total >= 8192) r = 8;
        else if (total >= 4096) r = 4;
        else r = 2;
    } else if (total >= 3072) {
        r = 8;
    } else if (k <= 2048) {
        r = 4;
    } else {
        r = 2;
    }
    const uint32_t outs = silu ? r / 2 : r;
    const uint32_t g = (n + outs - 1) / outs;
    *rows = r;
    *waves = w;
    *groups = g;
}

int gemv_launch(const ts_linear_args *a, void *stream) {
    int r;
    uint32_t w, g;
    const bool parts = a->w_dtype == TS_F32_PARTS, silu = (a->stages & TS_AFTER_SILU_MUL) || parts;
    gemv_plan(a->n, a->k, silu, a->w_dtype == TS_E4M3, &r, &w, &g);
    GemvParams p;
    p.x = a->x; p.w = a->w; p.w_scale = (const uint16_t *)a->w_scale; p.gain = a->gain; p.a0 = a->a0;
    p.out = a->out; p.m = a->m; p.n = a->n; p.k = a->k; p.stages = a->stages; p.eps = a->eps;
    p.out_bf16 = a->out_dtype == TS_BF16; p.waves = w; p.keys = a->workspace; p.pair_sum = parts;
    const int rc = linear_after(a, "lanes (gemv)", &p.after);
    if (rc) return rc;
    const bool xf = a->x_dtype == TS_F32, w8 = a->w_dtype == TS_E4M3;
    Kern k = xf ? (w8 ? pick_m<true, true>(a->m, r) : pick_m<true, false>(a->m, r))
                : (w8 ? pick_m<false, true>(a->m, r) : pick_m<false, false>(a->m, r));
    hipLaunchKernelGGL(k, dim3(g), dim3(64 * w), 0, (hipStream_t)stream, p);
    TS_CHECK_LAUNCH("lanes (gemv) launch");
    return TS_OK;
}

}  // namespace ts
