/*
 * TEST INFRASTRUCTURE ONLY. A plain-C restatement of tessera-interp, the
 * reference's CPU oracle (engine/ir/interp). Only tests/, the smoke check and
 * bench.py's cpu_baseline leg may load this library, and only as the checker.
 * The product path (libtessera_hip.so) never links or calls it.
 *
 * Every loop keeps the reference's summation order: one f32 accumulator per
 * output, starting at 0.0, adding x*y in ascending k
 * (engine/ir/interp/src/round.rs:8-34). Multi-threaded entry points split
 * over outputs only, so each output is summed in the same order and the result
 * is bit-identical to the single-threaded run.
 *
 * Pinning (what checks each function, in tests/test_oracle.py):
 *   narrow/widen bf16, e4m3      exhaustive code round trips, RNE ties, saturation
 *   noise                         closed form of the LCG
 *   product                       f64 brute force, integer-exact inputs, accumulator test
 *   attend / attend_rows          window_edges, rows_read_slots, decode_sees_past_keys,
 *                                 one-key and uniform-score invariants
 *   softmax, rms(norm), rope, act known-answer tests of cpu_test.rs
 *   top_k                         brute-force stable sort
 *   gather, take, mix             gather_rows, closed forms
 *   paged row                     closed form of kept.rs Paged::row
 *   f16, e8m0                     exhaustive f16 code round trips, numpy's RNE float16
 *                                 on random f32, e8m0 round-up closed forms
 *   e2m1                          the 16-code table, ties-to-even-code rounding on a
 *                                 dense grid (brute-force nearest), saturation
 *   block pack / dot              blocks_round_trip of block_test.rs for all seven forms
 *                                 (byte counts, round-trip share, dot == sum over
 *                                 unpacked), hand-built blocks with closed-form sums,
 *                                 code placement by form, the nvfp4 head, e8m0 round-up
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define EXPORT __attribute__((visibility("default")))

static int g_threads = 1;

EXPORT void or_set_threads(int n) { g_threads = n < 1 ? 1 : n; }

EXPORT int or_threads_available(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------ */
/* Narrow floats: engine/ir/graph/src/scalar.rs:20-59                  */
/* ------------------------------------------------------------------ */

static inline uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* 2^n as a double, for the subnormal step count. */
static double pow2d(int n) { return ldexp(1.0, n); }

static float widen_fmt(uint32_t bits, int E, int M, int INF, int NAN_) {
    int bias = (1 << (E - 1)) - 1;
    double steps = pow2d(bias - 1 + M);
    uint32_t ones = (1u << (E + M)) - 1;
    float sign = ((bits >> (E + M)) & 1) ? -1.0f : 1.0f;
    uint32_t exp = (bits >> M) & ((1u << E) - 1), man = bits & ((1u << M) - 1);
    uint32_t all = (1u << E) - 1;
    if (exp == 0) return sign * (float)((double)man / steps);
    if (exp == all && INF) return man == 0 ? sign * INFINITY : NAN;
    if (NAN_ && !INF && (bits & ones) == ones) return NAN;
    return sign * ((1.0f + (float)man / (float)(1u << M)) * (float)pow2d((int)exp - bias));
}

/* scalar.rs:20-44: RNE; subnormals by f64 rounding; saturation without INF. */
static uint32_t narrow_fmt(float x, int E, int M, int INF, int NAN_) {
    int bias = (1 << (E - 1)) - 1;
    uint32_t ones = (1u << (E + M)) - 1;
    uint32_t top = INF ? ones - (1u << M) : (NAN_ ? ones - 1 : ones);
    double steps = pow2d(bias - 1 + M);
    uint32_t sign = (f2u(x) >> 31) << (E + M);
    if (isnan(x)) {
        uint32_t quiet = (ones & ~((1u << M) - 1)) | (1u << (M - 1));
        return sign | (INF ? quiet : ones);
    }
    float a = fabsf(x);
    if (a < ldexpf(1.0f, 1 - bias)) {
        return sign | (uint32_t)nearbyint((double)a * steps); /* default mode: ties even */
    }
    int drop = 23 - M;
    uint32_t bits = f2u(a);
    uint32_t half = (1u << (drop - 1)) - 1 + ((bits >> drop) & 1);
    float r = u2f((bits + half) & ~((1u << drop) - 1));
    if (r > widen_fmt(top, E, M, INF, NAN_)) {
        uint32_t over = INF ? top + 1 : top;
        return sign | over;
    }
    uint32_t exp = (uint32_t)((int)(f2u(r) >> 23) - 127 + bias);
    return sign | (exp << M) | ((f2u(r) >> drop) & ((1u << M) - 1));
}

EXPORT uint16_t or_bf16_narrow(float x) { return (uint16_t)narrow_fmt(x, 8, 7, 1, 1); }
/* bf16 widening is exact: the top half of an f32. The general form above is the pinned
 * one; the shift is what the hot loops use, and the tests check both agree on all codes. */
EXPORT float or_bf16_widen_exact(uint16_t b) { return widen_fmt(b, 8, 7, 1, 1); }
static inline float widen16(uint16_t b) {
    float f = u2f((uint32_t)b << 16);
    return isnan(f) ? NAN : f;
}
EXPORT float or_bf16_widen(uint16_t b) { return widen16(b); }
EXPORT uint8_t or_e4m3_narrow(float x) { return (uint8_t)narrow_fmt(x, 4, 3, 0, 1); }
EXPORT float or_e4m3_widen(uint8_t b) { return widen_fmt(b, 4, 3, 0, 1); }

/* F16 (scalar.rs:114-117): IEEE binary16 through the same narrow/widen. */
EXPORT uint16_t or_f16_narrow(float x) { return (uint16_t)narrow_fmt(x, 5, 10, 1, 1); }
EXPORT float or_f16_widen(uint16_t b) { return widen_fmt(b, 5, 10, 1, 1); }

/* E8M0 (scalar.rs:139-161): a power-of-two scale, rounded up so a block never clips;
 * 0xFF is NaN. */
EXPORT uint8_t or_e8m0_narrow(float x) {
    if (isnan(x)) return 0xFF;
    uint32_t b = f2u(fabsf(x));
    int up = (int)(b >> 23) + ((b & 0x7FFFFF) != 0);
    return (uint8_t)(up < 0 ? 0 : (up > 254 ? 254 : up));
}
EXPORT float or_e8m0_widen(uint8_t e) { return e == 0xFF ? NAN : (float)pow2d((int)e - 127); }

/* ------------------------------------------------------------------ */
/* Block forms: engine/ir/mem/src/block.rs:1-291                       */
/* ------------------------------------------------------------------ */
/* The seven forms of block.rs:251-291, by id:
 *   0 q8_0      F16 scale,  I8 codes,     32 a block, halves
 *   1 mxfp8     E8M0 scale, E4M3 codes,   32
 *   2 int4_g32  F16 scale,  Nibble codes, 32, adjacent pairs
 *   3 q4_0      F16 scale,  Nibble codes, 32, halves
 *   4 nvfp4     E4M3 scale, E2M1 codes,   16, adjacent pairs, f32 head
 *   5 mxfp4     E8M0 scale, E2M1 codes,   32, adjacent pairs
 *   6 int4_g128 F16 scale,  Nibble codes, 128, adjacent pairs
 * A tensor is [head] then its blocks, in element order (a [n, k] matrix with k a
 * multiple of the block: row r's blocks start at head + r k / B block bytes). */
enum { SC_F16, SC_E8M0, SC_E4M3 };
enum { CD_I8, CD_E4M3, CD_NIB, CD_E2M1 };
typedef struct { int scale, code, B, halves, head; } BlkSpec;
static const BlkSpec kForms[7] = {
    {SC_F16, CD_I8, 32, 1, 0},   {SC_E8M0, CD_E4M3, 32, 0, 0}, {SC_F16, CD_NIB, 32, 0, 0},
    {SC_F16, CD_NIB, 32, 1, 0},  {SC_E4M3, CD_E2M1, 16, 0, 1}, {SC_E8M0, CD_E2M1, 32, 0, 0},
    {SC_F16, CD_NIB, 128, 0, 0},
};
static int blk_scale_bytes(int form) { return kForms[form].scale == SC_F16 ? 2 : 1; }
static int blk_bits(int form) { return kForms[form].code <= CD_E4M3 ? 8 : 4; }
EXPORT int or_block_size(int form) { return kForms[form].B; }
EXPORT int or_block_head(int form) { return kForms[form].head ? 4 : 0; }
EXPORT int or_block_bytes(int form) { return blk_scale_bytes(form) + kForms[form].B * blk_bits(form) / 8; }
EXPORT int64_t or_block_tensor_bytes(int form, int64_t n) {
    const int B = kForms[form].B;
    return or_block_head(form) + (n + B - 1) / B * or_block_bytes(form);
}

/* E2M1 (scalar.rs:132-135): 2 exponent bits, 1 mantissa bit, no inf, no NaN. */
EXPORT uint8_t or_e2m1_narrow(float x) { return (uint8_t)narrow_fmt(x, 2, 1, 0, 0); }
EXPORT float or_e2m1_widen(uint8_t b) { return widen_fmt(b & 15u, 2, 1, 0, 0); }

/* place (block.rs:131-137): 8-bit codes at byte j; nibbles paired by halves (j % (B/2),
 * shift 4 (j / (B/2))) or adjacent (j / 2, shift 4 (j % 2)). */
static void blk_place(int form, int j, int *byte, int *shift) {
    const BlkSpec *f = &kForms[form];
    if (blk_bits(form) == 8) { *byte = j; *shift = 0; return; }
    if (f->halves) { *byte = j % (f->B / 2); *shift = 4 * (j / (f->B / 2)); return; }
    *byte = j / 2; *shift = 4 * (j % 2);
}
static float blk_decode(int form, uint32_t code) {
    switch (kForms[form].code) {
    case CD_I8: return (float)(int8_t)(uint8_t)code;      /* I8 (block.rs:79-90) */
    case CD_E4M3: return or_e4m3_widen((uint8_t)code);     /* E4M3 (block.rs:66-76) */
    case CD_E2M1: return or_e2m1_widen((uint8_t)code);     /* E2M1 (block.rs:49-63) */
    default: return (float)code - 8.0f;                    /* Nibble (block.rs:95-104) */
    }
}
static uint32_t blk_encode(int form, float scaled) {
    switch (kForms[form].code) {
    case CD_I8: { /* round_ties_even, clamp to [-128, 127], as a byte */
        float r = nearbyintf(scaled);
        r = r < -128.0f ? -128.0f : (r > 127.0f ? 127.0f : r);
        if (isnan(scaled)) r = 0.0f; /* Rust's saturating cast: NaN -> 0 */
        return (uint32_t)(uint8_t)(int8_t)r;
    }
    case CD_E4M3: return or_e4m3_narrow(scaled);
    case CD_E2M1: return or_e2m1_narrow(scaled);
    default: { /* (scaled + 8.5).clamp(0, 15) as u32: truncation */
        float t = scaled + 8.5f;
        t = t < 0.0f ? 0.0f : (t > 15.0f ? 15.0f : t);
        if (isnan(t)) t = 0.0f;
        return (uint32_t)t;
    }
    }
}
/* Code::scale (block.rs:15-17: widest magnitude over the code's MAX) and
 * Nibble::scale (block.rs:107-113: the widest value, sign kept, over -8). */
static float blk_code_scale(int form, const float *b, int n) {
    const int code = kForms[form].code;
    if (code == CD_NIB) {
        float top = 0.0f;
        for (int i = 0; i < n; i++) if (fabsf(b[i]) > fabsf(top)) top = b[i];
        return top / -8.0f;
    }
    float m = 0.0f;
    for (int i = 0; i < n; i++) m = fmaxf(m, fabsf(b[i]));
    return m / (code == CD_I8 ? 127.0f : code == CD_E4M3 ? 448.0f : 6.0f);
}
static void blk_put(int form, float scale, uint8_t *at) {
    switch (kForms[form].scale) {
    case SC_E8M0: at[0] = or_e8m0_narrow(scale); return;
    case SC_E4M3: at[0] = or_e4m3_narrow(scale); return;
    default: {
        uint16_t h = or_f16_narrow(scale);
        at[0] = (uint8_t)h; at[1] = (uint8_t)(h >> 8);
    }
    }
}
static float blk_get(int form, const uint8_t *at) {
    switch (kForms[form].scale) {
    case SC_E8M0: return or_e8m0_widen(at[0]);
    case SC_E4M3: return or_e4m3_widen(at[0]);
    default: return or_f16_widen((uint16_t)(at[0] | (at[1] << 8)));
    }
}
/* head (block.rs:141-146): the f32 at the tensor's start, else 1.0. */
static float blk_head(int form, const uint8_t *bytes) {
    if (!kForms[form].head) return 1.0f;
    float h;
    memcpy(&h, bytes, 4);
    return h;
}

/* pack (block.rs:229-248, tensor_scale :148-158): the head is the widest block scale
 * over the scale type's MAX (E4M3: 448) when the form has one and it is not 0; each
 * block's scale is its code scale over the head, stored; codes are the values over
 * the stored scale times the head (0 when that is 0). `out` must be zeroed. */
EXPORT void or_block_pack(int form, const float *data, int64_t n, uint8_t *out) {
    const BlkSpec *f = &kForms[form];
    const int B = f->B, bb = or_block_bytes(form), sb = blk_scale_bytes(form), hb = or_block_head(form);
    float tensor = 1.0f;
    if (f->head) {
        float widest = 0.0f;
        for (int64_t b = 0; b * B < n; b++) {
            const int cnt = (int)(n - b * B < B ? n - b * B : B);
            widest = fmaxf(widest, fabsf(blk_code_scale(form, data + b * B, cnt)));
        }
        if (widest > 0.0f) tensor = widest / 448.0f;
        memcpy(out, &tensor, 4);
    }
    for (int64_t b = 0; b * B < n; b++) {
        const int cnt = (int)(n - b * B < B ? n - b * B : B);
        uint8_t *at = out + hb + b * bb;
        blk_put(form, blk_code_scale(form, data + b * B, cnt) / tensor, at);
        const float stored = blk_get(form, at) * tensor;
        for (int j = 0; j < cnt; j++) {
            const float scaled = stored == 0.0f ? 0.0f : data[b * B + j] / stored;
            int byte, shift;
            blk_place(form, j, &byte, &shift);
            at[sb + byte] |= (uint8_t)(blk_encode(form, scaled) << shift);
        }
    }
}

/* unpack (block.rs:219-225): head * scale * decode(code) for element `index`. */
EXPORT float or_block_unpack(int form, const uint8_t *bytes, int64_t index) {
    const int B = kForms[form].B;
    const uint8_t *at = bytes + or_block_head(form) + (index / B) * or_block_bytes(form);
    int byte, shift;
    blk_place(form, (int)(index % B), &byte, &shift);
    const uint32_t code = ((uint32_t)at[blk_scale_bytes(form) + byte] >> shift) & ((1u << blk_bits(form)) - 1);
    const float sw = blk_get(form, at) * blk_decode(form, code);
    return blk_head(form, bytes) * sw;
}

EXPORT void or_block_unpack_n(int form, const uint8_t *bytes, int64_t first, int64_t count, float *out) {
    for (int64_t i = 0; i < count; i++) out[i] = or_block_unpack(form, bytes, first + i);
}

/* dot (block.rs:202-217): from element `at` (a block start) of the tensor, per block
 * part = sum_j x_j decode(c_j) from 0.0 in j order; sum += scale * part in block
 * order; the head times the sum. */
EXPORT float or_block_dot(int form, const float *x, const uint8_t *bytes, int64_t at, int64_t n) {
    const int B = kForms[form].B, bb = or_block_bytes(form), sb = blk_scale_bytes(form);
    const uint32_t mask = (1u << blk_bits(form)) - 1;
    const float head = blk_head(form, bytes);
    float sum = 0.0f;
    for (int64_t b = 0; b * B < n; b++) {
        const uint8_t *blk = bytes + or_block_head(form) + (at / B + b) * bb;
        float part = 0.0f;
        for (int j = 0; j < B && b * B + j < n; j++) {
            int byte, shift;
            blk_place(form, j, &byte, &shift);
            const float prod = x[b * B + j] * blk_decode(form, ((uint32_t)blk[sb + byte] >> shift) & mask);
            part = part + prod;
        }
        const float sp = blk_get(form, blk) * part;
        sum = sum + sp;
    }
    return head * sum;
}

/* out[m, r] = dot(x[m], the tensor from element r k) for a [n, k] tensor (k a multiple
 * of the block). */
EXPORT void or_block_product(int form, int64_t m, int64_t n, int64_t k, const float *x, const uint8_t *w,
                             float *out) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t r = 0; r < n; r++)
        for (int64_t i = 0; i < m; i++) out[i * n + r] = or_block_dot(form, x + i * k, w, r * k, k);
}

EXPORT void or_bf16_narrow_n(const float *x, uint16_t *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = or_bf16_narrow(x[i]);
}
EXPORT void or_bf16_widen_n(const uint16_t *b, float *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = or_bf16_widen(b[i]);
}
EXPORT void or_e4m3_narrow_n(const float *x, uint8_t *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = or_e4m3_narrow(x[i]);
}
EXPORT void or_e4m3_widen_n(const uint8_t *b, float *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = or_e4m3_widen(b[i]);
}

/* ------------------------------------------------------------------ */
/* Noise: engine/ir/testkit/src/noise.rs:5-10                          */
/* ------------------------------------------------------------------ */

EXPORT void or_noise(uint64_t *state, float *out, int64_t n) {
    uint64_t s = *state;
    for (int64_t i = 0; i < n; i++) {
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        out[i] = (float)(s >> 40) / (float)(1ull << 23) - 1.0f;
    }
    *state = s;
}

/* ------------------------------------------------------------------ */
/* Accumulator and product: round.rs:8-34, cpu.rs:82-138               */
/* ------------------------------------------------------------------ */

/* Acc::dot with an f32 accumulator: sequential, from 0.0. */
static inline float dot_f32(const float *a, const float *b, int64_t k) {
    float s = 0.0f;
    for (int64_t i = 0; i < k; i++) s = s + a[i] * b[i];
    return s;
}

/* Acc::add for the narrow accumulators (round.rs:18-25). acc: 0 f32, 1 f16 (unused), 2 bf16. */
EXPORT float or_acc_sum(int acc, const float *v, int64_t n) {
    float s = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        s = s + v[i];
        if (acc == 2) s = or_bf16_widen(or_bf16_narrow(s));
        if (acc == 1) s = widen_fmt(narrow_fmt(s, 5, 10, 1, 1), 5, 10, 1, 1);
    }
    return s;
}

/* out[m,n] = sum_k x[m,k] * w[n,k], w already f32 (product, cpu.rs:108-138). */
EXPORT void or_product(int64_t m, int64_t n, int64_t k, const float *x, const float *w, float *out) {
    #pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
    for (int64_t c = 0; c < n; c++)
        for (int64_t r = 0; r < m; r++) out[r * n + c] = dot_f32(x + r * k, w + c * k, k);
}

/* The same product with w stored bf16 and widened per element (run.rs:232-237).
 * Eight rows share each widened weight row; each output keeps its own
 * accumulator and ascending-k order, so the result equals one dot per output. */
static void rows_dot(int64_t m, int64_t n, int64_t k, const float *x, const float *row, float *out, int64_t c) {
    int64_t r = 0;
    for (; r + 8 <= m; r += 8) {
        float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int64_t i = 0; i < k; i++) {
            const float w = row[i];
            for (int j = 0; j < 8; j++) s[j] = s[j] + x[(r + j) * k + i] * w;
        }
        for (int j = 0; j < 8; j++) out[(r + j) * n + c] = s[j];
    }
    for (; r < m; r++) out[r * n + c] = dot_f32(x + r * k, row, k);
}

/* Few rows: eight columns at a time, each with its own accumulator. */
static void cols_dot(int64_t m, int64_t n, int64_t k, const float *x, const uint16_t *w, float *out, int64_t c0,
                     float *rows) {
    for (int j = 0; j < 8; j++)
        for (int64_t i = 0; i < k; i++) rows[j * k + i] = widen16(w[(c0 + j) * k + i]);
    for (int64_t r = 0; r < m; r++) {
        float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        const float *xr = x + r * k;
        for (int64_t i = 0; i < k; i++)
            for (int j = 0; j < 8; j++) s[j] = s[j] + xr[i] * rows[j * k + i];
        for (int j = 0; j < 8; j++) out[r * n + c0 + j] = s[j];
    }
}

EXPORT void or_product_bf16w(int64_t m, int64_t n, int64_t k, const float *x, const uint16_t *w,
                             float *out) {
    #pragma omp parallel num_threads(g_threads) if (g_threads > 1)
    {
        float *row = (float *)malloc(sizeof(float) * (size_t)k * 8);
        if (m < 8) {
            #pragma omp for schedule(static)
            for (int64_t b = 0; b < n / 8; b++) cols_dot(m, n, k, x, w, out, b * 8, row);
            #pragma omp single
            for (int64_t c = n / 8 * 8; c < n; c++) {
                for (int64_t i = 0; i < k; i++) row[i] = widen16(w[c * k + i]);
                rows_dot(m, n, k, x, row, out, c);
            }
        } else {
            #pragma omp for schedule(static)
            for (int64_t c = 0; c < n; c++) {
                for (int64_t i = 0; i < k; i++) row[i] = widen16(w[c * k + i]);
                rows_dot(m, n, k, x, row, out, c);
            }
        }
        free(row);
    }
}

/* Per-output-channel fp8: w = e4m3(code) * scale[row], widened then multiplied in f32
 * (frontend/checkpoint/src/exlr8.rs:133-137 dequantizes this way at load). */
EXPORT void or_product_e4m3w(int64_t m, int64_t n, int64_t k, const float *x, const uint8_t *w,
                             const uint16_t *scale, float *out) {
    #pragma omp parallel num_threads(g_threads) if (g_threads > 1)
    {
        float *row = (float *)malloc(sizeof(float) * (size_t)k);
        #pragma omp for schedule(static)
        for (int64_t c = 0; c < n; c++) {
            float s = or_bf16_widen(scale[c]);
            for (int64_t i = 0; i < k; i++) row[i] = or_e4m3_widen(w[c * k + i]) * s;
            for (int64_t r = 0; r < m; r++) out[r * n + c] = dot_f32(x + r * k, row, k);
        }
        free(row);
    }
}

/* matmul_picked (cpu.rs:89-105): output row b multiplies matrix ids[b]-first, or zeros. */
EXPORT void or_product_picked_bf16w(int64_t rows, int64_t m, int64_t n, int64_t k, const float *x,
                                    const uint16_t *table, int64_t experts, const uint32_t *ids,
                                    int64_t first, float *out) {
    /* product(): rows = max(m, batches); x row = r / (rows / m). */
    int64_t per = rows / (m > 0 ? m : 1);
    #pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
    for (int64_t r = 0; r < rows; r++) {
        const float *xr = x + (r / per) * k;
        int64_t e = (int64_t)ids[r] - first;
        for (int64_t c = 0; c < n; c++) {
            if (e < 0 || e >= experts) { out[r * n + c] = 0.0f; continue; }
            const uint16_t *wr = table + (e * n + c) * k;
            float s = 0.0f;
            for (int64_t i = 0; i < k; i++) s = s + xr[i] * or_bf16_widen(wr[i]);
            out[r * n + c] = s;
        }
    }
}

/* ------------------------------------------------------------------ */
/* Row stages: cpu.rs:8-59, 353-447, 492-495                           */
/* ------------------------------------------------------------------ */

enum { ACT_GELU_TANH = 0, ACT_SILU = 1, ACT_SIGMOID = 2, ACT_RELU = 3, ACT_SOFTPLUS = 4,
       ACT_EXP = 5, ACT_TANH = 6 };

static float act1(int a, float x) {
    switch (a) {
    case ACT_GELU_TANH: {
        const float coef = 0.7978846f;
        return 0.5f * x * (1.0f + tanhf(coef * (x + 0.044715f * x * x * x)));
    }
    case ACT_SILU: return x / (1.0f + expf(-x));
    case ACT_SIGMOID: return 1.0f / (1.0f + expf(-x));
    case ACT_RELU: return x > 0.0f ? x : 0.0f;
    case ACT_SOFTPLUS: return fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x)));
    case ACT_EXP: return expf(x);
    case ACT_TANH: return tanhf(x);
    }
    return NAN;
}

EXPORT void or_act(int a, float *x, int64_t n) {
    for (int64_t i = 0; i < n; i++) x[i] = act1(a, x[i]);
}

/* softmax (cpu.rs:49-59): max fold, exp, sequential sum, divide. */
static void softmax_row(float *row, int64_t w) {
    float mx = -INFINITY;
    for (int64_t i = 0; i < w; i++) mx = fmaxf(mx, row[i]);
    float sum = 0.0f;
    for (int64_t i = 0; i < w; i++) { row[i] = expf(row[i] - mx); sum = sum + row[i]; }
    for (int64_t i = 0; i < w; i++) row[i] /= sum;
}

EXPORT void or_softmax(float *x, int64_t rows, int64_t width) {
    for (int64_t r = 0; r < rows; r++) softmax_row(x + r * width, width);
}

/* rms_inverse (cpu.rs:492-495). */
static float rms_inverse(const float *row, int64_t w, float eps) {
    float s = 0.0f;
    for (int64_t i = 0; i < w; i++) s = s + row[i] * row[i];
    float mean = s / (float)w;
    return 1.0f / sqrtf(mean + eps);
}

/* RmsNorm: v *= inv * g (cpu.rs:371-377). g == NULL gives Rms. */
EXPORT void or_rms_norm(float *x, int64_t rows, int64_t width, const float *g, float eps) {
    for (int64_t r = 0; r < rows; r++) {
        float *row = x + r * width;
        float inv = rms_inverse(row, width, eps);
        for (int64_t i = 0; i < width; i++) row[i] *= g ? inv * g[i] : inv;
    }
}

/* angle (cpu.rs:32-34). */
EXPORT float or_angle(int64_t pos, int64_t j, int64_t width, float theta) {
    return (float)pos * powf(theta, -((float)(2 * j)) / (float)width);
}

/* Rope (cpu.rs:36-47, 396-413): `len` elements split into one equal block per position;
 * each block rotates row by row (rows `width` wide). pairs: 0 = Adjacent (2j, 2j+1),
 * 1 = Halves (j, j+w/2). turned < 0 means every pair. */
EXPORT void or_rope(float *x, int64_t len, int64_t n_pos, const uint32_t *pos,
                         int64_t width, float theta, int pairs, int64_t turned) {
    int64_t span = len / (n_pos > 0 ? n_pos : 1);
    if (span < 1) span = 1;
    int64_t half = width / 2;
    int64_t t = turned < 0 ? width : turned;
    int64_t lim = half < t ? half : t;
    for (int64_t b = 0; b < n_pos; b++) {
        for (int64_t r0 = b * span; r0 + width <= (b + 1) * span; r0 += width) {
            float *row = x + r0;
            for (int64_t j = 0; j < lim; j++) {
                int64_t a = pairs ? j : 2 * j, c = pairs ? j + half : 2 * j + 1;
                float ang = or_angle(pos[b], j, width, theta);
                float sn = sinf(ang), cs = cosf(ang);
                float va = row[a], vb = row[c];
                row[a] = va * cs - vb * sn;
                row[c] = va * sn + vb * cs;
            }
        }
    }
}

/* ------------------------------------------------------------------ */
/* Attention: cpu.rs:61-77 (past_keys, seen), 141-225 (attend),        */
/* 293-351 (attend_rows)                                                */
/* ------------------------------------------------------------------ */

/* Keys::row (cpu.rs:149-167): scores, softmax, then o += p*v key by key. */
static void attend_one(const float *q, int64_t d, int64_t dv, float scale, const float *const *krows,
                       const float *const *vrows, int64_t nk, float *p, float *o) {
    for (int64_t j = 0; j < nk; j++) p[j] = dot_f32(q, krows[j], d) * scale;
    softmax_row(p, nk);
    for (int64_t j = 0; j < nk; j++)
        for (int64_t i = 0; i < dv; i++) o[i] = o[i] + p[j] * vrows[j][i];
}

/* seen (cpu.rs:71-77), with window (back, ahead) already resolved by the caller. */
static void seen(int64_t back, int64_t ahead, int64_t position, int64_t keys, int64_t *from, int64_t *to) {
    *from = position > back ? position - back : 0;
    int64_t t = position + ahead + 1;
    *to = t < keys ? t : keys;
}

/* attend (cpu.rs:172-225) for whole sequences. q [seqs,ctx,heads,d], k [seqs,keys,kvh,d],
 * v [seqs,keys,kvh,dv], out [seqs,ctx,heads,dv]. back/ahead: the mask window (use a huge
 * value for "all"). causal: 1 when query and key ends align. Returns -1 on a mismatch. */
EXPORT int or_attend(int64_t seqs, int64_t ctx, int64_t keys, int64_t heads, int64_t kv_heads,
                     int64_t d, int64_t dv, float scale, int64_t back, int64_t ahead, int causal,
                     const float *q, const float *k, const float *v, float *out) {
    int64_t past;
    if (keys >= ctx) past = keys - ctx;
    else if (!causal) past = 0;
    else return -1;
    int64_t group = heads / kv_heads;
    memset(out, 0, sizeof(float) * (size_t)(seqs * ctx * heads * dv));
    int rc = 0;
    #pragma omp parallel num_threads(g_threads) if (g_threads > 1)
    {
        float *p = (float *)malloc(sizeof(float) * (size_t)(keys + 1));
        const float **kr = (const float **)malloc(sizeof(void *) * (size_t)(keys + 1));
        const float **vr = (const float **)malloc(sizeof(void *) * (size_t)(keys + 1));
        #pragma omp for collapse(2) schedule(static)
        for (int64_t s = 0; s < seqs; s++)
            for (int64_t t = 0; t < ctx; t++) {
                int64_t from, to;
                seen(back, ahead, past + t, keys, &from, &to);
                for (int64_t h = 0; h < heads; h++) {
                    int64_t row = (s * ctx + t) * heads + h, nk = 0;
                    for (int64_t j = from; j < to; j++) {
                        int64_t at = (s * keys + j) * kv_heads + h / group;
                        kr[nk] = k + at * d;
                        vr[nk] = v + at * dv;
                        nk++;
                    }
                    attend_one(q + row * d, d, dv, scale, kr, vr, nk, p, out + row * dv);
                }
            }
        free(p); free(kr); free(vr);
    }
    return rc;
}

/* Paged::row (codegen/src/kept.rs:181-193). page is a power of two. */
EXPORT uint64_t or_paged_row(const uint32_t *table, uint32_t kept_pages, uint32_t page,
                             uint32_t slot, uint32_t pos) {
    uint32_t shift = (uint32_t)__builtin_ctz(page);
    uint64_t entry = (uint64_t)slot * kept_pages + (pos >> shift);
    return ((uint64_t)table[entry] << shift) | (pos & (page - 1));
}

/* attend_rows (cpu.rs:293-351). q [rows,heads,d]; kept K/V rows are addressed by
 * (slot, position): dense layout row = slot*keys + j when table == NULL, else the paged
 * row through `table` (kept_pages entries per slot, `page` rows per page). K rows are
 * [*, kv_heads, d], V rows [*, kv_heads, dv]. Returns -1 when a position is past keys. */
EXPORT int or_attend_rows(int64_t rows, int64_t heads, int64_t kv_heads, int64_t d, int64_t dv,
                          float scale, int64_t back, int64_t ahead, int64_t keys,
                          const float *q, const float *k, const float *v,
                          const uint32_t *slots, const uint32_t *positions,
                          const uint32_t *table, uint32_t kept_pages, uint32_t page, float *out) {
    for (int64_t r = 0; r < rows; r++)
        if ((int64_t)positions[r] >= keys) return -1;
    int64_t group = heads / kv_heads;
    memset(out, 0, sizeof(float) * (size_t)(rows * heads * dv));
    #pragma omp parallel num_threads(g_threads) if (g_threads > 1)
    {
        float *p = (float *)malloc(sizeof(float) * (size_t)(keys + 1));
        const float **kr = (const float **)malloc(sizeof(void *) * (size_t)(keys + 1));
        const float **vr = (const float **)malloc(sizeof(void *) * (size_t)(keys + 1));
        #pragma omp for collapse(2) schedule(static)
        for (int64_t r = 0; r < rows; r++)
            for (int64_t h = 0; h < heads; h++) {
                int64_t from, to;
                seen(back, ahead, positions[r], keys, &from, &to);
                int64_t row = r * heads + h, nk = 0;
                for (int64_t j = from; j < to; j++) {
                    uint64_t kept = table ? or_paged_row(table, kept_pages, page, slots[r], (uint32_t)j)
                                          : (uint64_t)slots[r] * (uint64_t)keys + (uint64_t)j;
                    int64_t at = (int64_t)kept * kv_heads + h / group;
                    kr[nk] = k + at * d;
                    vr[nk] = v + at * dv;
                    nk++;
                }
                attend_one(q + row * d, d, dv, scale, kr, vr, nk, p, out + row * dv);
            }
        free(p); free(kr); free(vr);
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* Indices: top_k (run.rs:577-591), take (cpu.rs:498-508),             */
/* gather (cpu.rs:511-525), mean/mix (cpu.rs:450-473)                   */
/* ------------------------------------------------------------------ */

/* Stable merge sort of indices by descending value (ties keep the lower index). */
static void sort_desc(uint32_t *ix, uint32_t *tmp, const float *row, int64_t n) {
    for (int64_t w = 1; w < n; w *= 2) {
        for (int64_t lo = 0; lo < n; lo += 2 * w) {
            int64_t mid = lo + w < n ? lo + w : n, hi = lo + 2 * w < n ? lo + 2 * w : n;
            int64_t a = lo, b = mid, o = lo;
            while (a < mid && b < hi) {
                /* take b first only when strictly greater: stability */
                if (row[ix[b]] > row[ix[a]]) tmp[o++] = ix[b++];
                else tmp[o++] = ix[a++];
            }
            while (a < mid) tmp[o++] = ix[a++];
            while (b < hi) tmp[o++] = ix[b++];
        }
        memcpy(ix, tmp, sizeof(uint32_t) * (size_t)n);
    }
}

/* ids[r, 0..k): row's largest finite entries best first; -inf and NaN skipped; spare = width. */
EXPORT void or_top_k(const float *x, int64_t rows, int64_t width, int64_t k, uint32_t *ids) {
    uint32_t *ix = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(width + 1));
    uint32_t *tmp = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(width + 1));
    for (int64_t r = 0; r < rows; r++) {
        const float *row = x + r * width;
        int64_t n = 0;
        for (int64_t i = 0; i < width; i++)
            if (row[i] > -INFINITY) ix[n++] = (uint32_t)i;
        sort_desc(ix, tmp, row, n);
        for (int64_t j = 0; j < k; j++) ids[r * k + j] = j < n ? ix[j] : (uint32_t)width;
    }
    free(ix); free(tmp);
}

/* take: each row's entries at ids; out-of-range reads 0. ids is [rows, picks]. */
EXPORT void or_take(const float *x, int64_t rows, int64_t width, const uint32_t *ids,
                    int64_t count, float *out) {
    int64_t picks = count / (rows > 0 ? rows : 1);
    if (picks < 1) picks = 1;
    for (int64_t j = 0; j < count; j++) {
        const float *row = x + (j / picks) * width;
        out[j] = ids[j] < (uint64_t)width ? row[ids[j]] : 0.0f;
    }
}

/* gather: rows of `table` (row_bytes each) at ids - first; others zero. */
EXPORT void or_gather(const void *table, int64_t rows, int64_t row_bytes, const uint32_t *ids,
                      int64_t count, int64_t first, void *out) {
    for (int64_t j = 0; j < count; j++) {
        int64_t r = (int64_t)ids[j] - first;
        uint8_t *o = (uint8_t *)out + j * row_bytes;
        if (r >= 0 && r < rows) memcpy(o, (const uint8_t *)table + r * row_bytes, (size_t)row_bytes);
        else memset(o, 0, (size_t)row_bytes);
    }
}

/* mean over `axis` of [outer, count, inner], weighted by w[outer, count] when given
 * (mix); the sum runs in ascending t. */
EXPORT void or_mix(const float *x, int64_t outer, int64_t count, int64_t inner, const float *w,
                   float *out) {
    for (int64_t o = 0; o < outer; o++)
        for (int64_t i = 0; i < inner; i++) {
            float s = 0.0f;
            for (int64_t t = 0; t < count; t++) {
                float wt = w ? w[o * count + t] : 1.0f / (float)count;
                s = s + x[(o * count + t) * inner + i] * wt;
            }
            out[o * inner + i] = s;
        }
}
