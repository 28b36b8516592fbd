// Block-scaled weight forms on the decode product (m <= 4 rows): the reference's
// seven block forms (q8_0, mxfp8, int4_g32, q4_0, nvfp4, mxfp4, int4_g128).
//
// Replaces the decode of a block form inside the few-row product: the reference's
// Block::dot (engine/ir/mem/src/block.rs:202-217) over the forms of block.rs:251-291,
// as the lanes rule reads them through a form's load (engine/plan/codegen/src/
// form.rs:10-93). blockform.h holds each form's layout and exact decode.
//
// gfx950 design. One wave per 4 weight rows. Blocks are 9 to 66 bytes, not 16-byte
// aligned: the wave streams its rows' bytes with coalesced 4-byte loads (all four rows
// in flight together) into its own LDS slices, one block per lane (64 blocks a
// slice), and lane l then decodes block l of each row. Each lane
// forms its block's part in the reference's order (x_j times the decoded code, summed
// from 0.0 in j order, no contraction), times the block scale; lane (row, m) then adds
// the contributions of activation row m in block order, and the head (nvfp4) scales
// the total. Every rounding step is the reference's, so the product is bit-identical
// to Block::dot for the same f32 activations. Rows of at most 32 blocks take the short
// form (block_gemv_short_kernel below): lanes over (row, block) pairs instead.
#include "blockform.h"

namespace ts {

namespace {

constexpr int kWaves = 4;
constexpr int kRows = 4;    // weight rows per wave, their loads overlapped

struct BlockParams {
    const void *x;
    const uint8_t *w;  // the packed tensor (head included)
    const float *a0;
    void *out;
    uint32_t m, n, k;
    uint32_t stages;
    int out_bf16;
    uint32_t wide;  // short form: rows of whole 16-byte chunks, 16-byte aligned (16-byte loads)
    ts_after after;  // stage chain (count 0: none)
};

// Blocks per LDS slice: one per lane (a 128-code block's part is one ordered sum, so
// it cannot be split over lanes; its slices take 66 KiB of LDS for the four waves).
template <int F>
constexpr int chunk_blocks() { return 64; }

// Waits for this wave's LDS traffic so the other lanes' writes are visible.
TS_DEV void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt not waited on
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// x[k0 .. k0 + P) of one row as f32 (exact for bf16 rows).
template <int P, bool XF32>
TS_DEV void load_x(const void *x, size_t at, float *xv) {
    if (XF32) {
        const float4 *xs = (const float4 *)((const float *)x + at);
#pragma unroll
        for (int q = 0; q < P / 4; q++) {
            const float4 t = xs[q];
            xv[4 * q] = t.x; xv[4 * q + 1] = t.y; xv[4 * q + 2] = t.z; xv[4 * q + 3] = t.w;
        }
    } else {
        const u32x4 *xs = (const u32x4 *)((const uint16_t *)x + at);
#pragma unroll
        for (int q = 0; q < P / 8; q++) {
            const u32x4 t = xs[q];
            const uint32_t u[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                xv[8 * q + 2 * e] = lo_bf16(u[e]);
                xv[8 * q + 2 * e + 1] = hi_bf16(u[e]);
            }
        }
    }
}

// e2m1 codes of byte T of w (low nibble first) as f32 (scale 1: exact).
template <int T>
TS_DEV ts_f32x2_t fp4_pair(uint32_t w) { return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, T); }

// Codes q P .. q P + P - 1 of the block whose codes start at byte `at` of the LDS
// words `w` (exact, before the scale), read as aligned words split by alignbyte
// instead of byte reads; the word after the block's codes must be readable.
template <int F, int P>
TS_DEV void codes_from_words(const uint32_t *w, uint32_t at, int q, float *wv) {
    using BF = BlockForm<F>;
    if (BF::BITS == 8) {
        const uint32_t off = at + q * P, w0 = off >> 2, sh = off & 3u;
        uint32_t d[P / 4 + 1];
#pragma unroll
        for (int e = 0; e <= P / 4; e++) d[e] = w[w0 + e];
#pragma unroll
        for (int e = 0; e < P / 4; e++) {
            const uint32_t v = __builtin_amdgcn_alignbyte(d[e + 1], d[e], sh);
            if (BF::CODE == kCodeI8) {
#pragma unroll
                for (int t = 0; t < 4; t++) wv[4 * e + t] = (float)((int32_t)(v << (24 - 8 * t)) >> 24);
            } else {
                e4m3x4_float(v, wv + 4 * e);
            }
        }
    } else {
        // Byte i of a piece holds codes 2 i, 2 i + 1 (low nibble first), or i and
        // i + B / 2 (q4_0's halves).
        const uint32_t off = at + q * (P / 2), w0 = off >> 2, sh = off & 3u;
        uint32_t d[P / 8 + 1];
#pragma unroll
        for (int e = 0; e <= P / 8; e++) d[e] = w[w0 + e];
#pragma unroll
        for (int e = 0; e < P / 8; e++) {
            const uint32_t v = __builtin_amdgcn_alignbyte(d[e + 1], d[e], sh);
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int i = 4 * e + t;
                if (BF::CODE == kCodeE2M1) {
                    const ts_f32x2_t c = t == 0 ? fp4_pair<0>(v) : t == 1 ? fp4_pair<1>(v)
                                       : t == 2 ? fp4_pair<2>(v) : fp4_pair<3>(v);
                    wv[2 * i] = c[0];
                    wv[2 * i + 1] = c[1];
                } else {
                    const float lo = (float)((v >> (8 * t)) & 15u) - 8.0f;
                    const float hi = (float)((v >> (8 * t + 4)) & 15u) - 8.0f;
                    if (BF::HALVES) {
                        wv[i] = lo;
                        wv[i + P / 2] = hi;
                    } else {
                        wv[2 * i] = lo;
                        wv[2 * i + 1] = hi;
                    }
                }
            }
        }
    }
}

template <int F, int M, bool XF32>
__global__ __launch_bounds__(kWaves * 64) void block_gemv_kernel(BlockParams p) {
#pragma clang fp contract(off)
    using BF = BlockForm<F>;
    constexpr int B = BF::B, BB = BF::BB, SB = BF::SB, CH = chunk_blocks<F>();
    constexpr int P = B < 32 ? B : 32;                   // elements decoded per piece
    constexpr int kSlice = CH * BB / 4;                  // words of one row's slice
    constexpr int kWords = (kSlice + 63) / 64;           // of them per lane
    // Each row's slice one word longer than its blocks: the aligned word reads of the
    // last block's codes.
    __shared__ __attribute__((aligned(16))) uint32_t stage[kWaves][kRows][kSlice + 4];
    __shared__ __attribute__((aligned(16))) float contrib[kWaves][kRows * M][CH];

    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t r0 = (blockIdx.x * kWaves + wave) * kRows;  // this wave's kRows rows
    if (r0 >= p.n) return;  // waves are independent: no group barrier below
    const uint32_t K = p.k, N = p.n, Mr = p.m, nb = K / B;
    const uint32_t nrows = min((uint32_t)kRows, N - r0);
    const uint8_t *rows = p.w + BF::HEAD;

    float run = 0.0f;  // lane rr * M + m: the running sum of output (m, r0 + rr)
    for (uint32_t c0 = 0; c0 < nb; c0 += CH) {
        const uint32_t cnt = min((uint32_t)CH, nb - c0), words = cnt * BB / 4;
        // Every word of the rows' slices in flight before any is written.
        uint32_t wt[kRows][kWords];
#pragma unroll
        for (int rr = 0; rr < kRows; rr++) {
            const uint32_t *src = (const uint32_t *)(rows + (size_t)(r0 + min((uint32_t)rr, nrows - 1)) * nb * BB) +
                                  (size_t)c0 * BB / 4;
#pragma unroll
            for (int q = 0; q < kWords; q++) {
                const uint32_t i = lane + 64 * q;
                wt[rr][q] = i < words ? __builtin_nontemporal_load(src + i) : 0u;
            }
        }
#pragma unroll
        for (int rr = 0; rr < kRows; rr++)
#pragma unroll
            for (int q = 0; q < kWords; q++)
                if (lane + 64 * q < words) stage[wave][rr][lane + 64 * q] = wt[rr][q];
        wave_lds_sync();
        if (lane < cnt) {
            const uint32_t k0 = (c0 + lane) * B;
#pragma unroll
            for (int m = 0; m < M; m++) {
                if ((uint32_t)m >= Mr) break;
                float part[kRows];
#pragma unroll
                for (int rr = 0; rr < kRows; rr++) part[rr] = 0.0f;
                // Block::dot's part: x_j times code j, summed from 0.0 in j order.
#pragma unroll
                for (int q = 0; q < B / P; q++) {
                    float xv[P];
                    load_x<P, XF32>(p.x, (size_t)m * K + k0 + q * P, xv);
#pragma unroll
                    for (int rr = 0; rr < kRows; rr++) {
                        float wv[P];
                        codes_from_words<F, P>(stage[wave][rr], lane * BB + SB, q, wv);
#pragma unroll
                        for (int j = 0; j < P; j++) part[rr] = part[rr] + xv[j] * wv[j];
                    }
                }
#pragma unroll
                for (int rr = 0; rr < kRows; rr++) {
                    const uint8_t *blk = (const uint8_t *)stage[wave][rr] + lane * BB;
                    contrib[wave][rr * M + m][lane] = block_scale<F>(blk) * part[rr];
                }
            }
        }
        wave_lds_sync();
        if (lane < kRows * M) {  // all contributions read first, then added in block order
            const float4 *cv = (const float4 *)contrib[wave][lane];
            float4 t[CH / 4];
#pragma unroll
            for (int q = 0; q < CH / 4; q++) t[q] = cv[q];
#pragma unroll
            for (int q = 0; q < CH / 4; q++)
                if ((uint32_t)(4 * q) < cnt) {  // cnt is a multiple of 4
                    run = run + t[q].x;
                    run = run + t[q].y;
                    run = run + t[q].z;
                    run = run + t[q].w;
                }
        }
        wave_lds_sync();  // the next slice overwrites stage and contrib
    }
    const uint32_t rr = lane / M, m = lane % M;
    if (lane >= kRows * M || rr >= nrows || m >= Mr) return;
    const float head = BF::HEAD ? *(const float *)p.w : 1.0f;  // Block::dot: head * sum
    float v = head * run;
    const size_t at = (size_t)m * N + r0 + rr;
    if (p.stages & TS_AFTER_ADD) v += p.a0[at];
    if (p.after.count) v = after_apply(p.after, v, at);
    if (p.out_bf16) ((uint16_t *)p.out)[at] = bf16_bits(v);
    else ((float *)p.out)[at] = v;
}

typedef __attribute__((address_space(3))) void block_lds_void;

constexpr uint32_t kShortBytes = 9200;  // LDS bytes of one wave's rows (short form; staged in 9 KiB + a word)

// Passes a wave of the short form with L lanes a row (64 / L rows a pass): 16 rows a
// wave, 8 at L = 32, so the rows' bytes fit kShortBytes. short_pick also takes 4 passes
// of 2 rows in twice the stage (or 2 passes) at L = 32 for rows too wide for 4 passes of
// 2 in one stage, and 4 passes at L = 8 for 128-code blocks.
constexpr int short_np(int L) { return L == 32 ? 4 : L == 16 ? 4 : 2; }

// Short rows (at most 32 blocks, e.g. 1024 codes of 32-code blocks, or of 128-code
// ones): L lanes a row (nb <= L), 64 / L rows a pass, so every lane decodes a block
// where the form above would leave 64 - nb lanes idle. A wave's NP passes (RT rows)
// are contiguous bytes: they go straight to LDS (global_load_lds, 16 bytes a lane when
// the rows are whole 16-byte chunks, else 4: no staging registers); a lane then runs
// its NP blocks (same block index, NP rows) as NP interleaved chains over one load of
// x. The arithmetic per block and the block-order sum of each output are those of
// block_gemv_kernel, so both give the same bits.
template <int F, int M, bool XF32, int L, int NP, uint32_t SBYTES = kShortBytes>
__global__ __launch_bounds__(kWaves * 64) void block_gemv_short_kernel(BlockParams p) {
#pragma clang fp contract(off)
    using BF = BlockForm<F>;
    constexpr int B = BF::B, BB = BF::BB, SB = BF::SB;
    constexpr int P = B < 32 ? B : 32;
    constexpr int G = 64 / L, RT = G * NP;
    static_assert(RT * M <= 64, "one lane an output");
    // Whole KiB (the loads' last instruction fills its KiB) and one word more: the
    // aligned word reads of the last block's codes.
    __shared__ __attribute__((aligned(16))) uint32_t stage[kWaves][(SBYTES + 1023) / 1024 * 256 + 4];
    __shared__ __attribute__((aligned(16))) float contrib[kWaves][RT * M][L];

    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t r0 = (blockIdx.x * kWaves + wave) * RT;  // this wave's RT rows
    if (r0 >= p.n) return;  // waves are independent: no group barrier below
    const uint32_t K = p.k, N = p.n, Mr = p.m, nb = K / B;
    const uint32_t nrows = min((uint32_t)RT, N - r0);
    const uint32_t words = nrows * (nb * BB / 4);
    const uint32_t *src = (const uint32_t *)(p.w + BF::HEAD + (size_t)r0 * nb * BB);
    char *base = (char *)stage[wave];
    if (p.wide) {  // 16-byte chunks (lane i of an instruction at 16 i)
        const uint32_t chunks = words / 4;
        for (uint32_t c0 = 0; c0 < chunks; c0 += 64) {
            const uint32_t i = min(c0 + lane, chunks - 1);  // past the end: a repeat, unused
            __builtin_amdgcn_global_load_lds((const void *)(src + 4 * i), (block_lds_void *)(base + 16 * c0), 16, 0, 0);
        }
    } else {
        for (uint32_t w0 = 0; w0 < words; w0 += 64) {
            const uint32_t i = min(w0 + lane, words - 1);  // past the end: a repeat, unused
            __builtin_amdgcn_global_load_lds((const void *)(src + i), (block_lds_void *)(base + 4 * w0), 4, 0, 0);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();

    const uint32_t b = lane % L, g = lane / L;
    if (b < nb) {
        const uint32_t k0 = b * B;
#pragma unroll
        for (int m = 0; m < M; m++) {
            if ((uint32_t)m >= Mr) break;
            float part[NP];
#pragma unroll
            for (int i = 0; i < NP; i++) part[i] = 0.0f;
            // Block::dot's part: x_j times code j, summed from 0.0 in j order.
#pragma unroll
            for (int q = 0; q < B / P; q++) {
                float xv[P];
                load_x<P, XF32>(p.x, (size_t)m * K + k0 + q * P, xv);
#pragma unroll
                for (int i = 0; i < NP; i++) {
                    const uint32_t rr = min(i * G + g, nrows - 1);  // rows past the end: unused
                    float wv[P];
                    codes_from_words<F, P>(stage[wave], (rr * nb + b) * BB + SB, q, wv);
#pragma unroll
                    for (int j = 0; j < P; j++) part[i] = part[i] + xv[j] * wv[j];
                }
            }
#pragma unroll
            for (int i = 0; i < NP; i++) {
                const uint32_t rr = i * G + g;
                const uint8_t *blk = (const uint8_t *)stage[wave] + (size_t)(min(rr, nrows - 1) * nb + b) * BB;
                contrib[wave][rr * M + m][b] = block_scale<F>(blk) * part[i];
            }
        }
    }
    wave_lds_sync();
    // Lane rr * M + m: output (m, r0 + rr), its blocks' contributions in block order.
    const uint32_t rr = lane / M, m = lane % M;
    if (lane >= RT * M || rr >= nrows || m >= Mr) return;
    const float *cv = contrib[wave][lane];
    float run = 0.0f;
    for (uint32_t j = 0; j < nb; j++) run = run + cv[j];
    const float head = BF::HEAD ? *(const float *)p.w : 1.0f;  // Block::dot: head * sum
    float v = head * run;
    const size_t at = (size_t)m * N + r0 + rr;
    if (p.stages & TS_AFTER_ADD) v += p.a0[at];
    if (p.after.count) v = after_apply(p.after, v, at);
    if (p.out_bf16) ((uint16_t *)p.out)[at] = bf16_bits(v);
    else ((float *)p.out)[at] = v;
}

using ShortKern = void (*)(BlockParams);

template <int F, bool XF32, int L, int NP = short_np(L), uint32_t SBYTES = kShortBytes>
ShortKern short_m(uint32_t m) {
    return m == 1 ? block_gemv_short_kernel<F, 1, XF32, L, NP, SBYTES>
         : m == 2 ? block_gemv_short_kernel<F, 2, XF32, L, NP, SBYTES>
                  : block_gemv_short_kernel<F, 4, XF32, L, NP, SBYTES>;
}

// L = 8 with 4 passes of 8 rows (32 rows a wave, 32 m outputs at most: m <= 2).
template <int F, bool XF32>
ShortKern short_l8_wide(uint32_t m) {
    return m == 1 ? block_gemv_short_kernel<F, 1, XF32, 8, 4, 2 * kShortBytes>
                  : block_gemv_short_kernel<F, 2, XF32, 8, 4, 2 * kShortBytes>;
}

// The short form for nb <= 32 blocks a row whose wave rows fit its stage, or NULL;
// *rows: the rows a wave of it takes.
template <int F>
ShortKern short_pick(uint32_t m, bool xf, uint32_t nb, uint32_t *rows) {
    using BF = BlockForm<F>;
    const int L = nb <= 8 ? 8 : nb <= 16 ? 16 : 32;
    if (nb > 32) return nullptr;
    *rows = (64 / L) * short_np(L);
    if ((uint64_t)*rows * nb * BF::BB > kShortBytes) {
        // Wide blocks (128 codes) at L = 32: 4 passes of 2 rows (8 rows a wave in twice
        // the stage, four chains a lane: 14336 x 4096 int4_g128 18.0 -> 13.2 us), else 2
        // passes (4 rows a wave). (8 passes of the 32-code forms' rows measured slower:
        // half the waves.)
        if (L == 32 && (uint64_t)8 * nb * BF::BB <= 2 * kShortBytes) {
            *rows = 8;
            return xf ? short_m<F, true, 32, 4, 2 * kShortBytes>(m) : short_m<F, false, 32, 4, 2 * kShortBytes>(m);
        }
        *rows = 4;
        if (L == 32 && (uint64_t)4 * nb * BF::BB <= kShortBytes)
            return xf ? short_m<F, true, 32, 2>(m) : short_m<F, false, 32, 2>(m);
        return nullptr;
    }
    if (L == 8) {
        // 128-code blocks: 4 passes of 8 rows (a wave's 32 rows in 17 KiB, two groups a
        // CU) instead of 2.
        if (BF::B == 128 && m <= 2 && (uint64_t)32 * nb * BF::BB <= 2 * kShortBytes) {
            *rows = 32;
            return xf ? short_l8_wide<F, true>(m) : short_l8_wide<F, false>(m);
        }
        return xf ? short_m<F, true, 8>(m) : short_m<F, false, 8>(m);
    }
    if (L == 16) return xf ? short_m<F, true, 16>(m) : short_m<F, false, 16>(m);
    return xf ? short_m<F, true, 32>(m) : short_m<F, false, 32>(m);
}

using Kern = void (*)(BlockParams);

template <int F, bool XF32>
Kern pick_m(uint32_t m) {
    return m == 1 ? block_gemv_kernel<F, 1, XF32>
         : m == 2 ? block_gemv_kernel<F, 2, XF32> : block_gemv_kernel<F, 4, XF32>;
}

template <int F>
Kern pick_x(uint32_t m, bool xf) {
    return xf ? pick_m<F, true>(m) : pick_m<F, false>(m);
}

template <int F>
constexpr BlockShape shape_of() {
    using BF = BlockForm<F>;
    return BlockShape{BF::B, BF::BB, BF::HEAD};
}

}  // namespace

bool block_form(int32_t dtype) { return dtype >= TS_Q8_0 && dtype <= TS_INT4_G128; }

BlockShape block_shape(int32_t dtype) {
    constexpr BlockShape s[7] = {shape_of<0>(), shape_of<1>(), shape_of<2>(), shape_of<3>(),
                                 shape_of<4>(), shape_of<5>(), shape_of<6>()};
    return s[dtype - TS_Q8_0];
}

int block_check(const ts_linear_args *a, const char *rule) {
    TS_REQUIRE(a && a->x && a->w && a->out, "%s (block form): null pointer", rule);
    const BlockShape bs = block_shape(a->w_dtype);
    TS_REQUIRE(a->n >= 1 && a->k >= 128 && a->k % (4 * bs.block) == 0,
               "%s (block form): k=%u must be a multiple of %u and at least 128", rule, a->k, 4 * bs.block);
    TS_REQUIRE(a->x_dtype == TS_F32 || a->x_dtype == TS_BF16, "%s (block form): x dtype %d", rule, a->x_dtype);
    TS_REQUIRE(a->out_dtype == TS_F32 || a->out_dtype == TS_BF16, "%s (block form): out dtype %d", rule,
               a->out_dtype);
    TS_REQUIRE(!(a->stages & TS_AFTER_ADD) || a->a0, "%s (block form): TS_AFTER_ADD needs a0", rule);
    TS_REQUIRE(aligned(a->x, 16) && aligned(a->w, 4), "%s (block form): x 16-byte and w 4-byte aligned", rule);
    return TS_OK;
}

int block_gemv_launch(const ts_linear_args *a, void *stream) {
    const int bad = block_check(a, "lanes");
    if (bad) return bad;
    TS_REQUIRE(a->m >= 1 && a->m <= 4, "lanes (block form): m=%u outside 1..4 (the decode product)", a->m);
    TS_REQUIRE((a->stages & ~TS_AFTER_ADD) == 0, "lanes (block form): stages %#x (only TS_AFTER_ADD)", a->stages);
    BlockParams p;
    p.x = a->x; p.w = (const uint8_t *)a->w; p.a0 = a->a0; p.out = a->out;
    p.m = a->m; p.n = a->n; p.k = a->k; p.stages = a->stages; p.out_bf16 = a->out_dtype == TS_BF16;
    const int rc = linear_after(a, "lanes (block form)", &p.after);
    if (rc) return rc;
    {
        const BlockShape bs = block_shape(a->w_dtype);
        p.wide = (a->k / bs.block) * bs.bytes % 16 == 0 && aligned((const uint8_t *)a->w + bs.head, 16);
    }
    const bool xf = a->x_dtype == TS_F32;
    const uint32_t nb = a->k / block_shape(a->w_dtype).block;
    ShortKern sk = nullptr;
    uint32_t rows = 0;
    switch (a->w_dtype) {
    case TS_Q8_0: sk = short_pick<0>(a->m, xf, nb, &rows); break;
    case TS_MXFP8: sk = short_pick<1>(a->m, xf, nb, &rows); break;
    case TS_INT4_G32: sk = short_pick<2>(a->m, xf, nb, &rows); break;
    case TS_Q4_0: sk = short_pick<3>(a->m, xf, nb, &rows); break;
    case TS_NVFP4: sk = short_pick<4>(a->m, xf, nb, &rows); break;
    case TS_MXFP4: sk = short_pick<5>(a->m, xf, nb, &rows); break;
    default: sk = short_pick<6>(a->m, xf, nb, &rows); break;
    }
    if (sk) {
        const uint32_t waves = (a->n + rows - 1) / rows;
        hipLaunchKernelGGL(sk, dim3((waves + kWaves - 1) / kWaves), dim3(kWaves * 64), 0, (hipStream_t)stream, p);
        TS_CHECK_LAUNCH("lanes (block form, short rows) launch");
        return TS_OK;
    }
    Kern k;
    switch (a->w_dtype) {
    case TS_Q8_0: k = pick_x<0>(a->m, xf); break;
    case TS_MXFP8: k = pick_x<1>(a->m, xf); break;
    case TS_INT4_G32: k = pick_x<2>(a->m, xf); break;
    case TS_Q4_0: k = pick_x<3>(a->m, xf); break;
    case TS_NVFP4: k = pick_x<4>(a->m, xf); break;
    case TS_MXFP4: k = pick_x<5>(a->m, xf); break;
    default: k = pick_x<6>(a->m, xf); break;
    }
    hipLaunchKernelGGL(k, dim3((a->n + kWaves * kRows - 1) / (kWaves * kRows)), dim3(kWaves * 64), 0, (hipStream_t)stream, p);
    TS_CHECK_LAUNCH("lanes (block form) launch");
    return TS_OK;
}

}  // namespace ts
