// The whole greedy decode step of a Qwen3-shaped decoder in one persistent launch.
//
// What it computes is the launch sequence of the graph runner (qwen3.hip), which
// is the reference's lowered decode step (engine/models/src/decoder.rs:327-391;
// engine/engine/src/lib.rs:401-470): per layer RmsNorm -> qkv product -> q/k
// RmsNorm per head, Halves RoPE, kept-row append, attention -> o product + residual
// -> RmsNorm -> gate/up products, silu(gate) * up -> down product + residual; then
// the final RmsNorm, the tied lm_head and the greedy pick (argmax.rs:74-129). The
// arithmetic of every stage is the one of the kernels it replaces (gemv.hip,
// attention.hip, rows.hip): f32 activations, bf16 weights widened exactly, f32 sums.
//
// Why one launch. At batch 1 every product only streams its weights (31 MB per
// layer), and a graph of 5 kernels per layer spends ~31 us per layer in per-kernel
// ramp and drain against ~4 us of HBM time. Here one group per CU lives for the
// whole decode call and:
//  * a group owns fixed rows of every matrix (ceil(N / groups) rows);
//  * two DMA waves stream those rows, phase after phase and layer after layer,
//    straight into a 128 KiB LDS ring with global_load_lds (no registers), up to a
//    ring ahead of the compute, so HBM stays busy while the compute waits for the
//    previous phase's activations;
//  * six compute waves hand activations between phases through "tagged" words in
//    HBM: each output value is one 8-byte store of (f32 value, u32 epoch) at agent
//    scope (coherent across XCDs), and a consumer polls the words it needs until
//    every epoch matches. The data is its own flag: no counters, no fences, no
//    cache write-back, one memory round trip per hand-off;
//  * all eight waves meet at hardware barriers. The DMA waves walk the same
//    schedule of barriers as the compute waves: before the barrier that starts a
//    phase they wait (vmcnt) for that phase's rows, after the barrier that ends it
//    they reuse its ring slots. Ring occupancy is known, never signalled;
//  * the first q_heads groups also run the attention of one q head each, with
//    the kept rows of earlier positions loaded before the q/k/v hand-off arrives;
//  * the lm_head rows stream through the same ring in chunks; every group publishes
//    its (max, index), and every group reduces all of them, so the next step's
//    token needs no extra hand-off.
// Waits are bounded: a poll that passes 2 s (100 MHz clock) sets the error word;
// every poll also watches that word, and a failed poll lets its group run on
// without waiting, so the grid always reaches its last barrier and ends. Groups
// are launched cooperatively (all resident), one per CU.
#include <string.h>

#include "common.h"
#include "decode_step.h"

namespace ts {
namespace {

typedef __attribute__((address_space(3))) void lds_void;

constexpr uint32_t kCW = 6;                    // compute waves
constexpr uint32_t kDW = 2;                    // DMA waves
constexpr uint32_t kCT = kCW * 64;             // compute threads
constexpr uint32_t kThreads = (kCW + kDW) * 64;
constexpr uint32_t kRing = 128;                // ring units of 1 KiB
constexpr uint32_t kMaxOut = 56;               // DMA loads in flight per wave (vmcnt holds 63)
constexpr uint32_t kBurst = 8;                 // DMA loads a wave issues per barrier
constexpr uint32_t kLmBurst = 24;              // the same in the lm_head chunks (7 us a token over 8)
constexpr uint32_t kRW = 4;                    // product rows per compute wave
constexpr uint32_t kChunk = kRW * kCW;         // lm_head rows per chunk
constexpr uint32_t kMaxXa = 3072;              // staged input floats (H, Hq*128 and F)
constexpr uint32_t kMaxH = 1024;
constexpr uint32_t kMaxPages = 512;
constexpr uint64_t kTimeout = 200000000ull;    // 2 s of the 100 MHz clock
constexpr int kNX = (kMaxXa + kCT - 1) / kCT;  // staged words per compute thread (widest input)
constexpr int kNH = (kMaxH + kCT - 1) / kCT;   // staged words per compute thread (hidden-wide input)
constexpr uint32_t kMaxGroups = 448;           // groups the step supports (2 pick words each)
constexpr int kNA = (2 * kMaxGroups + kCT - 1) / kCT;
constexpr int kPre = 7;                        // 4-key blocks per wave loaded before q arrives
static_assert(kCW >= 4 && kCW <= 8, "attention uses waves 0..3 and LDS partials for up to 8 waves");

// LDS layout (bytes).
constexpr uint32_t kRingOff = 0;
constexpr uint32_t kXaOff = kRingOff + kRing * 1024;
constexpr uint32_t kXrOff = kXaOff + kMaxXa * 4;
constexpr uint32_t kRedOff = kXrOff + kMaxH * 4;
constexpr uint32_t kTblOff = kRedOff + 1024 * 4;
constexpr uint32_t kSsqOff = kTblOff + kMaxPages * 4;
constexpr uint32_t kCtlOff = kSsqOff + 16 * 4;
constexpr uint32_t kLdsBytes = kCtlOff + 16 * 4;
// Control words.
constexpr uint32_t kAbort = 0;  // a wait of this group gave up
constexpr uint32_t kTok = 1;    // the step's token

TS_DEV uint32_t units(uint32_t bytes) { return (bytes + 1023) >> 10; }

// Rows [first, first + count) of N split over NG groups, ceil(N / NG) each.
struct Split {
    uint32_t first, count;
};
TS_DEV Split split(uint32_t n, uint32_t ng, uint32_t g) {
    const uint32_t per = (n + ng - 1) / ng;
    const uint32_t f = min(n, g * per);
    return {f, min(n, f + per) - f};
}

// This group's rows of every matrix, and the stream units they take.
struct Plan {
    Split q, o, f, v;  // qkv rows, o/down rows, gate (and up) rows, lm_head rows
    uint32_t uq, uo, ug, ud, layer, chunks, step;
    uint32_t QKV, QD;
};
TS_DEV uint32_t chunk_units(const DecodeStepArgs &p, const Plan &pl, uint32_t c) {
    return units(min(kChunk, pl.v.count - c * kChunk) * p.H * 2);
}
TS_DEV Plan plan(const DecodeStepArgs &p, uint32_t g) {
    Plan pl;
    pl.QD = p.Hq * 128;
    pl.QKV = (p.Hq + 2 * p.Hkv) * 128;
    pl.q = split(pl.QKV, p.NG, g);
    pl.o = split(p.H, p.NG, g);
    pl.f = split(p.F, p.NG, g);
    pl.v = split(p.V, p.NG, g);
    pl.uq = units(pl.q.count * p.H * 2);
    pl.uo = units(pl.o.count * pl.QD * 2);
    pl.ug = units(pl.f.count * p.H * 2);
    pl.ud = units(pl.o.count * p.F * 2);
    pl.layer = pl.uq + pl.uo + 2 * pl.ug + pl.ud;
    pl.chunks = (pl.v.count + kChunk - 1) / kChunk;
    pl.step = p.L * pl.layer;
    for (uint32_t c = 0; c < pl.chunks; c++) pl.step += chunk_units(p, pl, c);
    return pl;
}

// Hand-off word offsets: per layer qkv, attention, x after o, silu*up, x after down.
struct Hand {
    uint32_t qkv, att, x2, hf, xo, block, am;
};
TS_DEV Hand hand(const DecodeStepArgs &p, const Plan &pl) {
    Hand h;
    h.qkv = 0;
    h.att = pl.QKV;
    h.x2 = h.att + pl.QD;
    h.hf = h.x2 + p.H;
    h.xo = h.hf + p.F;
    h.block = h.xo + p.H;
    h.am = p.L * h.block;
    return h;
}

TS_DEV uint64_t ld_tag(const uint64_t *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
TS_DEV void st_tag(uint64_t *p, uint32_t bits, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
TS_DEV uint64_t now() { return __builtin_amdgcn_s_memrealtime(); }

// A barrier of all eight waves that also publishes this wave's LDS writes; global
// loads stay in flight (__syncthreads would wait for them).
TS_DEV void bar() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

struct Ctx {
    char *lds;
    float *xa, *xr, *red, *ssq;
    uint32_t *tbl;
    volatile uint32_t *ctl;
    uint32_t *err;
    uint32_t tid, wave, lane;
};

// One step of a bounded wait; false ends the wait (timed out here, or anywhere).
TS_DEV bool spin(Ctx &c, uint32_t &it, uint64_t &t0) {
    if (c.ctl[kAbort]) return false;
    ++it;
    if ((it & 255) == 0 && __hip_atomic_load(c.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
        c.ctl[kAbort] = 1u;
        return false;
    }
    if ((it & 1023) == 0) {
        const uint64_t t = now();
        if (!t0) {
            t0 = t;
        } else if (t - t0 > kTimeout) {
            c.ctl[kAbort] = 1u;
            __hip_atomic_store(c.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
    }
    __builtin_amdgcn_s_sleep(1);
    return true;
}

// Tagged words src[tid + kCT k] (k < NX, index < n) into v[k]: every load is
// issued, then the loads whose epoch is stale are reissued until none is. (A
// second round of loads kept in flight measured slower: it doubles the polling
// traffic every group puts on the memory system.)
template <int NX>
TS_DEV void poll(Ctx &c, const uint64_t *src, uint32_t n, uint32_t tag, float (&v)[NX]) {
    uint64_t w[NX];
#pragma unroll
    for (int k = 0; k < NX; k++) {
        const uint32_t i = c.tid + kCT * k;
        w[k] = i < n ? ld_tag(src + i) : ((uint64_t)tag << 32);
    }
    uint64_t t0 = 0;
    uint32_t it = 0;
    for (;;) {
        bool ready = true;
#pragma unroll
        for (int k = 0; k < NX; k++) ready &= (uint32_t)(w[k] >> 32) == tag;
        if (ready || !spin(c, it, t0)) break;
#pragma unroll
        for (int k = 0; k < NX; k++)
            if ((uint32_t)(w[k] >> 32) != tag) w[k] = ld_tag(src + c.tid + kCT * k);
    }
#pragma unroll
    for (int k = 0; k < NX; k++) v[k] = __uint_as_float((uint32_t)w[k]);
}

TS_DEV float dot8(u32x4 w, float4 a, float4 b, float acc) {
    acc += a.x * lo_bf16(w.x);
    acc += a.y * hi_bf16(w.x);
    acc += a.z * lo_bf16(w.y);
    acc += a.w * hi_bf16(w.y);
    acc += b.x * lo_bf16(w.z);
    acc += b.y * hi_bf16(w.z);
    acc += b.z * lo_bf16(w.w);
    acc += b.w * hi_bf16(w.w);
    return acc;
}

TS_DEV const u32x4 *ring_at(const char *lds, uint32_t u0, uint32_t byte) {
    const uint32_t u = u0 + (byte >> 10);
    return (const u32x4 *)(lds + kRingOff + ((u & (kRing - 1)) << 10) + (byte & 1023));
}

// Partial dot products of NR rows of this wave with xa[0, K), over pieces [j0, j1)
// of 8 values: every LDS read of an iteration is issued before its math.
template <int NR>
TS_DEV void dots(const Ctx &c, const uint32_t (&u0)[kRW], const uint32_t (&rr)[kRW], uint32_t j0, uint32_t j1,
                 float (&acc)[kRW]) {
    const float4 *x4 = (const float4 *)c.xa;
#pragma unroll 2
    for (uint32_t j = j0 + c.lane; j < j1; j += 64) {
        const float4 a = x4[2 * j], b = x4[2 * j + 1];
        u32x4 w[NR];
#pragma unroll
        for (int i = 0; i < NR; i++) w[i] = *ring_at(c.lds, u0[i], rr[i] + j * 16);
#pragma unroll
        for (int i = 0; i < NR; i++) acc[i] = dot8(w[i], a, b, acc[i]);
    }
}

// Partial dot products of R rows (R <= kRW kCW) with xa[0, K): rows r < Ra are rows
// of the stream segment at unit ua, rows r >= Ra rows r - Ra of the segment at ub.
// With R >= kCW wave w owns rows w + kCW i; fewer rows split k across S = kCW / R
// waves. Row r's value is the sum over s < S of red[r * S + s] (in that order).
TS_DEV uint32_t gemv_part(Ctx &c, uint32_t ua, uint32_t Ra, uint32_t ub, uint32_t R, uint32_t K, float *red) {
    if (R == 0) return 1;
    const uint32_t P = K >> 3, rowb = K * 2;
    const uint32_t S = R >= kCW ? 1 : kCW / R;
    uint32_t u0[kRW], rr[kRW], nr, j0 = 0, j1 = P;
    float acc[kRW];
    if (S > 1) {
        nr = c.wave < R * S ? 1 : 0;
        const uint32_t r = min(c.wave / S, R - 1), s = c.wave % S, per = (P + S - 1) / S;
        j0 = min(P, s * per);
        j1 = min(P, j0 + per);
#pragma unroll
        for (int i = 0; i < kRW; i++) {
            u0[i] = r < Ra ? ua : ub;
            rr[i] = (r < Ra ? r : r - Ra) * rowb;
        }
    } else {
        nr = c.wave < R ? (R - c.wave + kCW - 1) / kCW : 0;
#pragma unroll
        for (int i = 0; i < kRW; i++) {
            const uint32_t r = min(c.wave + kCW * i, R - 1);
            u0[i] = r < Ra ? ua : ub;
            rr[i] = (r < Ra ? r : r - Ra) * rowb;
        }
    }
#pragma unroll
    for (int i = 0; i < kRW; i++) acc[i] = 0.0f;
    switch (nr) {  // uniform across the wave
    case 1: dots<1>(c, u0, rr, j0, j1, acc); break;
    case 2: dots<2>(c, u0, rr, j0, j1, acc); break;
    case 3: dots<3>(c, u0, rr, j0, j1, acc); break;
    case 4: dots<4>(c, u0, rr, j0, j1, acc); break;
    default: break;
    }
#pragma unroll
    for (int i = 0; i < kRW; i++) {
        if ((uint32_t)i < nr) {
            const float t = wave_sum(acc[i]);
            if (c.lane == 0) red[c.wave + kCW * i] = t;
        }
    }
    return S;
}

TS_DEV float row_value(const float *red, uint32_t r, uint32_t S) {
    float v = 0.0f;
    for (uint32_t s = 0; s < S; s++) v += red[r * S + s];
    return v;
}

// Stage an input vector of n <= 3072 values: xa[i] = v * g[i], xr[i] = v when
// keep_raw, and the partial sums of squares of the RmsNorm; read back after the
// next barrier by norm_inv.
template <int NX>
TS_DEV void stage(Ctx &c, const float (&v)[NX], uint32_t n, const float (&g)[NX], bool keep_raw) {
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < NX; k++) {
        const uint32_t i = c.tid + kCT * k;
        if (i < n) {
            c.xa[i] = v[k] * g[k];
            if (keep_raw) c.xr[i] = v[k];
            ss += v[k] * v[k];
        }
    }
    ss = wave_sum(ss);
    if (c.lane == 0) c.ssq[c.wave] = ss;
}

// 1/sqrt(mean(v^2) + eps): the RmsNorm scale, folded into the products' results
// (sum_k (x_k inv g_k) w_k = inv sum_k (x_k g_k) w_k).
TS_DEV float norm_inv(const Ctx &c, uint32_t n, float eps) {
    float t = 0.0f;
    for (uint32_t w = 0; w < kCW; w++) t += c.ssq[w];
    return 1.0f / sqrtf(t / (float)n + eps);
}

// RmsNorm over a 128-wide head held as (d, d + 64) in lane d, then the Halves
// rotation of that pair (engine/ir/interp/src/cpu.rs:36-47, 371-377).
TS_DEV void norm_rope(float &a, float &b, float ga, float gb, float cs, float sn, float eps) {
    const float s = wave_sum(a * a + b * b);
    const float inv = 1.0f / sqrtf(s / 128.0f + eps);
    a = a * (inv * ga);
    b = b * (inv * gb);
    const float ra = a * cs - b * sn, rb = a * sn + b * cs;
    a = ra;
    b = rb;
}

// Optional phase stamps of the first step (thread 0 of every group): slot 2 ph
// when the phase's input is staged, 2 ph + 1 when its outputs are stored, 8 when
// the group's attention is done; row L: lm_head input, chunks done, token.
TS_DEV void mark(const DecodeStepArgs &p, const Ctx &c, uint32_t g, uint32_t t, uint32_t l, uint32_t k) {
    if (p.marks && t == 0 && c.tid == 0) p.marks[((size_t)g * (p.L + 2) + l) * 10 + k] = now();
}

constexpr uint32_t kAttBars = 4;  // barriers of attention()

// Sums (maxima) over the four 16-lane rows of a wave, in every lane: lanes j, j + 16,
// j + 32 and j + 48 end with the same total (gfx950 permlane swaps: VALU, no LDS).
TS_DEV float rows4_sum(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
TS_DEV float rows4_max(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Attention of q head `h` (kv head a = h / 2) at position pos over kept rows
// [0, pos] (engine/ir/interp/src/cpu.rs:141-167, 293-351): the raw q/k/v rows
// come from the qkv hand-off; q and the new k are normalized and rotated, the new
// k and v rows are appended (bf16, by the even head of the pair), and the head's
// output is published. One group per q head: the two heads of a GQA pair run
// side by side on two CUs (each loads the pair's kept rows) instead of one
// after the other on one.
// Lanes: key = lane / 16 of a 4-key block, dims 8 (lane % 16) .. +8; a wave takes
// blocks wave + kCW i, kPre of them per softmax pass (one max and one sum per pass,
// then the running (max, sum, acc) rescaled once per pass).
TS_DEV void attention(const DecodeStepArgs &p, const Plan &pl, const Hand &hd, Ctx &c, uint32_t l, uint32_t h,
                      uint32_t pos, uint32_t tag) {
    const uint32_t lane = c.lane, wave = c.wave, a = h >> 1;
#define AMARK(k) do { if (l == 5 && tag == p.epoch) mark(p, c, h, 0, p.L + 1, k); } while (0)
    AMARK(0);
    const uint32_t kr = lane >> 4, part = lane & 15;
    const uint32_t Hkv = p.Hkv, shift = p.page_shift, mask = (1u << shift) - 1;
    const uint16_t *kc = p.k_cache[l], *vc = p.v_cache[l];
    const uint32_t nblk = (pos >> 2) + 1;                                 // 4-key blocks in [0, pos]
    const uint32_t mine = nblk > wave ? (nblk - wave + kCW - 1) / kCW : 0;  // this wave's blocks
    float *raw = c.xa + 2560, *qs = c.xa, *pm = c.xa + 384, *pl_ = c.xa + 400, *po = c.xa + 512;
    uint16_t *kn = (uint16_t *)(c.xa + 256), *vn = (uint16_t *)(c.xa + 320);
    const uint32_t last = pos ? pos - 1 : 0u;  // kept rows before pos exist; pos arrives in LDS

    // Kept rows of earlier positions: the first kPre blocks of this wave, now.
    u32x4 kk[kPre], vv[kPre];
#pragma unroll
    for (int i = 0; i < kPre; i++) {
        const uint32_t key = min(4 * (wave + kCW * i) + kr, last);
        const uint64_t row = ((uint64_t)c.tbl[key >> shift] << shift) | (key & mask);
        const size_t e = (row * Hkv + a) * 128 + 8 * part;
        kk[i] = *(const u32x4 *)(kc + e);
        vv[i] = *(const u32x4 *)(vc + e);
    }
    float ga = 0.0f, gb = 0.0f;
    if (wave == 0) { ga = p.q_norm[l][lane]; gb = p.q_norm[l][lane + 64]; }
    if (wave == 1) { ga = p.k_norm[l][lane]; gb = p.k_norm[l][lane + 64]; }
    const float2 cs = ((const float2 *)p.rope)[(size_t)pos * 64 + lane];
    AMARK(1);
    // q head h, then k and v of head a: 384 words in 3 runs of 128, one per thread.
    static_assert(kCT >= 384, "one hand-off word per thread");
    if (c.tid < 384) {
        const uint64_t *blk = p.hand + hd.qkv + (size_t)l * hd.block;
        const uint32_t r = c.tid >> 7, d = c.tid & 127;
        const uint32_t gi = r == 0 ? h * 128 + d : (r == 1 ? pl.QD + a * 128 + d : pl.QD + (Hkv + a) * 128 + d);
        uint64_t w = ld_tag(blk + gi);
        uint64_t t0 = 0;
        uint32_t it = 0;
        while ((uint32_t)(w >> 32) != tag && spin(c, it, t0)) w = ld_tag(blk + gi);
        raw[c.tid] = __uint_as_float((uint32_t)w);
    }
    AMARK(2);
    bar();  // 1
    AMARK(3);
    if (wave < 3) {
        float x0 = raw[wave * 128 + lane], x1 = raw[wave * 128 + lane + 64];
        if (wave < 2) norm_rope(x0, x1, ga, gb, cs.x, cs.y, p.eps);
        if (wave == 0) {
            qs[lane] = x0;
            qs[lane + 64] = x1;
        } else {
            const uint16_t b0 = bf16_bits(x0), b1 = bf16_bits(x1);
            uint16_t *dst = wave == 1 ? kn : vn;
            dst[lane] = b0;
            dst[lane + 64] = b1;
            // The new row joins the kept rows (Store::append, engine/ir/interp/src/run.rs:122-198),
            // written once per pair (the odd head computes the same row).
            if ((h & 1) == 0) {
                const uint64_t row = ((uint64_t)c.tbl[pos >> shift] << shift) | (pos & mask);
                uint16_t *cache = (wave == 1 ? p.k_cache[l] : p.v_cache[l]) + (row * Hkv + a) * 128;
                // Agent scope: the odd head reads this row at the next step from
                // another CU (perhaps another XCD, whose L2 this store would miss).
                __hip_atomic_store(cache + lane, b0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(cache + lane + 64, b1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    bar();  // 2
    AMARK(4);

    float q[8];
    {
        const float4 t0 = *(const float4 *)&qs[8 * part], t1 = *(const float4 *)&qs[8 * part + 4];
        q[0] = t0.x; q[1] = t0.y; q[2] = t0.z; q[3] = t0.w;
        q[4] = t1.x; q[5] = t1.y; q[6] = t1.z; q[7] = t1.w;
    }
    const u32x4 knew = *(const u32x4 *)(kn + 8 * part), vnew = *(const u32x4 *)(vn + 8 * part);
    float m = -INFINITY, ls = 0.0f, o[8];
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = 0.0f;

    for (uint32_t i0 = 0; i0 < mine; i0 += kPre) {
        if (i0) {  // later passes (contexts past kCW kPre blocks): load this pass now
#pragma unroll
            for (int i = 0; i < kPre; i++) {
                const uint32_t key = min(4 * (wave + kCW * (i0 + i)) + kr, last);
                const uint64_t row = ((uint64_t)c.tbl[key >> shift] << shift) | (key & mask);
                const size_t e = (row * Hkv + a) * 128 + 8 * part;
                kk[i] = *(const u32x4 *)(kc + e);
                vv[i] = *(const u32x4 *)(vc + e);
            }
        }
        float sc[kPre];
        bool ok[kPre];
#pragma unroll
        for (int i = 0; i < kPre; i++) {
            const uint32_t key = 4 * (wave + kCW * (i0 + i)) + kr;
            ok[i] = key <= pos;  // past the wave's blocks too: key >= 4 nblk > pos
            const u32x4 kv = key == pos ? knew : kk[i];
            const uint32_t kw[4] = {kv.x, kv.y, kv.z, kv.w};
            float s0 = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                s0 += q[2 * e] * lo_bf16(kw[e]);
                s0 += q[2 * e + 1] * hi_bf16(kw[e]);
            }
            sc[i] = ok[i] ? row16_sum(s0) * p.scale : -INFINITY;
        }
        float bm = sc[0];
#pragma unroll
        for (int i = 1; i < kPre; i++) bm = fmaxf(bm, sc[i]);
        const float mn = fmaxf(m, rows4_max(bm));  // finite: key 4 wave <= pos
        const float alpha = m == -INFINITY ? 0.0f : expf(m - mn);
        float acc[8], sum = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) acc[e] = 0.0f;
#pragma unroll
        for (int i = 0; i < kPre; i++) {
            const float pk = ok[i] ? expf(sc[i] - mn) : 0.0f;
            sum += pk;
            const u32x4 vx = (4 * (wave + kCW * (i0 + i)) + kr) == pos ? vnew : vv[i];
            const uint32_t vw[4] = {ok[i] ? vx.x : 0u, ok[i] ? vx.y : 0u, ok[i] ? vx.z : 0u, ok[i] ? vx.w : 0u};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                acc[2 * e] += pk * lo_bf16(vw[e]);
                acc[2 * e + 1] += pk * hi_bf16(vw[e]);
            }
        }
        ls = ls * alpha + rows4_sum(sum);
        m = mn;
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = o[e] * alpha + acc[e];
    }
    AMARK(5);
    // Sum the four key rows; lanes of row 0 hold the wave's 128 partial sums.
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = rows4_sum(o[e]);
    if (kr == 0) {
        *(float4 *)&po[wave * 128 + 8 * part] = make_float4(o[0], o[1], o[2], o[3]);
        *(float4 *)&po[wave * 128 + 8 * part + 4] = make_float4(o[4], o[5], o[6], o[7]);
    }
    if (lane == 0) {
        pm[wave] = m;
        pl_[wave] = ls;
    }
    bar();  // 3
    AMARK(6);
    if (c.tid < 128) {
        const uint32_t d = c.tid;
        float M = -INFINITY;
        for (uint32_t w = 0; w < kCW; w++) M = fmaxf(M, pm[w]);
        float L = 0.0f, O = 0.0f;
        for (uint32_t w = 0; w < kCW; w++) {
            const float f = pm[w] == -INFINITY ? 0.0f : expf(pm[w] - M);
            L += pl_[w] * f;
            O += po[w * 128 + d] * f;
        }
        st_tag(p.hand + hd.att + (size_t)l * hd.block + h * 128 + d, __float_as_uint(O / L), tag);
    }
    AMARK(7);
    bar();  // 4: the next phase stages its input over this scratch
    AMARK(8);
}

TS_DEV void better(float &bv, uint32_t &bi, float v, uint32_t i) {
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}
TS_DEV void wave_best(float &bv, uint32_t &bi) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float v = __shfl_xor(bv, o, 64);
        const uint32_t i = __shfl_xor(bi, o, 64);
        better(bv, bi, v, i);
    }
}

// One product phase of a layer.
struct Phase {
    const uint64_t *in;  // tagged input; null: the embedding row of the step's token
    const float *gain;   // RmsNorm gain; null: none
    uint64_t *out;       // tagged outputs, from row `first`
    uint32_t n, ua, Ra, ub, R, K, first;
    uint32_t kind;       // 0: value * inv; 1: xr[first + r] + value; 2: silu(gate) * up
    bool keep_raw;
};

// Stage the input, barrier (the DMA waves have landed the rows), products,
// barrier, publish.
template <int NX>
TS_DEV void run_phase(const DecodeStepArgs &p, Ctx &c, const Phase &f, uint32_t tag, uint32_t tok, uint32_t g,
                      uint32_t t, uint32_t l, uint32_t ph) {
    float v[NX], gv[NX];
#pragma unroll
    for (int k = 0; k < NX; k++) {
        const uint32_t i = c.tid + kCT * k;
        gv[k] = f.gain && i < f.n ? f.gain[i] : 1.0f;
    }
    if (f.in) {
        poll(c, f.in, f.n, tag, v);
    } else {
#pragma unroll
        for (int k = 0; k < NX; k++) {
            const uint32_t i = c.tid + kCT * k;
            v[k] = i < f.n ? bf16_float(p.embed[(size_t)tok * f.n + i]) : 0.0f;
        }
    }
    stage(c, v, f.n, gv, f.keep_raw);
    mark(p, c, g, t, l, 2 * ph);
    bar();
    const float inv = f.gain ? norm_inv(c, f.n, p.eps) : 1.0f;
    const uint32_t S = gemv_part(c, f.ua, f.Ra, f.ub, f.R, f.K, c.red);
    bar();
    const uint32_t outs = f.kind == 2 ? f.Ra : f.R;
    if (c.tid < outs) {
        const float x = row_value(c.red, c.tid, S);
        float y;
        if (f.kind == 0) {
            y = x * inv;
        } else if (f.kind == 1) {
            y = c.xr[f.first + c.tid] + x;
        } else {
            const float gt = x * inv, up = row_value(c.red, f.Ra + c.tid, S) * inv;
            y = gt / (1.0f + expf(-gt)) * up;
        }
        st_tag(f.out + f.first + c.tid, __float_as_uint(y), tag);
    }
    mark(p, c, g, t, l, 2 * ph + 1);
}

// The compute waves of group g. Barrier schedule per step (mirrored by dma()):
// per layer 2 per phase x 4 phases (+ kAttBars after phase 0 in groups below
// kv_heads); then 1 for the lm_head input, 1 per chunk, 2 for the token.
TS_DEV void compute(const DecodeStepArgs &p, Ctx &c, uint32_t g) {
    const Plan pl = plan(p, g);
    const Hand hd = hand(p, pl);
    const uint32_t H = p.H, F = p.F;
    const uint32_t pos0 = p.pos[0];
    uint32_t tok = p.tok[0];
    uint32_t U = 0;  // stream cursor (units)
    for (uint32_t t = 0; t < p.steps; t++) {
        const uint32_t tag = p.epoch + t, pos = pos0 + t;
        for (uint32_t l = 0; l < p.L; l++) {
            uint64_t *blk = p.hand + (size_t)l * hd.block;
            const uint32_t Uq = U, Uo = Uq + pl.uq, Ug = Uo + pl.uo, Uu = Ug + pl.ug, Ud = Uu + pl.ug;
            U = Ud + pl.ud;
            for (uint32_t ph = 0; ph < 4; ph++) {
                Phase f;
                if (ph == 0) {  // RmsNorm(ln1), qkv rows
                    f = {l ? blk - hd.block + hd.xo : nullptr, p.ln1[l], blk + hd.qkv, H, Uq, pl.q.count, Uq,
                         pl.q.count, H, pl.q.first, 0u, true};
                } else if (ph == 1) {  // o rows + residual
                    f = {blk + hd.att, nullptr, blk + hd.x2, pl.QD, Uo, pl.o.count, Uo, pl.o.count, pl.QD,
                         pl.o.first, 1u, false};
                } else if (ph == 2) {  // RmsNorm(ln2), gate and up rows, silu(gate) * up
                    f = {blk + hd.x2, p.ln2[l], blk + hd.hf, H, Ug, pl.f.count, Uu, 2 * pl.f.count, H, pl.f.first,
                         2u, true};
                } else {  // down rows + residual
                    f = {blk + hd.hf, nullptr, blk + hd.xo, F, Ud, pl.o.count, Ud, pl.o.count, F, pl.o.first, 1u,
                         false};
                }
                if (ph & 1)
                    run_phase<kNX>(p, c, f, tag, tok, g, t, l, ph);
                else
                    run_phase<kNH>(p, c, f, tag, tok, g, t, l, ph);
                if (ph == 0 && g < p.Hq) {
                    attention(p, pl, hd, c, l, g, pos, tag);
                    mark(p, c, g, t, l, 8);
                }
            }
        }
        // --- final RmsNorm, lm_head rows, greedy pick ---
        {
            float v[kNH], gn[kNH];
#pragma unroll
            for (int k = 0; k < kNH; k++) {
                const uint32_t i = c.tid + kCT * k;
                gn[k] = i < H ? p.norm[i] : 1.0f;
            }
            poll(c, p.hand + (size_t)(p.L - 1) * hd.block + hd.xo, H, tag, v);
            stage(c, v, H, gn, false);
        }
        mark(p, c, g, t, p.L, 0);
        bar();  // lm input staged; chunk 0 landed
        const float inv = norm_inv(c, H, p.eps);
        float bv = -INFINITY;
        uint32_t bi = p.V;
        for (uint32_t ch = 0; ch < pl.chunks; ch++) {
            const uint32_t r0 = ch * kChunk, rows = min(kChunk, pl.v.count - r0);
            const uint32_t Uc = U;
            U += units(rows * H * 2);
            // Chunks alternate halves of the partials: wave 0 reads chunk ch's after
            // the barrier while the other waves write chunk ch + 1's.
            float *red = c.red + (ch & 1) * 64;
            const uint32_t S = gemv_part(c, Uc, rows, Uc, rows, H, red);
            bar();  // chunk ch consumed; chunk ch + 1 landed
            if (c.wave == 0) {
                float v = -INFINITY;
                uint32_t i = p.V;
                if (c.lane < rows) {
                    const uint32_t row = pl.v.first + r0 + c.lane;
                    const float x = row_value(red, c.lane, S) * inv;
                    p.logits[row] = x;
                    if (x > -INFINITY) { v = x; i = row; }  // NaN and -inf never win
                }
                wave_best(v, i);
                better(bv, bi, v, i);
            }
        }
        mark(p, c, g, t, p.L, 1);
        uint64_t *am = p.hand + hd.am;
        if (c.tid == 0) {
            st_tag(am + 2 * g, __float_as_uint(bv), tag);
            st_tag(am + 2 * g + 1, bi, tag);
        }
        {
            float v[kNA];
            poll(c, am, 2 * p.NG, tag, v);
#pragma unroll
            for (int k = 0; k < kNA; k++)
                if (c.tid + kCT * k < 2 * p.NG) c.red[128 + c.tid + kCT * k] = v[k];
        }
        bar();
        if (c.wave == 0) {
            float v = -INFINITY;
            uint32_t i = p.V;
            for (uint32_t w = c.lane; w < p.NG; w += 64) {
                const float x = c.red[128 + 2 * w];
                const uint32_t xi = __float_as_uint(c.red[128 + 2 * w + 1]);
                if (xi < p.V) better(v, i, x, xi);
            }
            wave_best(v, i);
            if (c.lane == 0) c.ctl[kTok] = i;
        }
        bar();
        mark(p, c, g, t, p.L, 2);
        tok = c.ctl[kTok];
        if (tok >= p.V) tok = 0;  // no finite logit (an aborted launch): any row of the table
        if (g == 0 && c.tid == 0) p.hist[pos + 1] = tok;
    }
    if (g == 0 && c.tid == 0) {
        p.pos[0] = pos0 + p.steps;
        p.tok[0] = tok;
    }
}

// Wait until at most n of this wave's DMA loads are in flight (n rounded down to a
// multiple of 8: the vmcnt field is an immediate).
TS_DEV void wait_vm(uint32_t n) {
    switch (n >> 3) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(16)" ::: "memory"); break;
    case 3: asm volatile("s_waitcnt vmcnt(24)" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(32)" ::: "memory"); break;
    case 5: asm volatile("s_waitcnt vmcnt(40)" ::: "memory"); break;
    case 6: asm volatile("s_waitcnt vmcnt(48)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(56)" ::: "memory"); break;
    }
}

// A DMA wave: streams the units u with u % 2 == dw of the group's weight stream
// (per step and layer the qkv, o, gate, up and down rows, then the lm_head rows
// in chunks) into ring slot u % kRing, and walks the compute's barrier schedule.
struct Dma {
    const DecodeStepArgs *p;
    Plan pl;
    uint32_t dw, lane, ring;
    uint32_t total;      // units of the whole launch
    uint32_t U;          // next unit to issue
    uint32_t freed;      // units whose slots may be reused: unit u needs u < freed + kRing
    uint32_t mine;       // this wave's units issued so far
    uint32_t inflight;   // of those, possibly still in flight
    uint32_t burst;      // loads per wave issued ahead of need per barrier
    // the segment under the cursor
    uint32_t seg, seg_u, seg_n, seg_bytes;
    const char *seg_base;

    TS_DEV void open_segment() {
        const DecodeStepArgs &a = *p;
        const uint32_t per = 5 * a.L + pl.chunks, js = __builtin_amdgcn_readfirstlane(seg % per), H = a.H, F = a.F;
        if (js < 5 * a.L) {
            const uint32_t l = js / 5, s = js % 5;
            if (s == 0) {
                seg_base = (const char *)(a.qkv[l] + (size_t)pl.q.first * H); seg_bytes = pl.q.count * H * 2;
            } else if (s == 1) {
                seg_base = (const char *)(a.o[l] + (size_t)pl.o.first * pl.QD); seg_bytes = pl.o.count * pl.QD * 2;
            } else if (s == 4) {
                seg_base = (const char *)(a.down[l] + (size_t)pl.o.first * F); seg_bytes = pl.o.count * F * 2;
            } else {
                seg_base = (const char *)(a.gate_up[l] + (size_t)((s == 3 ? F : 0) + pl.f.first) * H);
                seg_bytes = pl.f.count * H * 2;
            }
        } else {
            const uint32_t r0 = (js - 5 * a.L) * kChunk;
            seg_base = (const char *)(a.embed + (size_t)(pl.v.first + r0) * H);
            seg_bytes = min(kChunk, pl.v.count - r0) * H * 2;
        }
        seg_n = units(seg_bytes);
        seg_u = 0;
    }

    // Issue the next units the ring has room for: at least those below `need`, else
    // at most kBurst of this wave's per barrier (a long burst would hold the barrier
    // up; the compute meets a dozen barriers per layer).
    TS_DEV void issue(uint32_t need) {
        const uint32_t limit = min(total, min(freed + kRing, max(U + 2 * burst, need)));
        while (U < limit) {
            if (seg_u >= seg_n) {
                seg++;
                open_segment();
                continue;
            }
            const uint32_t n = min(seg_n - seg_u, limit - U);
            // this wave's units of the run: U + k with (U + k) % 2 == dw
            for (uint32_t k = (U & 1) == dw ? 0u : 1u; k < n; k += 2) {
                if (inflight >= kMaxOut) {
                    wait_vm(kMaxOut - 8);
                    inflight = kMaxOut - 8;
                }
                const uint32_t off = min((seg_u + k) * 1024 + lane * 16, seg_bytes - 16);
                __builtin_amdgcn_global_load_lds((const void *)(seg_base + off),
                                                 (lds_void *)(uintptr_t)(ring + (((U + k) & (kRing - 1)) << 10)), 16,
                                                 0, 0);
                mine++;
                inflight++;
            }
            seg_u += n;
            U += n;
        }
    }

    // The barrier after which the compute reads units [0, need) and before which it
    // has released units [0, free).
    TS_DEV void barrier(uint32_t need, uint32_t free) {
        issue(need);  // every unit below `need` is issued (the ring holds a phase)
        const uint32_t below = dw == 0 ? (need + 1) >> 1 : need >> 1;  // this wave's units < need
        const uint32_t after = mine - min(mine, below);
        if (after < inflight) {
            wait_vm(after);
            inflight = after & ~7u;
        }
        bar();
        if (free > freed) freed = free;
    }
};

TS_DEV void dma(const DecodeStepArgs &p, uint32_t g, uint32_t dw, uint32_t lane, uint32_t ring) {
    Dma d;
    d.p = &p;
    d.pl = plan(p, g);
    d.dw = dw;
    d.lane = lane;
    d.ring = ring;
    d.total = d.pl.step * p.steps;
    d.U = 0;
    d.freed = 0;
    d.mine = 0;
    d.inflight = 0;
    d.burst = kBurst;
    d.seg = 0;
    d.open_segment();
    const Plan &pl = d.pl;
    uint32_t U = 0;  // the compute's cursor
    for (uint32_t t = 0; t < p.steps; t++) {
        for (uint32_t l = 0; l < p.L; l++) {
            const uint32_t ends[4] = {U + pl.uq, U + pl.uq + pl.uo, U + pl.uq + pl.uo + 2 * pl.ug, U + pl.layer};
            for (uint32_t ph = 0; ph < 4; ph++) {
                d.barrier(ends[ph], 0);  // staged input; the phase's rows landed
                d.barrier(0, ends[ph]);  // products done; its rows released
                if (ph == 0 && g < p.Hq)
                    for (uint32_t b = 0; b < kAttBars; b++) d.barrier(0, 0);
            }
            U += pl.layer;
        }
        d.barrier(pl.chunks ? U + chunk_units(p, pl, 0) : 0, 0);  // lm input; chunk 0 landed
        // The lm_head chunks: little compute per barrier, so the DMA waves keep the
        // ring as full as their loads in flight allow.
        d.burst = kLmBurst;
        for (uint32_t ch = 0; ch < pl.chunks; ch++) {
            const uint32_t next = U + chunk_units(p, pl, ch);
            const uint32_t need = ch + 1 < pl.chunks ? next + chunk_units(p, pl, ch + 1) : 0;
            d.barrier(need, next);
            U = next;
        }
        d.burst = kBurst;
        d.barrier(0, 0);
        d.barrier(0, 0);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

__global__ __launch_bounds__(kThreads) void decode_step_kernel(DecodeStepArgs p) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    // The wave index is uniform: readfirstlane lets the compiler keep what derives
    // from it (the DMA cursors, the segment pointers) in scalar registers; as
    // vector values, the per-layer pointer loads of the DMA waves became vector
    // loads followed by a wait for every load in flight.
    const uint32_t tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63,
                   g = blockIdx.x;
    volatile uint32_t *ctl = (volatile uint32_t *)(lds + kCtlOff);
    uint32_t *tbl = (uint32_t *)(lds + kTblOff);
    if (tid < 16) ctl[tid] = 0u;
    if (g < p.Hq)
        for (uint32_t i = tid; i < p.kept_pages; i += kThreads) tbl[i] = p.table[i];
    __syncthreads();
    if (wave >= kCW) {
        const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)lds;
        dma(p, g, wave - kCW, lane, base + kRingOff);
        return;
    }
    Ctx c;
    c.lds = lds;
    c.xa = (float *)(lds + kXaOff);
    c.xr = (float *)(lds + kXrOff);
    c.red = (float *)(lds + kRedOff);
    c.ssq = (float *)(lds + kSsqOff);
    c.tbl = tbl;
    c.ctl = ctl;
    c.err = p.error;
    c.tid = tid;
    c.wave = wave;
    c.lane = lane;
    compute(p, c, g);
}

}  // namespace

size_t decode_step_hand_words(uint32_t H, uint32_t L, uint32_t Hq, uint32_t Hkv, uint32_t F, uint32_t NG) {
    const size_t block = (size_t)(Hq + 2 * Hkv) * 128 + Hq * 128 + 2 * H + F;
    return L * block + 2 * (size_t)NG;
}

int decode_step_supported(uint32_t H, uint32_t L, uint32_t Hq, uint32_t Hkv, uint32_t D, uint32_t F,
                          uint32_t kept_pages) {
    uint32_t ng = 0;
    int rc = decode_step_groups(&ng);
    if (rc != TS_OK) return rc;
    if (D != 128 || Hkv == 0 || Hq != 2 * Hkv || Hq > ng || ng > kMaxGroups) return 1;
    if (L > kStepMaxLayers || H > kMaxH || H % 8 || F % 8 || F > kMaxXa || Hq * 128 > kMaxXa) return 1;
    if (kept_pages > kMaxPages) return 1;
    // No group may own more than kRW kCW rows of a phase, and every phase's rows
    // must fit half the ring.
    const uint32_t QKV = (Hq + 2 * Hkv) * 128;
    const uint32_t rq = (QKV + ng - 1) / ng, ro = (H + ng - 1) / ng, rf = (F + ng - 1) / ng;
    if (rq > kRW * kCW || ro > kRW * kCW || 2 * rf > kRW * kCW) return 1;
    auto u = [](uint64_t b) { return (b + 1023) / 1024; };
    if (u((uint64_t)rq * H * 2) > kRing / 2 || u((uint64_t)ro * Hq * 256) > kRing / 2 ||
        2 * u((uint64_t)rf * H * 2) > kRing / 2 || u((uint64_t)ro * F * 2) > kRing / 2 ||
        u((uint64_t)kChunk * H * 2) > kRing / 2)
        return 1;
    return TS_OK;
}

int decode_step_groups(uint32_t *groups) {
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return hip_status(e, "decode_step: device attributes");
    *groups = (uint32_t)cus;
    return TS_OK;
}

int decode_step_launch(const DecodeStepArgs *a, void *stream) {
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void *)decode_step_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
        if (e != hipSuccess) return hip_status(e, "decode_step: shared memory attribute");
        attr = true;
    }
    DecodeStepArgs args = *a;
    void *params[] = {&args};
    hipError_t e = hipLaunchCooperativeKernel((const void *)decode_step_kernel, dim3(a->NG), dim3(kThreads), params,
                                              kLdsBytes, (hipStream_t)stream);
    if (e != hipSuccess) return hip_status(e, "decode_step: cooperative launch");
    return TS_OK;
}

}  // namespace ts
