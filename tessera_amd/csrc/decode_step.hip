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
// Why one launch, and why roles. At batch 1 every product only streams its weights
// (31 MB a layer, ~4 us of HBM time), while each stage needs the whole output of the
// one before: the step is a chain of ~140 chip-wide hand-offs, and their latency,
// not HBM, sets its speed. A hand-off among all 256 CUs measured ~2.2 us on MI355X,
// among 32 ~1.3 us. So each group (one per CU, resident for the whole call) has one
// role for the whole launch:
//  * qkv, o, gate/up or down: the group owns fixed rows of that matrix in every
//    layer and keeps them in registers (<= 96 VGPRs a lane). Right after a layer's
//    products it issues the loads of the next layer's rows into the same registers,
//    so they land during the ~10 us until that layer comes round: no weight latency
//    on the chain, and each hand-off runs between two role sets of 32..96 groups;
//  * attention: one group per q head (both heads of a kv head append the same new k/v
//    row, bit for bit, and each reads back only rows it wrote: no cross-CU ordering);
//  * every group then streams its rows of the tied lm_head; every group publishes
//    its (max, index), and the groups that need the token reduce all of them.
// Hand-offs are "tagged" words in HBM: each value is one 8-byte store of (f32 value,
// u32 epoch) at agent scope (coherent across XCDs), and a consumer polls the words it
// needs until every epoch matches: the data is its own flag. Waits are bounded: a
// poll that passes 2 s (100 MHz clock) sets the error word; every poll also watches
// that word, and a failed poll lets its group run on without waiting, so the grid
// always ends. Groups are launched cooperatively (all resident), one per CU.
#include <string.h>

#include <algorithm>

#include "common.h"
#include "decode_step.h"

namespace ts {
namespace {

constexpr uint32_t kW = 8;                      // waves per group
constexpr uint32_t kT = kW * 64;                // threads per group
constexpr uint32_t kMaxH = 1024;                // hidden (2 chunks of 8 per lane)
constexpr uint32_t kMaxQD = 2048;               // q heads x 128 (4 chunks per lane)
constexpr uint32_t kMaxF = 3072;                // ffn (6 chunks per lane)
constexpr uint32_t kMaxPages = 512;
constexpr uint32_t kLdsBytes = 96 * 1024;       // more than half the CU's LDS: one group per CU
constexpr uint64_t kTimeout = 200000000ull;     // 2 s of the 100 MHz clock
constexpr int kPre = 5;                         // 4-key blocks per wave per attention pass
constexpr uint32_t kMaxLm = 1024;               // lm_head rows a group holds
constexpr int kLmDepth = 4;                     // lm_head row tiles in flight per wave
constexpr uint64_t kPrefetchDelay = 70;         // 0.7 us of the 100 MHz clock
// 16-row tiles a group holds per product role (gate/up: gate tiles then up tiles).
constexpr int kTilesQkv = 4, kTilesO = 2, kTilesGu = 4, kTilesDn = 2;

enum Role : uint32_t { kQkv = 0, kO = 1, kGu = 2, kDn = 3, kAtt = 4 };

// LDS layout (bytes).
// A staged part is kXsCol bf16 long: 16 bytes past kMaxF, so the three parts one
// fragment read touches start on different banks (kMaxF * 2 bytes is a multiple of 256).
constexpr uint32_t kXsCol = kMaxF + 8;
constexpr uint32_t kXsOff = 0;                             // staged inputs, 3 bf16 parts [2][3][kXsCol]
constexpr uint32_t kResOff = kXsOff + 2 * 3 * kXsCol * 2;  // residual rows [2][64]
constexpr uint32_t kSsqOff = kResOff + 2 * 64 * 4;        // sums of squares [2][kW]
constexpr uint32_t kPartOff = kSsqOff + 2 * kW * 4;       // per-wave row partials [2][kW][64]
constexpr uint32_t kLmPartOff = kPartOff + 2 * kW * 64 * 4;  // lm_head row partials [kW][kMaxLm]
constexpr uint32_t kTblOff = kLmPartOff + kW * kMaxLm * 4;  // page table [kMaxPages]
constexpr uint32_t kAttOff = kTblOff + kMaxPages * 4;     // attention scratch
constexpr uint32_t kAttBytes = 512 * 4 + 2 * 128 * 4 + 2 * 128 * 2 + 2 * kW * 2 * 4 + 2 * kW * 128 * 4;
constexpr uint32_t kBestOff = kAttOff + kAttBytes;        // per-wave (max, index) [kW][2]
constexpr uint32_t kPickOff = kBestOff + kW * 2 * 4;      // every group's (max, index) [2 * groups]
constexpr uint32_t kCtlOff = kPickOff + 2 * kStepMaxGroups * 4;
constexpr uint32_t kLdsUsed = kCtlOff + 16 * 4;
static_assert(kLdsUsed <= kLdsBytes, "LDS layout");
// Control words.
constexpr uint32_t kAbort = 0;  // a wait of this group gave up
constexpr uint32_t kTok = 1;    // the step's token

// Rows [first, first + count) of N split over n parts, ceil(N / n) each.
struct Split {
    uint32_t first, count;
};
__host__ __device__ inline Split split(uint32_t n, uint32_t parts, uint32_t i) {
    const uint32_t per = (n + parts - 1) / parts;
    const uint32_t f = i * per < n ? i * per : n;
    return {f, (f + per < n ? f + per : n) - f};
}

// Hand-off word offsets: per layer qkv, attention, x after o, silu*up, x after down;
// then two words per group for the greedy pick.
struct Hand {
    uint32_t qkv, att, x2, hf, xo, block, am;
};
TS_DEV Hand hand(const DecodeStepArgs &p) {
    Hand h;
    h.qkv = 0;
    h.att = (p.Hq + 2 * p.Hkv) * 128;
    h.x2 = h.att + p.Hq * 128;
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

// A wave-uniform address as a scalar value (a load then takes it as its scalar base and
// only the lane's offset in a vector register).
TS_DEV const char *uniform(const void *ptr) {
    const uint64_t v = (uint64_t)ptr;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const char *)(((uint64_t)hi << 32) | lo);
}

// A barrier of the group's waves that publishes their LDS writes; global loads stay
// in flight (__syncthreads would wait for them, draining the weight prefetch).
TS_DEV void bar() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

struct Ctx {
    char *lds;
    volatile uint32_t *ctl;
    uint32_t *err;
    uint32_t *tbl;
    uint32_t tid, wave, lane, g;
    uint32_t ph;  // staging parity
    TS_DEV uint16_t *xs() const { return (uint16_t *)(lds + kXsOff) + (ph & 1) * 3 * kXsCol; }
    TS_DEV float *res() const { return (float *)(lds + kResOff) + (ph & 1) * 64; }
    TS_DEV float *ssq() const { return (float *)(lds + kSsqOff) + (ph & 1) * kW; }
    TS_DEV float *part() const { return (float *)(lds + kPartOff) + (ph & 1) * kW * 64; }
};

// Sums (maxima) over the four 16-lane rows of a wave, in every lane.
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

// Whole-wave total in every lane on the VALU alone: DPP within rows of 16, then the
// gfx950 permlane swaps across rows (no LDS round trips, unlike a shuffle).
TS_DEV float wave_total(float v) { return rows4_sum(row16_sum(v)); }

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
    // No sleep between polls: C1 2437 against 2412 tok/s with s_sleep 1 (longer sleeps
    // measured slower still).
    return true;
}

// The words a thread takes of an input vector: base + stride k, k < NX. Group-wide
// (base tid, stride kT) or one wave's own range (base 32 KS wave + lane, stride 64).
struct Words {
    uint32_t base, stride;
};
TS_DEV Words group_words(const Ctx &c) { return {c.tid, kT}; }

// Tagged words src[w.base + w.stride k] (k < NX, index < n) into v[k], and (extra
// non-null) one more word into *xv: every load is issued, then the loads whose epoch
// is stale are reissued until none is.
template <int NX>
TS_DEV void poll(Ctx &c, Words ws, const uint64_t *src, uint32_t n, uint32_t tag, float (&v)[NX],
                 const uint64_t *extra = nullptr, float *xv = nullptr) {
    uint64_t w[NX], x;
#pragma unroll
    for (int k = 0; k < NX; k++) {
        const uint32_t i = ws.base + ws.stride * k;
        w[k] = i < n ? ld_tag(src + i) : ((uint64_t)tag << 32);
    }
    x = extra ? ld_tag(extra) : ((uint64_t)tag << 32);
    uint64_t t0 = 0;
    uint32_t it = 0;
    for (;;) {
        bool ready = (uint32_t)(x >> 32) == tag;
#pragma unroll
        for (int k = 0; k < NX; k++) ready &= (uint32_t)(w[k] >> 32) == tag;
        if (ready || !spin(c, it, t0)) break;
#pragma unroll
        for (int k = 0; k < NX; k++)
            if ((uint32_t)(w[k] >> 32) != tag) w[k] = ld_tag(src + ws.base + ws.stride * k);
        if ((uint32_t)(x >> 32) != tag) x = ld_tag(extra);
    }
#pragma unroll
    for (int k = 0; k < NX; k++) v[k] = __uint_as_float((uint32_t)w[k]);
    if (extra) *xv = __uint_as_float((uint32_t)x);
}

// One tagged word (thread-private wait).
TS_DEV float poll1(Ctx &c, const uint64_t *src, uint32_t tag) {
    uint64_t w = ld_tag(src);
    uint64_t t0 = 0;
    uint32_t it = 0;
    while ((uint32_t)(w >> 32) != tag && spin(c, it, t0)) w = ld_tag(src);
    return __uint_as_float((uint32_t)w);
}

// Gains of the words this thread stages (1 without a gain), loaded before the poll.
template <int NX>
TS_DEV void gains(const Ctx &c, Words ws, const float *g, uint32_t n, float (&gv)[NX]) {
#pragma unroll
    for (int k = 0; k < NX; k++) {
        const uint32_t i = ws.base + ws.stride * k;
        gv[k] = g && i < n ? g[i] : 1.0f;
    }
}

// Stage an input of n values: x = v * g (the preloaded gains) as three bf16 parts,
// x = hi + mid + lo (8 + 8 + 8 mantissa bits: exact for normal values), the B
// operand columns of the matrix-unit products; and the group's partial sums of
// squares of v (read after the next barrier by norm_inv).
template <int NX>
TS_DEV void stage(Ctx &c, Words ws, const float (&v)[NX], uint32_t n, const float (&g)[NX]) {
    float ss = 0.0f;
    uint16_t *xs = c.xs();
#pragma unroll
    for (int k = 0; k < NX; k++) {
        const uint32_t i = ws.base + ws.stride * k;
        if (i < n) {
            const float x = v[k] * g[k];
            const uint16_t hi = bf16_bits(x);
            const float r1 = x - bf16_float(hi);
            const uint16_t mid = bf16_bits(r1);
            xs[i] = hi;
            xs[kXsCol + i] = mid;
            xs[2 * kXsCol + i] = bf16_bits(r1 - bf16_float(mid));
            ss += v[k] * v[k];
        }
    }
    ss = wave_total(ss);
    if (c.lane == 0) c.ssq()[c.wave] = ss;
}

// 1/sqrt(mean(v^2) + eps): the RmsNorm scale, folded into the products' results
// (sum_k (x_k inv g_k) w_k = inv sum_k (x_k g_k) w_k).
TS_DEV float norm_inv(const float *ssq, uint32_t n, float eps) {
    float t = 0.0f;
    for (uint32_t w = 0; w < kW; w++) t += ssq[w];
    return 1.0f / sqrtf(t / (float)n + eps);
}

// Optional phase stamps of the first step (thread 0 of every group): row l, slot k.
TS_DEV void mark(const DecodeStepArgs &p, const Ctx &c, uint32_t t, uint32_t l, uint32_t k) {
    if (p.marks && t == 0 && c.tid == 0) {
        p.marks[((size_t)c.g * (p.L + 2) + l) * 10 + k] = now();
    }
}

TS_DEV void better(float &bv, uint32_t &bi, float v, uint32_t i) {
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

// 16-row tiles of lm_head rows per group (every group the same count; rows past a
// group's share are zeros in the packed copy).
__host__ __device__ inline uint32_t lm_tiles(uint32_t V, uint32_t NG) { return ((V + NG - 1) / NG + 15) / 16; }

// ---------------------------------------------------------------------------
// Products on the matrix unit. A 16-row tile of weights is the A operand of
// v_mfma_f32_16x16x32_bf16 (lane l: row l % 16, k 8 (l / 16) .. +8 of a 32-deep
// k-step); the input is the B operand with three live columns, its three bf16
// parts (x = hi + mid + lo, exact): columns 0, 1, 2 hold them, the rest zero. Lane l
// of the result holds column l % 16, rows 4 (l / 16) .. +3, so rows' sums are
// columns 0 + 1 + 2: lanes 0, 16, 32, 48 after two DPP swaps. A wave owns
// a range of k-steps of every tile; the waves' partials meet in LDS and are summed
// in wave order.
// ---------------------------------------------------------------------------

// B fragment of k-step ks from the staged input: column 0 the high parts of k values
// ks * 32 + 8 (l / 16) .. +8, column 1 the middle, column 2 the low, the rest zero.
// Branch-free: every lane reads (the other columns a part that exists) and zeroes by
// select, so a role's reads of all its k-steps issue back to back before the MFMAs.
TS_DEV u32x4 x_frag(const Ctx &c, const uint16_t *xs, uint32_t ks, uint32_t K) {
    const uint32_t col = c.lane & 15, k0 = ks * 32 + (c.lane >> 4) * 8;
    const bool live = col < 3 && k0 < K;
    const u32x4 v = *(const u32x4 *)&xs[(col < 3 ? col : 0) * kXsCol + (k0 < K ? k0 : 0)];
    return live ? v : u32x4{0, 0, 0, 0};
}

// The tile's row sums (columns 0 + 1 + 2) into part[t * 16 + row] from lanes 0, 16,
// 32, 48.
TS_DEV void tile_out(const Ctx &c, f32x4 acc, float *part, uint32_t t) {
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float a = acc[i] + dpp_f(acc[i], 0);  // columns 0 + 1 (and 2 + 3 in lane 2)
        v[i] = a + dpp_f(a, 1);                     // + columns 2 + 3 (3 is zero)
    }
    if ((c.lane & 15) == 0) {
        float *dst = part + t * 16 + 4 * (c.lane >> 4);
        *(float4 *)dst = make_float4(v[0], v[1], v[2], v[3]);
    }
}

// ---------------------------------------------------------------------------
// The lm_head rows of this group and the group's best (value, index), published.
// Wave w streams k-steps [4 w, 4 w + 4) of every 16-row tile, kLmDepth tiles in
// flight; the row sums meet in LDS.
// ---------------------------------------------------------------------------
TS_DEV void lm_rows(const DecodeStepArgs &p, Ctx &c, const Hand &hd, uint32_t t, uint32_t tag) {
    const uint32_t H = p.H;
    const Split rows = split(p.V, p.NG, c.g);
    const uint32_t tiles = (rows.count + 15) / 16;
    constexpr int KS = 4;  // k-steps per wave (H <= 1024)
    float *part = (float *)(c.lds + kLmPartOff) + c.wave * kMaxLm;
    u32x4 a0[KS], a1[KS], a2[KS], a3[KS];
    // The packed lm_head tiles of this group (decode_step_pack, role 4).
    const uint32_t KSt = H / 32, LT = lm_tiles(p.V, p.NG);
    const char *P = (const char *)p.lm_packed + (size_t)c.g * LT * KSt * 1024;
    auto load = [&](uint32_t ti, u32x4 (&a)[KS]) {
#pragma unroll
        for (int j = 0; j < KS; j++) {
            const uint32_t ks = c.wave * KS + j;
            const u32x4 *blk = (const u32x4 *)uniform(P + ((size_t)ti * KSt + ks) * 1024);
            a[j] = ks < KSt ? __builtin_nontemporal_load(blk + c.lane) : u32x4{0, 0, 0, 0};
        }
    };
    // The first tiles' loads do not need the input: issued before it is polled.
    if (tiles > 0) load(0, a0);
    if (tiles > 1) load(1, a1);
    if (tiles > 2) load(2, a2);
    {
        float v[2], gv[2];
        gains<2>(c, group_words(c), p.norm, H, gv);
        const uint64_t *blk = p.hand + (size_t)(p.L - 1) * hd.block;
        poll<2>(c, group_words(c), blk + hd.xo, H, tag, v);
        stage<2>(c, group_words(c), v, H, gv);
    }
    mark(p, c, t, p.L, 0);
    bar();
    const float inv = norm_inv(c.ssq(), H, p.eps);
    const uint16_t *xs = c.xs();
    c.ph++;
    u32x4 xb[KS];
#pragma unroll
    for (int j = 0; j < KS; j++) xb[j] = x_frag(c, xs, c.wave * KS + j, H);
    auto use = [&](uint32_t ti, const u32x4 (&a)[KS]) {
        f32x4 acc = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < KS; j++) acc = mfma16(as_bf16x8(a[j]), as_bf16x8(xb[j]), acc);
        tile_out(c, acc, part, ti);
    };
    for (uint32_t i = 0; i < tiles; i += 4) {
        if (i + 3 < tiles) load(i + 3, a3);
        use(i, a0);
        if (i + 1 >= tiles) break;
        if (i + 4 < tiles) load(i + 4, a0);
        use(i + 1, a1);
        if (i + 2 >= tiles) break;
        if (i + 5 < tiles) load(i + 5, a1);
        use(i + 2, a2);
        if (i + 3 >= tiles) break;
        if (i + 6 < tiles) load(i + 6, a2);
        use(i + 3, a3);
    }
    mark(p, c, t, p.L, 1);
    bar();
    // Row r: the waves' partials in wave order, then the best of this thread's rows.
    const float *lp = (const float *)(c.lds + kLmPartOff);
    float bv = -INFINITY;
    uint32_t bi = p.V;
    for (uint32_t r = c.tid; r < rows.count; r += kT) {
        float x = 0.0f;
#pragma unroll
        for (uint32_t w = 0; w < kW; w++) x += lp[w * kMaxLm + r];
        x *= inv;
        const uint32_t row = rows.first + r;
        p.logits[row] = x;
        if (x > -INFINITY) better(bv, bi, x, row);  // NaN and -inf never win
    }
#ifdef TS_FINE
    mark(p, c, t, p.L, 3);
#endif
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const uint32_t oi = __shfl_xor(bi, o, 64);
        better(bv, bi, ov, oi);
    }
    float *best = (float *)(c.lds + kBestOff);
    if (c.lane == 0) {
        best[2 * c.wave] = bv;
        best[2 * c.wave + 1] = __uint_as_float(bi);
    }
    bar();
    uint64_t *am = p.hand + hd.am;
    if (c.tid == 0) {
        float v = -INFINITY;
        uint32_t i = p.V;
        for (uint32_t w = 0; w < kW; w++) better(v, i, best[2 * w], __float_as_uint(best[2 * w + 1]));
        st_tag(am + 2 * c.g, __float_as_uint(v), tag);
        st_tag(am + 2 * c.g + 1, i, tag);
    }
#ifdef TS_FINE
    mark(p, c, t, p.L, 4);
#endif
}

// Every group's best, reduced in group order (ties to the lower index): the token.
TS_DEV uint32_t pick(const DecodeStepArgs &p, Ctx &c, const Hand &hd, uint32_t t, uint32_t tag) {
    uint64_t *am = p.hand + hd.am;
    float *pk = (float *)(c.lds + kPickOff);
    for (uint32_t i = c.tid; i < 2 * p.NG; i += kT) pk[i] = poll1(c, am + i, tag);
#ifdef TS_FINE
    mark(p, c, t, p.L, 5);
#endif
    bar();
    if (c.wave == 0) {
        float v = -INFINITY;
        uint32_t i = p.V;
        for (uint32_t w = c.lane; w < p.NG; w += 64) {
            const uint32_t xi = __float_as_uint(pk[2 * w + 1]);
            if (xi < p.V) better(v, i, pk[2 * w], xi);
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(v, o, 64);
            const uint32_t oi = __shfl_xor(i, o, 64);
            better(v, i, ov, oi);
        }
        if (c.lane == 0) c.ctl[kTok] = i;
    }
    bar();
    mark(p, c, t, p.L, 2);
    const uint32_t tok = c.ctl[kTok];
    return tok < p.V ? tok : 0u;  // no finite logit (an aborted launch): any row of the table
}

// ---------------------------------------------------------------------------
// Product roles. The group's outputs [s.first, s.first + s.count) of one matrix, as
// TILES 16-row tiles (gate/up: TILES / 2 gate tiles, then the matching up tiles),
// held in registers: wave w keeps k-steps [KS w, KS w + KS) of every tile. Per
// layer: each wave polls the input words of its own k-steps (the RmsNorm gains loaded
// first; o and down also poll their residual rows), stages them, and runs its MFMAs
// without waiting for the other waves; the partials go to LDS, one barrier, each
// output is summed over the waves by one thread (with the RmsNorm scale from the
// waves' sums of squares) and published by consecutive threads (whole lines per
// store instruction); then the next layer's tiles are loaded into the same registers.
// ---------------------------------------------------------------------------
template <uint32_t KIND, int TILES, int KS, int NX>
TS_DEV void product_role(const DecodeStepArgs &p, Ctx &c, const Hand &hd, uint32_t idx, uint32_t count) {
    const uint32_t H = p.H, F = p.F, QD = p.Hq * 128, QKV = (p.Hq + 2 * p.Hkv) * 128;
    const uint32_t N = KIND == kQkv ? QKV : (KIND == kGu ? F : H);
    const uint32_t K = KIND == kQkv || KIND == kGu ? H : (KIND == kO ? QD : F);
    const Split s = split(N, count, idx);
    constexpr int OT = KIND == kGu ? TILES / 2 : TILES;  // tiles of outputs
    static_assert(NX * 64 == KS * 32, "a wave polls exactly the words of its k-steps");
    const Words ws = {32 * KS * c.wave + c.lane, 64};  // this wave's input words
    u32x4 w[TILES][KS];
    // The packed tiles (decode_step_pack): tile t, k-step ks of this group is 1 KB at
    // ((idx * TILES + t) * KSt + ks) KiB, lane l's 16 bytes at l * 16.
    const uint32_t KSt = K / 32;
    auto load = [&](uint32_t l) {
        const char *P = (const char *)p.packed[l][KIND] + (size_t)idx * TILES * KSt * 1024;
#pragma unroll
        for (int t = 0; t < TILES; t++) {

#pragma unroll
            for (int j = 0; j < KS; j++) {
                const uint32_t ks = c.wave * KS + j;
                const u32x4 *blk = (const u32x4 *)uniform(P + ((size_t)t * KSt + ks) * 1024);
                w[t][j] = ks < KSt ? __builtin_nontemporal_load(blk + c.lane) : u32x4{0, 0, 0, 0};
            }
        }
    };
    load(0);

    uint32_t tok = p.tok[0];
    const uint32_t pos0 = p.pos[0];
    for (uint32_t t = 0; t < p.steps; t++) {
        const uint32_t tag = p.epoch + t;
        for (uint32_t l = 0; l < p.L; l++) {
            const uint64_t *blk = p.hand + (size_t)l * hd.block;
            const uint64_t *prev = l ? blk - hd.block : nullptr;
            // Input (the RmsNorm gains loaded first), and for o and down the residual
            // rows (one word a thread, polled with the input).
            float v[NX], gv[NX];
            const uint32_t n = K;
            gains<NX>(c, ws, KIND == kQkv ? p.ln1[l] : (KIND == kGu ? p.ln2[l] : nullptr), n, gv);
            const bool has_res = (KIND == kO || KIND == kDn) && c.tid < s.count;
            const uint64_t *res_src = nullptr;
            float rv = 0.0f;
            if (has_res) {
                if (KIND == kO) {
                    if (prev) res_src = prev + hd.xo + s.first + c.tid;
                    else rv = bf16_float(p.embed[(size_t)tok * H + s.first + c.tid]);
                } else {
                    res_src = blk + hd.x2 + s.first + c.tid;
                }
            }
            if (KIND == kQkv && !prev) {
#pragma unroll
                for (int k = 0; k < NX; k++) {
                    const uint32_t i = ws.base + ws.stride * k;
                    v[k] = i < n ? bf16_float(p.embed[(size_t)tok * H + i]) : 0.0f;
                }
            } else {
                const uint64_t *in = KIND == kQkv ? prev + hd.xo
                                                  : (KIND == kO ? blk + hd.att : (KIND == kGu ? blk + hd.x2 : blk + hd.hf));
                // The whole input is polled from the start (a light wait first on one
                // word a wave of the stage before the input's producers measured 2433
                // against 2450 tok/s once polls stopped sleeping).
                poll<NX>(c, ws, in, n, tag, v, res_src, &rv);
            }
            if (has_res) c.res()[c.tid] = rv;
            stage<NX>(c, ws, v, n, gv);
            mark(p, c, t, l, 0);
            // No barrier: a wave's fragments come from the words it staged itself
            // (LDS operations of one wave complete in order), so each wave starts its
            // MFMAs once its own words are in; the residual words and the sums of
            // squares are read after the barrier that ends the products.
            const uint16_t *xs = c.xs();
            const float *res = c.res(), *ssq = c.ssq();
            c.ph++;
            if (s.count) {
#ifdef TS_FINE
                mark(p, c, t, l, 2);
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                mark(p, c, t, l, 3);
#endif
                float *part = c.part();
                f32x4 acc[TILES];
#pragma unroll
                for (int t2 = 0; t2 < TILES; t2++) acc[t2] = f32x4{0, 0, 0, 0};
                // The input fragments in chunks of CH k-steps, the next chunk's reads
                // issued before this chunk's MFMAs (the order pinned: the LDS latency
                // then hides under matrix work instead of preceding every step).
                constexpr int CH = KS < 4 ? KS : 4;
                u32x4 xb[2][CH];
#pragma unroll
                for (int j = 0; j < CH; j++) xb[0][j] = x_frag(c, xs, c.wave * KS + j, K);
#pragma unroll
                for (int j0 = 0; j0 < KS; j0 += CH) {
                    const int cur = (j0 / CH) & 1;
                    if (j0 + CH < KS) {
#pragma unroll
                        for (int j = 0; j < CH; j++) xb[cur ^ 1][j] = x_frag(c, xs, c.wave * KS + j0 + CH + j, K);
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int j = 0; j < CH; j++)
#pragma unroll
                        for (int t2 = 0; t2 < TILES; t2++)
                            acc[t2] = mfma16(as_bf16x8(w[t2][j0 + j]), as_bf16x8(xb[cur][j]), acc[t2]);
                    __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
                for (int t2 = 0; t2 < TILES; t2++) tile_out(c, acc[t2], part + c.wave * 64, t2);
#ifdef TS_FINE
                mark(p, c, t, l, 4);
#endif
                bar();
                if (c.tid < s.count) {
                    const uint32_t o = c.tid;
                    float x = 0.0f;
#pragma unroll
                    for (uint32_t w2 = 0; w2 < kW; w2++) x += part[w2 * 64 + o];
                    const float inv = KIND == kQkv || KIND == kGu ? norm_inv(ssq, n, p.eps) : 1.0f;
                    float y;
                    if (KIND == kQkv) {
                        y = x * inv;
                    } else if (KIND == kGu) {
                        float u = 0.0f;
#pragma unroll
                        for (uint32_t w2 = 0; w2 < kW; w2++) u += part[w2 * 64 + OT * 16 + o];
                        const float gt = x * inv, up = u * inv;
                        y = gt / (1.0f + expf(-gt)) * up;
                    } else {
                        y = res[o] + x;
                    }
                    uint64_t *out = (uint64_t *)(blk + (KIND == kQkv ? hd.qkv : (KIND == kO ? hd.x2
                                                                                : (KIND == kGu ? hd.hf : hd.xo))));
                    st_tag(out + s.first + o, __float_as_uint(y), tag);
                }
                mark(p, c, t, l, 1);
                // The next layer's tiles (the first layer's after the lm_head).
#ifndef TS_NOPF
                // Held back kPrefetchDelay first: issued at once, every role's prefetch
                // lands in the hand-off that follows its publish and slows those polls.
                {
                    const uint64_t t0 = now();
                    while (now() - t0 < kPrefetchDelay) __builtin_amdgcn_s_sleep(8);
                }
                if (l + 1 < p.L) load(l + 1);
#endif
            }
        }
        lm_rows(p, c, hd, t, tag);
        // The first layer's tiles, issued once the lm_head has streamed (its registers
        // are free then) and after the token's poll (the memory counter retires in
        // order: a poll issued behind them would wait for them).
        if (KIND == kQkv || KIND == kO) tok = pick(p, c, hd, t, tag);
#ifndef TS_NOPF
        load(0);  // unconditional (also after the last step): the registers are dead across the lm_head
#endif
        if (KIND == kQkv && idx == 0 && c.tid == 0) {
            p.hist[pos0 + t + 1] = tok;
            if (t + 1 == p.steps) {
                p.pos[0] = pos0 + p.steps;
                p.tok[0] = tok;
            }
        }
    }
}

// RmsNorm over a 128-wide head held as (d, d + 64) in lane d, then the Halves
// rotation of that pair (engine/ir/interp/src/cpu.rs:36-47, 371-377).
TS_DEV void norm_rope(float &a, float &b, float ga, float gb, float cs, float sn, float eps) {
    const float s = wave_total(a * a + b * b);
    const float inv = 1.0f / sqrtf(s / 128.0f + eps);
    a = a * (inv * ga);
    b = b * (inv * gb);
    const float ra = a * cs - b * sn, rb = a * sn + b * cs;
    a = ra;
    b = rb;
}

// ---------------------------------------------------------------------------
// Attention role: q head h (kv head a = h / (heads / kv heads)) at position pos over
// kept rows [0, pos] (engine/ir/interp/src/cpu.rs:141-167, 293-351). Lanes: key
// lane / 16 of a 4-key block, dims 8 (lane % 16) .. +8; wave w takes blocks w + kW i.
// Scores in base 2 (dot(q, k) * scale * log2 e, v_exp_f32). The raw q/k/v rows come
// from the qkv hand-off; q and the new k are normalized and rotated, and the new k
// and v rows appended (bf16) after the head's output is published. Every q head of
// kv head a appends the same row: the same words through the same arithmetic give
// the same bits, so the row's value never depends on which write lands last. A
// group's own append is waited for (vmcnt) before the barrier that ends the layer,
// and the row is read only at later steps (reads stop at pos - 1 until it exists),
// through this CU's caches, which never held it before.
// ---------------------------------------------------------------------------
TS_DEV void att_role(const DecodeStepArgs &p, Ctx &c, const Hand &hd, uint32_t h) {
    const uint32_t lane = c.lane, wave = c.wave;
    const uint32_t kr = lane >> 4, part = lane & 15;
    const uint32_t Hkv = p.Hkv, a = h / (p.Hq / Hkv), shift = p.page_shift, mask = (1u << shift) - 1;
    const uint32_t QD = p.Hq * 128;
    float *raw = (float *)(c.lds + kAttOff);   // [384]: q h, k a, v a
    float *qs = raw + 384;                     // [128]
    uint16_t *kn = (uint16_t *)(qs + 128);     // [128]
    uint16_t *vn = kn + 128;                   // [128]
    float *pm = (float *)(vn + 128);           // [kW]
    float *pl = pm + kW;                       // [kW]
    float *po = pl + kW;                       // [kW][128]
    const uint32_t pos0 = p.pos[0];
    const float sl2 = p.scale * 1.4426950408889634f;
    for (uint32_t t = 0; t < p.steps; t++) {
        const uint32_t tag = p.epoch + t, pos = pos0 + t;
        const uint32_t last = pos ? pos - 1 : 0u;   // kept rows before pos exist
        const uint32_t nblk = (pos >> 2) + 1;       // 4-key blocks in [0, pos]
        const uint32_t mine = nblk > wave ? (nblk - wave + kW - 1) / kW : 0;
        const float2 cs = ((const float2 *)p.rope)[(size_t)pos * 64 + lane];
        for (uint32_t l = 0; l < p.L; l++) {
            const uint16_t *kc = p.k_cache[l], *vc = p.v_cache[l];
            // Kept rows of earlier positions: this wave's first kPre blocks, now.
            u32x4 kk[kPre], vv[kPre];
#pragma unroll
            for (int i = 0; i < kPre; i++) {
                const uint32_t key = min(4 * (wave + kW * i) + kr, last);
                const uint64_t row = ((uint64_t)c.tbl[key >> shift] << shift) | (key & mask);
                const size_t e = (row * Hkv + a) * 128 + 8 * part;
                kk[i] = *(const u32x4 *)(kc + e);
                vv[i] = *(const u32x4 *)(vc + e);
            }
            float ga = 0.0f, gb = 0.0f;
            if (wave == 0) { ga = p.q_norm[l][lane]; gb = p.q_norm[l][lane + 64]; }
            if (wave == 1) { ga = p.k_norm[l][lane]; gb = p.k_norm[l][lane + 64]; }
            // q head h, then k and v of head a: one word a thread.
            if (c.tid < 384) {
                const uint64_t *blk = p.hand + hd.qkv + (size_t)l * hd.block;
                const uint32_t r = c.tid >> 7, d = c.tid & 127;
                const uint32_t gi = r == 0 ? h * 128 + d : QD + ((r - 1) * Hkv + a) * 128 + d;
                raw[c.tid] = poll1(c, blk + gi, tag);
            }
            mark(p, c, t, l, 0);
            bar();
            if (wave < 3) {
                float x0 = raw[wave * 128 + lane], x1 = raw[wave * 128 + lane + 64];
                if (wave < 2) norm_rope(x0, x1, ga, gb, cs.x, cs.y, p.eps);
                if (wave == 0) {
                    qs[lane] = x0;
                    qs[lane + 64] = x1;
                } else {
                    uint16_t *dst = wave == 1 ? kn : vn;
                    dst[lane] = bf16_bits(x0);
                    dst[lane + 64] = bf16_bits(x1);
                }
            }
            bar();
#ifdef TS_FINE
            mark(p, c, t, l, 2);
#endif
            float q[8];
            {
                const float4 q0 = *(const float4 *)&qs[8 * part], q1 = *(const float4 *)&qs[8 * part + 4];
                q[0] = q0.x; q[1] = q0.y; q[2] = q0.z; q[3] = q0.w;
                q[4] = q1.x; q[5] = q1.y; q[6] = q1.z; q[7] = q1.w;
            }
            const u32x4 knew = *(const u32x4 *)(kn + 8 * part), vnew = *(const u32x4 *)(vn + 8 * part);
            float m = -INFINITY, ls = 0.0f, o[8];
#pragma unroll
            for (int e = 0; e < 8; e++) o[e] = 0.0f;

            for (uint32_t i0 = 0; i0 < mine; i0 += kPre) {
                if (i0) {  // contexts past kW kPre blocks: load this pass now
#pragma unroll
                    for (int i = 0; i < kPre; i++) {
                        const uint32_t key = min(4 * (wave + kW * (i0 + i)) + kr, last);
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
                    const uint32_t key = 4 * (wave + kW * (i0 + i)) + kr;
                    ok[i] = key <= pos;
                    const u32x4 kv = key == pos ? knew : kk[i];
                    const uint32_t kw[4] = {kv.x, kv.y, kv.z, kv.w};
                    float s0 = 0.0f;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        s0 += q[2 * e] * lo_bf16(kw[e]);
                        s0 += q[2 * e + 1] * hi_bf16(kw[e]);
                    }
                    sc[i] = ok[i] ? row16_sum(s0) * sl2 : -INFINITY;
                }
                float bm = sc[0];
#pragma unroll
                for (int i = 1; i < kPre; i++) bm = fmaxf(bm, sc[i]);
                const float mn = fmaxf(m, rows4_max(bm));  // finite: key 4 wave <= pos
                const float alpha = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - mn);
                float acc[8], sum = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; e++) acc[e] = 0.0f;
#pragma unroll
                for (int i = 0; i < kPre; i++) {
                    const float pk = ok[i] ? __builtin_amdgcn_exp2f(sc[i] - mn) : 0.0f;
                    sum += pk;
                    const u32x4 vx = (4 * (wave + kW * (i0 + i)) + kr) == pos ? vnew : vv[i];
                    const uint32_t vw[4] = {ok[i] ? vx.x : 0u, ok[i] ? vx.y : 0u, ok[i] ? vx.z : 0u,
                                            ok[i] ? vx.w : 0u};
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
#ifdef TS_FINE
            mark(p, c, t, l, 3);
#endif
            // Sum the four key rows; lanes of row 0 hold the wave's partial sums.
#pragma unroll
            for (int e = 0; e < 8; e++) o[e] = rows4_sum(o[e]);
            if (kr == 0) {
                float *dst = po + wave * 128 + 8 * part;
                *(float4 *)dst = make_float4(o[0], o[1], o[2], o[3]);
                *(float4 *)(dst + 4) = make_float4(o[4], o[5], o[6], o[7]);
            }
            if (lane == 0) {
                pm[wave] = m;
                pl[wave] = ls;
            }
            bar();
#ifdef TS_FINE
            mark(p, c, t, l, 4);
#endif
            if (c.tid < 128) {
                const uint32_t d = c.tid;
                float M = -INFINITY;
                for (uint32_t w = 0; w < kW; w++) M = fmaxf(M, pm[w]);
                float L = 0.0f, O = 0.0f;
                for (uint32_t w = 0; w < kW; w++) {
                    const float f = pm[w] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(pm[w] - M);
                    L += pl[w] * f;
                    O += po[w * 128 + d] * f;
                }
                st_tag(p.hand + hd.att + (size_t)l * hd.block + h * 128 + d, __float_as_uint(O / L), tag);
            }
            mark(p, c, t, l, 1);
            // Then the new row joins the kept rows (Store::append,
            // engine/ir/interp/src/run.rs:122-198), off the chain.
            if (wave == 1 || wave == 2) {
                const uint16_t *src = wave == 1 ? kn : vn;
                const uint64_t row = ((uint64_t)c.tbl[pos >> shift] << shift) | (pos & mask);
                uint16_t *cache = (wave == 1 ? p.k_cache[l] : p.v_cache[l]) + (row * Hkv + a) * 128;
                ((uint32_t *)cache)[lane] = ((const uint32_t *)src)[lane];
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            }
            bar();  // the scratch is reused by the next layer
        }
        lm_rows(p, c, hd, t, tag);
    }
}

// Groups without a role: the lm_head only.
TS_DEV void idle_role(const DecodeStepArgs &p, Ctx &c, const Hand &hd) {
    for (uint32_t t = 0; t < p.steps; t++) lm_rows(p, c, hd, t, p.epoch + t);
}

__global__ __launch_bounds__(kT) void decode_step_kernel(DecodeStepArgs p) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const uint32_t tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const uint32_t g = blockIdx.x;
    Ctx c;
    c.lds = lds;
    c.ctl = (volatile uint32_t *)(lds + kCtlOff);
    c.err = p.error;
    c.tbl = (uint32_t *)(lds + kTblOff);
    c.tid = tid;
    c.wave = wave;
    c.lane = lane;
    c.g = g;
    c.ph = 0;
    if (tid < 16) c.ctl[tid] = 0u;
    uint32_t role = kAtt + 1, idx = 0;
#pragma unroll
    for (uint32_t r = 0; r <= kAtt; r++)
        if (g >= p.role_first[r] && g < p.role_first[r] + p.role_count[r]) { role = r; idx = g - p.role_first[r]; }
    if (role == kAtt)
        for (uint32_t i = tid; i < p.kept_pages; i += kT) c.tbl[i] = p.table[i];
    __syncthreads();
    const Hand hd = hand(p);
    switch (role) {
    case kQkv: product_role<kQkv, kTilesQkv, kMaxH / 256, kMaxH / kT>(p, c, hd, idx, p.role_count[kQkv]); break;
    case kO: product_role<kO, kTilesO, kMaxQD / 256, kMaxQD / kT>(p, c, hd, idx, p.role_count[kO]); break;
    case kGu: product_role<kGu, kTilesGu, kMaxH / 256, kMaxH / kT>(p, c, hd, idx, p.role_count[kGu]); break;
    case kDn: product_role<kDn, kTilesDn, kMaxF / 256, kMaxF / kT>(p, c, hd, idx, p.role_count[kDn]); break;
    case kAtt: att_role(p, c, hd, idx); break;
    default: idle_role(p, c, hd); break;
    }
}

// Outputs a group of each product role can hold.
constexpr uint32_t kCap[4] = {16 * kTilesQkv, 16 * kTilesO, 16 * kTilesGu / 2, 16 * kTilesDn};

// Groups per role: the fewest that hold every output (attention: one per q head),
// then spare groups to the role whose groups carry the most weight bytes, in the
// fewest that lower that load.
bool plan_roles(uint32_t H, uint32_t Hq, uint32_t Hkv, uint32_t F, uint32_t NG, uint32_t *first, uint32_t *count) {
    const uint32_t QKV = (Hq + 2 * Hkv) * 128, QD = Hq * 128;
    const uint64_t n[4] = {QKV, H, F, H};
    const uint64_t bytes[4] = {2ull * H, 2ull * QD, 4ull * H, 2ull * F};  // per output
    uint32_t c[4];
    uint32_t used = Hq;
    for (int r = 0; r < 4; r++) {
        c[r] = (uint32_t)((n[r] + kCap[r] - 1) / kCap[r]);
        used += c[r];
    }
    if (used > NG) return false;
    auto load = [&](int r, uint32_t k) { return ((n[r] + k - 1) / k) * bytes[r]; };
    uint32_t spare = NG - used;
    bool done[4] = {false, false, false, false};
    for (;;) {
        int best = -1;
        for (int r = 0; r < 4; r++)
            if (!done[r] && (best < 0 || load(r, c[r]) > load(best, c[best]))) best = r;
        if (best < 0) break;
        uint32_t k = c[best] + 1;
        while (k <= c[best] + spare && load(best, k) >= load(best, c[best])) k++;
        if (k > c[best] + spare) {
            done[best] = true;
            continue;
        }
        spare -= k - c[best];
        c[best] = k;
    }
    uint32_t at = 0;
    for (int r = 0; r < 4; r++) {
        first[r] = at;
        count[r] = c[r];
        at += c[r];
    }
    first[kAtt] = at;
    count[kAtt] = Hq;
    return true;
}


// Packed copy of one role's matrix (decode_step_pack): thread i writes the 16 bytes of
// lane i % 64 of block i / 64 = (group, tile, k-step).
__global__ __launch_bounds__(256) void pack_kernel(const uint16_t *W, uint16_t *dst, uint32_t N, uint32_t K,
                                                   uint32_t groups, uint32_t tiles, uint32_t up_off, uint32_t gu,
                                                   uint64_t chunks) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= chunks) return;
    const uint32_t KSt = K / 32, lane = (uint32_t)(i & 63);
    const uint64_t blk = i >> 6;
    const uint32_t ks = (uint32_t)(blk % KSt), t = (uint32_t)((blk / KSt) % tiles), g = (uint32_t)(blk / KSt / tiles);
    const Split s = split(N, groups, g);
    const uint32_t ot = gu ? tiles / 2 : tiles;
    const uint32_t o = (t % ot) * 16 + (lane & 15);
    u32x4 v = {0, 0, 0, 0};
    if (o < s.count) {
        const uint32_t row = s.first + o + (gu && t >= ot ? up_off : 0u);
        v = *(const u32x4 *)(W + (size_t)row * K + ks * 32 + (lane >> 4) * 8);
    }
    *((u32x4 *)dst + i) = v;
}

struct PackShape {
    uint32_t N, K, groups, tiles, up_off, gu;
};

bool pack_shape(uint32_t H, uint32_t Hq, uint32_t Hkv, uint32_t F, uint32_t V, uint32_t NG, uint32_t role,
                PackShape *ps) {
    uint32_t first[5], count[5];
    if (!plan_roles(H, Hq, Hkv, F, NG, first, count)) return false;
    const uint32_t QKV = (Hq + 2 * Hkv) * 128, QD = Hq * 128;
    switch (role) {
    case kQkv: *ps = {QKV, H, count[kQkv], kTilesQkv, 0, 0}; break;
    case kO: *ps = {H, QD, count[kO], kTilesO, 0, 0}; break;
    case kGu: *ps = {F, H, count[kGu], kTilesGu, F, 1}; break;
    case kDn: *ps = {H, F, count[kDn], kTilesDn, 0, 0}; break;
    case 4: *ps = {V, H, NG, lm_tiles(V, NG), 0, 0}; break;
    default: return false;
    }
    return true;
}

}  // namespace

size_t decode_step_hand_words(uint32_t H, uint32_t L, uint32_t Hq, uint32_t Hkv, uint32_t F, uint32_t NG) {
    const size_t block = (size_t)(Hq + 2 * Hkv) * 128 + Hq * 128 + 2 * H + F;
    return L * block + 2 * (size_t)NG;
}

int decode_step_supported(uint32_t H, uint32_t L, uint32_t Hq, uint32_t Hkv, uint32_t D, uint32_t F, uint32_t V,
                          uint32_t kept_pages) {
    uint32_t ng = 0;
    int rc = decode_step_groups(&ng);
    if (rc != TS_OK) return rc;
    if ((V + ng - 1) / ng > kMaxLm) return 1;
    if (D != 128 || Hkv == 0 || Hq % Hkv || ng > kStepMaxGroups) return 1;
    if (H % 32 || F % 32) return 1;  // whole 32-deep k-steps
    if (L > kStepMaxLayers || H > kMaxH || H % 8 || F % 8 || F > kMaxF || Hq * 128 > kMaxQD) return 1;
    if (kept_pages > kMaxPages) return 1;
    uint32_t first[5], count[5];
    return plan_roles(H, Hq, Hkv, F, ng, first, count) ? TS_OK : 1;
}

size_t decode_step_packed_elems(uint32_t H, uint32_t Hq, uint32_t Hkv, uint32_t F, uint32_t V, uint32_t NG,
                                uint32_t role) {
    PackShape ps;
    if (!pack_shape(H, Hq, Hkv, F, V, NG, role, &ps)) return 0;
    return (size_t)ps.groups * ps.tiles * (ps.K / 32) * 512;
}

int decode_step_pack(const uint16_t *W, uint16_t *dst, uint32_t H, uint32_t Hq, uint32_t Hkv, uint32_t F, uint32_t V,
                     uint32_t NG, uint32_t role, void *stream) {
    PackShape ps;
    if (!pack_shape(H, Hq, Hkv, F, V, NG, role, &ps) || ps.K % 32)
        return fail(TS_ERR_ARG, "decode_step_pack: role %u does not fit %u groups", role, NG);
    const uint64_t chunks = (uint64_t)ps.groups * ps.tiles * (ps.K / 32) * 64;
    hipLaunchKernelGGL(pack_kernel, dim3((uint32_t)((chunks + 255) / 256)), dim3(256), 0, (hipStream_t)stream, W, dst,
                       ps.N, ps.K, ps.groups, ps.tiles, ps.up_off, ps.gu, chunks);
    TS_CHECK_LAUNCH("decode_step_pack launch");
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
    // Raised once per process; C++ makes the static's initialisation thread-safe, and
    // every call returns the stored outcome.
    static const hipError_t attr =
        hipFuncSetAttribute((const void *)decode_step_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (attr != hipSuccess) return hip_status(attr, "decode_step: shared memory attribute");
    DecodeStepArgs args = *a;
    if (!plan_roles(a->H, a->Hq, a->Hkv, a->F, a->NG, args.role_first, args.role_count))
        return fail(TS_ERR_ARG, "decode_step: %u groups cannot hold this shape", a->NG);
    void *params[] = {&args};
    hipError_t e = hipLaunchCooperativeKernel((const void *)decode_step_kernel, dim3(a->NG), dim3(kT), params,
                                              kLdsBytes, (hipStream_t)stream);
    if (e != hipSuccess) return hip_status(e, "decode_step: cooperative launch");
    return TS_OK;
}

}  // namespace ts
