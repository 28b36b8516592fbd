// Ragged-row attention over kept (paged) K/V: the decode kernel.
//
// Replaces the reference's attend_rows rule (one 256-thread group per
// (row, head), a block reduction per key: engine/rules/attention/src/attend.rs:
// 126-270) and flash_rows for decode rows (flash.rs:506-591). Semantics follow
// the interpreter: keys [max(0, pos - back), pos] of the row's slot, scores
// dot(q, k) * scale, softmax, sum of p * v (engine/ir/interp/src/cpu.rs:
// 141-167, 293-351). Kept rows are addressed through the page table as
// engine/plan/codegen/src/kept.rs:181-193 does.
//
// gfx950 design (HBM-bound: every K/V byte read once):
//  * One group per (row, kv head, key partition): all G = heads/kv_heads query
//    heads that share the kv head ride along, so K/V are read once per GQA group.
//  * Keys go 16 at a time (one page-aligned block; pages hold >= 16 rows so a
//    block is one table lookup). Scores S[16 heads, 16 keys] come from four
//    v_mfma_f32_16x16x32_bf16 steps per q part: each lane loads 64 contiguous
//    bytes of one key row (B operand), q is split into two bf16 parts.
//  * Online softmax per head in registers (16-lane butterflies, base 2 on
//    v_exp_f32), then P*V on
//    the vector ALUs: a lane owns 2 adjacent head dims, so each V row is one
//    256-byte coalesced load across the wave.
//  * A group's waves (up to 8) split its keys and merge (max, sum, acc) in LDS.
//    Short contexts (the batch-1 decode) take one group per (row, kv head).
//    Long ones split keys across groups too: each writes its partial to the
//    workspace and a second small kernel merges them in partition order. Past
//    2048 keys (no fused step) attend_long_kernel streams many key blocks per wave
//    with the next block's loads in flight. A
//    kernel boundary orders the two: a device-wide fence inside one kernel costs
//    more than the merge launch.
#include <string.h>

#include <algorithm>
#include <mutex>

#include "common.h"

#ifdef TS_MARKS
// Debug builds: a device ledger for TS_MARK, read back by tessera_hip_debug_marks.
static uint64_t *ts_debug_marks() {
    static uint64_t *ledger = nullptr;
    if (!ledger && hipMalloc((void **)&ledger, 16 * 65536 * sizeof(uint64_t)) != hipSuccess) ledger = nullptr;
    return ledger;
}
extern "C" int tessera_hip_debug_marks(uint64_t *host, uint32_t count) {
    uint64_t *d = ts_debug_marks();
    if (!d) return -1;
    return hipMemcpy(host, d, count * sizeof(uint64_t), hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}
#endif

namespace {

constexpr int kMaxWaves = 8;  // 512 threads: room for two blocks of K/V in registers
// Softmax in base 2: scores times scale log2(e), exponentials on v_exp_f32 (2^x), so
// every running maximum and partial's maximum (and the merges) are base 2.
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMaxG = 16;

struct RowsParams {
    const float *q;
    const uint16_t *k, *v;
    float *out;
    const uint32_t *slots, *positions, *table;
    float *partials;     // [rows][kv_heads][parts][G][2 + 128] when split across groups
    uint32_t rows, keys, heads, kv_heads, G, back, kept_pages, page_shift;
    uint32_t wave_keys;  // keys per wave per partition (multiple of 16)
    float scale;
    // The fused decode step: raw q/k/v product rows, per-head gains, RoPE.
    const float *qkv;
    const float *q_gain, *k_gain;
    const float *rope;  // [positions][64] (cos, sin) pairs
    float eps;
    uint64_t *marks;    // TS_MARK ledger (debug builds)
    uint32_t max_position;
    uint32_t *status;   // TS_STATUS_* bits, or NULL
};

TS_DEV uint64_t kept_row(const RowsParams &p, uint32_t slot, uint32_t pos) {
    if (!p.table) return (uint64_t)slot * p.keys + pos;
    const uint64_t entry = (uint64_t)slot * p.kept_pages + (pos >> p.page_shift);
    return ((uint64_t)p.table[entry] << p.page_shift) | (pos & ((1u << p.page_shift) - 1));
}

// A row the slot cannot hold (the interpreter refuses a read at >= keys,
// engine/ir/interp/src/cpu.rs:323-327), past the stated bound that sized the split,
// or past the slot's table row.
TS_DEV bool refused(const RowsParams &p, uint32_t pos) {
    return pos >= p.keys || pos > p.max_position || (p.table && (pos >> p.page_shift) >= p.kept_pages);
}

// A refused row loads nothing: its output is NaN (directly, or as an empty partial
// that the merge turns into 0 / 0), and the refusal is reported in *status.
TS_DEV void refuse_row(const RowsParams &p, uint32_t r, uint32_t kvh, uint32_t part, uint32_t parts, uint32_t G) {
    if (threadIdx.x == 0 && p.status) atomicOr(p.status, TS_STATUS_POSITION);
    const size_t gi = (size_t)r * p.kv_heads + kvh;
    for (uint32_t e = threadIdx.x; e < G * 130; e += blockDim.x) {
        if (parts == 1) {
            if (e < G * 128) p.out[((size_t)r * p.heads + kvh * G + e / 128) * 128 + e % 128] = __builtin_nanf("");
        } else {
            p.partials[(gi * parts + part) * G * 130 + e] = (e % 130 == 0) ? -INFINITY : 0.0f;
        }
    }
}

// RmsNorm over one 128-wide head held as (d, d+64) in lane d of a wave, then
// the Halves rotation of that pair by the tabled angle (engine/ir/interp/src/
// cpu.rs:36-47, 371-377; the table is the reference's `angles` stage,
// engine/rules/kernels/src/rope.rs:10-58).
TS_DEV void norm_rope(float &a, float &b, float ga, float gb, float cs, float sn, float eps) {
    const float s = wave_sum(a * a + b * b);
    const float inv = 1.0f / sqrtf(s / 128.0f + eps);
    a = a * (inv * ga);
    b = b * (inv * gb);
    const float ra = a * cs - b * sn, rb = a * sn + b * cs;
    a = ra;
    b = rb;
}

template <int G, bool STEP, int NB>
__global__ __launch_bounds__(kMaxWaves * 64) void attend_rows_kernel(RowsParams p) {
    constexpr int kWaves = (64 / G) < kMaxWaves ? (64 / G) : kMaxWaves;  // LDS bound: waves x G <= 64
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    const uint32_t part = blockIdx.x, kvh = blockIdx.y, r = blockIdx.z, parts = gridDim.x;
    const uint32_t col = lane & 15, grp = lane >> 4;

    __shared__ __attribute__((aligned(16))) float sp[kWaves][G][16];  // p[head][key] of the current block
    __shared__ float sm[kWaves][G], sl[kWaves][G];
    __shared__ __attribute__((aligned(16))) float so[kWaves][G][128];
    __shared__ __attribute__((aligned(16))) float sq[STEP ? G : 1][128];          // fused step: q heads
    __shared__ __attribute__((aligned(16))) uint16_t snew[STEP ? 2 : 1][128];     // fused step: new k, v

    TS_MARK(p.marks, 0);
    const uint32_t pos = p.positions[r], slot = p.slots[r];
    if (refused(p, pos)) {  // uniform: one row per group
        refuse_row(p, r, kvh, part, parts, G);
        return;
    }
    const uint32_t from = pos > p.back ? pos - p.back : 0;
    const uint32_t wk0 = (part * waves + wave) * (16 * NB);
    const uint32_t pmask = (1u << p.page_shift) - 1;

    // Loads are issued in the order their values are needed, because the memory
    // counter retires them in order: page-table entries, then the fused step's
    // inputs, then this wave's K/V blocks. Every load is unconditional (addresses
    // clamped to rows that exist, results masked later) so the compiler can wait
    // for exactly the loads a value needs instead of all of them.
    bool live[NB];
    uint32_t kbc[NB], page_of[NB];
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
        const uint32_t kb = wk0 + 16 * nb;
        live[nb] = kb <= pos && kb + 16 > from;  // uniform across the wave
        kbc[nb] = min(kb, pos) & ~15u;           // a 16-aligned block whose page exists
        page_of[nb] = p.table ? p.table[(uint64_t)slot * p.kept_pages + (kbc[nb] >> p.page_shift)] : 0u;
    }
    // Fused step inputs: wave w < G + 2 takes item w (q heads, new k, new v); the
    // host launches at least G + 2 waves whenever the LDS budget allows.
    constexpr bool kOneItem = G + 2 <= kWaves;
    const uint32_t item = min(wave, (uint32_t)G + 1);
    const size_t qkv_base = (size_t)r * (p.heads + 2 * p.kv_heads) * 128;
    float ra = 0.0f, rb = 0.0f, qga = 0.0f, qgb = 0.0f, kga = 0.0f, kgb = 0.0f;
    float2 cs = make_float2(1.0f, 0.0f);
    if (STEP) {
        const uint32_t rowh = item < (uint32_t)G ? kvh * G + item
                                                 : (item == (uint32_t)G ? p.heads + kvh : p.heads + p.kv_heads + kvh);
        const float *src = p.qkv + qkv_base + (size_t)rowh * 128;
        ra = src[lane];
        rb = src[lane + 64];
        cs = ((const float2 *)p.rope)[(size_t)pos * 64 + lane];
        qga = p.q_gain[lane];
        qgb = p.q_gain[lane + 64];
        kga = p.k_gain[lane];
        kgb = p.k_gain[lane + 64];
    }
    u32x4 kk[NB][4];
    u32x4 vq[NB][4];  // V: load j holds key 4j + lane/16 of the block, dims 8*(lane%16)..+8
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
        // 16 rows of one page (pages hold >= 16 rows); dense rows clamp at the
        // slot's capacity. Rows outside [from, pos] are masked where they are used.
        const uint64_t row0 = p.table ? (((uint64_t)page_of[nb] << p.page_shift) | (kbc[nb] & pmask))
                                      : (uint64_t)slot * p.keys + kbc[nb];
        const uint32_t room = p.table ? 15u : p.keys - 1 - min(kbc[nb], p.keys - 1);
        const uint16_t *kr = p.k + ((row0 + min(col, room)) * p.kv_heads + kvh) * 128 + 32 * grp;
#pragma unroll
        for (int j = 0; j < 4; j++) kk[nb][j] = *((const u32x4 *)kr + j);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t i = 4 * j + grp;
            vq[nb][j] = *(const u32x4 *)(p.v + ((row0 + min(i, room)) * p.kv_heads + kvh) * 128 + 8 * col);
        }
    }

    if (STEP) {
        for (uint32_t it = item; it < (uint32_t)G + 2; it += waves) {
            if (!kOneItem && it != item) {  // fewer waves than items: later items load here
                const uint32_t rowh = it < (uint32_t)G ? kvh * G + it
                                                       : (it == (uint32_t)G ? p.heads + kvh : p.heads + p.kv_heads + kvh);
                const float *src = p.qkv + qkv_base + (size_t)rowh * 128;
                ra = src[lane];
                rb = src[lane + 64];
            }
            if (it == item && wave > (uint32_t)G + 1) break;  // spare wave: no item of its own
            float a = ra, b = rb;
            if (it < (uint32_t)G) {
                norm_rope(a, b, qga, qgb, cs.x, cs.y, p.eps);
                sq[it][lane] = a;
                sq[it][lane + 64] = b;
            } else if (it == (uint32_t)G) {
                norm_rope(a, b, kga, kgb, cs.x, cs.y, p.eps);
                snew[0][lane] = bf16_bits(a);
                snew[0][lane + 64] = bf16_bits(b);
            } else {
                snew[1][lane] = bf16_bits(a);
                snew[1][lane + 64] = bf16_bits(b);
            }
            if (kOneItem) break;
        }
        __syncthreads();
        TS_MARK(p.marks, 1);
    }

    // q operand: row (head) col of the group, d-group grp; two bf16 parts.
    // Read as 16-byte vectors from a row that exists, then zeroed past G.
    u32x4 qh[4], ql[4];
    {
        const bool ok = col < G;
        const uint32_t qrow = ok ? col : 0;
        const float4 *qr = STEP ? (const float4 *)&sq[qrow][32 * grp]
                                : (const float4 *)(p.q + ((size_t)r * p.heads + kvh * G + qrow) * 128 + 32 * grp);
        float4 qv[8];
#pragma unroll
        for (int i = 0; i < 8; i++) qv[i] = qr[i];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float f[8] = {qv[2 * j].x, qv[2 * j].y, qv[2 * j].z, qv[2 * j].w,
                                qv[2 * j + 1].x, qv[2 * j + 1].y, qv[2 * j + 1].z, qv[2 * j + 1].w};
            uint32_t h[4], l[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float a = ok ? f[2 * e] : 0.0f, b = ok ? f[2 * e + 1] : 0.0f;
                const float ha = bf16_round(a), hb = bf16_round(b);
                h[e] = pack_bf16x2(ha, hb);
                l[e] = pack_bf16x2(a - ha, b - hb);
            }
            qh[j] = u32x4{h[0], h[1], h[2], h[3]};
            ql[j] = u32x4{l[0], l[1], l[2], l[3]};
        }
    }

#ifdef TS_MARKS
    __builtin_amdgcn_s_waitcnt(0xc070);  // debug marks only: wait for every load, then stamp
    TS_MARK(p.marks, 8);
#endif
    // Online softmax state: this lane's 4 head rows (4*grp + i) in the S layout.
    float m[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; i++) { m[i] = -INFINITY; l[i] = 0.0f; }
    // Accumulator: heads h < G; lane holds dims 8*(lane%16)..+8 summed over the
    // keys with index = lane/16 (mod 4); the four lane groups add up at the end.
    float o[G][8];
#pragma unroll
    for (int h = 0; h < G; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) o[h][e] = 0.0f;

#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
        if (!live[nb]) continue;  // uniform across the wave
        const uint32_t kb = wk0 + 16 * nb;
        const uint32_t key = kb + col;
        if (STEP && key == pos) {
#pragma unroll
            for (int j = 0; j < 4; j++) kk[nb][j] = *((const u32x4 *)&snew[0][32 * grp] + j);
        }
        f32x4 s = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            s = mfma16(as_bf16x8(qh[j]), as_bf16x8(kk[nb][j]), s);
            s = mfma16(as_bf16x8(ql[j]), as_bf16x8(kk[nb][j]), s);
        }
        const bool valid = key >= from && key <= pos;
        float alpha[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float si = valid ? s[i] * (p.scale * kLog2e) : -INFINITY;  // base 2
            const float mn = fmaxf(m[i], row16_max(si));
            alpha[i] = (mn == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m[i] - mn);
            const float pi = (mn == -INFINITY || !valid) ? 0.0f : __builtin_amdgcn_exp2f(si - mn);
            l[i] = l[i] * alpha[i] + row16_sum(pi);
            m[i] = mn;
            const uint32_t h = 4 * grp + i;
            if (h < G) sp[wave][h][col] = pi;
        }
        // The wave reads back its own LDS writes: in order within a wave, no barrier.
        __builtin_amdgcn_wave_barrier();
        // alpha of head h lives in lanes of row-group h/4 (any column): broadcast it.
#pragma unroll
        for (int h = 0; h < G; h++) {
            const float a = __shfl(alpha[h & 3], (h >> 2) * 16, 64);
#pragma unroll
            for (int e = 0; e < 8; e++) o[h][e] *= a;
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t i = 4 * j + grp, kpos = kb + i;
            u32x4 v = vq[nb][j];
            if (STEP && kpos == pos) v = *(const u32x4 *)&snew[1][8 * col];
            const bool ok = kpos >= from && kpos <= pos;  // p is zero outside; keep v finite too
            const uint32_t w4[4] = {ok ? v.x : 0u, ok ? v.y : 0u, ok ? v.z : 0u, ok ? v.w : 0u};
#pragma unroll
            for (int h = 0; h < G; h++) {
                const float pk = sp[wave][h][i];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    o[h][2 * e] += pk * lo_bf16(w4[e]);
                    o[h][2 * e + 1] += pk * hi_bf16(w4[e]);
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
        TS_MARK(p.marks, 2 + nb);
    }

    // Merge the waves of this group.
    if (col == 0) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t h = 4 * grp + i;
            if (h < G) { sm[wave][h] = m[i]; sl[wave][h] = l[i]; }
        }
    }
#pragma unroll
    for (int h = 0; h < G; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float v = o[h][e];
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            o[h][e] = v;
        }
    if (grp == 0) {
#pragma unroll
        for (int h = 0; h < G; h++) {
            *(float4 *)&so[wave][h][8 * col] = make_float4(o[h][0], o[h][1], o[h][2], o[h][3]);
            *(float4 *)&so[wave][h][8 * col + 4] = make_float4(o[h][4], o[h][5], o[h][6], o[h][7]);
        }
    }
    __syncthreads();
    TS_MARK(p.marks, 10);

    const uint32_t t = threadIdx.x;
    const size_t gi = (size_t)r * p.kv_heads + kvh;
    float *mine = p.partials ? p.partials + (gi * parts + part) * G * 130 : nullptr;
    for (uint32_t e = t; e < G * 128; e += blockDim.x) {
        const uint32_t h = e / 128, d = e % 128;
        float M = -INFINITY;
        for (uint32_t w = 0; w < waves; w++) M = fmaxf(M, sm[w][h]);
        float L = 0.0f, O = 0.0f;
        for (uint32_t w = 0; w < waves; w++) {
            const float f = (sm[w][h] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(sm[w][h] - M);
            L += sl[w][h] * f;
            O += so[w][h][d] * f;
        }
        if (parts == 1) {
            p.out[((size_t)r * p.heads + kvh * G + h) * 128 + d] = O / L;
        } else {
            mine[h * 130 + 2 + d] = O;
            if (d == 0) { mine[h * 130] = M; mine[h * 130 + 1] = L; }
        }
    }
    if (STEP && part == 0) {
        // The new row joins the kept rows (Store::append, engine/ir/interp/src/
        // run.rs:122-198). Stored last: a store the compiler cannot prove apart from
        // the K/V loads would otherwise wait for all of them.
        const uint64_t row = kept_row(p, slot, pos);
        for (uint32_t i = threadIdx.x; i < 128; i += blockDim.x) {
            const uint32_t which = i >> 6;
            uint16_t *dst = (uint16_t *)(which == 0 ? p.k : p.v) + (row * p.kv_heads + kvh) * 128;
            ((uint32_t *)dst)[i & 63] = ((const uint32_t *)snew[which])[i & 63];
        }
    }
    TS_MARK(p.marks, 11);
}

// Long contexts (no fused step): each wave streams L iterations of 32 keys (two
// 16-key blocks), loading iteration it + 1 while it computes iteration it; the
// group's page-table entries are copied to LDS once; a group whose keys all lie
// outside the row's range writes an empty partial and leaves without loading.
// Same per-block math and partial layout as attend_rows_kernel.
// Two waves a group and about sixteen groups a (row, kv head) at the C3 decode shape:
// 121-123 us against 130-131 with 8 waves and four groups, the same keys a wave
// (smaller groups spread the ragged rows' work over the CUs more evenly; 1 wave and
// 32 groups 127, 4 waves and 8 groups 124-126).
constexpr int kLongWaves = 2;
constexpr uint32_t kLongPages = 1024;  // page-table entries a group keeps in LDS

template <int G>
struct LongBuf {
    u32x4 kk[2][4], vq[2][4];
};

template <int G>
__global__ __launch_bounds__(kLongWaves * 64) void attend_long_kernel(RowsParams p, uint32_t iters) {
    static_assert(G * kLongWaves <= 64, "LDS budget: waves x G <= 64");
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t part = blockIdx.x, kvh = blockIdx.y, r = blockIdx.z, parts = gridDim.x;
    const uint32_t col = lane & 15, grp = lane >> 4;

    __shared__ __attribute__((aligned(16))) float sp[kLongWaves][G][32];  // p[head][key] of the current pair
    __shared__ float sm[kLongWaves][G], sl[kLongWaves][G];
    __shared__ __attribute__((aligned(16))) float so[kLongWaves][G][128];
    __shared__ uint32_t stab[kLongPages];

    const uint32_t pos = p.positions[r], slot = p.slots[r];
    if (refused(p, pos)) {  // uniform: one row per group
        refuse_row(p, r, kvh, part, parts, G);
        return;
    }
    const uint32_t from = pos > p.back ? pos - p.back : 0;
    const uint32_t span_keys = kLongWaves * 32 * iters;  // keys of one group
    const uint32_t g0 = part * span_keys, g1 = g0 + span_keys;
    const size_t gi = (size_t)r * p.kv_heads + kvh;
    float *mine = p.partials + (gi * parts + part) * G * 130;
    if (g0 > pos || g1 <= from) {  // nothing in range: an empty partial for the merge
        for (uint32_t e = threadIdx.x; e < G * 130; e += blockDim.x) mine[e] = (e % 130 == 0) ? -INFINITY : 0.0f;
        return;
    }
    const uint32_t pmask = (1u << p.page_shift) - 1;
    const uint32_t p0 = g0 >> p.page_shift;
    if (p.table) {
        const uint32_t np = min((min(g1, pos + 1) - 1) >> p.page_shift, p.kept_pages - 1) - p0 + 1;
        for (uint32_t i = threadIdx.x; i < np; i += blockDim.x)
            stab[i] = p.table[(uint64_t)slot * p.kept_pages + p0 + i];
        __syncthreads();
    }
    const uint32_t w0 = g0 + wave * 32 * iters;  // this wave's first key

    // Block at kb (clamped into [0, pos] so its page exists): K 4 x 16B per lane (key
    // col, d 32 grp..+32), V 4 x 16B (key 4j + grp, d 8 col..+8).
    auto load = [&](uint32_t kb, u32x4 (&kk)[4], u32x4 (&vq)[4]) {
        const uint32_t kbc = min(kb, pos) & ~15u;
        const uint64_t row0 = p.table ? (((uint64_t)stab[(kbc >> p.page_shift) - p0] << p.page_shift) | (kbc & pmask))
                                      : (uint64_t)slot * p.keys + kbc;
        const uint32_t room = p.table ? 15u : p.keys - 1 - min(kbc, p.keys - 1);
        const uint16_t *kr = p.k + ((row0 + min(col, room)) * p.kv_heads + kvh) * 128 + 32 * grp;
#pragma unroll
        for (int j = 0; j < 4; j++) kk[j] = *((const u32x4 *)kr + j);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t i = 4 * j + grp;
            vq[j] = *(const u32x4 *)(p.v + ((row0 + min(i, room)) * p.kv_heads + kvh) * 128 + 8 * col);
        }
    };
    LongBuf<G> buf[2];
    load(w0, buf[0].kk[0], buf[0].vq[0]);
    load(w0 + 16, buf[0].kk[1], buf[0].vq[1]);

    // q operand: row (head) col of the group, d-group grp; two bf16 parts.
    u32x4 qh[4], ql[4];
    {
        const bool ok = col < G;
        const float4 *qr = (const float4 *)(p.q + ((size_t)r * p.heads + kvh * G + (ok ? col : 0)) * 128 + 32 * grp);
        float4 qv[8];
#pragma unroll
        for (int i = 0; i < 8; i++) qv[i] = qr[i];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float f[8] = {qv[2 * j].x, qv[2 * j].y, qv[2 * j].z, qv[2 * j].w,
                                qv[2 * j + 1].x, qv[2 * j + 1].y, qv[2 * j + 1].z, qv[2 * j + 1].w};
            uint32_t h[4], l[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float a = ok ? f[2 * e] : 0.0f, b = ok ? f[2 * e + 1] : 0.0f;
                const float ha = bf16_round(a), hb = bf16_round(b);
                h[e] = pack_bf16x2(ha, hb);
                l[e] = pack_bf16x2(a - ha, b - hb);
            }
            qh[j] = u32x4{h[0], h[1], h[2], h[3]};
            ql[j] = u32x4{l[0], l[1], l[2], l[3]};
        }
    }

    float m[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; i++) { m[i] = -INFINITY; l[i] = 0.0f; }
    float o[G][8];
#pragma unroll
    for (int h = 0; h < G; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) o[h][e] = 0.0f;

    // Two 16-key blocks (32 keys from kb): scores on the matrix unit, one online
    // softmax update over both (one max and one sum reduction, one rescale of o),
    // P*V on the VALU.
    auto pair = [&](uint32_t kb, const LongBuf<G> &b) {
        if (kb > pos || kb + 32 <= from) return;  // uniform across the wave
        f32x4 sc[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            sc[t] = f32x4{0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                sc[t] = mfma16(as_bf16x8(qh[j]), as_bf16x8(b.kk[t][j]), sc[t]);
                sc[t] = mfma16(as_bf16x8(ql[j]), as_bf16x8(b.kk[t][j]), sc[t]);
            }
        }
        const uint32_t key0 = kb + col, key1 = kb + 16 + col;
        const bool valid0 = key0 >= from && key0 <= pos, valid1 = key1 >= from && key1 <= pos;
        float alpha[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float s0 = valid0 ? sc[0][i] * (p.scale * kLog2e) : -INFINITY;  // base 2
            const float s1 = valid1 ? sc[1][i] * (p.scale * kLog2e) : -INFINITY;
            const float mn = fmaxf(m[i], row16_max(fmaxf(s0, s1)));
            const bool none = mn == -INFINITY;
            alpha[i] = none ? 1.0f : __builtin_amdgcn_exp2f(m[i] - mn);
            const float p0 = (none || !valid0) ? 0.0f : __builtin_amdgcn_exp2f(s0 - mn);
            const float p1 = (none || !valid1) ? 0.0f : __builtin_amdgcn_exp2f(s1 - mn);
            l[i] = l[i] * alpha[i] + row16_sum(p0 + p1);
            m[i] = mn;
            const uint32_t h = 4 * grp + i;
            if (h < G) { sp[wave][h][col] = p0; sp[wave][h][16 + col] = p1; }
        }
        __builtin_amdgcn_wave_barrier();  // the wave reads back its own LDS writes
#pragma unroll
        for (int h = 0; h < G; h++) {
            const float a = __shfl(alpha[h & 3], (h >> 2) * 16, 64);
#pragma unroll
            for (int e = 0; e < 8; e++) o[h][e] *= a;
        }
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t i = 4 * j + grp, kpos = kb + 16 * t + i;
                const bool ok = kpos >= from && kpos <= pos;  // p is zero outside; keep v finite too
                const u32x4 v = b.vq[t][j];
                const uint32_t w4[4] = {ok ? v.x : 0u, ok ? v.y : 0u, ok ? v.z : 0u, ok ? v.w : 0u};
#pragma unroll
                for (int h = 0; h < G; h++) {
                    const float pk = sp[wave][h][16 * t + i];
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        o[h][2 * e] += pk * lo_bf16(w4[e]);
                        o[h][2 * e + 1] += pk * hi_bf16(w4[e]);
                    }
                }
            }
        __builtin_amdgcn_wave_barrier();
    };

    // Iterations in pairs so each buffer stays in registers: load it + 1 into the
    // other buffer, then compute it.
    for (uint32_t it = 0; it < iters; it += 2) {
        const uint32_t kb0 = w0 + 32 * it;
        if (it + 1 < iters) {
            load(kb0 + 32, buf[1].kk[0], buf[1].vq[0]);
            load(kb0 + 48, buf[1].kk[1], buf[1].vq[1]);
        }
        pair(kb0, buf[0]);
        if (it + 1 >= iters) break;
        if (it + 2 < iters) {
            load(kb0 + 64, buf[0].kk[0], buf[0].vq[0]);
            load(kb0 + 80, buf[0].kk[1], buf[0].vq[1]);
        }
        pair(kb0 + 32, buf[1]);
    }

    // Merge the waves of this group into its partial.
    if (col == 0) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t h = 4 * grp + i;
            if (h < G) { sm[wave][h] = m[i]; sl[wave][h] = l[i]; }
        }
    }
#pragma unroll
    for (int h = 0; h < G; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float v = o[h][e];
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            o[h][e] = v;
        }
    if (grp == 0) {
#pragma unroll
        for (int h = 0; h < G; h++) {
            *(float4 *)&so[wave][h][8 * col] = make_float4(o[h][0], o[h][1], o[h][2], o[h][3]);
            *(float4 *)&so[wave][h][8 * col + 4] = make_float4(o[h][4], o[h][5], o[h][6], o[h][7]);
        }
    }
    __syncthreads();
    for (uint32_t e = threadIdx.x; e < G * 128; e += blockDim.x) {
        const uint32_t h = e / 128, d = e % 128;
        float M = -INFINITY;
        for (uint32_t w = 0; w < kLongWaves; w++) M = fmaxf(M, sm[w][h]);
        float L = 0.0f, O = 0.0f;
        for (uint32_t w = 0; w < kLongWaves; w++) {
            const float f = (sm[w][h] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(sm[w][h] - M);
            L += sl[w][h] * f;
            O += so[w][h][d] * f;
        }
        mine[h * 130 + 2 + d] = O;
        if (d == 0) { mine[h * 130] = M; mine[h * 130 + 1] = L; }
    }
}

// Merges the partitions of one (row, kv head) in partition order.
template <int G>
__global__ __launch_bounds__(256) void attend_rows_merge(RowsParams p, uint32_t parts) {
    const uint32_t kvh = blockIdx.x, r = blockIdx.y;
    const size_t gi = (size_t)r * p.kv_heads + kvh;
    const float *all = p.partials + gi * parts * G * 130;
    for (uint32_t e = threadIdx.x; e < G * 128; e += blockDim.x) {
        const uint32_t h = e / 128, d = e % 128;
        // Up to 16 partitions: every (m, l, o) loaded at once, one round trip (the same
        // max and the same sums in partition order as the batched loop below).
        constexpr uint32_t kOne = 16;
        if (parts <= kOne) {
            float mq[kOne], lq[kOne], oq[kOne];
#pragma unroll
            for (uint32_t j = 0; j < kOne; j++) {
                const float *pq = all + (min(j, parts - 1) * G + h) * 130;  // clamped: read, not used
                mq[j] = pq[0];
                lq[j] = pq[1];
                oq[j] = pq[2 + d];
            }
            float M = -INFINITY;
#pragma unroll
            for (uint32_t j = 0; j < kOne; j++)
                if (j < parts) M = fmaxf(M, mq[j]);
            float L = 0.0f, O = 0.0f;
#pragma unroll
            for (uint32_t j = 0; j < kOne; j++)
                if (j < parts) {
                    const float f = (mq[j] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mq[j] - M);
                    L += lq[j] * f;
                    O += oq[j] * f;
                }
            p.out[((size_t)r * p.heads + kvh * G + h) * 128 + d] = O / L;
            continue;
        }
        // Partitions in batches of 8 with every load of a batch issued before use
        // (clamped indices are read, not used); sums stay in partition order.
        constexpr uint32_t kB = 8;
        float M = -INFINITY;
        for (uint32_t q0 = 0; q0 < parts; q0 += kB) {
            float mq[kB];
#pragma unroll
            for (uint32_t j = 0; j < kB; j++) mq[j] = all[(min(q0 + j, parts - 1) * G + h) * 130];
#pragma unroll
            for (uint32_t j = 0; j < kB; j++)
                if (q0 + j < parts) M = fmaxf(M, mq[j]);
        }
        float L = 0.0f, O = 0.0f;
        for (uint32_t q0 = 0; q0 < parts; q0 += kB) {
            float mq[kB], lq[kB], oq[kB];
#pragma unroll
            for (uint32_t j = 0; j < kB; j++) {
                const float *pq = all + (min(q0 + j, parts - 1) * G + h) * 130;
                mq[j] = pq[0];
                lq[j] = pq[1];
                oq[j] = pq[2 + d];
            }
#pragma unroll
            for (uint32_t j = 0; j < kB; j++)
                if (q0 + j < parts) {
                    const float f = (mq[j] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mq[j] - M);
                    L += lq[j] * f;
                    O += oq[j] * f;
                }
        }
        p.out[((size_t)r * p.heads + kvh * G + h) * 128 + d] = O / L;
    }
}

struct Split {
    uint32_t wave_keys, parts, waves;  // wave_keys: 16 or 32 (one or two blocks per wave)
    uint32_t iters;                    // > 0: the long-context kernel, iters x 32 keys per wave
};

// Spans beyond this go to attend_long_kernel (without the fused step, G <= 4).
constexpr uint32_t kLongSpan = 2048;

Split split(const ts_rows_args *a, bool step) {
    const uint32_t G = a->heads / a->kv_heads;
    const uint32_t max_waves = (64 / G) < (uint32_t)kMaxWaves ? 64 / G : kMaxWaves;
    const uint32_t span = a->max_position + 1;
    Split s;
    // One block per wave while a group covers the span, else two.
    s.wave_keys = span <= max_waves * 16 ? 16 : 32;
    s.parts = (span + max_waves * s.wave_keys - 1) / (max_waves * s.wave_keys);
    s.waves = s.parts == 1 ? (span + s.wave_keys - 1) / s.wave_keys : max_waves;
    // The fused step gives each of its G + 2 rows (q heads, new k, new v) a wave.
    if (step && s.waves < G + 2) s.waves = (G + 2) < max_waves ? G + 2 : max_waves;
    s.iters = 0;
    if (!step && span > kLongSpan && G <= 4) {
        // Long contexts: each wave streams iters x 32 keys (iters ~ span / 1024), a
        // group kLongWaves waves of them: ~16 groups per (row, kv head).
        s.iters = std::max(1u, std::min(32u, span / (16 * kLongWaves * 32)));
        s.wave_keys = 32;
        s.waves = kLongWaves;
        s.parts = (span + kLongWaves * 32 * s.iters - 1) / (kLongWaves * 32 * s.iters);
    }
    return s;
}

int check(const ts_rows_args *a) {
    TS_REQUIRE(a && a->q && a->k && a->v && a->out && a->slots && a->positions, "attend_rows: null pointer");
    TS_REQUIRE(a->width == 128, "attend_rows: head width %u (128 supported)", a->width);
    TS_REQUIRE(a->kv_heads >= 1 && a->heads % a->kv_heads == 0, "attend_rows: %u heads over %u kv heads",
               a->heads, a->kv_heads);
    TS_REQUIRE(a->heads / a->kv_heads <= kMaxG, "attend_rows: %u query heads per kv head (at most %d)",
               a->heads / a->kv_heads, kMaxG);
    TS_REQUIRE(a->q_dtype == TS_F32 && a->kv_dtype == TS_BF16 && a->out_dtype == TS_F32,
               "attend_rows: q f32, kept rows bf16, out f32 supported");
    TS_REQUIRE(!a->kept_table || (a->page >= 16 && (a->page & (a->page - 1)) == 0),
               "attend_rows: page %u must be a power of two >= 16", a->page);
    TS_REQUIRE(a->keys >= 1, "attend_rows: keys (the positions a slot holds) must be >= 1");
    TS_REQUIRE(ts::aligned(a->k, 16) && ts::aligned(a->v, 16) && ts::aligned(a->q, 16),
               "attend_rows: q, k, v must be 16-byte aligned");
    TS_REQUIRE(a->kv_heads <= 65535 && a->rows <= 65535, "attend_rows: grid limits");
    return TS_OK;
}

// Bytes of split-KV partials a launch with split s writes: [rows][kv_heads][parts][G][130].
size_t partials_bytes(const ts_rows_args *a, const Split &s) {
    if (s.parts <= 1) return 0;
    const size_t G = a->heads / a->kv_heads;
    const size_t groups = (size_t)a->rows * a->kv_heads;
    return groups * s.parts * G * 130 * sizeof(float);
}

}  // namespace

// One size serves both entry points (tessera_hip_attend_rows and the fused
// tessera_hip_attend_step split the same span differently past 2048 keys): the
// larger of the two.
extern "C" size_t tessera_hip_attend_rows_workspace(const ts_rows_args *a) {
    if (!a || a->kv_heads == 0 || a->heads % a->kv_heads) return 0;
    return std::max(partials_bytes(a, split(a, false)), partials_bytes(a, split(a, true)));
}

namespace {

template <int G, bool STEP>
void (*pick_nb(uint32_t wave_keys))(RowsParams) {
    return wave_keys == 16 ? attend_rows_kernel<G, STEP, 1> : attend_rows_kernel<G, STEP, 2>;
}

template <bool STEP>
int launch_rows(const ts_rows_args *a, RowsParams &p, void *stream) {
    Split s = split(a, STEP);
    p.q = (const float *)a->q; p.k = (const uint16_t *)a->k; p.v = (const uint16_t *)a->v;
    p.out = (float *)a->out; p.slots = a->slots; p.positions = a->positions; p.table = a->kept_table;
    p.rows = a->rows; p.keys = a->keys; p.heads = a->heads; p.kv_heads = a->kv_heads;
    p.G = a->heads / a->kv_heads; p.back = a->back; p.kept_pages = a->kept_pages;
    p.page_shift = a->kept_table ? (uint32_t)__builtin_ctz(a->page) : 0;
    p.wave_keys = s.wave_keys; p.scale = a->scale;
    p.max_position = a->max_position; p.status = a->status;
    p.partials = nullptr;
#ifdef TS_MARKS
    p.marks = ts_debug_marks();
#endif
    if (s.parts > 1) {
        const size_t need = partials_bytes(a, s);  // what this launch writes
        if (!a->workspace || a->workspace_bytes < need)
            return ts::fail(TS_ERR_WORKSPACE, "attend_rows: workspace of %zu bytes needed", need);
        p.partials = (float *)a->workspace;
    }
    void (*k)(RowsParams) = nullptr;
    void (*merge)(RowsParams, uint32_t) = nullptr;
    switch (p.G) {
    case 1: k = pick_nb<1, STEP>(s.wave_keys); merge = attend_rows_merge<1>; break;
    case 2: k = pick_nb<2, STEP>(s.wave_keys); merge = attend_rows_merge<2>; break;
    case 4: k = pick_nb<4, STEP>(s.wave_keys); merge = attend_rows_merge<4>; break;
    case 8: k = pick_nb<8, STEP>(s.wave_keys); merge = attend_rows_merge<8>; break;
    case 16: k = pick_nb<16, STEP>(s.wave_keys); merge = attend_rows_merge<16>; break;
    default: return ts::fail(TS_ERR_ARG, "attend_rows: %u query heads per kv head (1, 2, 4, 8 or 16)", p.G);
    }
    if (!STEP && s.iters) {
        void (*kl)(RowsParams, uint32_t) = nullptr;
        switch (p.G) {
        case 1: kl = attend_long_kernel<1>; break;
        case 2: kl = attend_long_kernel<2>; break;
        default: kl = attend_long_kernel<4>; break;
        }
        hipLaunchKernelGGL(kl, dim3(s.parts, a->kv_heads, a->rows), dim3(kLongWaves * 64), 0, (hipStream_t)stream, p,
                           s.iters);
    } else {
        hipLaunchKernelGGL(k, dim3(s.parts, a->kv_heads, a->rows), dim3(s.waves * 64), 0, (hipStream_t)stream, p);
    }
    TS_CHECK_LAUNCH("attend_rows launch");
    if (s.parts > 1) {
        hipLaunchKernelGGL(merge, dim3(a->kv_heads, a->rows), dim3(256), 0, (hipStream_t)stream, p, s.parts);
        TS_CHECK_LAUNCH("attend_rows merge launch");
    }
    return TS_OK;
}

}  // namespace

extern "C" int tessera_hip_attend_rows(const ts_rows_args *a, void *stream) {
    int rc = check(a);
    if (rc) return rc;
    if (a->rows == 0) return TS_OK;
    RowsParams p;
    memset(&p, 0, sizeof p);
    return launch_rows<false>(a, p, stream);
}

extern "C" int tessera_hip_attend_step(const ts_step_args *s, void *stream) {
    TS_REQUIRE(s, "attend_step: null args");
    const ts_rows_args *a = &s->rows;
    const float *qkv = s->qkv, *q_gain = s->q_gain, *k_gain = s->k_gain, *rope_table = s->rope_table;
    const uint32_t rope_rows = s->rope_rows;
    const float eps = s->eps;
    TS_REQUIRE(a && qkv && q_gain && k_gain && rope_table, "attend_step: null pointer");
    TS_REQUIRE(a->max_position < rope_rows, "attend_step: positions up to %u but the angle table has %u rows",
               a->max_position, rope_rows);
    ts_rows_args b = *a;
    b.q = qkv;  // q comes from the product rows; only checked for alignment
    int rc = check(&b);
    if (rc) return rc;
    if (a->rows == 0) return TS_OK;
    RowsParams p;
    memset(&p, 0, sizeof p);
    p.qkv = qkv; p.q_gain = q_gain; p.k_gain = k_gain; p.rope = rope_table; p.eps = eps;
    return launch_rows<true>(&b, p, stream);
}

// ---------------------------------------------------------------------------
// The entry point that allocates nothing: split-KV partials in a fixed device
// array instead of a caller's workspace.
// ---------------------------------------------------------------------------
namespace {

constexpr size_t kScratchBytes = size_t(16) << 20;  // partials of up to 16 MiB per launch
constexpr int kMaxDevices = 64;

// One copy per GPU the library runs on, held until the process ends. In host code
// this name is only a stand-in: its device address comes from hipGetSymbolAddress.
__device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex scratch_mu;
void *scratch_at[kMaxDevices] = {};

// The current device's address of `scratch`, looked up once per device with that
// device current.
int scratch_ptr(void **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return ts::hip_status(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return ts::fail(TS_ERR_ARG, "attend_rows_noalloc: device %d", dev);
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_at[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return ts::hip_status(e, "hipGetSymbolAddress(scratch)");
        scratch_at[dev] = p;
    }
    *out = scratch_at[dev];
    return TS_OK;
}

}  // namespace

extern "C" size_t tessera_hip_attend_rows_noalloc_limit(void) { return kScratchBytes; }

extern "C" int tessera_hip_attend_rows_noalloc(const ts_rows_args *a, void *stream) {
    int rc = check(a);
    if (rc) return rc;
    if (a->rows == 0) return TS_OK;
    const size_t need = partials_bytes(a, split(a, false));
    if (need > kScratchBytes)
        return ts::fail(TS_ERR_WORKSPACE,
                        "attend_rows_noalloc: %zu bytes of partials needed, the fixed scratch holds %zu "
                        "(fewer rows or a shorter max_position; or tessera_hip_attend_rows with a workspace)",
                        need, kScratchBytes);
    void *ptr = nullptr;
    if ((rc = scratch_ptr(&ptr))) return rc;
    ts_rows_args b = *a;
    b.workspace = ptr;  // the partials are written in full before the merge reads them: no clearing
    b.workspace_bytes = kScratchBytes;
    RowsParams p;
    memset(&p, 0, sizeof p);
    return launch_rows<false>(&b, p, stream);
}
