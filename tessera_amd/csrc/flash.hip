// Ragged-row attention over kept (paged) K/V for many rows: the prefill kernel.
//
// Replaces the reference's flash / flash_rows rules (engine/rules/attention/
// src/flash.rs:156-503 score tiles + online softmax, :506-591 ragged rows over
// kept_row, :595-807 sizes and propose). The reference refuses them on gfx950
// (no matrix tile row for gfx9_5). Semantics: the interpreter's attend_rows
// (engine/ir/interp/src/cpu.rs:293-351): row (slot, pos) sees keys
// [max(0, pos - back), pos] of its slot, p = softmax(dot(q, k) * scale).
//
// gfx950 design:
//  * One 256-thread group per (64 query rows, head); each wave owns 16 rows.
//    The 64 rows must belong to one slot (the prefill shape: runs of one slot).
//  * Keys stream in 32-row blocks. K goes to LDS as rows ([key][d], 16-byte chunks
//    XOR-swizzled by key). V goes to LDS transposed ([d][key]) so the P*V operand is
//    one 16-byte read per lane: each lane octet loads an 8 keys x 8 d block,
//    transposes it across the octet with lane shuffles and writes 16 bytes per lane
//    (16-bit scattered writes bank-conflicted 16 ways and cost more than the MFMAs).
//  * The group's page-table entries are copied to LDS once.
//  * S = Q K^T: 2 key tiles x 4 d-steps of v_mfma_f32_16x16x32_bf16 per q part
//    (bf16 q as is; f32 q split into two exact bf16 parts). Online softmax per row
//    with 16-lane butterflies. P (bf16; two parts for f32 q) is staged through the
//    wave's own LDS into the A layout; O[16 rows, 128] += P V in 8 MFMA column tiles.
//  * The next key block's K/V loads are issued before the current block computes,
//    and the barriers wait for LDS only, so HBM latency hides under the MFMAs.
#include "common.h"

namespace {

constexpr int kRows = 64;   // query rows per group
constexpr int kKeys = 32;   // keys per block

struct FlashParams {
    const void *q;
    const uint16_t *k, *v;
    float *out;
    const uint32_t *slots, *positions, *table;
    uint32_t rows, keys, heads, kv_heads, back, kept_pages, page_shift;
    float scale;
};

TS_DEV uint64_t kept_row(const FlashParams &p, uint32_t slot, uint32_t pos) {
    if (!p.table) return (uint64_t)slot * p.keys + pos;
    const uint64_t entry = (uint64_t)slot * p.kept_pages + (pos >> p.page_shift);
    return ((uint64_t)p.table[entry] << p.page_shift) | (pos & ((1u << p.page_shift) - 1));
}

constexpr uint32_t kMaxPages = 1024;  // page-table entries a group keeps in LDS

// Row of the kept K/V for key position pos (stab: the group's LDS copy of its page
// table range from page p0, or NULL to read the table).
TS_DEV uint64_t key_row(const FlashParams &p, uint32_t slot, uint32_t pos, const uint32_t *stab, uint32_t p0) {
    return stab ? ((uint64_t)stab[(pos >> p.page_shift) - p0] << p.page_shift) | (pos & ((1u << p.page_shift) - 1))
                : kept_row(p, slot, pos);
}

// K and V of one 32-key block in flight, 16 bytes (8 d values) per load. K: thread t
// holds key idx / 16, chunk idx % 16 (idx = t + 256 c). V: wave w's load c covers keys
// 8 kg + (l & 7) and chunks 8 cg + (l >> 3), g = 2w + c, kg = g & 3, cg = g >> 2, so
// each lane octet holds an 8 keys x 8 d block for the transpose in stage_v. Keys past
// the last row's position may sit in pages never written: they load as zeros.
TS_DEV void fetch_kv(const FlashParams &p, uint32_t slot, uint32_t kvh, uint32_t kb, uint32_t hi, const uint32_t *stab,
                     uint32_t p0, u32x4 (&kr)[2], u32x4 (&vr)[2]) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int c2 = 0; c2 < 2; c2++) {
        const uint32_t idx = threadIdx.x + 256 * c2, key = idx >> 4, chunk = idx & 15, pos = kb + key;
        kr[c2] = u32x4{0, 0, 0, 0};
        if (pos <= hi && (p.table || pos < p.keys)) {
            const uint64_t row = key_row(p, slot, pos, stab, p0);
            kr[c2] = *(const u32x4 *)(p.k + (row * p.kv_heads + kvh) * 128 + chunk * 8);
        }
        const uint32_t g = 2 * wave + c2, vkey = 8 * (g & 3) + (lane & 7), vchunk = 8 * (g >> 2) + (lane >> 3);
        const uint32_t vpos = kb + vkey;
        vr[c2] = u32x4{0, 0, 0, 0};
        if (vpos <= hi && (p.table || vpos < p.keys)) {
            const uint64_t row = key_row(p, slot, vpos, stab, p0);
            vr[c2] = *(const u32x4 *)(p.v + (row * p.kv_heads + kvh) * 128 + vchunk * 8);
        }
    }
}

// 8 x 8 transpose of bf16 across the 8 lanes of an octet: lane j holds row j (8 values
// in 4 words) in, column j out. Three butterfly stages swap the off-diagonal blocks
// between lanes j and j ^ 4, j ^ 2, j ^ 1.
TS_DEV u32x4 transpose8(u32x4 v, uint32_t j) {
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
    {  // lanes ^ 4: words {2, 3} of the low lane <-> words {0, 1} of the high lane
        const bool up = j & 4;
        const uint32_t s0 = up ? w[0] : w[2], s1 = up ? w[1] : w[3];
        const uint32_t r0 = __shfl_xor(s0, 4), r1 = __shfl_xor(s1, 4);
        if (up) { w[0] = r0; w[1] = r1; } else { w[2] = r0; w[3] = r1; }
    }
    {  // lanes ^ 2: words {1, 3} of the low lane <-> words {0, 2} of the high lane
        const bool up = j & 2;
        const uint32_t s0 = up ? w[0] : w[1], s1 = up ? w[2] : w[3];
        const uint32_t r0 = __shfl_xor(s0, 2), r1 = __shfl_xor(s1, 2);
        if (up) { w[0] = r0; w[2] = r1; } else { w[1] = r0; w[3] = r1; }
    }
    {  // lanes ^ 1: the high halves of the low lane <-> the low halves of the high lane
        const bool up = j & 1;
        const uint32_t s0 = up ? (w[0] & 0xffffu) | (w[1] << 16) : (w[0] >> 16) | (w[1] & 0xffff0000u);
        const uint32_t s1 = up ? (w[2] & 0xffffu) | (w[3] << 16) : (w[2] >> 16) | (w[3] & 0xffff0000u);
        const uint32_t r0 = __shfl_xor(s0, 1), r1 = __shfl_xor(s1, 1);
        if (up) {
            w[0] = (w[0] & 0xffff0000u) | (r0 & 0xffffu);
            w[1] = (w[1] & 0xffff0000u) | (r0 >> 16);
            w[2] = (w[2] & 0xffff0000u) | (r1 & 0xffffu);
            w[3] = (w[3] & 0xffff0000u) | (r1 >> 16);
        } else {
            w[0] = (w[0] & 0xffffu) | (r0 << 16);
            w[1] = (w[1] & 0xffffu) | (r0 & 0xffff0000u);
            w[2] = (w[2] & 0xffffu) | (r1 << 16);
            w[3] = (w[3] & 0xffffu) | (r1 & 0xffff0000u);
        }
    }
    return u32x4{w[0], w[1], w[2], w[3]};
}

// Byte offset of (d, 8-key group kg) in V^T: rows of 32 keys (64 bytes), 16-byte
// groups XOR-swizzled by d / 4 so 16 consecutive d rows hit distinct banks.
TS_DEV uint32_t vt_at(uint32_t d, uint32_t kg) { return d * 64 + ((kg ^ ((d >> 2) & 3)) << 4); }

template <bool QF32>
__global__ __launch_bounds__(256) void flash_rows_kernel(FlashParams p) {
    __shared__ __attribute__((aligned(16))) uint16_t sk[kKeys][128];     // K rows, swizzled chunks
    __shared__ __attribute__((aligned(16))) char svt[128 * kKeys * 2];  // V transposed (vt_at)
    __shared__ __attribute__((aligned(16))) uint16_t sp[4][QF32 ? 2 : 1][16][kKeys];  // P parts per wave
    __shared__ uint32_t srange[2];
    __shared__ uint32_t stab_s[kMaxPages];  // this group's page-table entries

    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, t = threadIdx.x;
    const uint32_t col = lane & 15, grp = lane >> 4;
    const uint32_t h = blockIdx.y, G = p.heads / p.kv_heads, kvh = h / G;
    const uint32_t r0 = blockIdx.x * kRows;
    const uint32_t slot = p.slots[r0];

    // This wave's rows: r0 + 16*wave + i. Row i's position for masking.
    const uint32_t my_row = r0 + 16 * wave + col;  // A-operand row of this lane
    const bool row_ok = my_row < p.rows;

    // Key range of the whole group: [lo, hi].
    if (t == 0) { srange[0] = 0xffffffffu; srange[1] = 0; }
    __syncthreads();
    if (t < kRows && r0 + t < p.rows) {
        const uint32_t pos = p.positions[r0 + t];
        atomicMin(&srange[0], pos > p.back ? pos - p.back : 0);
        atomicMax(&srange[1], pos);
    }
    __syncthreads();
    const uint32_t lo = srange[0] & ~(kKeys - 1), hi = srange[1];
    // The page numbers of keys [lo, hi] into LDS once, so no key block waits on a
    // dependent table load.
    const uint32_t p0 = p.table ? lo >> p.page_shift : 0, np = p.table ? (hi >> p.page_shift) - p0 + 1 : 0;
    const uint32_t *stab = nullptr;
    if (p.table && np <= kMaxPages) {
        for (uint32_t i = t; i < np; i += 256) stab_s[i] = p.table[(uint64_t)slot * p.kept_pages + p0 + i];
        __syncthreads();
        stab = stab_s;
    }

    // q operand, loaded once: bf16 q as is; f32 q as two exact bf16 parts.
    u32x4 qh[4], ql[4];
    if (!QF32) {
        const uint16_t *qr = (const uint16_t *)p.q + ((size_t)(row_ok ? my_row : 0) * p.heads + h) * 128 + 32 * grp;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            qh[j] = row_ok ? *(const u32x4 *)(qr + 8 * j) : u32x4{0, 0, 0, 0};
            ql[j] = u32x4{0, 0, 0, 0};
        }
    } else {
        const float *qr = (const float *)p.q + ((size_t)(row_ok ? my_row : 0) * p.heads + h) * 128 + 32 * grp;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            uint32_t hh[4], ll[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float a = row_ok ? qr[8 * j + 2 * e] : 0.0f, b = row_ok ? qr[8 * j + 2 * e + 1] : 0.0f;
                float ha = bf16_round(a), hb = bf16_round(b);
                hh[e] = pack_bf16x2(ha, hb);
                ll[e] = pack_bf16x2(a - ha, b - hb);
            }
            qh[j] = u32x4{hh[0], hh[1], hh[2], hh[3]};
            ql[j] = u32x4{ll[0], ll[1], ll[2], ll[3]};
        }
    }
    // Positions of the 4 rows this lane holds in the S/D layout (rows 4*grp + i).
    uint32_t rpos[4], rfrom[4];
    bool rlive[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t r = r0 + 16 * wave + 4 * grp + i;
        rlive[i] = r < p.rows;
        rpos[i] = rlive[i] ? p.positions[r] : 0;
        rfrom[i] = rpos[i] > p.back ? rpos[i] - p.back : 0;
    }

    float m[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; i++) { m[i] = -INFINITY; l[i] = 0.0f; }
    f32x4 o[8];
#pragma unroll
    for (int d = 0; d < 8; d++) o[d] = f32x4{0, 0, 0, 0};

    u32x4 kr[2], vr[2];
    fetch_kv(p, slot, kvh, lo, hi, stab, p0, kr, vr);
    for (uint32_t kb = lo; kb <= hi; kb += kKeys) {
        // Every wave is done reading the previous block's K and V^T.
        lds_barrier();
#pragma unroll
        for (int c2 = 0; c2 < 2; c2++) {
            const uint32_t idx = t + 256 * c2, key = idx >> 4, chunk = idx & 15;
            *(u32x4 *)&sk[key][(chunk ^ (key & 15)) * 8] = kr[c2];
            // V: after the octet transpose lane j holds d = 8 vchunk + j for keys
            // 8 kg .. 8 kg + 7: one 16-byte write.
            const uint32_t g = 2 * wave + c2, vchunk = 8 * (g >> 2) + (lane >> 3);
            *(u32x4 *)(svt + vt_at(vchunk * 8 + (lane & 7), g & 3)) = transpose8(vr[c2], lane & 7);
        }
        // The next block's loads fly while this one computes (the barrier below
        // waits for LDS only).
        if (kb + kKeys <= hi) fetch_kv(p, slot, kvh, kb + kKeys, hi, stab, p0, kr, vr);
        lds_barrier();

        // S for two 16-key tiles.
        f32x4 s[2];
#pragma unroll
        for (int kt = 0; kt < 2; kt++) {
            s[kt] = f32x4{0, 0, 0, 0};
            const uint32_t key = kt * 16 + col;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t chunk = grp * 4 + j;  // d [32*grp + 8j, +8): q's order
                const bf16x8 kf = as_bf16x8(*(const u32x4 *)&sk[key][(chunk ^ (key & 15)) * 8]);
                s[kt] = mfma16(as_bf16x8(qh[j]), kf, s[kt]);
                if (QF32) s[kt] = mfma16(as_bf16x8(ql[j]), kf, s[kt]);
            }
        }
        // Online softmax per row; write P parts for the A layout.
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float sv[2];
            float mx = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
                const uint32_t kpos = kb + kt * 16 + col;
                const bool ok = rlive[i] && kpos <= rpos[i] && kpos >= rfrom[i];
                sv[kt] = ok ? s[kt][i] * p.scale : -INFINITY;
                mx = fmaxf(mx, sv[kt]);
            }
            mx = row16_max(mx);
            const float mn = fmaxf(m[i], mx);
            const float alpha = (mn == -INFINITY) ? 1.0f : expf(m[i] - mn);
            float sum = 0.0f;
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
                const float pv = (sv[kt] == -INFINITY) ? 0.0f : expf(sv[kt] - mn);
                sum += pv;
                const float ph = bf16_round(pv);
                sp[wave][0][4 * grp + i][kt * 16 + col] = bf16_bits(ph);
                if (QF32) sp[wave][QF32 ? 1 : 0][4 * grp + i][kt * 16 + col] = bf16_bits(pv - ph);
            }
            sum = row16_sum(sum);
            l[i] = l[i] * alpha + sum;
            m[i] = mn;
#pragma unroll
            for (int d = 0; d < 8; d++) o[d][i] *= alpha;
        }
        // P (rows x 32 keys) as the A operand: lane row col, keys 8*grp..+8. sp[wave]
        // is this wave's own: its LDS operations run in order, no barrier needed.
        const bf16x8 ph = as_bf16x8(*(const u32x4 *)&sp[wave][0][col][8 * grp]);
        const bf16x8 pl = as_bf16x8(*(const u32x4 *)&sp[wave][QF32 ? 1 : 0][col][8 * grp]);
#pragma unroll
        for (int d = 0; d < 8; d++) {
            const bf16x8 vf = as_bf16x8(*(const u32x4 *)(svt + vt_at(d * 16 + col, grp)));
            o[d] = mfma16(ph, vf, o[d]);
            if (QF32) o[d] = mfma16(pl, vf, o[d]);
        }
    }

    // O / l. D layout: column (d) col of tile d, rows 4*grp + i.
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (!rlive[i]) continue;
        const uint32_t r = r0 + 16 * wave + 4 * grp + i;
        float *dst = p.out + ((size_t)r * p.heads + h) * 128;
        const float inv = 1.0f / l[i];
#pragma unroll
        for (int d = 0; d < 8; d++) dst[d * 16 + col] = o[d][i] * inv;
    }
}

}  // namespace

extern "C" int tessera_hip_flash_rows(const ts_rows_args *a, void *stream) {
    TS_REQUIRE(a && a->q && a->k && a->v && a->out && a->slots && a->positions, "flash_rows: null pointer");
    TS_REQUIRE(a->width == 128, "flash_rows: head width %u (128 supported)", a->width);
    TS_REQUIRE(a->kv_heads >= 1 && a->heads % a->kv_heads == 0, "flash_rows: %u heads over %u kv heads",
               a->heads, a->kv_heads);
    TS_REQUIRE((a->q_dtype == TS_F32 || a->q_dtype == TS_BF16) && a->kv_dtype == TS_BF16 && a->out_dtype == TS_F32,
               "flash_rows: q f32 or bf16, kept rows bf16, out f32 supported");
    TS_REQUIRE(!a->kept_table || (a->page >= 16 && (a->page & (a->page - 1)) == 0),
               "flash_rows: page %u must be a power of two >= 16", a->page);
    TS_REQUIRE(a->kept_table || a->keys >= 1, "flash_rows: dense kept rows need keys");
    TS_REQUIRE(ts::aligned(a->k, 16) && ts::aligned(a->v, 16) && ts::aligned(a->q, 16),
               "flash_rows: q, k, v must be 16-byte aligned");
    TS_REQUIRE(a->heads <= 65535, "flash_rows: grid limits");
    if (a->rows == 0) return TS_OK;
    FlashParams p;
    p.q = a->q; p.k = (const uint16_t *)a->k; p.v = (const uint16_t *)a->v;
    p.out = (float *)a->out; p.slots = a->slots; p.positions = a->positions; p.table = a->kept_table;
    p.rows = a->rows; p.keys = a->keys; p.heads = a->heads; p.kv_heads = a->kv_heads; p.back = a->back;
    p.kept_pages = a->kept_pages; p.page_shift = a->kept_table ? (uint32_t)__builtin_ctz(a->page) : 0;
    p.scale = a->scale;
    const auto kern = a->q_dtype == TS_F32 ? flash_rows_kernel<true> : flash_rows_kernel<false>;
    hipLaunchKernelGGL(kern, dim3((a->rows + kRows - 1) / kRows, a->heads), dim3(256), 0, (hipStream_t)stream, p);
    TS_CHECK_LAUNCH("flash_rows launch");
    return TS_OK;
}
