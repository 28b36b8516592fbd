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
//  * Keys stream in 32-row blocks (two page lookups). K goes to LDS as rows
//    ([key][d], 16-byte chunks XOR-swizzled by key), V goes to LDS transposed
//    ([d][key]) so the P*V operand is one 16-byte read per lane.
//  * S = Q K^T: 2 key tiles x 4 d-steps of v_mfma_f32_16x16x32_bf16 per q part
//    (q f32 split into two exact bf16 parts). Online softmax per row with
//    16-lane butterflies. P (two bf16 parts) is staged through LDS into the A
//    layout; O[16 rows, 128] += P V in 8 MFMA column tiles.
#include "common.h"

namespace {

constexpr int kRows = 64;   // query rows per group
constexpr int kKeys = 32;   // keys per block

struct FlashParams {
    const float *q;
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

__global__ __launch_bounds__(256) void flash_rows_kernel(FlashParams p) {
    __shared__ __attribute__((aligned(16))) uint16_t sk[kKeys][128];     // K rows, swizzled chunks
    __shared__ __attribute__((aligned(16))) uint16_t svt[128][kKeys];    // V transposed
    __shared__ __attribute__((aligned(16))) uint16_t sp[4][2][16][kKeys];  // P parts per wave
    __shared__ uint32_t srange[2];

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

    // q operand (two bf16 parts), loaded once.
    u32x4 qh[4], ql[4];
    {
        const float *qr = p.q + ((size_t)(row_ok ? my_row : 0) * p.heads + h) * 128 + 32 * grp;
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

    for (uint32_t kb = lo; kb <= hi; kb += kKeys) {
        // Stage K rows and V^T: 32 keys x 16 chunks of 8 = 512 chunks, 2 per thread.
        __syncthreads();
#pragma unroll
        for (int c2 = 0; c2 < 2; c2++) {
            const uint32_t idx = t + 256 * c2, key = idx >> 4, chunk = idx & 15;
            const uint32_t pos = kb + key;
            u32x4 kv = u32x4{0, 0, 0, 0}, vv = u32x4{0, 0, 0, 0};
            // Keys past the last row's position may sit in pages never written: skip them.
            if (pos <= hi && (p.table || pos < p.keys)) {
                const uint64_t row = kept_row(p, slot, pos);
                const size_t off = (row * p.kv_heads + kvh) * 128 + chunk * 8;
                kv = *(const u32x4 *)(p.k + off);
                vv = *(const u32x4 *)(p.v + off);
            }
            *(u32x4 *)&sk[key][(chunk ^ (key & 15)) * 8] = kv;
            const uint32_t w4[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                svt[chunk * 8 + 2 * e][key] = (uint16_t)(w4[e] & 0xffff);
                svt[chunk * 8 + 2 * e + 1][key] = (uint16_t)(w4[e] >> 16);
            }
        }
        __syncthreads();

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
                s[kt] = mfma16(as_bf16x8(ql[j]), kf, s[kt]);
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
                sp[wave][1][4 * grp + i][kt * 16 + col] = bf16_bits(pv - ph);
            }
            sum = row16_sum(sum);
            l[i] = l[i] * alpha + sum;
            m[i] = mn;
#pragma unroll
            for (int d = 0; d < 8; d++) o[d][i] *= alpha;
        }
        // P (rows x 32 keys) as the A operand: lane row col, keys 8*grp..+8.
        __syncthreads();
        const bf16x8 ph = as_bf16x8(*(const u32x4 *)&sp[wave][0][col][8 * grp]);
        const bf16x8 pl = as_bf16x8(*(const u32x4 *)&sp[wave][1][col][8 * grp]);
#pragma unroll
        for (int d = 0; d < 8; d++) {
            const bf16x8 vf = as_bf16x8(*(const u32x4 *)&svt[d * 16 + col][8 * grp]);
            o[d] = mfma16(ph, vf, o[d]);
            o[d] = mfma16(pl, vf, o[d]);
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
    TS_REQUIRE(a->q_dtype == TS_F32 && a->kv_dtype == TS_BF16 && a->out_dtype == TS_F32,
               "flash_rows: q f32, kept rows bf16, out f32 supported");
    TS_REQUIRE(!a->kept_table || (a->page >= 16 && (a->page & (a->page - 1)) == 0),
               "flash_rows: page %u must be a power of two >= 16", a->page);
    TS_REQUIRE(a->kept_table || a->keys >= 1, "flash_rows: dense kept rows need keys");
    TS_REQUIRE(ts::aligned(a->k, 16) && ts::aligned(a->v, 16) && ts::aligned(a->q, 16),
               "flash_rows: q, k, v must be 16-byte aligned");
    TS_REQUIRE(a->heads <= 65535, "flash_rows: grid limits");
    if (a->rows == 0) return TS_OK;
    FlashParams p;
    p.q = (const float *)a->q; p.k = (const uint16_t *)a->k; p.v = (const uint16_t *)a->v;
    p.out = (float *)a->out; p.slots = a->slots; p.positions = a->positions; p.table = a->kept_table;
    p.rows = a->rows; p.keys = a->keys; p.heads = a->heads; p.kv_heads = a->kv_heads; p.back = a->back;
    p.kept_pages = a->kept_pages; p.page_shift = a->kept_table ? (uint32_t)__builtin_ctz(a->page) : 0;
    p.scale = a->scale;
    hipLaunchKernelGGL(flash_rows_kernel, dim3((a->rows + kRows - 1) / kRows, a->heads), dim3(256), 0,
                       (hipStream_t)stream, p);
    TS_CHECK_LAUNCH("flash_rows launch");
    return TS_OK;
}
