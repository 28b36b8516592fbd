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
//  * One group per (128 query rows, q heads of one kv head): 4 waves per q head, each
//    wave owns 32 rows (two 16-query MFMA tiles); with GQA pairs a group of 8 waves
//    covers both heads of the pair. Each K/V block is loaded once for all of that
//    MFMA work (64 rows and one head per group measured 1.8x slower).
//  * Rows may be packed ragged (prompts back to back): a group whose rows belong to
//    several slots makes one pass over the keys per distinct slot, in order of first
//    appearance, as the reference's flash_rows does (flash.rs:504-591); a pass
//    touches only its own rows' softmax state, and waves with none of them idle
//    through it. The common case, one slot per group, is one pass.
//  * Keys stream in 64-row blocks, two resident in LDS: block b + 1's K and V rows go
//    straight from memory to LDS (global_load_lds, no staging registers or LDS
//    stores) while block b computes, one barrier per block. Rows sit in LDS as [key][d]
//    with 16-byte chunks XOR-swizzled by key (the swizzle picks each lane's source
//    chunk, since a wave's 1 KiB lands contiguously); the V^T operand of
//    O^T += V^T P^T comes out of LDS already transposed through gfx950's
//    ds_read_b64_tr_b16. Fragment offsets are computed once per lane.
//  * The group's page-table entries are copied to LDS once.
//  * S^T = K Q^T: 4 key tiles x 4 d-steps of v_mfma_f32_16x16x32_bf16 per q part
//    (bf16 q as is; f32 q split into two exact bf16 parts). Online softmax per query
//    in base 2 with a lazy reference point (moved only when a score passes it by
//    2^8, so most blocks skip rescaling O); P^T (bf16; two parts for f32 q) feeds
//    O^T += V^T P^T straight from registers (the layout notes at flash_rows_kernel).
#include "common.h"

namespace {

constexpr int kQT = 2;              // 16-query tiles per wave
constexpr int kRows = 64 * kQT;     // query rows per group (4 waves)
constexpr int kKeys = 64;   // keys per block (two 32-key MFMA steps of P V)
constexpr float kSlack = 8.0f;  // base-2 headroom of the softmax reference point

struct FlashParams {
    const void *q;
    const uint16_t *k, *v;
    float *out;
    const uint32_t *slots, *positions, *table;
    uint32_t rows, keys, heads, kv_heads, back, kept_pages, page_shift, max_position;
    float scale;
    uint32_t *status;
    // Whole sequences (seq_rows > 0, slots and positions NULL): row r is query r %
    // seq_rows of sequence r / seq_rows, at position past + r % seq_rows, and sees keys
    // [pos - back, pos + ahead] of its sequence (engine/ir/interp/src/cpu.rs:61-77
    // seen); a row whose window holds no key writes zeros. Ragged rows: ahead = 0.
    uint32_t ahead, seq_rows, past;
};

// The slot and position of row r, and the last key its window reaches.
TS_DEV uint32_t row_slot(const FlashParams &p, uint32_t r) { return p.seq_rows ? r / p.seq_rows : p.slots[r]; }
TS_DEV uint32_t row_pos(const FlashParams &p, uint32_t r) {
    return p.seq_rows ? p.past + r % p.seq_rows : p.positions[r];
}
TS_DEV uint32_t row_to(const FlashParams &p, uint32_t pos) {
    return p.seq_rows ? (uint32_t)min((uint64_t)pos + p.ahead, (uint64_t)p.keys - 1) : pos;
}

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

typedef __attribute__((address_space(3))) void flash_lds_void;

// Bytes of one key block buffer in LDS: 64 K rows then 64 V rows of 256 bytes, the
// 16-byte chunks of row key at chunk ^ kswz(key).
constexpr uint32_t kBlockBytes = 2 * kKeys * 256;

// The chunk swizzle of a key row: a permutation of the key's low four bits (bits 0, 1
// to 2, 3; bit 2 to 1; bit 3 to 0). K fragment reads (16 keys of one chunk) see 16
// distinct slots because it is one-to-one; the transposing V reads (4 consecutive
// keys of one 16-lane block, chunks 2d and 2d + 1) see 8 distinct slots in each block
// and 16 across two blocks, where XOR by key & 15 put two keys on one bank.
TS_DEV uint32_t kswz(uint32_t key) {
    return ((key & 3) << 2) | (((key >> 2) & 1) << 1) | ((key >> 3) & 1);
}

// Sums and maxima over the four 16-lane rows of a wave, in every lane (gfx950
// permlane swaps: VALU).
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

// V^T operand straight from row-major V with gfx950's transposing LDS read
// (ds_read_b64_tr_b16): within each 16-lane block, lane i receives element i % 4 of
// the 8-byte pieces addressed by lanes i / 4 + 4 e, e = 0..3. Lane L = 4 e + c of
// block g addresses key k0 + e, d = d0 + 4 c, so lane i ends with d0 + i of keys
// k0 .. k0 + 3: four consecutive keys of one d, as the MFMA A operand wants.
typedef short ts_v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) ts_v4i16 lds_v4i16;
TS_DEV u32x2 read_vt4(const char *a) {
    const ts_v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)a);
    return __builtin_bit_cast(u32x2, v);
}

// Row groups this order-by-cost considers (beyond it: launch order).
constexpr uint32_t kMaxOrder = 256;

// The (row group << 16 | head group) of this block, widest key span first. Causal
// prefill groups differ up to rows / 64 times in work and one 8-wave group fills a CU,
// so launch order leaves a tail; every block ranks the row groups by the key blocks
// they span (the positions come from L2) and takes, for its linear id L, the group of
// rank L / gridDim.y and head group L % gridDim.y: the widest first, head groups
// fastest (consecutive blocks go to different XCDs, each then keeps one head group's
// keys in its L2). Ties keep row order. Every block computes the same ranking, so
// the mapping is a permutation of the grid.
TS_DEV uint32_t widest_first(const FlashParams &p, uint32_t lane, uint32_t wave, uint32_t waves) {
    __shared__ uint32_t slo[kMaxOrder], shi[kMaxOrder], scost[kMaxOrder], ssel;
    const uint32_t ng = gridDim.x, nh = gridDim.y;
    if (ng <= 1 || ng > kMaxOrder) return (blockIdx.x << 16) | blockIdx.y;
    const uint32_t L = blockIdx.x + ng * blockIdx.y, target = L / nh;
    for (uint32_t u = threadIdx.x; u < ng; u += 64 * waves) { slo[u] = 0xffffffffu; shi[u] = 0; }
    if (threadIdx.x == 0) ssel = target;  // every rank is taken; set for form's sake
    __syncthreads();
    // One wave a 64-row half group at a time, eight halves' positions loaded before
    // any is reduced: the span [min from, max pos] of the group's rows (positions
    // clamped to the bound; refused rows only widen it).
    for (uint32_t h0 = wave; h0 < 2 * ng; h0 += 8 * waves) {
        uint32_t his[8], los[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const uint32_t half = h0 + u * waves, r = 64 * half + lane;
            his[u] = 0;
            los[u] = 0xffffffffu;
            if (half < 2 * ng && r < p.rows) {
                const uint32_t pos = min(row_pos(p, r), p.max_position);
                his[u] = row_to(p, pos);
                los[u] = pos > p.back ? pos - p.back : 0;
            }
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            uint32_t hi = his[u], lo = los[u];
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                hi = max(hi, (uint32_t)__shfl_xor((int)hi, o, 64));
                lo = min(lo, (uint32_t)__shfl_xor((int)lo, o, 64));
            }
            const uint32_t half = h0 + u * waves;
            if (lane == 0 && half < 2 * ng && lo <= hi) {
                atomicMin(&slo[half >> 1], lo);
                atomicMax(&shi[half >> 1], hi);
            }
        }
    }
    __syncthreads();
    // Rank by the key blocks spanned (an upper bound for a group of several slots).
    for (uint32_t g = threadIdx.x; g < ng; g += 64 * waves)
        scost[g] = slo[g] <= shi[g] ? (shi[g] >> 6) - (slo[g] >> 6) + 1 : 0u;
    __syncthreads();
    for (uint32_t g = threadIdx.x; g < ng; g += 64 * waves) {
        const uint32_t c = scost[g];
        uint32_t rank = 0;
        for (uint32_t j = 0; j < ng; j++) {
            const uint32_t cj = scost[j];
            rank += (cj > c) | ((cj == c) & (j < g));
        }
        if (rank == target) ssel = g;
    }
    __syncthreads();
    return (ssel << 16) | (L % nh);
}

// The transposed formulation: S^T = K Q^T and O^T = V^T P^T. With K as the A
// operand (rows = keys) and Q^T as B (columns = queries), the S^T accumulator lane
// (query col, group g) holds keys 4 g + i of each 16-key tile: after the softmax
// those P^T values are, packed as they are, the B operand of the P V product over
// keys {4 g + i, 16 + 4 g + i} of each 32-key step (no staging of P through LDS), and the O^T
// accumulator gives each lane 4 adjacent d of its query (16-byte stores).
// HG q heads of one kv head per group (GQA): 4 HG waves, wave w on head h0 + w / 4; the
// block's K and V are loaded and staged once for all of them.
template <bool QF32, int HG>
__global__ __launch_bounds__(256 * HG) void flash_rows_kernel(FlashParams p) {
    constexpr int kWaves = 4 * HG;
    constexpr int kNI = kKeys * 256 / 1024 / kWaves;  // 1 KiB K (and V) loads per wave and block
    extern __shared__ __attribute__((aligned(16))) char kv_lds[];  // 2 x kBlockBytes
    __shared__ uint32_t srange[kRows][2];   // key range of each pass
    __shared__ uint32_t sslot[kRows];       // slot of each row; then the slot of each pass
    __shared__ uint32_t spass[kRows];       // pass of each row (kNoPass: dead or refused)
    __shared__ uint32_t snpass, smixed;
    __shared__ uint32_t stab_s[kMaxPages];  // this group's page-table entries

    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), t = threadIdx.x;
    const uint32_t col = lane & 15, grp = lane >> 4;
    const uint32_t rg = widest_first(p, lane, wave, kWaves), hp = rg & 0xffffu;
    const uint32_t G = p.heads / p.kv_heads, h = hp * HG + (wave >> 2), kvh = h / G;
    const uint32_t qw = wave & 3;  // the wave's 16 kQT rows within the group's kRows
    const uint32_t r0 = (rg >> 16) * kRows;
    constexpr uint32_t kNoPass = 0xffffffffu;

    // Passes: one per distinct slot among the group's rows, numbered in order of first
    // appearance. A row the slot cannot hold (position >= keys, past the stated bound
    // or past the slot's table row: the interpreter refuses such reads,
    // engine/ir/interp/src/cpu.rs:323-327) takes no pass, loads nothing, writes NaN and
    // sets the status bit.
    bool ok_t = false;
    uint32_t slot_t = 0;
    if (t < kRows) {
        srange[t][0] = 0xffffffffu;
        srange[t][1] = 0;
        spass[t] = kNoPass;
        if (r0 + t < p.rows) {
            const uint32_t pos = row_pos(p, r0 + t);
            if (p.seq_rows) {  // whole sequences: served when the window holds a key
                ok_t = pos < p.keys + (uint64_t)p.back && (pos > p.back ? pos - p.back : 0) <= row_to(p, pos);
            } else {
                ok_t = !(pos >= p.keys || pos > p.max_position || (p.table && (pos >> p.page_shift) >= p.kept_pages));
                if (!ok_t && p.status) atomicOr(p.status, TS_STATUS_POSITION);
            }
            slot_t = row_slot(p, r0 + t);
        }
    }
    if (t == 0) { smixed = 0; snpass = 0; }
    __syncthreads();
    if (t < kRows) sslot[t] = ok_t ? slot_t : 0;
    if (t < kRows && ok_t) spass[t] = 0;  // provisional: whether the row is served
    __syncthreads();
    const uint32_t lead0 = [&] {  // first served row's slot (any, when none is served)
        for (uint32_t j = 0; j < kRows; j++)
            if (spass[j] == 0) return sslot[j];
        return 0u;
    }();
    if (ok_t && slot_t != lead0) smixed = 1;
    __syncthreads();
    if (!smixed) {
        if (t == 0) snpass = 1;
        if (t < kRows && ok_t) spass[t] = 0;
    } else {
        // The leader of a row: the first served row of its slot. Leaders count the
        // leaders before them (their pass); each row then takes its leader's pass.
        uint32_t leader = kNoPass;
        if (t < kRows && ok_t) {
            for (uint32_t j = 0; j <= t; j++)
                if (spass[j] != kNoPass && sslot[j] == slot_t) { leader = j; break; }
        }
        __syncthreads();
        // Reuse spass: 1 marks a leader.
        if (t < kRows) spass[t] = (ok_t && leader == t) ? 1u : 0u;
        __syncthreads();
        uint32_t mine = kNoPass;
        if (t < kRows && ok_t) {
            mine = 0;
            for (uint32_t j = 0; j < leader; j++) mine += spass[j];
        }
        __syncthreads();
        if (t < kRows) spass[t] = mine;
        if (t < kRows && ok_t && leader == t) atomicAdd(&snpass, 1u);
        __syncthreads();
        if (t < kRows && ok_t && leader == t) sslot[mine] = slot_t;  // pass -> slot (mine <= t)
    }
    __syncthreads();
    if (!smixed && t == 0) sslot[0] = lead0;
    if (t < kRows && ok_t) {
        const uint32_t pos = row_pos(p, r0 + t);
        atomicMin(&srange[spass[t]][0], pos > p.back ? pos - p.back : 0);
        atomicMax(&srange[spass[t]][1], row_to(p, pos));
    }
    __syncthreads();
    const uint32_t npass = snpass;

    // The scale's sign goes into q (exact: a sign flip of every bf16 / f32 value), so
    // the scores are scaled by sl >= 0 and a maximum of raw scores is one of scaled
    // ones. A zero scale becomes 2^-100 (every p equal to 1 within f32 rounding for
    // any finite score below 2^75), so masked -inf scores stay -inf.
    const uint32_t qsign = p.scale < 0.0f ? 0x80008000u : 0u;
    const float sl = p.scale == 0.0f ? 0x1p-100f : fabsf(p.scale) * 1.4426950408889634f;  // to base 2

    // This wave's queries: r0 + 16 kQT wave + 16 qt + col. The q operand
    // (B, columns = queries), loaded once: lane group g holds d 32 g + 8 j .. + 8 for
    // d-step j; bf16 q as is, f32 q as two exact bf16 parts.
    u32x4 qh[kQT][4], ql[kQT][4];
    uint32_t rpos[kQT], rfrom[kQT], rpass[kQT];
    bool rlive[kQT];  // the row is served (exists and is not refused)
#pragma unroll
    for (int qt = 0; qt < kQT; qt++) {
        const uint32_t i = 16 * kQT * qw + 16 * qt + col, r = r0 + i;
        rpass[qt] = spass[i];
        rlive[qt] = rpass[qt] != kNoPass;
        const uint32_t pos = rlive[qt] ? row_pos(p, r) : 0;
        rpos[qt] = row_to(p, pos);  // the last key the row sees
        rfrom[qt] = pos > p.back ? pos - p.back : 0;
        if (!QF32) {
            const uint16_t *qr = (const uint16_t *)p.q + ((size_t)(rlive[qt] ? r : 0) * p.heads + h) * 128 + 32 * grp;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const u32x4 w = rlive[qt] ? *(const u32x4 *)(qr + 8 * j) : u32x4{0, 0, 0, 0};
                qh[qt][j] = u32x4{w.x ^ qsign, w.y ^ qsign, w.z ^ qsign, w.w ^ qsign};
                ql[qt][j] = u32x4{0, 0, 0, 0};
            }
        } else {
            const float *qr = (const float *)p.q + ((size_t)(rlive[qt] ? r : 0) * p.heads + h) * 128 + 32 * grp;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                uint32_t hh[4], ll[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float a = rlive[qt] ? qr[8 * j + 2 * e] : 0.0f, b = rlive[qt] ? qr[8 * j + 2 * e + 1] : 0.0f;
                    if (qsign) { a = -a; b = -b; }
                    float ha = bf16_round(a), hb = bf16_round(b);
                    hh[e] = pack_bf16x2(ha, hb);
                    ll[e] = pack_bf16x2(a - ha, b - hb);
                }
                qh[qt][j] = u32x4{hh[0], hh[1], hh[2], hh[3]};
                ql[qt][j] = u32x4{ll[0], ll[1], ll[2], ll[3]};
            }
        }
    }

    // LDS byte offsets of this lane's fragments within a block buffer: K as S^T's A
    // operand (key 16 kt + col, d chunk 4 grp + j) and V^T as the A operand of P V
    // (keys 32 st + 4 grp + col / 4 and + 16, d 16 d + 4 (col & 3)).
    uint32_t koff[4];
#pragma unroll
    for (int j = 0; j < 4; j++) koff[j] = col * 256 + (((4 * grp + j) ^ kswz(col)) << 4);
    const uint32_t vk = 4 * grp + (col >> 2), vbase = vk * 256 + 8 * (col & 1), vc = (col & 3) >> 1;

    float m[kQT], l[kQT];
#pragma unroll
    for (int qt = 0; qt < kQT; qt++) { m[qt] = -INFINITY; l[qt] = 0.0f; }
    f32x4 o[kQT][8];  // O^T: [query tile][d tile], lane: query col, d 4 grp + i
#pragma unroll
    for (int qt = 0; qt < kQT; qt++)
#pragma unroll
        for (int d = 0; d < 8; d++) o[qt][d] = f32x4{0, 0, 0, 0};

    for (uint32_t pass = 0; pass < npass; pass++) {
    const uint32_t slot = sslot[pass];
    uint32_t lo = srange[pass][0], hi = srange[pass][1];
    lo &= ~(kKeys - 1);
    bool act[kQT];  // rows of this pass
#pragma unroll
    for (int qt = 0; qt < kQT; qt++) act[qt] = rlive[qt] && rpass[qt] == pass;
    bool any = false;
#pragma unroll
    for (int qt = 0; qt < kQT; qt++) any |= act[qt];
    const bool wave_on = __builtin_amdgcn_ballot_w64(any) != 0;  // else: stage and wait only
    // The page numbers of keys [lo, hi] into LDS once, so no key block waits on a
    // dependent table load.
    if (pass) __syncthreads();  // every wave is done with the previous pass's table
    const uint32_t p0 = p.table ? lo >> p.page_shift : 0, np = p.table ? (hi >> p.page_shift) - p0 + 1 : 0;
    const uint32_t *stab = nullptr;
    if (p.table && np <= kMaxPages) {
        for (uint32_t i = t; i < np; i += 256 * HG) stab_s[i] = p.table[(uint64_t)slot * p.kept_pages + p0 + i];
        __syncthreads();
        stab = stab_s;
    }
    // Block kb's K and V rows straight into LDS buffer buf (global_load_lds: lane i of
    // a wave's 1 KiB segment lands at 16 i, so the swizzle picks the source chunk).
    // Keys past hi read row hi instead (written, finite; masked below).
    auto fetch = [&](uint32_t kb, uint32_t buf) {
        char *base = kv_lds + buf * kBlockBytes;
#pragma unroll
        for (int c = 0; c < kNI; c++) {
            const uint32_t sg = c * kWaves + wave, key = 4 * sg + (lane >> 4), chunk = (lane & 15) ^ kswz(key & 15);
            const uint64_t row = key_row(p, slot, min(kb + key, hi), stab, p0);
            const size_t e = (row * p.kv_heads + kvh) * 128 + chunk * 8;
            __builtin_amdgcn_global_load_lds((const void *)(p.k + e), (flash_lds_void *)(base + sg * 1024), 16, 0, 0);
            __builtin_amdgcn_global_load_lds((const void *)(p.v + e),
                                             (flash_lds_void *)(base + kKeys * 256 + sg * 1024), 16, 0, 0);
        }
    };
    fetch(lo, 0);
    for (uint32_t kb = lo, b = 0; kb <= hi; kb += kKeys, b++) {
        // Block b has landed (its loads are the only ones outstanding); the barrier
        // also ends every wave's reads of the buffer refilled next (block b - 1).
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (kb + kKeys <= hi) fetch(kb + kKeys, (b + 1) & 1);
        if (!wave_on) continue;
        const char *kbuf = kv_lds + (b & 1) * kBlockBytes, *vbuf = kbuf + kKeys * 256;

        // S^T for four 16-key tiles x the query tiles.
        f32x4 s[4][kQT];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
#pragma unroll
            for (int qt = 0; qt < kQT; qt++) s[kt][qt] = f32x4{0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const bf16x8 kf = as_bf16x8(*(const u32x4 *)(kbuf + koff[j] + kt * 16 * 256));
#pragma unroll
                for (int qt = 0; qt < kQT; qt++) {
                    s[kt][qt] = mfma16(kf, as_bf16x8(qh[qt][j]), s[kt][qt]);
                    if (QF32) s[kt][qt] = mfma16(kf, as_bf16x8(ql[qt][j]), s[kt][qt]);
                }
            }
        }
        // Online softmax per query (a lane's column), over its 16 keys and the
        // lanes of its column in the other three row groups, in base 2: scores are
        // scaled by scale * log2(e) and exponentiated with v_exp_f32 (exp(x) =
        // 2^(x log2 e)); m and l keep the base-2 running max and the sum.
        // A block wholly inside every query's window of the wave skips the masks.
        bool inside = true;
#pragma unroll
        for (int qt = 0; qt < kQT; qt++)  // rows of other passes keep their masks
            inside &= act[qt] ? (kb + kKeys - 1 <= rpos[qt] && kb >= rfrom[qt]) : !rlive[qt];
        inside = __builtin_amdgcn_ballot_w64(!inside) == 0;  // uniform
        bf16x8 ph[2][kQT], pl[2][kQT];
#pragma unroll
        for (int qt = 0; qt < kQT; qt++) {
            const int hi_off = (int)rpos[qt] - (int)kb, lo_off = (int)rfrom[qt] - (int)kb;
            // One uniform branch a block: the masks only where a block meets a window's
            // edge (a per-score short-circuit test compiled to a branch a score). The
            // scores stay raw (sl >= 0: the sign of the scale is in q), masked ones -inf
            // in place.
            if (!inside) {
#pragma unroll
                for (int kt = 0; kt < 4; kt++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int k = kt * 16 + 4 * (int)grp + i;
                        const bool ok = act[qt] & (k <= hi_off) & (k >= lo_off);
                        s[kt][qt][i] = ok ? s[kt][qt][i] : -INFINITY;
                    }
            }
            float mx;
            {
                float t[4];
#pragma unroll
                for (int kt = 0; kt < 4; kt++)
                    t[kt] = fmaxf(fmaxf(s[kt][qt][0], s[kt][qt][1]), fmaxf(s[kt][qt][2], s[kt][qt][3]));
                mx = fmaxf(fmaxf(t[0], t[1]), fmaxf(t[2], t[3]));
            }
            mx = rows4_max(mx) * sl;  // -inf stays -inf (sl > 0)
            // The reference point m moves only when a score passes it by more than
            // kSlack (base 2): p = 2^(score - m) then stays below 2^kSlack, and most
            // blocks leave l and O unscaled (O / l does not depend on the choice of m).
            const bool raise = mx > m[qt] + kSlack;
            const float mn = raise ? mx : m[qt];
            const float alpha = raise ? __builtin_amdgcn_exp2f(m[qt] - mn) : 1.0f;  // 0 from m = -inf
            const float mo = mn == -INFINITY ? 0.0f : mn;  // exp2(-inf - 0) = 0 for masked keys
            float part[4];  // sums of p by 16-key tile, then as a tree
#pragma unroll
            for (int st = 0; st < 2; st++) {
                uint32_t hw[4], lw[4];
#pragma unroll
                for (int tt = 0; tt < 2; tt++)
#pragma unroll
                    for (int i = 0; i < 4; i += 2) {
                        const int kt = 2 * st + tt;
                        // 2^(score - m) = 2^(s sl - mo): one fma; a masked -inf gives 0.
                        const float pa = __builtin_amdgcn_exp2f(fmaf(s[kt][qt][i], sl, -mo));
                        const float pb = __builtin_amdgcn_exp2f(fmaf(s[kt][qt][i + 1], sl, -mo));
                        part[kt] = i == 0 ? pa + pb : part[kt] + (pa + pb);
                        // p in [0, 2^kSlack] (never NaN for finite scores): the
                        // plain round-to-nearest-even conversion, no NaN fix-up.
                        hw[2 * tt + i / 2] = __builtin_bit_cast(
                            uint32_t, __builtin_convertvector(ts_f32x2{pa, pb}, ts_bf16x2));
                        if (QF32) {
                            const float ha = bf16_float((uint16_t)(hw[2 * tt + i / 2] & 0xffffu));
                            const float hb = bf16_float((uint16_t)(hw[2 * tt + i / 2] >> 16));
                            lw[2 * tt + i / 2] = pack_bf16x2(pa - ha, pb - hb);
                        } else {
                            lw[2 * tt + i / 2] = 0u;
                        }
                    }
                ph[st][qt] = as_bf16x8(u32x4{hw[0], hw[1], hw[2], hw[3]});
                pl[st][qt] = as_bf16x8(u32x4{lw[0], lw[1], lw[2], lw[3]});
            }
            const float sum = rows4_sum((part[0] + part[1]) + (part[2] + part[3]));
            l[qt] = l[qt] * alpha + sum;
            m[qt] = mn;
            // Rescale O only when some query of the wave moved its reference point.
            if (__builtin_amdgcn_ballot_w64(raise) != 0) {
#pragma unroll
                for (int d = 0; d < 8; d++) o[qt][d] *= alpha;
            }
        }
        // O^T += V^T P^T: A = V^T rows d, keys in P^T's order (one 16-byte read per
        // 32-key step).
#pragma unroll
        for (int d = 0; d < 8; d++) {
#pragma unroll
            for (int st = 0; st < 2; st++) {
                // Positions 8 grp .. + 3 and + 4 .. + 7 of step st hold keys
                // 32 st + 4 grp + i and 32 st + 16 + 4 grp + i (P^T's order).
                const char *va_at = vbuf + vbase + (((2 * d + vc) ^ kswz(vk)) << 4) + 32 * st * 256;
                const u32x2 va = read_vt4(va_at), vb = read_vt4(va_at + 16 * 256);
                const bf16x8 vf = as_bf16x8(u32x4{va.x, va.y, vb.x, vb.y});
#pragma unroll
                for (int qt = 0; qt < kQT; qt++) {
                    o[qt][d] = mfma16(vf, ph[st][qt], o[qt][d]);
                    if (QF32) o[qt][d] = mfma16(vf, pl[st][qt], o[qt][d]);
                }
            }
        }
    }

    }  // pass

    // O / l: lane (query col of tile qt) holds d = 16 dt + 4 grp + i. Refused rows
    // write NaN; whole-sequence rows that see no key write zeros.
#pragma unroll
    for (int qt = 0; qt < kQT; qt++) {
        const uint32_t r = r0 + 16 * kQT * qw + 16 * qt + col;
        if (r >= p.rows) continue;
        float *dst = p.out + ((size_t)r * p.heads + h) * 128;
        const float inv = rlive[qt] ? 1.0f / l[qt] : p.seq_rows ? 0.0f : __builtin_nanf("");
#pragma unroll
        for (int d = 0; d < 8; d++) *(f32x4 *)(dst + d * 16 + 4 * grp) = o[qt][d] * inv;
    }
}

int flash_launch(const FlashParams &p, bool f32, void *stream, const char *rule) {
    // Two q heads per group when the kv heads are shared in pairs (or more, evenly).
    const int hg = (p.heads / p.kv_heads) % 2 == 0 ? 2 : 1;
    const auto kern = hg == 2 ? (f32 ? flash_rows_kernel<true, 2> : flash_rows_kernel<false, 2>)
                              : (f32 ? flash_rows_kernel<true, 1> : flash_rows_kernel<false, 1>);
    // The key blocks' dynamic LDS, raised once per process (thread-safe static
    // initialisation; every call returns the stored outcome).
    static const hipError_t attr = [] {
        for (const auto k : {flash_rows_kernel<true, 2>, flash_rows_kernel<false, 2>, flash_rows_kernel<true, 1>,
                             flash_rows_kernel<false, 1>}) {
            const hipError_t e = hipFuncSetAttribute((const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                     2 * kBlockBytes);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }();
    if (attr != hipSuccess) return ts::hip_status(attr, "flash: shared memory attribute");
    hipLaunchKernelGGL(kern, dim3((p.rows + kRows - 1) / kRows, p.heads / hg), dim3(256 * hg), 2 * kBlockBytes,
                       (hipStream_t)stream, p);
    const hipError_t e = hipPeekAtLastError();
    if (e != hipSuccess) return ts::hip_status(e, rule);
    return TS_OK;
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
    TS_REQUIRE(a->keys >= 1, "flash_rows: keys (the positions a slot holds) must be >= 1");
    TS_REQUIRE(ts::aligned(a->k, 16) && ts::aligned(a->v, 16) && ts::aligned(a->q, 16),
               "flash_rows: q, k, v must be 16-byte aligned");
    TS_REQUIRE(a->heads <= 65535, "flash_rows: grid limits");
    // The block order packs a row group in 16 bits (65535 groups of 128 rows).
    TS_REQUIRE(a->rows <= 65535u * 128u, "flash_rows: %u rows in one launch (at most %u)", a->rows, 65535u * 128u);
    if (a->rows == 0) return TS_OK;
    FlashParams p;
    p.q = a->q; p.k = (const uint16_t *)a->k; p.v = (const uint16_t *)a->v;
    p.out = (float *)a->out; p.slots = a->slots; p.positions = a->positions; p.table = a->kept_table;
    p.rows = a->rows; p.keys = a->keys; p.heads = a->heads; p.kv_heads = a->kv_heads; p.back = a->back;
    p.kept_pages = a->kept_pages; p.page_shift = a->kept_table ? (uint32_t)__builtin_ctz(a->page) : 0;
    p.scale = a->scale; p.max_position = a->max_position; p.status = a->status;
    p.ahead = 0; p.seq_rows = 0; p.past = 0;
    return flash_launch(p, a->q_dtype == TS_F32, stream, "flash_rows");
}

extern "C" int tessera_hip_flash(const ts_flash_args *a, void *stream) {
    TS_REQUIRE(a && a->q && a->k && a->v && a->out, "flash: null pointer");
    TS_REQUIRE(a->width == 128, "flash: head width %u (128 supported)", a->width);
    TS_REQUIRE(a->kv_heads >= 1 && a->heads % a->kv_heads == 0, "flash: %u heads over %u kv heads", a->heads,
               a->kv_heads);
    TS_REQUIRE((a->q_dtype == TS_F32 || a->q_dtype == TS_BF16) && a->kv_dtype == TS_BF16 && a->out_dtype == TS_F32,
               "flash: q f32 or bf16, k and v bf16, out f32 supported");
    TS_REQUIRE(a->keys >= 1 && a->rows >= 1, "flash: rows %u, keys %u", a->rows, a->keys);
    // interp's attend (cpu.rs:61-77): query and key ends align when the keys cover the
    // rows; fewer keys than rows are refused for masks whose ends align (causal, back).
    TS_REQUIRE(a->keys >= a->rows || !a->causal, "flash: %u rows over %u keys with a causal mask", a->rows, a->keys);
    TS_REQUIRE(ts::aligned(a->k, 16) && ts::aligned(a->v, 16) && ts::aligned(a->q, 16),
               "flash: q, k, v must be 16-byte aligned");
    TS_REQUIRE(a->heads <= 65535, "flash: grid limits");
    const uint64_t total = (uint64_t)a->seqs * a->rows;
    TS_REQUIRE(total <= 65535u * 128u, "flash: %llu rows in one launch (at most %u)", (unsigned long long)total,
               65535u * 128u);
    TS_REQUIRE((uint64_t)a->seqs * a->keys < (1ull << 32), "flash: %u sequences of %u keys", a->seqs, a->keys);
    if (total == 0) return TS_OK;
    FlashParams p;
    p.q = a->q; p.k = (const uint16_t *)a->k; p.v = (const uint16_t *)a->v; p.out = (float *)a->out;
    p.slots = p.positions = p.table = nullptr;
    p.rows = (uint32_t)total; p.keys = a->keys; p.heads = a->heads; p.kv_heads = a->kv_heads;
    p.back = a->back; p.ahead = a->ahead; p.kept_pages = 0; p.page_shift = 0; p.scale = a->scale;
    p.status = nullptr;
    p.seq_rows = a->rows;
    p.past = a->keys >= a->rows ? a->keys - a->rows : 0;
    p.max_position = p.past + a->rows - 1;
    return flash_launch(p, a->q_dtype == TS_F32, stream, "flash");
}
