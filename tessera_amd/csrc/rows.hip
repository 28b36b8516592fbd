// Row stages and index kernels: RmsNorm, RoPE, the fused q/k norm + rope +
// kept-row append, embedding gather, argmax and top-k.
//
// Reference semantics: engine/ir/interp/src/cpu.rs:32-59 (angle, turn,
// softmax), 353-447 (stages), 492-525 (rms_inverse, take, gather) and
// engine/ir/interp/src/run.rs:577-591 (top_k). Each kernel cites its rule.
#include "common.h"

namespace {

// ---------------------------------------------------------------------------
// RmsNorm: one wave per row (rms_norm.rs:9-69 / lane_norm.rs:10-96 do a thread
// or a 32-lane group per row; a 64-lane wave with a butterfly sum here).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rms_norm_kernel(const float *x, const float *g, float *out,
                                                       uint32_t rows, uint32_t width, float eps) {
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *xr = x + (size_t)row * width;
    float s = 0.0f;
    for (uint32_t i = lane; i < width; i += 64) s += xr[i] * xr[i];
    s = wave_sum(s);
    const float inv = 1.0f / sqrtf(s / (float)width + eps);
    float *o = out + (size_t)row * width;
    for (uint32_t i = lane; i < width; i += 64) o[i] = xr[i] * (inv * g[i]);
}

// angle(pos, j, width, theta) = pos * theta^(-2j/width) (cpu.rs:32-34).
TS_DEV float rope_angle(uint32_t pos, uint32_t j, uint32_t width, float theta) {
    return (float)pos * powf(theta, -((float)(2 * j)) / (float)width);
}

// In-place rotation of one [width] row by its position (cpu.rs:36-47).
__global__ __launch_bounds__(256) void rope_kernel(float *x, const uint32_t *positions, uint32_t rows,
                                                   uint32_t heads, uint32_t width, float theta,
                                                   int halves) {
    const uint32_t half = width / 2;
    const uint64_t total = (uint64_t)rows * heads * half;
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const uint32_t j = (uint32_t)(i % half);
    const uint64_t rh = i / half;
    const uint32_t r = (uint32_t)(rh / heads);
    float *row = x + rh * width;
    const uint32_t a = halves ? j : 2 * j, b = halves ? j + half : 2 * j + 1;
    float sn, cs;
    sincosf(rope_angle(positions[r], j, width, theta), &sn, &cs);
    const float va = row[a], vb = row[b];
    row[a] = va * cs - vb * sn;
    row[b] = va * sn + vb * cs;
}

// The angle table: (cos, sin) of angle(pos, j, width, theta) for every position
// and pair, computed once (the reference's `angles` stage, rope.rs:10-58).
__global__ __launch_bounds__(256) void rope_table_kernel(float2 *t, uint32_t positions, uint32_t width, float theta) {
    const uint32_t half = width / 2;
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)positions * half) return;
    float sn, cs;
    sincosf(rope_angle((uint32_t)(i / half), (uint32_t)(i % half), width, theta), &sn, &cs);
    t[i] = make_float2(cs, sn);
}

// ---------------------------------------------------------------------------
// q/k RmsNorm per head, Halves RoPE, then k and v appended to the kept rows.
// One wave per (row, head) with width 128: lane j holds the pair (j, j+64),
// exactly the Halves rotation pair, so the rotation needs no exchange.
// ---------------------------------------------------------------------------
struct QkParams {
    const float *qkv;
    const float *q_gain, *k_gain;
    float *q_out;
    uint16_t *k_cache, *v_cache;
    const uint32_t *slots, *positions, *table;
    uint32_t rows, heads, kv_heads, keys, kept_pages, page_shift;
    float eps, theta;
};

TS_DEV uint64_t kept_row(const uint32_t *table, uint32_t kept_pages, uint32_t page_shift, uint32_t keys,
                         uint32_t slot, uint32_t pos) {
    if (!table) return (uint64_t)slot * keys + pos;
    const uint64_t entry = (uint64_t)slot * kept_pages + (pos >> page_shift);
    return ((uint64_t)table[entry] << page_shift) | (pos & ((1u << page_shift) - 1));
}

__global__ __launch_bounds__(256) void qk_norm_rope_append_kernel(QkParams p) {
    const uint32_t per_row = p.heads + 2 * p.kv_heads;
    const uint32_t wid = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (wid >= p.rows * per_row) return;
    const uint32_t r = wid / per_row, h = wid % per_row;
    const float *src = p.qkv + (size_t)r * per_row * 128 + (size_t)h * 128;
    float a = src[lane], b = src[lane + 64];
    const uint32_t pos = p.positions[r];
    if (h < p.heads + p.kv_heads) {
        const bool is_q = h < p.heads;
        const float *g = is_q ? p.q_gain : p.k_gain;
        const float s = wave_sum(a * a + b * b);
        const float inv = 1.0f / sqrtf(s / 128.0f + p.eps);
        a = a * (inv * g[lane]);
        b = b * (inv * g[lane + 64]);
        float sn, cs;
        sincosf(rope_angle(pos, lane, 128, p.theta), &sn, &cs);
        const float ra = a * cs - b * sn, rb = a * sn + b * cs;
        if (is_q) {
            float *o = p.q_out + ((size_t)r * p.heads + h) * 128;
            o[lane] = ra;
            o[lane + 64] = rb;
            return;
        }
        a = ra;
        b = rb;
    }
    const bool is_k = h < p.heads + p.kv_heads;
    const uint32_t kvh = is_k ? h - p.heads : h - p.heads - p.kv_heads;
    // A position the slot cannot hold appends nothing (the interpreter refuses the
    // write, engine/ir/interp/src/run.rs:122-198); the attention that reads it refuses
    // the row too and reports it.
    if (pos >= p.keys || (p.table && (pos >> p.page_shift) >= p.kept_pages)) return;
    const uint64_t row = kept_row(p.table, p.kept_pages, p.page_shift, p.keys, p.slots[r], pos);
    uint16_t *dst = (is_k ? p.k_cache : p.v_cache) + (row * p.kv_heads + kvh) * 128;
    dst[lane] = bf16_bits(a);
    dst[lane + 64] = bf16_bits(b);
}

// ---------------------------------------------------------------------------
// Embedding gather: bf16 table rows widened to f32 (exact).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gather_kernel(const uint16_t *table, const uint32_t *ids, float *out,
                                                     uint32_t count, uint32_t table_rows, uint32_t width,
                                                     uint32_t first) {
    const uint32_t r = blockIdx.y;
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= count || i >= width) return;
    const uint32_t id = ids[r];
    const bool in = id >= first && id - first < table_rows;
    out[(size_t)r * width + i] = in ? bf16_float(table[(size_t)(id - first) * width + i]) : 0.0f;
}

// ---------------------------------------------------------------------------
// Argmax: the first index of the largest finite entry (strictly greater wins
// in ascending order; NaN and -inf never win; none gives `width`).
// Pass 1: groups of 256 threads reduce 4096-wide spans to (value, index).
// Pass 2: one wave per row reduces the spans.
// ---------------------------------------------------------------------------
constexpr uint32_t kSpan = 4096;

TS_DEV void better(float &bv, uint32_t &bi, float v, uint32_t i) {
    // (v, i) beats (bv, bi) when larger, or equal with a lower index.
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

TS_DEV void wave_best(float &bv, uint32_t &bi) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float v = __shfl_xor(bv, o, 64);
        uint32_t i = __shfl_xor(bi, o, 64);
        better(bv, bi, v, i);
    }
}

__global__ __launch_bounds__(256) void argmax_spans(const float *x, float *vals, uint32_t *idx, uint32_t rows,
                                                    uint32_t width, uint32_t spans) {
    const uint32_t r = blockIdx.y, s = blockIdx.x;
    const float *xr = x + (size_t)r * width;
    float bv = -INFINITY;
    uint32_t bi = width;
    const uint32_t end = min(width, (s + 1) * kSpan);
    for (uint32_t i = s * kSpan + threadIdx.x; i < end; i += 256) {
        float v = xr[i];
        if (v > -INFINITY) better(bv, bi, v, i);  // NaN and -inf fail the test
    }
    wave_best(bv, bi);
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        bv = sv[0]; bi = si[0];
        for (int w = 1; w < 4; w++) better(bv, bi, sv[w], si[w]);
        vals[(size_t)r * spans + s] = bv;
        idx[(size_t)r * spans + s] = bi;
    }
}

__global__ __launch_bounds__(64) void argmax_finish(const float *vals, const uint32_t *idx, uint32_t *ids,
                                                    uint32_t spans, uint32_t width) {
    const uint32_t r = blockIdx.x;
    float bv = -INFINITY;
    uint32_t bi = width;
    for (uint32_t s = threadIdx.x; s < spans; s += 64) {
        float v = vals[(size_t)r * spans + s];
        uint32_t i = idx[(size_t)r * spans + s];
        if (i < width) better(bv, bi, v, i);
    }
    wave_best(bv, bi);
    if (threadIdx.x == 0) ids[r] = bi;
}

// ---------------------------------------------------------------------------
// top_k by rank: entry i's rank is the count of valid entries ahead of it
// (larger, or equal with a lower index); ranks below k write their index.
// One 256-thread group per row, the row staged in LDS.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void top_k_kernel(const float *x, uint32_t *ids, uint32_t rows, uint32_t width,
                                                    uint32_t k) {
    __shared__ float row[1024];
    __shared__ uint32_t valid_s;
    const uint32_t r = blockIdx.x;
    if (threadIdx.x == 0) valid_s = 0;
    __syncthreads();
    uint32_t mine = 0;
    for (uint32_t i = threadIdx.x; i < width; i += 256) {
        float v = x[(size_t)r * width + i];
        bool ok = v > -INFINITY;
        row[i] = ok ? v : NAN;  // NaN marks an entry that takes no rank
        mine += ok;
    }
    atomicAdd(&valid_s, mine);
    __syncthreads();
    const uint32_t valid = valid_s;
    for (uint32_t i = threadIdx.x; i < width; i += 256) {
        const float v = row[i];
        if (!(v == v)) continue;
        uint32_t rank = 0;
        for (uint32_t j = 0; j < width; j++) {
            const float u = row[j];
            rank += (u > v) || (u == v && j < i);
        }
        if (rank < k) ids[(size_t)r * k + rank] = i;
    }
    for (uint32_t s = valid + threadIdx.x; s < k; s += 256) ids[(size_t)r * k + s] = width;
}

}  // namespace

extern "C" int tessera_hip_rms_norm(const ts_norm_args *a, void *stream) {
    TS_REQUIRE(a, "rms_norm: null args");
    const float *x = a->x, *gain = a->gain;
    float *out = a->out;
    const uint32_t rows = a->rows, width = a->width;
    const float eps = a->eps;
    TS_REQUIRE(x && gain && out, "rms_norm: null pointer");
    TS_REQUIRE(width >= 1, "rms_norm: width 0");
    if (rows == 0) return TS_OK;
    hipLaunchKernelGGL(rms_norm_kernel, dim3((rows + 3) / 4), dim3(256), 0, (hipStream_t)stream, x, gain, out,
                       rows, width, eps);
    TS_CHECK_LAUNCH("rms_norm launch");
    return TS_OK;
}

extern "C" int tessera_hip_rope(const ts_rope_args *a, void *stream) {
    TS_REQUIRE(a, "rope: null args");
    float *x = a->x;
    const uint32_t *positions = a->positions;
    const uint32_t rows = a->rows, heads = a->heads, width = a->width;
    const float theta = a->theta;
    const int32_t halves = a->halves;
    TS_REQUIRE(x && positions, "rope: null pointer");
    TS_REQUIRE(width >= 2 && width % 2 == 0, "rope: width %u must be even", width);
    const uint64_t total = (uint64_t)rows * heads * (width / 2);
    if (total == 0) return TS_OK;
    hipLaunchKernelGGL(rope_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, x,
                       positions, rows, heads, width, theta, (int)halves);
    TS_CHECK_LAUNCH("rope launch");
    return TS_OK;
}

extern "C" int tessera_hip_rope_table(const ts_angles_args *a, void *stream) {
    TS_REQUIRE(a, "rope_table: null args");
    float *table = a->table;
    const uint32_t positions = a->positions, width = a->width;
    const float theta = a->theta;
    TS_REQUIRE(table, "rope_table: null pointer");
    TS_REQUIRE(width >= 2 && width % 2 == 0, "rope_table: width %u must be even", width);
    const uint64_t n = (uint64_t)positions * (width / 2);
    if (n == 0) return TS_OK;
    hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (float2 *)table, positions, width, theta);
    TS_CHECK_LAUNCH("rope_table launch");
    return TS_OK;
}

extern "C" int tessera_hip_qk_norm_rope_append(const ts_qk_args *a, void *stream) {
    TS_REQUIRE(a, "qk_norm_rope_append: null args");
    const float *qkv = a->qkv, *q_gain = a->q_gain, *k_gain = a->k_gain;
    float *q_out = a->q_out;
    void *k_cache = a->k_cache, *v_cache = a->v_cache;
    const uint32_t *slots = a->slots, *positions = a->positions, *kept_table = a->kept_table;
    const uint32_t rows = a->rows, heads = a->heads, kv_heads = a->kv_heads, width = a->width, keys = a->keys;
    const uint32_t kept_pages = a->kept_pages, page = a->page;
    const float eps = a->eps, theta = a->theta;
    TS_REQUIRE(qkv && q_gain && k_gain && q_out && k_cache && v_cache && slots && positions,
               "qk_norm_rope_append: null pointer");
    TS_REQUIRE(width == 128, "qk_norm_rope_append: head width %u (128 supported)", width);
    TS_REQUIRE(kv_heads >= 1 && heads % kv_heads == 0, "qk_norm_rope_append: %u heads over %u kv heads", heads,
               kv_heads);
    TS_REQUIRE(!kept_table || (page >= 1 && (page & (page - 1)) == 0), "qk_norm_rope_append: page %u", page);
    if (rows == 0) return TS_OK;
    QkParams p;
    p.qkv = qkv; p.q_gain = q_gain; p.k_gain = k_gain; p.q_out = q_out;
    p.k_cache = (uint16_t *)k_cache; p.v_cache = (uint16_t *)v_cache;
    p.slots = slots; p.positions = positions; p.table = kept_table;
    p.rows = rows; p.heads = heads; p.kv_heads = kv_heads; p.keys = keys; p.kept_pages = kept_pages;
    p.page_shift = kept_table ? (uint32_t)__builtin_ctz(page) : 0;
    p.eps = eps; p.theta = theta;
    const uint32_t waves = rows * (heads + 2 * kv_heads);
    hipLaunchKernelGGL(qk_norm_rope_append_kernel, dim3((waves + 3) / 4), dim3(256), 0, (hipStream_t)stream, p);
    TS_CHECK_LAUNCH("qk_norm_rope_append launch");
    return TS_OK;
}

extern "C" int tessera_hip_gather(const ts_gather_args *a, void *stream) {
    TS_REQUIRE(a, "gather: null args");
    const void *table = a->table;
    const uint32_t *ids = a->ids;
    float *out = a->out;
    const uint32_t count = a->count, table_rows = a->table_rows, width = a->width, first = a->first;
    TS_REQUIRE(table && ids && out, "gather: null pointer");
    if (count == 0 || width == 0) return TS_OK;
    TS_REQUIRE(count <= 65535, "gather: %u rows (at most 65535 per call)", count);
    hipLaunchKernelGGL(gather_kernel, dim3((width + 255) / 256, count), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t *)table, ids, out, count, table_rows, width, first);
    TS_CHECK_LAUNCH("gather launch");
    return TS_OK;
}

__global__ void argmax_keys_kernel(uint64_t *keys, uint32_t *ids, uint32_t rows, uint32_t width) {
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const uint64_t key = keys[r];
    ids[r] = key ? ~(uint32_t)key : width;
    keys[r] = 0;
}

extern "C" int tessera_hip_argmax_keys(const ts_keys_args *a, void *stream) {
    TS_REQUIRE(a, "argmax_keys: null args");
    uint64_t *keys = a->keys;
    uint32_t *ids = a->ids;
    const uint32_t rows = a->rows, width = a->width;
    TS_REQUIRE(keys && ids, "argmax_keys: null pointer");
    if (rows == 0) return TS_OK;
    hipLaunchKernelGGL(argmax_keys_kernel, dim3((rows + 255) / 256), dim3(256), 0, (hipStream_t)stream, keys, ids,
                       rows, width);
    TS_CHECK_LAUNCH("argmax_keys launch");
    return TS_OK;
}

extern "C" size_t tessera_hip_argmax_workspace(const ts_argmax_args *a) {
    if (!a) return 0;
    const uint32_t rows = a->rows, width = a->width;
    const size_t spans = (width + kSpan - 1) / kSpan;
    return (size_t)rows * spans * (sizeof(float) + sizeof(uint32_t));
}

extern "C" int tessera_hip_argmax(const ts_argmax_args *a, void *stream) {
    TS_REQUIRE(a, "argmax: null args");
    const float *x = a->x;
    uint32_t *ids = a->ids;
    const uint32_t rows = a->rows, width = a->width;
    void *workspace = a->workspace;
    const size_t workspace_bytes = a->workspace_bytes;
    TS_REQUIRE(x && ids, "argmax: null pointer");
    TS_REQUIRE(width >= 1, "argmax: width 0");
    if (rows == 0) return TS_OK;
    TS_REQUIRE(rows <= 65535, "argmax: %u rows (at most 65535)", rows);
    const size_t need = tessera_hip_argmax_workspace(a);
    if (!workspace || workspace_bytes < need)
        return ts::fail(TS_ERR_WORKSPACE, "argmax: workspace of %zu bytes needed", need);
    const uint32_t spans = (width + kSpan - 1) / kSpan;
    float *vals = (float *)workspace;
    uint32_t *idx = (uint32_t *)((char *)vals + (size_t)rows * spans * sizeof(float));
    hipLaunchKernelGGL(argmax_spans, dim3(spans, rows), dim3(256), 0, (hipStream_t)stream, x, vals, idx, rows,
                       width, spans);
    TS_CHECK_LAUNCH("argmax launch");
    hipLaunchKernelGGL(argmax_finish, dim3(rows), dim3(64), 0, (hipStream_t)stream, vals, idx, ids, spans, width);
    TS_CHECK_LAUNCH("argmax finish launch");
    return TS_OK;
}

extern "C" int tessera_hip_top_k(const ts_top_k_args *a, void *stream) {
    TS_REQUIRE(a, "top_k: null args");
    const float *x = a->x;
    uint32_t *ids = a->ids;
    const uint32_t rows = a->rows, width = a->width, k = a->k;
    TS_REQUIRE(x && ids, "top_k: null pointer");
    TS_REQUIRE(width >= 1 && width <= 1024, "top_k: width %u outside 1..1024", width);
    TS_REQUIRE(k >= 1 && k <= 1024, "top_k: k %u", k);
    if (rows == 0) return TS_OK;
    hipLaunchKernelGGL(top_k_kernel, dim3(rows), dim3(256), 0, (hipStream_t)stream, x, ids, rows, width, k);
    TS_CHECK_LAUNCH("top_k launch");
    return TS_OK;
}
