// Routing for picked products (the MoE layer), and the small row stages around it.
//
// The reference computes a picked product one thread per output element, each row
// on the matrix its id names (engine/rules/linear/src/picked.rs:28-60; interp
// matmul_picked, engine/ir/interp/src/cpu.rs:89-105). Here the rows are first sorted
// by matrix with a stable counting sort (bit-exact: the order inside a matrix is the
// row order), so each matrix's rows run through the matrix unit as dense row tiles
// against one read of that matrix (the PICK mode of the tiled kernel).
//
// Sort layout in the caller's workspace (u32 words), B = count + 1 buckets (the
// last holds rows whose id is outside this rank's matrices; they read zeros):
//   offs[chunks][B]   per 256-row chunk, the first sorted position of its rows in
//                     each bucket (counts, then turned into positions in place)
//   row_start[B + 1]  first sorted position of each bucket; row_start[B] = rows
//   tile_start[count + 1]  first row tile of each matrix; tile_start[count] = total
//   perm[rows]        perm[pos] = the row at sorted position pos
#include "after.h"

namespace ts {

namespace {

constexpr uint32_t kChunk = 256;  // rows per sort chunk (one group)
constexpr uint32_t kScan = 1024;  // threads of the single scan group

TS_DEV uint32_t bucket_of(uint32_t id, uint32_t first, uint32_t count) {
    return (id >= first && id - first < count) ? id - first : count;
}

__global__ __launch_bounds__(kChunk) void route_count(const uint32_t *ids, uint32_t rows, uint32_t first,
                                                      uint32_t count, uint32_t *offs) {
    extern __shared__ uint32_t hist[];
    const uint32_t B = count + 1;
    for (uint32_t b = threadIdx.x; b < B; b += kChunk) hist[b] = 0;
    __syncthreads();
    const uint32_t r = blockIdx.x * kChunk + threadIdx.x;
    if (r < rows) atomicAdd(&hist[bucket_of(ids[r], first, count)], 1u);
    __syncthreads();
    for (uint32_t b = threadIdx.x; b < B; b += kChunk) offs[(size_t)blockIdx.x * B + b] = hist[b];
}

// Exclusive scan of per-thread segment sums held in part[kScan] (in place).
TS_DEV void scan_parts(uint32_t *part) {
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t s = 0;
        for (uint32_t i = 0; i < kScan; i++) {
            const uint32_t v = part[i];
            part[i] = s;
            s += v;
        }
    }
    __syncthreads();
}

// One group: per bucket, chunk counts -> positions within the bucket; bucket totals
// -> row_start; row tiles per matrix -> tile_start; then positions made absolute.
__global__ __launch_bounds__(kScan) void route_scan(uint32_t *offs, uint32_t chunks, uint32_t rows, uint32_t count,
                                                    uint32_t tile_rows, uint32_t *row_start, uint32_t *tile_start) {
    __shared__ uint32_t part[kScan], tpart[kScan];
    const uint32_t B = count + 1, t = threadIdx.x;
    const uint32_t per = (B + kScan - 1) / kScan, b0 = t * per, b1 = min(B, b0 + per);
    // Totals of this thread's buckets (each bucket's chunk prefix in place). The
    // counts are loaded 16 at a time before any is rewritten: a load after a store to
    // the same array would otherwise wait for the store, one memory round trip per chunk.
    constexpr uint32_t kBatch = 16;
    uint32_t seg = 0, tseg = 0;
    for (uint32_t b = b0; b < b1; b++) {
        uint32_t s = 0;
        for (uint32_t c0 = 0; c0 < chunks; c0 += kBatch) {
            uint32_t v[kBatch];
#pragma unroll
            for (uint32_t i = 0; i < kBatch; i++) v[i] = c0 + i < chunks ? offs[(size_t)(c0 + i) * B + b] : 0u;
#pragma unroll
            for (uint32_t i = 0; i < kBatch; i++)
                if (c0 + i < chunks) {
                    offs[(size_t)(c0 + i) * B + b] = s;
                    s += v[i];
                }
        }
        row_start[b] = s;  // total for now
        seg += s;
        tseg += b < count ? (s + tile_rows - 1) / tile_rows : 0;
    }
    part[t] = seg;
    tpart[t] = tseg;
    scan_parts(part);
    scan_parts(tpart);
    uint32_t base = part[t], tbase = tpart[t];
    for (uint32_t b = b0; b < b1; b++) {
        const uint32_t tot = row_start[b];
        row_start[b] = base;
        for (uint32_t c0 = 0; c0 < chunks; c0 += kBatch) {
            uint32_t v[kBatch];
#pragma unroll
            for (uint32_t i = 0; i < kBatch; i++) v[i] = c0 + i < chunks ? offs[(size_t)(c0 + i) * B + b] : 0u;
#pragma unroll
            for (uint32_t i = 0; i < kBatch; i++)
                if (c0 + i < chunks) offs[(size_t)(c0 + i) * B + b] = v[i] + base;
        }
        if (b < count) {
            tile_start[b] = tbase;
            tbase += (tot + tile_rows - 1) / tile_rows;
        }
        base += tot;
    }
    if (t == kScan - 1) {
        row_start[B] = rows;
        tile_start[count] = tbase;
    }
}

// Inclusive prefix sum over the 64 lanes of a wave.
TS_DEV uint32_t wave_scan(uint32_t v, uint32_t lane) {
#pragma unroll
    for (uint32_t d = 1; d < 64; d <<= 1) {
        const uint32_t u = __shfl_up(v, d, 64);
        if (lane >= d) v += u;
    }
    return v;
}

// route_scan for up to kFastChunks chunks and kFastBuckets buckets, one coalesced
// load and one coalesced store of the counts: wave w takes chunks [kFastCW w, +kFastCW)
// with lane l on buckets l, l + 64, ... (the [chunk][bucket] layout's contiguous
// direction); the waves' sums per bucket are scanned over the waves in LDS, one
// wave scans the bucket totals and row tiles, and every wave stores absolute
// positions.
constexpr uint32_t kFastWaves = kScan / 64, kFastCW = 8, kFastBS = 5;
constexpr uint32_t kFastChunks = kFastWaves * kFastCW, kFastBuckets = 64 * kFastBS;
__global__ __launch_bounds__(kScan) void route_scan_fast(uint32_t *offs, uint32_t chunks, uint32_t rows,
                                                         uint32_t count, uint32_t tile_rows, uint32_t *row_start,
                                                         uint32_t *tile_start) {
    __shared__ uint32_t wsum[kFastWaves][kFastBuckets], tot_s[kFastBuckets], base_s[kFastBuckets];
    const uint32_t B = count + 1, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t v[kFastBS][kFastCW];
#pragma unroll
    for (uint32_t j = 0; j < kFastBS; j++) {
        const uint32_t b = 64 * j + lane;
#pragma unroll
        for (uint32_t i = 0; i < kFastCW; i++) {
            const uint32_t c = kFastCW * wave + i;
            v[j][i] = b < B && c < chunks ? offs[(size_t)c * B + b] : 0u;
        }
    }
#pragma unroll
    for (uint32_t j = 0; j < kFastBS; j++) {
        uint32_t sum = 0;
#pragma unroll
        for (uint32_t i = 0; i < kFastCW; i++) sum += v[j][i];
        wsum[wave][64 * j + lane] = sum;
    }
    __syncthreads();
    if (threadIdx.x < B) {  // one thread a bucket: the waves' sums, exclusive, in wave order
        const uint32_t b = threadIdx.x;
        uint32_t run = 0;
        for (uint32_t w = 0; w < kFastWaves; w++) {
            const uint32_t x = wsum[w][b];
            wsum[w][b] = run;
            run += x;
        }
        tot_s[b] = run;
    }
    __syncthreads();
    if (wave == 0) {
        constexpr uint32_t kPer = kFastBS;  // consecutive buckets a lane
        uint32_t rs = 0, ts = 0;
        for (uint32_t i = 0; i < kPer; i++) {
            const uint32_t b = lane * kPer + i;
            if (b < B) {
                rs += tot_s[b];
                ts += b < count ? (tot_s[b] + tile_rows - 1) / tile_rows : 0;
            }
        }
        uint32_t rb = wave_scan(rs, lane) - rs, tb = wave_scan(ts, lane) - ts;
        for (uint32_t i = 0; i < kPer; i++) {
            const uint32_t b = lane * kPer + i;
            if (b < B) {
                base_s[b] = rb;
                row_start[b] = rb;
                if (b < count) tile_start[b] = tb;
                rb += tot_s[b];
                tb += b < count ? (tot_s[b] + tile_rows - 1) / tile_rows : 0;
            }
        }
        if (lane == 63) {
            row_start[B] = rows;
            tile_start[count] = tb;
        }
    }
    __syncthreads();
#pragma unroll
    for (uint32_t j = 0; j < kFastBS; j++) {
        const uint32_t b = 64 * j + lane;
        if (b >= B) continue;
        uint32_t at = base_s[b] + wsum[wave][b];
#pragma unroll
        for (uint32_t i = 0; i < kFastCW; i++) {
            const uint32_t c = kFastCW * wave + i;
            if (c < chunks) offs[(size_t)c * B + b] = at;
            at += v[j][i];
        }
    }
}

// Stable placement: a row's position is its chunk's first position in its bucket
// plus the rows of the same bucket before it in the chunk.
__global__ __launch_bounds__(kChunk) void route_place(const uint32_t *ids, uint32_t rows, uint32_t first,
                                                      uint32_t count, const uint32_t *offs, uint32_t *perm) {
    __shared__ uint32_t bk[kChunk];
    const uint32_t t = threadIdx.x, r = blockIdx.x * kChunk + t;
    const uint32_t b = r < rows ? bucket_of(ids[r], first, count) : 0xffffffffu;
    bk[t] = b;
    __syncthreads();
    if (r >= rows) return;
    uint32_t rank = 0;
    for (uint32_t j = 0; j < t; j++) rank += bk[j] == b;
    perm[offs[(size_t)blockIdx.x * (count + 1) + b] + rank] = r;
}

// Rows whose id is outside this rank's matrices read zeros (cpu.rs:100-102).
__global__ __launch_bounds__(256) void zero_absent(const uint32_t *perm, const uint32_t *row_start, uint32_t count,
                                                   void *out, uint32_t n, int out_bf16, ts_after after) {
    const uint32_t from = row_start[count], to = row_start[count + 1];
    const uint64_t total = (uint64_t)(to - from) * n;
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < total; i += (uint64_t)gridDim.x * 256) {
        const uint32_t pos = from + (uint32_t)(i / n), col = (uint32_t)(i % n);
        const size_t at = (size_t)perm[pos] * n + col;
        const float v = after.count ? after_apply(after, 0.0f, at) : 0.0f;
        if (out_bf16) ((uint16_t *)out)[at] = bf16_bits(v);
        else ((float *)out)[at] = v;
    }
}

// take (cpu.rs:498-508): out[j] = x[j / picks][ids[j]], zero out of range.
__global__ __launch_bounds__(256) void take_kernel(const float *x, const uint32_t *ids, float *out, uint32_t rows,
                                                   uint32_t width, uint32_t picks) {
    const uint64_t j = blockIdx.x * 256ull + threadIdx.x;
    if (j >= (uint64_t)rows * picks) return;
    const uint32_t id = ids[j];
    out[j] = id < width ? x[(j / picks) * width + id] : 0.0f;
}

// softmax (cpu.rs:49-59): max by f32::max from -inf (NaN ignored), exp(v - max),
// sequential sum, divide. One thread per row, in the reference's order.
__global__ __launch_bounds__(256) void softmax_kernel(const float *x, float *out, uint32_t rows, uint32_t width) {
#pragma clang fp contract(off)
    const uint32_t r = blockIdx.x * 256 + threadIdx.x;
    if (r >= rows) return;
    const float *row = x + (size_t)r * width;
    float *o = out + (size_t)r * width;
    float mx = -INFINITY;
    for (uint32_t i = 0; i < width; i++) mx = fmaxf(mx, row[i]);
    float sum = 0.0f;
    for (uint32_t i = 0; i < width; i++) {
        const float v = expf(row[i] - mx);
        o[i] = v;
        sum = sum + v;
    }
    for (uint32_t i = 0; i < width; i++) o[i] = o[i] / sum;
}

// mix / weighted mean (cpu.rs:450-473): out[o, i] = sum_t x[o, t, i] * w[o, t], in t
// order from 0, each product rounded before the add (no fused multiply-add).
// Four adjacent columns a thread (16-byte loads, every pick's load issued before the
// adds) when inner is a multiple of 4 and the buffers 16-byte aligned.
__global__ __launch_bounds__(256) void mix4_kernel(const float *x, const float *w, float *out, uint32_t outer,
                                                   uint32_t count, uint32_t inner) {
#pragma clang fp contract(off)  // the reference rounds each product before the add
    const uint32_t q = inner / 4;
    const uint64_t j = blockIdx.x * 256ull + threadIdx.x;
    if (j >= (uint64_t)outer * q) return;
    const uint32_t o = (uint32_t)(j / q), i = (uint32_t)(j % q) * 4;
    const float even = 1.0f / (float)count;
    float4 s = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    constexpr uint32_t kB = 8;  // picks in flight
    for (uint32_t t0 = 0; t0 < count; t0 += kB) {
        float4 v[kB];
#pragma unroll
        for (uint32_t u = 0; u < kB; u++)
            if (t0 + u < count) v[u] = *(const float4 *)(x + ((size_t)o * count + t0 + u) * inner + i);
#pragma unroll
        for (uint32_t u = 0; u < kB; u++)
            if (t0 + u < count) {
                const float wt = w ? w[(size_t)o * count + t0 + u] : even;
                s.x = s.x + v[u].x * wt;
                s.y = s.y + v[u].y * wt;
                s.z = s.z + v[u].z * wt;
                s.w = s.w + v[u].w * wt;
            }
    }
    *(float4 *)(out + (size_t)o * inner + i) = s;
}

__global__ __launch_bounds__(256) void mix_kernel(const float *x, const float *w, float *out, uint32_t outer,
                                                  uint32_t count, uint32_t inner) {
#pragma clang fp contract(off)  // the reference rounds each product before the add
    const uint64_t j = blockIdx.x * 256ull + threadIdx.x;
    if (j >= (uint64_t)outer * inner) return;
    const uint32_t o = (uint32_t)(j / inner), i = (uint32_t)(j % inner);
    const float even = 1.0f / (float)count;
    float s = 0.0f;
    for (uint32_t t = 0; t < count; t++) {
        const float wt = w ? w[(size_t)o * count + t] : even;
        const float prod = x[((size_t)o * count + t) * inner + i] * wt;
        s = s + prod;
    }
    out[j] = s;
}

}  // namespace

size_t route_words(uint32_t rows, uint32_t count) {
    const size_t chunks = (rows + kChunk - 1) / kChunk, B = (size_t)count + 1;
    return chunks * B + (B + 1) + ((size_t)count + 1) + rows;
}

int route_launch(const uint32_t *ids, uint32_t rows, uint32_t first, uint32_t count, uint32_t tile_rows, void *ws,
                 Route *route, void *stream) {
    const uint32_t chunks = (rows + kChunk - 1) / kChunk, B = count + 1;
    uint32_t *offs = (uint32_t *)ws;
    route->row_start = offs + (size_t)chunks * B;
    route->tile_start = route->row_start + (B + 1);
    route->perm = route->tile_start + (count + 1);
    const hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(route_count, dim3(chunks), dim3(kChunk), B * sizeof(uint32_t), s, ids, rows, first, count,
                       offs);
    if (chunks <= kFastChunks && B <= kFastBuckets)
        hipLaunchKernelGGL(route_scan_fast, dim3(1), dim3(kScan), 0, s, offs, chunks, rows, count, tile_rows,
                           route->row_start, route->tile_start);
    else
        hipLaunchKernelGGL(route_scan, dim3(1), dim3(kScan), 0, s, offs, chunks, rows, count, tile_rows,
                           route->row_start, route->tile_start);
    hipLaunchKernelGGL(route_place, dim3(chunks), dim3(kChunk), 0, s, ids, rows, first, count, offs, route->perm);
    TS_CHECK_LAUNCH("picked routing");
    return TS_OK;
}

int zero_absent_launch(const Route &route, uint32_t count, void *out, uint32_t n, int out_bf16, const ts_after &after,
                       void *stream) {
    hipLaunchKernelGGL(zero_absent, dim3(64), dim3(256), 0, (hipStream_t)stream, route.perm, route.row_start, count,
                       out, n, out_bf16, after);
    TS_CHECK_LAUNCH("picked zero rows");
    return TS_OK;
}

}  // namespace ts

extern "C" int tessera_hip_take(const ts_take_args *a, void *stream) {
    TS_REQUIRE(a, "take: null args");
    const float *x = a->x;
    const uint32_t *ids = a->ids;
    float *out = a->out;
    const uint32_t rows = a->rows, width = a->width, picks = a->picks;
    TS_REQUIRE(x && ids && out, "take: null pointer");
    const uint64_t total = (uint64_t)rows * picks;
    if (total == 0) return TS_OK;
    TS_REQUIRE(total < (1ull << 40), "take: %llu entries", (unsigned long long)total);
    hipLaunchKernelGGL(ts::take_kernel, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, x,
                       ids, out, rows, width, picks);
    TS_CHECK_LAUNCH("take launch");
    return TS_OK;
}

extern "C" int tessera_hip_softmax(const ts_softmax_args *a, void *stream) {
    TS_REQUIRE(a, "softmax: null args");
    const float *x = a->x;
    float *out = a->out;
    const uint32_t rows = a->rows, width = a->width;
    TS_REQUIRE(x && out, "softmax: null pointer");
    TS_REQUIRE(width >= 1 && width <= 4096, "softmax: width %u (routing widths, 1..4096)", width);
    if (rows == 0) return TS_OK;
    hipLaunchKernelGGL(ts::softmax_kernel, dim3((rows + 255) / 256), dim3(256), 0, (hipStream_t)stream, x, out, rows,
                       width);
    TS_CHECK_LAUNCH("softmax launch");
    return TS_OK;
}

extern "C" int tessera_hip_mix(const ts_mix_args *a, void *stream) {
    TS_REQUIRE(a, "mix: null args");
    const float *x = a->x, *weights = a->weights;
    float *out = a->out;
    const uint32_t outer = a->outer, count = a->count, inner = a->inner;
    TS_REQUIRE(x && out, "mix: null pointer");
    TS_REQUIRE(count >= 1, "mix: count 0");
    const uint64_t total = (uint64_t)outer * inner;
    if (total == 0) return TS_OK;
    if (inner % 4 == 0 && ts::aligned(x, 16) && ts::aligned(out, 16)) {
        const uint64_t quads = total / 4;
        hipLaunchKernelGGL(ts::mix4_kernel, dim3((uint32_t)((quads + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                           x, weights, out, outer, count, inner);
    } else {
        hipLaunchKernelGGL(ts::mix_kernel, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                           x, weights, out, outer, count, inner);
    }
    TS_CHECK_LAUNCH("mix launch");
    return TS_OK;
}
