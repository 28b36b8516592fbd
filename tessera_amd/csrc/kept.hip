// Page copies of the kept rows: the copy-on-write step of the page pool.
//
// Pool::grow (engine/ir/kv/src/pool.rs:193-223) moves a run off a partial last page
// that another run still holds: the run gets a fresh page and a PageCopy {from, to,
// rows} whose rows must be copied "before the launch writes". This kernel makes
// those copies on the device for every kept-row buffer at once (the K and V of each
// layer), in stream order ahead of the launch that appends, so no host round trip
// and no per-layer launch is needed.
//
// gfx950 design: HBM-bound byte moves. One group per (copy, buffer); each thread
// moves 16-byte vectors, 256 threads cover 4 KiB per pass (a 16-row page of 8 kv
// heads x 128 bf16 is 32 KiB: 8 passes, all loads of a pass issued before its
// stores). Copies with a page or row count out of range, or whose pages overlap
// another copy's target, are skipped and reported in the status word.
#include "common.h"
#include "../../include/tessera_kv.h"

namespace {

struct CopyParams {
    void *const *buffers;
    const ts_kv_copy *copies;
    uint32_t buffer_count, copy_count, page, row_bytes, pages;
    uint32_t *status;
};

__global__ __launch_bounds__(256) void kv_copy_kernel(CopyParams p) {
    const uint32_t c = blockIdx.x / p.buffer_count, b = blockIdx.x % p.buffer_count;
    const ts_kv_copy cp = p.copies[c];
    bool bad = cp.from >= p.pages || cp.to >= p.pages || cp.rows > p.page ||
               (cp.from == cp.to && cp.rows > 0) || ((uintptr_t)p.buffers[b] & 15);
    // Copies of one call run at once: a page another copy reads or writes may not be
    // this copy's target, nor its source another's target (the result would depend
    // on timing). Both copies of such a pair are skipped and reported.
    for (uint32_t j = 0; j < p.copy_count; j++) {
        if (j == c) continue;
        const ts_kv_copy o = p.copies[j];
        bad |= o.to == cp.to || o.from == cp.to || o.to == cp.from;
    }
    if (bad || cp.rows == 0) {
        if (bad && threadIdx.x == 0 && p.status) atomicOr(p.status, TS_KV_STATUS_COPY);
        return;
    }
    const size_t page_bytes = (size_t)p.page * p.row_bytes;
    const u32x4 *src = (const u32x4 *)((const char *)p.buffers[b] + cp.from * page_bytes);
    u32x4 *dst = (u32x4 *)((char *)p.buffers[b] + cp.to * page_bytes);
    const uint32_t vecs = (uint32_t)(cp.rows * p.row_bytes / 16);
    constexpr uint32_t kPer = 4;  // vectors in flight per thread
    for (uint32_t i0 = 0; i0 < vecs; i0 += 256 * kPer) {
        u32x4 v[kPer];
#pragma unroll
        for (uint32_t j = 0; j < kPer; j++) {
            const uint32_t i = i0 + j * 256 + threadIdx.x;
            if (i < vecs) v[j] = src[i];
        }
#pragma unroll
        for (uint32_t j = 0; j < kPer; j++) {
            const uint32_t i = i0 + j * 256 + threadIdx.x;
            if (i < vecs) dst[i] = v[j];
        }
    }
}

}  // namespace

extern "C" int tessera_hip_kv_copy(const ts_kv_copy_args *a, void *stream) {
    TS_REQUIRE(a, "kv_copy: null arguments");
    if (a->copy_count == 0 || a->buffer_count == 0) return TS_OK;
    TS_REQUIRE(a->buffers && a->copies, "kv_copy: null pointer");
    TS_REQUIRE(a->page >= 1 && a->pages >= 1, "kv_copy: page %u, pages %u", a->page, a->pages);
    TS_REQUIRE(a->row_bytes >= 16 && a->row_bytes % 16 == 0, "kv_copy: row bytes %u (a multiple of 16)",
               a->row_bytes);
    TS_REQUIRE((uint64_t)a->copy_count * a->buffer_count <= 0x7fffffffu, "kv_copy: grid limits");
    CopyParams p;
    p.buffers = a->buffers; p.copies = a->copies; p.buffer_count = a->buffer_count; p.copy_count = a->copy_count;
    p.page = a->page; p.row_bytes = a->row_bytes; p.pages = a->pages; p.status = a->status;
    hipLaunchKernelGGL(kv_copy_kernel, dim3(a->copy_count * a->buffer_count), dim3(256), 0, (hipStream_t)stream, p);
    TS_CHECK_LAUNCH("kv_copy launch");
    return TS_OK;
}
