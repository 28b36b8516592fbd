/*
 * tessera_kv: the page pool behind paged kept rows (host side, C ABI).
 *
 * Replaces: tessera-kv's Pool (engine/ir/kv/src/pool.rs:71-450). Same calls,
 * same page order (lowest free page first; retained runs are evicted oldest
 * first), same copy-on-write of a shared partial last page, same refusals, and
 * every refusal leaves the pool unchanged. The pages a run holds become the
 * rows of its slot in the kept-row page table that the attention kernels read
 * (table[slot * kept_pages + i] = pages[i]).
 *
 * Not thread-safe: one pool per scheduler thread, as in the reference.
 */
#ifndef TESSERA_KV_H
#define TESSERA_KV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes (pool.rs:25-40 Error variants). The payload of the last refusal
 * is tessera_kv_error_value(): NoRoom -> pages needed; PastWorst -> rows (and
 * tessera_kv_error_value2() -> worst); PastSource -> source rows. */
enum {
    TS_KV_OK = 0,
    TS_KV_NO_ROOM = 1,
    TS_KV_PAST_WORST = 2,
    TS_KV_PAST_SOURCE = 3,
    TS_KV_LIVE = 4,
    TS_KV_RETAINED = 5,
    TS_KV_UNKNOWN = 6,
};

typedef struct ts_kv_pool ts_kv_pool;

/* A run's place in the pool; stale ids fail with TS_KV_UNKNOWN (pool.rs:7-11). */
typedef struct {
    uint32_t at;
    uint32_t generation;
} ts_kv_run;

/* Rows to copy between pages before the launch writes (pool.rs:17-22). */
typedef struct {
    uint32_t from;
    uint32_t to;
    uint64_t rows;
} ts_kv_copy;

/* pool.rs:55-66. */
typedef struct {
    uint64_t size, active, worst, live_runs, kept_runs;
} ts_kv_stats;

/* Pool::new (pool.rs:83-93). */
ts_kv_pool *tessera_kv_new(uint32_t pages, uint32_t page);
void tessera_kv_free(ts_kv_pool *p);

/* Pool::reserve (pool.rs:140-155). */
int tessera_kv_reserve(ts_kv_pool *p, uint64_t tag, uint64_t rows, uint64_t worst, ts_kv_run *out);
/* Pool::fork (pool.rs:157-191). */
int tessera_kv_fork(ts_kv_pool *p, ts_kv_run source, uint64_t rows, uint64_t worst, ts_kv_run *out);
/* Pool::grow (pool.rs:193-223): at most one copy, written to *copy when *n_copies is 1. */
int tessera_kv_grow(ts_kv_pool *p, ts_kv_run run, uint64_t rows, ts_kv_copy *copy, uint32_t *n_copies);
/* Pool::truncate (pool.rs:225-245). */
int tessera_kv_truncate(ts_kv_pool *p, ts_kv_run run, uint64_t rows);
/* Pool::retain (pool.rs:247-260). */
int tessera_kv_retain(ts_kv_pool *p, ts_kv_run run);
/* Pool::adopt (pool.rs:262-293). */
int tessera_kv_adopt(ts_kv_pool *p, ts_kv_run run, uint64_t rows, uint64_t worst, ts_kv_run *out);
/* Pool::release (pool.rs:295-301). */
int tessera_kv_release(ts_kv_pool *p, ts_kv_run run);

/* Pool::pages / rows / tag (pool.rs:95-105). *pages stays valid until the next call. */
int tessera_kv_pages(const ts_kv_pool *p, ts_kv_run run, const uint32_t **pages, uint32_t *count);
int tessera_kv_rows(const ts_kv_pool *p, ts_kv_run run, uint64_t *rows);
int tessera_kv_tag(const ts_kv_pool *p, ts_kv_run run, uint64_t *tag);

/* Pool::spare / promised / stats / digest (pool.rs:107-138, 304-322). */
uint64_t tessera_kv_spare(const ts_kv_pool *p);
uint64_t tessera_kv_promised(const ts_kv_pool *p);
void tessera_kv_get_stats(const ts_kv_pool *p, ts_kv_stats *out);
uint64_t tessera_kv_digest(const ts_kv_pool *p);
/* Pool::consistent (pool.rs:432-449): 1 when holder counts, the free set and every promise agree. */
int tessera_kv_consistent(const ts_kv_pool *p);

uint64_t tessera_kv_error_value(const ts_kv_pool *p);
uint64_t tessera_kv_error_value2(const ts_kv_pool *p);

/* ----------------------------------------------------------------------------
 * Device side: the copies Pool::grow asks for, made on the GPU.
 * ------------------------------------------------------------------------- */

/* Status bit (ORed into ts_kv_copy_args.status): a copy named a page >= pages, more
 * rows than a page, a page onto itself, a buffer not 16-byte aligned, or a target page
 * that another copy of the same call reads or writes (copies run at once); it was
 * skipped. */
#define TS_KV_STATUS_COPY 2u

typedef struct {
    void *const *buffers;      /* device array [buffer_count] of kept-row buffers (e.g. K and V of each layer),
                                  each [pages * page, row_bytes] */
    const ts_kv_copy *copies;  /* device array [copy_count], as Pool::grow returned them */
    uint32_t buffer_count, copy_count;
    uint32_t page;             /* rows per page */
    uint32_t row_bytes;        /* bytes of one kept row (kv_heads * width * 2 for bf16), a multiple of 16 */
    uint32_t pages;            /* pages each buffer holds */
    uint32_t *status;          /* device word or NULL */
} ts_kv_copy_args;

/* Rows [0, rows) of page `from` to page `to` in every buffer, for every copy, stream
 * ordered before the launch that appends (one launch, no host round trip; graph
 * capturable). Copies of one call must not overlap each other's pages.
 * Replaces: the "make the copies before the launch" step of Pool::grow
 * (engine/ir/kv/src/pool.rs:193-223); the reference's engine refuses grows that need
 * a copy (engine/engine/src/kept.rs:127-141) and uploads only the table
 * (engine/engine/src/lanes.rs:60-66). */
int tessera_hip_kv_copy(const ts_kv_copy_args *a, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TESSERA_KV_H */
