/*
 * libtessera_hip: gfx950 (MI355X) kernels for tessera's matmul and attention
 * hot path, behind a plain C ABI.
 *
 * Conventions (all entry points):
 *  - Every pointer is a device pointer unless stated; the caller owns all
 *    memory. No entry point allocates, frees, copies to/from the host or
 *    synchronizes: each only enqueues kernels on `stream` (a hipStream_t, NULL
 *    for the null stream), so every call may be captured into a HIP graph.
 *  - Scratch (split-K / split-KV partials) comes from a caller-owned
 *    `workspace` of at least the bytes the matching *_workspace() call reports.
 *    It carries nothing between calls (no counters, no state), so one
 *    workspace serves any sequence of stream-ordered calls; calls that run
 *    concurrently (different streams) need separate workspaces.
 *  - Return 0 on success; a positive value is a passed-through hipError_t; a
 *    negative value is an argument error (TS_ERR_*). The message for the last
 *    failure on the calling thread is tessera_hip_last_error(). Nothing aborts.
 *  - Argument order inside each struct follows the reference Launch order:
 *    the step's reads, epilogue operands, the output, then the u32 counts.
 */
#ifndef TESSERA_HIP_H
#define TESSERA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TS_OK 0
#define TS_ERR_ARG (-1)       /* unsupported shape, dtype, alignment or null pointer */
#define TS_ERR_ARCH (-2)      /* the current device is not gfx950 */
#define TS_ERR_WORKSPACE (-3) /* workspace missing or too small */

/* Storage types (engine/ir/mem/src/form.rs forms used on this path). The block forms
 * (engine/ir/mem/src/block.rs:251-291) hold the [n, k] weights as one packed tensor:
 * an optional 4-byte f32 head, then k/B blocks per row, each one scale then B codes,
 * rows back to back (k a multiple of 4 B and at least 128); w_scale is unused:
 *   TS_Q8_0       34 B a block: f16 scale, 32 signed bytes
 *   TS_MXFP8      33 B a block: e8m0 scale, 32 e4m3 codes
 *   TS_INT4_G32   18 B a block: f16 scale, 32 nibbles (code - 8), element 2q low, 2q+1 high
 *   TS_Q4_0       18 B a block: f16 scale, 32 nibbles (code - 8), element q low, q+16 high
 *   TS_NVFP4       9 B a block: e4m3 scale, 16 e2m1 nibbles (2q low, 2q+1 high); f32 head
 *   TS_MXFP4      17 B a block: e8m0 scale, 32 e2m1 nibbles (2q low, 2q+1 high)
 *   TS_INT4_G128  66 B a block: f16 scale, 128 nibbles (code - 8), 2q low, 2q+1 high
 * tessera_hip_lanes / tessera_hip_linear / tessera_hip_tiled accept them at any m. */
enum { TS_F32 = 0, TS_BF16 = 1, TS_E4M3 = 2, TS_U32 = 3, TS_Q8_0 = 4, TS_MXFP8 = 5, TS_INT4_G32 = 6,
       TS_Q4_0 = 7, TS_NVFP4 = 8, TS_MXFP4 = 9, TS_INT4_G128 = 10, TS_F32_PARTS = 11 };
/* TS_F32_PARTS: f32 weights as tessera_hip_pack_f32 lays them out, [2n, k] bf16: rows
 * 0..n-1 the high parts bf16(w), rows n..2n-1 the low parts bf16(w - bf16(w)) (w to
 * about 16 significant bits, every part exact on the matrix unit); the product sums
 * x . hi + x . lo. Not with TS_AFTER_SILU_MUL, not for picked products. */

/* Fused stages around a product (engine/plan/lower/src/kernels/map.rs:20-59 MapStage,
 * applied by `finish` at the store, map.rs:155-185). */
#define TS_AFTER_ADD 1u       /* out = sum + a0[m, n] (the residual add; a0 may alias out) */
#define TS_AFTER_SILU_MUL 2u  /* w holds 2n rows, gate rows then up rows; out = silu(g) * u */
#define TS_BEFORE_RMS_NORM 4u /* x rows pass through RmsNorm with `gain` before the product */
#define TS_AFTER_ARGMAX 8u    /* m <= 4, f32 out, no SiLU pair: out as usual, and each row's
                                 greedy pick folded into workspace key[m] (uint64; zero before
                                 the launch): tessera_hip_argmax_keys reads and clears them */

/* A general chain of elementwise stages, run on a product's sum before its store or
 * over an input by tessera_hip_map (engine/plan/lower/src/kernels/map.rs:40-59 MapStage,
 * applied at the store by `finish`, map.rs:155-185; the Finished site,
 * engine/plan/lower/src/sites/matmul.rs:117-200). The chain reads 1 + (its Add and Mul
 * stages) values: read 0 starts v, and each Add / Mul stage reads the next one. Read
 * `sum` is the product's sum (tessera_hip_map: its input x); the others are
 * operand[0], operand[1], ... in order. Each stage is one f32 operation rounded on its
 * own (no fused multiply-add), as the interpreter evaluates Stage::Add / Mul / Scale /
 * Act (engine/ir/interp/src/cpu.rs:8-29,353-390):
 *   TS_MAP_ADD    v = v + next read        TS_MAP_SCALE  v = v * by
 *   TS_MAP_MUL    v = v * next read        TS_MAP_ACT    v = act(v), act = TS_ACT_*
 * Activations (cpu.rs:8-29): GeluTanh 0.5 x (1 + tanh(0.7978846 (x + 0.044715 x^3))),
 * Silu x / (1 + e^-x), Sigmoid 1 / (1 + e^-x), Relu max(x, 0), Softplus
 * max(x, 0) + log1p(e^-|x|), Exp e^x, Tanh tanh x. */
#define TS_MAP_STAGES 8
#define TS_MAP_OPERANDS 4
enum { TS_MAP_ADD = 0, TS_MAP_MUL = 1, TS_MAP_SCALE = 2, TS_MAP_ACT = 3 };
enum { TS_ACT_GELU_TANH = 0, TS_ACT_SILU = 1, TS_ACT_SIGMOID = 2, TS_ACT_RELU = 3, TS_ACT_SOFTPLUS = 4,
       TS_ACT_EXP = 5, TS_ACT_TANH = 6 };
typedef struct {
    int32_t op;   /* TS_MAP_* */
    int32_t act;  /* TS_ACT_*, TS_MAP_ACT only */
    float by;     /* TS_MAP_SCALE only */
} ts_map_stage;
typedef struct {
    const float *operand[TS_MAP_OPERANDS]; /* f32, as long as the output (a product's [m, n]) */
    uint32_t spans[TS_MAP_OPERANDS];       /* tessera_hip_map only: 0 = as long as x; s > 0: operand j
                                              is read at i % s (1: a scalar). Products need 0 (the
                                              Finished site refuses repeating operands) */
    uint32_t count;                        /* stages, <= TS_MAP_STAGES */
    uint32_t sum;                          /* which read is the sum (or x), <= operands */
    ts_map_stage stage[TS_MAP_STAGES];
} ts_after;

/* Version of this ABI; bumped on any struct layout change. */
#define TS_ABI_VERSION 4

/* Checks that the current device is gfx950 and records its properties.
 * Replaces: the platform probe of engine/gpu/gpukit/src/rocm/context.rs:60-106
 * (arch, lanes, group bytes). */
int tessera_hip_init(void);

/* Thread-local text of the last failure.
 * Replaces: Runtime::check's error text, engine/gpu/gpukit/src/rocm/hip.rs:98-106. */
const char *tessera_hip_last_error(void);

int tessera_hip_abi_version(void);

/* ----------------------------------------------------------------------------
 * Linear: out[m, n] = after(sum_k before(x)[m, k] * w[n, k])
 * x: [m, k] f32 or bf16 (f32 is split into two exact bf16 parts on the matrix
 * unit, as the reference's tiled_parts splits f32 rows into bf16 slabs).
 * w: [n, k] bf16, or e4m3 with a bf16 scale per output row (w_scale [n]).
 * out: [m, n] f32 or bf16.
 * ------------------------------------------------------------------------- */
typedef struct {
    const void *x;        /* [m, k] */
    const void *w;        /* [n, k], or [2n, k] with TS_AFTER_SILU_MUL */
    const void *w_scale;  /* [n] (or [2n]) bf16, e4m3 weights only */
    const float *gain;    /* [k] f32, TS_BEFORE_RMS_NORM only */
    const float *a0;      /* [m, n] f32, TS_AFTER_ADD only; may alias out */
    void *out;            /* [m, n] */
    void *workspace;
    size_t workspace_bytes;
    uint32_t m, n, k;
    int32_t x_dtype, w_dtype, out_dtype;
    uint32_t stages;      /* TS_AFTER_* | TS_BEFORE_* bits */
    float eps;            /* RmsNorm epsilon */
    const ts_after *after; /* host struct or NULL: a stage chain on the sum (after the SiLU pair
                              when TS_AFTER_SILU_MUL is set); not with TS_AFTER_ADD / ARGMAX */
} ts_linear_args;

/* Picks `lanes` for m <= 64 and `tiled` otherwise (the cost select of
 * engine/plan/lower/src/cost.rs between the two rules). */
int tessera_hip_linear(const ts_linear_args *a, void *stream);
size_t tessera_hip_linear_workspace(const ts_linear_args *a);

/* Few rows (m <= 64): m <= 4 on the vector ALU (a wave streams whole weight
 * rows; block-form weights decode there too, bit-identical to the reference's
 * Block::dot, engine/ir/mem/src/block.rs:202-219); 5..64 on the matrix unit: a wave per 16 output columns, x staged once
 * per group in LDS, weights streamed once with 64-byte runs per lane, k split
 * across groups when the columns alone do not cover the chip (partials in the
 * workspace, summed in split order by a second kernel: deterministic).
 * TS_BEFORE_RMS_NORM needs f32 x and m <= 16.
 * Replaces: rule "lanes" (engine/rules/linear/src/lanes.rs:17-143) and "thin"
 * (engine/rules/linear/src/thin.rs:11-104). */
int tessera_hip_lanes(const ts_linear_args *a, void *stream);
size_t tessera_hip_lanes_workspace(const ts_linear_args *a);

/* Many rows: LDS-staged, double-buffered MFMA tiles.
 * Replaces: rule "tiled" (engine/rules/linear/src/tiled.rs:281-345,441-453,611-672)
 * including tiled_parts (tiled.rs:43-49,186-278). */
int tessera_hip_tiled(const ts_linear_args *a, void *stream);

/* ----------------------------------------------------------------------------
 * Picked: row r multiplies matrix ids[r] - first of a stored set (the MoE expert
 * products). out[r, c] = sum_k x[r / repeat, k] * w[ids[r] - first][offset + c, k];
 * rows whose id is outside [first, first + count) read zeros.
 * w: [count, stride, k] bf16, or e4m3 with a bf16 scale per stored row
 * (w_scale [count, stride]). With TS_AFTER_SILU_MUL the matrix rows offset..
 * offset+n are the gates and offset+n..offset+2n the ups: out = silu(g) * u.
 * x: [rows / repeat, k] f32 or bf16; out: [rows, n] f32 or bf16.
 * Rows are sorted by matrix (a stable counting sort, in the workspace), then each
 * matrix's rows run as dense MFMA row tiles against one read of its weights.
 * ------------------------------------------------------------------------- */
typedef struct {
    const void *x;        /* [rows / repeat, k] */
    const void *w;        /* [count, stride, k] */
    const void *w_scale;  /* [count, stride] bf16, e4m3 weights only */
    const uint32_t *ids;  /* [rows] */
    void *out;            /* [rows, n] */
    void *workspace;
    size_t workspace_bytes;
    uint32_t rows, n, k;
    uint32_t count;       /* matrices of the set held here */
    uint32_t stride;      /* rows per stored matrix */
    uint32_t offset;      /* first matrix row used */
    uint32_t repeat;      /* consecutive rows sharing one x row (the picks per token) */
    uint32_t first;       /* id of this set's first matrix */
    int32_t x_dtype, w_dtype, out_dtype;
    uint32_t stages;      /* 0 or TS_AFTER_SILU_MUL */
    const ts_after *after; /* host struct or NULL: a stage chain on each output (operands
                              [rows, n], indexed as out) */
} ts_picked_args;

/* Replaces: rule "picked" (engine/rules/linear/src/picked.rs:28-60,106-122) on the
 * site Picked (engine/plan/lower/src/sites/matmul.rs:10-24,66-96). */
int tessera_hip_picked(const ts_picked_args *a, void *stream);
size_t tessera_hip_picked_workspace(const ts_picked_args *a);

/* ----------------------------------------------------------------------------
 * Ragged-row attention over kept (paged) K/V.
 * Row r (slot s, position p) attends keys [max(0, p - back), p] of slot s; the
 * key at position j lives at kept row table[s*kept_pages + (j >> log2 page)]
 * * page + (j & (page-1)) (engine/plan/codegen/src/kept.rs:181-193), or at
 * s*keys + j when kept_table is NULL. Scores are dot(q, k) * scale.
 * q: [rows, heads, width] f32; K/V rows: [*, kv_heads, width] bf16;
 * out: [rows, heads, width] f32. Head h reads kv head h / (heads / kv_heads).
 * ------------------------------------------------------------------------- */
typedef struct {
    const void *q;
    const void *k;
    const void *v;
    void *out;
    const uint32_t *slots;      /* [rows] */
    const uint32_t *positions;  /* [rows] */
    const uint32_t *kept_table; /* [slot count * kept_pages], or NULL for dense */
    void *workspace;
    size_t workspace_bytes;
    uint32_t rows;              /* queries */
    uint32_t keys;              /* positions a slot may hold (the kept context) */
    uint32_t heads, kv_heads;
    uint32_t width;             /* head dim: 128 */
    uint32_t back;              /* keys a row sees before its own; UINT32_MAX = causal */
    uint32_t kept_pages;        /* table entries per slot */
    uint32_t page;              /* rows per page (power of two, >= 16) */
    float scale;
    int32_t q_dtype, kv_dtype, out_dtype;
    uint32_t max_position;      /* an upper bound on positions[] (sizes the split) */
    uint32_t *status;           /* device word or NULL: TS_STATUS_* bits are OR-ed in */
} ts_rows_args;

/* Device-side refusals of the attention kernels (ts_rows_args.status). A row whose
 * position is >= keys, > max_position, or past its slot's kept_pages * page is refused,
 * as the interpreter refuses a read at >= keys (engine/ir/interp/src/cpu.rs:323-327):
 * the row loads nothing, writes NaN outputs (and appends nothing), and the bit below is
 * set in *status. The caller clears the word and reads it back when it wants to know. */
#define TS_STATUS_POSITION 1u

/* Decode: few rows, each key range split across workgroups, partial
 * (max, sum, acc) merged by the last group to finish.
 * Replaces: rule "attend" / attend_rows (engine/rules/attention/src/attend.rs:126-270)
 * and flash_rows for decode rows (flash.rs:506-591). */
int tessera_hip_attend_rows(const ts_rows_args *a, void *stream);
size_t tessera_hip_attend_rows_workspace(const ts_rows_args *a);

/* attend_rows with no workspace and no allocation: the split-KV partials live in a
 * fixed device array of tessera_hip_attend_rows_noalloc_limit() bytes (16 MiB; one
 * copy per GPU, held until the process ends). a->workspace is ignored. Launches whose
 * partials would pass the limit (rows * kv_heads * partitions * heads/kv_heads * 520
 * bytes; e.g. 32 rows at 8192 keys, 16 partitions, need 4.3 MB) fail with TS_ERR_WORKSPACE. Calls
 * on one GPU share the array: calls that overlap in time on that GPU (different
 * streams) race; stream-ordered calls do not.
 * No counterpart in the reference: for callers that cannot allocate (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). */
int tessera_hip_attend_rows_noalloc(const ts_rows_args *a, void *stream);
size_t tessera_hip_attend_rows_noalloc_limit(void);

/* The decode step of a Qwen3 layer in one launch: per-head RmsNorm (q_gain /
 * k_gain, eps) and Halves RoPE (angles from rope_table, rows >= max_position + 1,
 * as tessera_hip_rope_table fills it) of q and of the new k from the raw q/k/v
 * product rows qkv [rows, (heads + 2*kv_heads) * width] f32; the new k and v rows
 * written (bf16) into the kept rows at (slot, position) (a->k and a->v are
 * written); then attend_rows over the kept rows, the new row included. a->q is
 * ignored. Same split and workspace as tessera_hip_attend_rows. Every row must
 * read only keys kept by earlier launches plus its own: rows of one launch may not
 * share a slot (the decode shape: one new row per slot).
 * Replaces: the q_norm/k_norm RmsNorm + rope + Append + attend_rows chain of
 * engine/models/src/shared.rs:109-145 and engine/ir/interp/src/run.rs:122-198. */
typedef struct {
    ts_rows_args rows;          /* as for attend_rows; rows.q is ignored */
    const float *qkv;           /* [rows, (heads + 2 kv_heads) * width] f32 */
    const float *q_gain, *k_gain; /* [width] f32 */
    const float *rope_table;    /* tessera_hip_rope_table's output */
    uint32_t rope_rows;         /* positions the table holds (> rows.max_position) */
    float eps;
} ts_step_args;
int tessera_hip_attend_step(const ts_step_args *a, void *stream);

/* Prefill: 128-row query blocks on the matrix unit, keys streamed page by page
 * with online softmax. Rows may be packed ragged, back to back: a block whose rows
 * belong to several slots takes one pass over the keys per distinct slot, as the
 * reference does.
 * Replaces: rule "flash" / flash_rows (engine/rules/attention/src/flash.rs:416-503,
 * 506-591, 595-807). */
int tessera_hip_flash_rows(const ts_rows_args *a, void *stream);

/* ----------------------------------------------------------------------------
 * Elementwise chains not fused into a product.
 * out[i] = chain(x[i], operands at i) for i < len, with `after` as above (read
 * `after.sum` is x; operands with spans repeat). out may alias x or an operand.
 * Replaces: rule "map" / kernel Map (engine/plan/lower/src/kernels/map.rs:60-65,
 * 187-260), e.g. the q pre-scale Map Scale(1/sqrt(d)) of
 * engine/rules/attention/src/lib.rs:22-31.
 * ------------------------------------------------------------------------- */
typedef struct {
    const float *x;   /* [len] */
    float *out;       /* [len] */
    uint32_t len;
    ts_after after;   /* by value */
} ts_map_args;
int tessera_hip_map(const ts_map_args *a, void *stream);

/* f32 weights to the TS_F32_PARTS layout, once at load: out [2n, k] bf16 from w [n, k]
 * f32 (high parts, then low parts; both round to nearest even).
 * Replaces: the F32 form the reference's tiled / lanes rules read directly
 * (engine/plan/codegen/src/form.rs:224-229), laid out for the matrix unit. */
typedef struct {
    const float *w;  /* [n, k] */
    void *out;       /* [2n, k] bf16 */
    uint32_t n, k;
} ts_pack_args;
int tessera_hip_pack_f32(const ts_pack_args *a, void *stream);

/* ----------------------------------------------------------------------------
 * Whole-sequence attention with any mask (the reference's flash on the Attend site,
 * engine/rules/attention/src/flash.rs:416-503; semantics of interp's attend,
 * engine/ir/interp/src/cpu.rs:61-77,172-225, masks engine/ir/graph/src/node.rs:162-
 * 181). Query i of a sequence sits at position past + i, past = keys - rows when the
 * keys cover the rows (ends aligned), else 0 (refused for causal masks); it sees keys
 * [pos - back, pos + ahead] of its sequence, p = softmax(dot(q, k) * scale); a query
 * whose window holds no key writes zeros. Masks: Causal (back UINT32_MAX, ahead 0,
 * causal 1), Bidirectional (UINT32_MAX, UINT32_MAX, 0), Within(n) (n, n, 0), Back(n)
 * (n, 0, 1). Head h reads kv head h / (heads / kv_heads).
 * ------------------------------------------------------------------------- */
typedef struct {
    const void *q;      /* [seqs, rows, heads, width] f32 or bf16 */
    const void *k;      /* [seqs, keys, kv_heads, width] bf16 */
    const void *v;      /* [seqs, keys, kv_heads, width] bf16 */
    void *out;          /* [seqs, rows, heads, width] f32 */
    uint32_t seqs, rows, keys, heads, kv_heads;
    uint32_t width;     /* 128 */
    uint32_t back, ahead;
    int32_t causal;     /* the mask is causal (Causal, Back): more rows than keys is refused */
    float scale;
    int32_t q_dtype, kv_dtype, out_dtype;
} ts_flash_args;

/* Same kernel as tessera_hip_flash_rows: 128-row query blocks on the matrix unit, keys
 * streamed in 64-key blocks with online softmax.
 * Replaces: rule "flash" on whole sequences (engine/rules/attention/src/flash.rs:
 * 416-503, 775-807). */
int tessera_hip_flash(const ts_flash_args *a, void *stream);

/* ----------------------------------------------------------------------------
 * Row stages and indices. Each takes one argument struct, fields in the reference
 * Launch order (reads, outputs, then counts and scalars), and the stream.
 * ------------------------------------------------------------------------- */

/* out = x * rsqrt(mean(x^2) + eps) * gain, per row of `width`; x/out f32.
 * Replaces: "rms_norm" / "lane_norm" (engine/rules/kernels/src/rms_norm.rs:9-69,
 * lane_norm.rs:10-96). out may alias x. */
typedef struct {
    const float *x, *gain;  /* reads: [rows, width], [width] */
    float *out;             /* [rows, width] */
    uint32_t rows, width;
    float eps;
} ts_norm_args;
int tessera_hip_rms_norm(const ts_norm_args *a, void *stream);

/* Rotates (j, j + width/2) pairs (Halves) or (2j, 2j+1) (Adjacent) of each
 * [rows, heads, width] row in place by angle pos * theta^(-2j/width).
 * Replaces: "angles" + "rope" (engine/rules/kernels/src/rope.rs:10-125). */
typedef struct {
    float *x;                   /* [rows, heads, width], rotated in place */
    const uint32_t *positions;  /* [rows] */
    uint32_t rows, heads, width;
    float theta;
    int32_t halves;             /* 1: Halves pairs, 0: Adjacent */
} ts_rope_args;
int tessera_hip_rope(const ts_rope_args *a, void *stream);

/* The angle table: table[(pos * width/2 + j) * 2 + {0, 1}] = (cos, sin) of
 * pos * theta^(-2j/width) for pos < positions, j < width/2.
 * Replaces: the "angles" stage (engine/rules/kernels/src/rope.rs:10-58). */
typedef struct {
    float *table;  /* [positions][width / 2][2] */
    uint32_t positions, width;
    float theta;
} ts_angles_args;
int tessera_hip_rope_table(const ts_angles_args *a, void *stream);

/* The step between the q/k/v product and attention for a Qwen3 layer: per head
 * RmsNorm (q_gain / k_gain, eps) then Halves RoPE on q and k, then the new k
 * and v rows written (bf16) into the kept rows at (slot, position).
 * qkv: [rows, (heads + 2*kv_heads) * width] f32 (q heads, then k, then v).
 * q_out: [rows, heads, width] f32.
 * Replaces: the q_norm/k_norm RmsNorm + rope + Append chain
 * (engine/models/src/shared.rs:109-145, engine/ir/interp/src/run.rs:122-198). */
typedef struct {
    const float *qkv, *q_gain, *k_gain;                  /* reads */
    float *q_out;                                        /* [rows, heads, width] */
    void *k_cache, *v_cache;                             /* kept rows, bf16 (written) */
    const uint32_t *slots, *positions, *kept_table;      /* kept_table may be NULL (dense) */
    uint32_t rows, heads, kv_heads, width, keys, kept_pages, page;
    float eps, theta;
} ts_qk_args;
int tessera_hip_qk_norm_rope_append(const ts_qk_args *a, void *stream);

/* Embedding rows: out[r, :] = f32(table[ids[r] - first, :]), zeros outside the
 * table. table bf16 [rows_in_table, width].
 * Replaces: "gather" (engine/rules/kernels/src/gather.rs; interp cpu.rs:511-525). */
typedef struct {
    const void *table;    /* bf16 [table_rows, width] */
    const uint32_t *ids;  /* [count] */
    float *out;           /* [count, width] */
    uint32_t count, table_rows, width, first;
} ts_gather_args;
int tessera_hip_gather(const ts_gather_args *a, void *stream);

/* out[j] = x[j / picks, ids[j]], zero when ids[j] >= width; x [rows, width],
 * ids/out [rows, picks]. Replaces: interp take (engine/ir/interp/src/cpu.rs:498-508)
 * as the MoE layer uses it (engine/models/src/decoder.rs:78). */
typedef struct {
    const float *x;       /* [rows, width] */
    const uint32_t *ids;  /* [rows, picks] */
    float *out;           /* [rows, picks] */
    uint32_t rows, width, picks;
} ts_take_args;
int tessera_hip_take(const ts_take_args *a, void *stream);

/* Row softmax in the reference's order: max from -inf (NaN ignored), exp(v - max),
 * sequential sum, divide. One thread per row: routing widths (<= 4096).
 * Replaces: interp softmax (engine/ir/interp/src/cpu.rs:49-59). out may alias x. */
typedef struct {
    const float *x;  /* [rows, width] */
    float *out;      /* [rows, width], may alias x */
    uint32_t rows, width;
} ts_softmax_args;
int tessera_hip_softmax(const ts_softmax_args *a, void *stream);

/* out[o, i] = sum_t x[o, t, i] * weights[o, t] (t in order from 0, no fused
 * multiply-add: bit-exact), or the mean when weights is NULL. x [outer, count, inner].
 * Replaces: mean / mix (engine/ir/interp/src/cpu.rs:450-473), the MoE combine. */
typedef struct {
    const float *x, *weights;  /* [outer, count, inner], [outer, count] or NULL (mean) */
    float *out;                /* [outer, inner] */
    uint32_t outer, count, inner;
} ts_mix_args;
int tessera_hip_mix(const ts_mix_args *a, void *stream);

/* ids[r] = first index of the largest finite entry of row r (NaN and -inf
 * skipped; `width` when none). x f32 [rows, width].
 * Replaces: "peaks" + "argmax" (engine/rules/kernels/src/argmax.rs:74-129). */
typedef struct {
    const float *x;  /* [rows, width] */
    uint32_t *ids;   /* [rows] */
    void *workspace;
    size_t workspace_bytes;
    uint32_t rows, width;
} ts_argmax_args;
int tessera_hip_argmax(const ts_argmax_args *a, void *stream);
size_t tessera_hip_argmax_workspace(const ts_argmax_args *a);

/* ids[r] from the keys a product with TS_AFTER_ARGMAX folded (the same pick as
 * tessera_hip_argmax over its output row: first index of the largest entry, NaN and
 * -inf skipped, `width` when none), then keys[r] = 0 for the next product.
 * No counterpart in the reference: argmax fused into the lm_head product, so the
 * logits are not read back (engine/rules/kernels/src/argmax.rs:74-129 reads them). */
typedef struct {
    uint64_t *keys;  /* [rows]: read, then cleared */
    uint32_t *ids;   /* [rows] */
    uint32_t rows, width;
} ts_keys_args;
int tessera_hip_argmax_keys(const ts_keys_args *a, void *stream);

/* ids[r, 0..k): the row's k largest finite entries, best first, ties to the
 * lower index, NaN/-inf skipped, spare slots = width. x f32 [rows, width],
 * width <= 1024, k <= 32.
 * Replaces: "top_k" (engine/rules/kernels/src/argmax.rs:39-72; interp run.rs:577-591). */
typedef struct {
    const float *x;  /* [rows, width] */
    uint32_t *ids;   /* [rows, k] */
    uint32_t rows, width, k;
} ts_top_k_args;
int tessera_hip_top_k(const ts_top_k_args *a, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TESSERA_HIP_H */
