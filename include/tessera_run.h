/*
 * tessera_run: the host runner for a Qwen3-shaped decoder on one gfx950 GPU.
 *
 * Replaces, for this path, the reference's device Runner and decode loop:
 * tessera-run's device::Runner (engine/plan/run/src/device.rs:91-245,390-400:
 * buffers owned and zeroed at replan, launches bound in Launch order, the whole
 * step captured once into a HIP graph and replayed) driven by
 * tessera-engine's Engine::step / generate (engine/engine/src/lib.rs:315-498),
 * over the Qwen3 graph of engine/models/src/decoder.rs:160-391 (tied embedding,
 * q/k RmsNorm per head then Halves RoPE, SwiGLU, RmsNorm before each block).
 *
 * Memory: every device buffer is allocated at open (weights, kept rows in
 * pages, activations, one workspace); prefill and decode allocate nothing.
 * Kept rows: [pages * page, kv_heads, head_dim] bf16 per layer for K and V,
 * addressed through the page table that the pool (tessera_kv.h) assigns.
 * Errors: the status conventions of tessera_hip.h.
 */
#ifndef TESSERA_RUN_H
#define TESSERA_RUN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    uint32_t vocab, hidden, layers, heads, kv_heads, head_dim, ffn;
    float eps, theta;
    uint32_t max_context; /* kept rows one slot may hold */
    uint32_t page;        /* rows per kept page (power of two >= 16) */
    uint32_t max_prompt;  /* rows one prefill may carry */
} ts_qwen3_config;

typedef struct ts_qwen3 ts_qwen3;

/* Qwen3-0.6B's sizes (engine/models/src/decoder.rs:160-170, Config::qwen3). */
void tessera_qwen3_default_config(ts_qwen3_config *c);

/* Allocates everything and fills the weights from `seed`: every matrix
 * N(0, 0.02), every RmsNorm gain 1 + N(0, 0.02), all rounded to bf16 (gains are
 * kept as the f32 value of that bf16). */
int tessera_qwen3_open(const ts_qwen3_config *c, uint64_t seed, ts_qwen3 **out);
void tessera_qwen3_close(ts_qwen3 *m);

/* Device pointer, bytes and dtype (TS_BF16 / TS_F32) of a weight: name is one of
 * "embed", "norm" (layer ignored) or "ln1", "qkv", "q_norm", "k_norm", "o",
 * "ln2", "gate_up", "down" for `layer`. "qkv" stacks q, k then v rows;
 * "gate_up" stacks gate rows then up rows. */
int tessera_qwen3_weight(ts_qwen3 *m, const char *name, uint32_t layer, void **ptr, uint64_t *bytes,
                         int32_t *dtype);

/* Copies the first `bytes` of a weight (or "k_cache" / "v_cache" of a layer) to host. */
int tessera_qwen3_read(ts_qwen3 *m, const char *name, uint32_t layer, void *host, uint64_t bytes);

/* Resets the slot, runs the prompt (host token ids) through every layer, keeps
 * its K/V rows and writes the greedy next token to *next. */
int tessera_qwen3_prefill(ts_qwen3 *m, const uint32_t *tokens, uint32_t count, uint32_t *next);

/* `steps` greedy decode steps after the prefill, each one replay of the step's
 * HIP graph (or eager launches when graphs are off). Tokens are written to
 * tokens_out (host) when it is not NULL. Synchronizes before returning. */
int tessera_qwen3_decode(ts_qwen3 *m, uint32_t steps, uint32_t *tokens_out);

/* Replaces the next decode step's input token (by default the previous step's greedy
 * pick) with `token`: teacher forcing, as when a caller feeds its own sequence. The
 * reference's decode loop feeds back its pick (engine/engine/src/lib.rs:401-470); this
 * lets a caller, and the tests, drive the same step with any token. */
int tessera_qwen3_set_token(ts_qwen3 *m, uint32_t token);

/* The last step's logits (f32, vocab entries) copied to host. */
int tessera_qwen3_logits(ts_qwen3 *m, float *host, uint64_t count);

/* 1: capture the decode step into a HIP graph (default); 0: eager launches. */
int tessera_qwen3_set_graph(ts_qwen3 *m, int on);

/* 1: run decode steps as one persistent launch per decode call (every layer, the
 * lm_head and the greedy pick of all `steps` tokens in one grid of one group per
 * CU; the default when the shape fits: head_dim 128, two q heads per kv head,
 * hidden <= 1024, ffn <= 3072, at most 32 layers); 0: the graph of kernels (or
 * eager launches, see tessera_qwen3_set_graph). Returns an error for 1 when the
 * shape does not fit. No counterpart in the reference, whose decode step is a
 * graph of its lowered kernels (engine/plan/run/src/device.rs:227-245). */
int tessera_qwen3_set_step(ts_qwen3 *m, int on);
/* 1 when decode runs the persistent step. */
int tessera_qwen3_step_mode(ts_qwen3 *m);

/* Device time (ms) of the last tessera_qwen3_decode call's steps, from HIP events
 * recorded on the runner's stream around the persistent launch (or the graph
 * replays); -1 when the call was not timed. No counterpart in the reference
 * (its runner reports wall time, engine/plan/run/src/device.rs:227-245). */
float tessera_qwen3_decode_ms(ts_qwen3 *m);

/* Debug: the persistent step writes phase stamps (100 MHz clock) of the first
 * step of each later launch to `marks` (device memory of groups * (layers + 2)
 * * 10 words; NULL stops it); *groups receives the grid size. */
int tessera_qwen3_step_marks(ts_qwen3 *m, uint64_t *marks, uint32_t *groups);

/* The runner's stream (a hipStream_t). */
void *tessera_qwen3_stream(ts_qwen3 *m);

/* Current position (the next token's kept row) and the page table of the slot. */
uint32_t tessera_qwen3_position(ts_qwen3 *m);
int tessera_qwen3_pages(ts_qwen3 *m, uint32_t *host, uint32_t count);

#ifdef __cplusplus
}
#endif

#endif /* TESSERA_RUN_H */
