// The Qwen3 decode runner: device memory, seeded weights, prefill, and the
// greedy decode step captured once into a HIP graph.
//
// Launch sequence per decode token (engine/models/src/decoder.rs:327-391 as
// lowered by the rules, with the fusions the rules allow):
//   gather(embed, tok)                              -> x          [1, H]
//   per layer:
//     lanes(x, qkv, before RmsNorm(ln1))            -> qkv        [1, (Hq+2Hkv)*D]
//     qk_norm_rope_append(qkv)                      -> q; K/V rows at (slot, pos)
//     attend_rows(q, K, V)                          -> attn       [1, Hq*D]
//     lanes(attn, o, after +x)                      -> x
//     lanes(x, gate_up, before RmsNorm(ln2), silu*) -> h          [1, F]
//     lanes(h, down, after +x)                      -> x
//   lanes(x, embed, before RmsNorm(norm), argmax)   -> logits     [1, V], key
//   advance: tok from key; pos + 1
// Position and token live in device memory, so one captured graph serves
// every step (engine/plan/run/src/device.rs:227-245 captures per size binding).
#include <string.h>

#include <vector>

#include "../../include/tessera_kv.h"
#include "../../include/tessera_run.h"
#include "common.h"
#include "decode_step.h"

#include <algorithm>

namespace {

// splitmix64: a counter-based hash, so every weight element is a pure function
// of (seed, tensor, index) and generation order does not matter.
TS_DEV uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// N(mean, std) by Box-Muller from two 24-bit uniforms in (0, 1], rounded to bf16.
TS_DEV float seeded_normal(uint64_t seed, uint64_t tensor, uint64_t i) {
    const uint64_t h = mix64(seed ^ mix64(tensor * 0x100000001b3ull + i));
    const float u1 = ((float)(h >> 40) + 1.0f) * (1.0f / 16777216.0f);
    const float u2 = ((float)((h >> 16) & 0xffffff) + 0.5f) * (1.0f / 16777216.0f);
    return sqrtf(-2.0f * logf(u1)) * cosf(6.28318530717958647692f * u2);
}

__global__ void init_bf16_kernel(uint16_t *w, uint64_t n, uint64_t seed, uint64_t tensor, float std) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        w[i] = bf16_bits(std * seeded_normal(seed, tensor, i));
}

__global__ void init_gain_kernel(float *g, uint64_t n, uint64_t seed, uint64_t tensor, float std) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        g[i] = bf16_round(1.0f + std * seeded_normal(seed, tensor, i));
}

// The greedy token from the key the lm_head product folded (TS_AFTER_ARGMAX), and the
// key cleared for the next product.
TS_DEV uint32_t take_token(uint64_t *key, uint32_t *tok, uint32_t vocab) {
    const uint64_t k = key[0];
    const uint32_t t = k ? ~(uint32_t)k : vocab;
    key[0] = 0;
    tok[0] = t;
    return t;
}

// After a decode step: the new token, recorded, and the next position.
__global__ void advance_kernel(uint64_t *key, uint32_t *tok, uint32_t *pos, uint32_t *hist, uint32_t vocab) {
    const uint32_t p = pos[0] + 1;
    hist[p] = take_token(key, tok, vocab);
    pos[0] = p;
}

// After a prefill of `count` rows: the first new token sits at position count.
__global__ void start_kernel(uint64_t *key, uint32_t *tok, uint32_t *pos, uint32_t *hist, uint32_t count,
                             uint32_t vocab) {
    pos[0] = count;
    hist[count] = take_token(key, tok, vocab);
}

// The next step's input token set from the host (teacher forcing), recorded at its position.
__global__ void set_token_kernel(uint32_t *tok, uint32_t *hist, uint32_t at, uint32_t t) {
    tok[0] = t;
    hist[at] = t;
}

struct Layer {
    float *ln1, *q_norm, *k_norm, *ln2;
    uint16_t *qkv, *o, *gate_up, *down;
    uint16_t *k_cache, *v_cache;
};

}  // namespace

struct ts_qwen3 {
    ts_qwen3_config c;
    hipStream_t stream = nullptr;
    std::vector<void *> allocs;
    uint16_t *embed = nullptr;
    float *norm = nullptr;
    std::vector<Layer> layers;
    // activations
    float *x, *xn, *qkv, *q, *attn, *h, *logits, *rope;
    uint32_t *d_tok, *d_pos, *d_slot, *d_hist, *d_prompt, *d_prompt_pos, *d_prompt_slot, *d_table;
    uint64_t *d_key = nullptr;  // the lm_head product's folded argmax (zero between steps)
    void *ws = nullptr;
    size_t ws_bytes = 0;
    void **d_buffers = nullptr;  // the K and V kept-row buffers of every layer (page copies)
    ts_kv_copy *d_copy = nullptr;
    ts_kv_pool *pool = nullptr;
    ts_kv_run run{0, 0};
    bool have_run = false;
    uint32_t kept_pages = 0, total_pages = 0;
    bool use_graph = true;
    hipGraphExec_t graph = nullptr;
    uint32_t position = 0;
    // The persistent step (decode_step.hip): hand-off words, error word, epoch.
    bool step_ok = false;   // the shape fits the persistent kernel
    bool use_step = false;  // decode runs it (default when it fits)
    uint64_t *hand = nullptr;
    uint32_t *d_error = nullptr;
    std::vector<uint16_t *> packed;    // the step's packed weights, [layer][qkv, o, gate/up, down]
    uint16_t *lm_packed = nullptr;     // and its packed lm_head rows
    uint32_t epoch = 1, groups = 0;
    uint64_t *step_marks = nullptr;  // debug: phase stamps of the next persistent launch
    hipEvent_t ev0 = nullptr, ev1 = nullptr;  // around the last decode call's device work
    float decode_ms = -1.0f;

    template <class T>
    int alloc(T **p, size_t count) {
        void *v = nullptr;
        hipError_t e = hipMalloc(&v, count * sizeof(T) + 16);
        if (e != hipSuccess) return ts::hip_status(e, "hipMalloc");
        allocs.push_back(v);
        *p = (T *)v;
        return TS_OK;
    }
};

namespace {

int launch_init_bf16(ts_qwen3 *m, uint16_t *w, uint64_t n, uint64_t seed, uint64_t id) {
    hipLaunchKernelGGL(init_bf16_kernel, dim3(1024), dim3(256), 0, m->stream, w, n, seed, id, 0.02f);
    TS_CHECK_LAUNCH("init weights");
    return TS_OK;
}

int launch_init_gain(ts_qwen3 *m, float *g, uint64_t n, uint64_t seed, uint64_t id) {
    hipLaunchKernelGGL(init_gain_kernel, dim3(64), dim3(256), 0, m->stream, g, n, seed, id, 0.02f);
    TS_CHECK_LAUNCH("init gains");
    return TS_OK;
}

ts_linear_args lin(const void *x, const void *w, void *out, uint32_t rows, uint32_t n, uint32_t k, ts_qwen3 *m) {
    ts_linear_args a;
    memset(&a, 0, sizeof a);
    a.x = x; a.w = w; a.out = out; a.m = rows; a.n = n; a.k = k;
    a.x_dtype = TS_F32; a.w_dtype = TS_BF16; a.out_dtype = TS_F32;
    a.workspace = m->ws; a.workspace_bytes = m->ws_bytes;
    a.eps = m->c.eps;
    return a;
}

ts_rows_args rows_args(ts_qwen3 *m, const Layer &L, uint32_t rows, const uint32_t *slots, const uint32_t *pos,
                       uint32_t max_position) {
    ts_rows_args r;
    memset(&r, 0, sizeof r);
    r.q = m->q; r.k = L.k_cache; r.v = L.v_cache; r.out = m->attn;
    r.slots = slots; r.positions = pos; r.kept_table = m->d_table;
    r.workspace = m->ws; r.workspace_bytes = m->ws_bytes;
    r.rows = rows; r.keys = m->kept_pages * m->c.page; r.heads = m->c.heads; r.kv_heads = m->c.kv_heads;
    r.width = m->c.head_dim; r.back = 0xffffffffu; r.kept_pages = m->kept_pages; r.page = m->c.page;
    r.scale = 1.0f / sqrtf((float)m->c.head_dim);
    r.q_dtype = TS_F32; r.kv_dtype = TS_BF16; r.out_dtype = TS_F32;
    r.max_position = max_position;
    return r;
}

#define TRY(expr)                   \
    do {                            \
        int _rc = (expr);           \
        if (_rc != TS_OK) return _rc; \
    } while (0)

// The layers for `rows` rows at (slots, pos). Decode rows (<= 16) fuse the
// RmsNorm into the product; prefill rows normalize first and use the tiled rule.
int run_layers(ts_qwen3 *m, uint32_t rows, const uint32_t *slots, const uint32_t *pos, uint32_t max_position) {
    const ts_qwen3_config &c = m->c;
    const uint32_t H = c.hidden, D = c.head_dim, QKV = (c.heads + 2 * c.kv_heads) * D, QD = c.heads * D;
    const bool fused = rows <= 16;
    void *s = m->stream;
    for (uint32_t l = 0; l < c.layers; l++) {
        const Layer &L = m->layers[l];
        ts_linear_args a = lin(fused ? m->x : m->xn, L.qkv, m->qkv, rows, QKV, H, m);
        if (fused) {
            a.stages = TS_BEFORE_RMS_NORM;
            a.gain = L.ln1;
        } else {
            const ts_norm_args n = {m->x, L.ln1, m->xn, rows, H, c.eps};
            TRY(tessera_hip_rms_norm(&n, s));
        }
        TRY(tessera_hip_linear(&a, s));
        ts_rows_args r = rows_args(m, L, rows, slots, pos, max_position);
        if (rows == 1) {
            // q/k norm, RoPE, the kept-row append and attention in one launch (a row
            // may only read keys appended by earlier launches, so one row per slot).
            const ts_step_args st = {r, m->qkv, L.q_norm, L.k_norm, m->rope, c.max_context, c.eps};
            TRY(tessera_hip_attend_step(&st, s));
        } else {
            const ts_qk_args q = {m->qkv, L.q_norm, L.k_norm, m->q, L.k_cache, L.v_cache, slots, pos,
                                  m->d_table, rows, c.heads, c.kv_heads, D, m->kept_pages * c.page,
                                  m->kept_pages, c.page, c.eps, c.theta};
            TRY(tessera_hip_qk_norm_rope_append(&q, s));
            TRY(fused ? tessera_hip_attend_rows(&r, s) : tessera_hip_flash_rows(&r, s));
        }
        a = lin(m->attn, L.o, m->x, rows, H, QD, m);
        a.stages = TS_AFTER_ADD;
        a.a0 = m->x;
        TRY(tessera_hip_linear(&a, s));
        a = lin(fused ? m->x : m->xn, L.gate_up, m->h, rows, c.ffn, H, m);
        a.stages = TS_AFTER_SILU_MUL;
        if (fused) {
            a.stages |= TS_BEFORE_RMS_NORM;
            a.gain = L.ln2;
        } else {
            const ts_norm_args n = {m->x, L.ln2, m->xn, rows, H, c.eps};
            TRY(tessera_hip_rms_norm(&n, s));
        }
        TRY(tessera_hip_linear(&a, s));
        a = lin(m->h, L.down, m->x, rows, H, c.ffn, m);
        a.stages = TS_AFTER_ADD;
        a.a0 = m->x;
        TRY(tessera_hip_linear(&a, s));
    }
    return TS_OK;
}

// Logits of one row (`row` of x), the greedy pick folded into d_key by the same
// product (start_kernel / advance_kernel turn it into the token).
int head(ts_qwen3 *m, uint32_t row) {
    const ts_qwen3_config &c = m->c;
    ts_linear_args a = lin(m->x + (size_t)row * c.hidden, m->embed, m->logits, 1, c.vocab, c.hidden, m);
    a.stages = TS_BEFORE_RMS_NORM | TS_AFTER_ARGMAX;
    a.gain = m->norm;
    a.workspace = m->d_key;
    a.workspace_bytes = 8;
    return tessera_hip_linear(&a, m->stream);
}

int decode_step(ts_qwen3 *m) {
    const ts_qwen3_config &c = m->c;
    const ts_gather_args g = {m->embed, m->d_tok, m->x, 1, c.vocab, c.hidden, 0};
    TRY(tessera_hip_gather(&g, m->stream));
    TRY(run_layers(m, 1, m->d_slot, m->d_pos, c.max_context - 1));
    TRY(head(m, 0));
    hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(1), 0, m->stream, m->d_key, m->d_tok, m->d_pos, m->d_hist,
                       c.vocab);
    TS_CHECK_LAUNCH("advance");
    return TS_OK;
}

// `steps` decode steps in one persistent launch (decode_step.hip).
int launch_step(ts_qwen3 *m, uint32_t steps) {
    const ts_qwen3_config &c = m->c;
    ts::DecodeStepArgs a;
    memset(&a, 0, sizeof a);
    for (uint32_t l = 0; l < c.layers; l++) {
        const Layer &L = m->layers[l];
        a.ln1[l] = L.ln1; a.ln2[l] = L.ln2; a.q_norm[l] = L.q_norm; a.k_norm[l] = L.k_norm;
        a.k_cache[l] = L.k_cache; a.v_cache[l] = L.v_cache;
        for (uint32_t r = 0; r < 4; r++) a.packed[l][r] = m->packed[(size_t)l * 4 + r];
    }
    a.lm_packed = m->lm_packed;
    a.embed = m->embed; a.norm = m->norm; a.rope = m->rope; a.table = m->d_table;
    a.tok = m->d_tok; a.pos = m->d_pos; a.hist = m->d_hist; a.logits = m->logits;
    a.hand = m->hand; a.error = m->d_error; a.marks = m->step_marks;
    a.H = c.hidden; a.L = c.layers; a.Hq = c.heads; a.Hkv = c.kv_heads; a.F = c.ffn; a.V = c.vocab;
    a.NG = m->groups; a.kept_pages = m->kept_pages; a.page_shift = (uint32_t)__builtin_ctz(c.page);
    a.steps = steps; a.epoch = m->epoch;
    a.eps = c.eps; a.scale = 1.0f / sqrtf((float)c.head_dim);
    TRY(ts::decode_step_launch(&a, m->stream));
    m->epoch += steps;
    return TS_OK;
}

size_t workspace_need(ts_qwen3 *m) {
    const ts_qwen3_config &c = m->c;
    ts_argmax_args am{};
    am.rows = 1;
    am.width = c.vocab;
    size_t need = tessera_hip_argmax_workspace(&am);
    const uint32_t H = c.hidden, D = c.head_dim;
    const uint32_t shapes[][2] = {{(c.heads + 2 * c.kv_heads) * D, H}, {H, c.heads * D}, {c.ffn, H},
                                  {H, c.ffn}, {c.vocab, H}};
    // Split partials grow with the rows: size for one row and for the most rows a
    // launch can carry to the few-row kernels (up to 64).
    const uint32_t row_counts[] = {1, std::min<uint32_t>(c.max_prompt, 64)};
    for (uint32_t rows : row_counts)
        for (auto &sh : shapes) {
            ts_linear_args a = lin(nullptr, nullptr, nullptr, rows, sh[0], sh[1], m);
            if (sh[0] == c.ffn && sh[1] == H) a.stages = TS_AFTER_SILU_MUL;
            size_t w = tessera_hip_linear_workspace(&a);
            if (w > need) need = w;
        }
    Layer L{};
    ts_rows_args r = rows_args(m, L, 1, nullptr, nullptr, c.max_context - 1);
    size_t w = tessera_hip_attend_rows_workspace(&r);
    if (w > need) need = w;
    return need;
}

}  // namespace

extern "C" void tessera_qwen3_default_config(ts_qwen3_config *c) {
    c->vocab = 151936; c->hidden = 1024; c->layers = 28; c->heads = 16; c->kv_heads = 8; c->head_dim = 128;
    c->ffn = 3072; c->eps = 1e-6f; c->theta = 1e6f; c->max_context = 160; c->page = 16; c->max_prompt = 128;
}

extern "C" int tessera_qwen3_open(const ts_qwen3_config *cfg, uint64_t seed, ts_qwen3 **out) {
    TS_REQUIRE(cfg && out, "qwen3_open: null argument");
    TS_REQUIRE(cfg->head_dim == 128, "qwen3_open: head_dim %u (128 supported)", cfg->head_dim);
    TS_REQUIRE(cfg->hidden % 8 == 0 && cfg->ffn % 8 == 0, "qwen3_open: hidden and ffn must be multiples of 8");
    TS_REQUIRE(cfg->page >= 16 && (cfg->page & (cfg->page - 1)) == 0, "qwen3_open: page %u", cfg->page);
    TS_REQUIRE(cfg->max_context >= 2 && cfg->max_prompt >= 1 && cfg->max_prompt < cfg->max_context,
               "qwen3_open: max_prompt %u must be below max_context %u", cfg->max_prompt, cfg->max_context);
    TS_REQUIRE(cfg->kv_heads >= 1 && cfg->heads % cfg->kv_heads == 0, "qwen3_open: heads");
    int rc = tessera_hip_init();
    if (rc) return rc;
    ts_qwen3 *m = new ts_qwen3();
    m->c = *cfg;
    const ts_qwen3_config &c = m->c;
    auto fail = [&](int code) {
        tessera_qwen3_close(m);
        return code;
    };
    hipError_t e = hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking);
    if (e != hipSuccess) return fail(ts::hip_status(e, "hipStreamCreate"));
    const uint32_t H = c.hidden, D = c.head_dim, QKV = (c.heads + 2 * c.kv_heads) * D, QD = c.heads * D;
    m->kept_pages = (c.max_context + c.page - 1) / c.page;
    m->total_pages = m->kept_pages;
    const size_t kv_rows = (size_t)m->total_pages * c.page;
    uint64_t id = 1;
    if ((rc = m->alloc(&m->embed, (size_t)c.vocab * H))) return fail(rc);
    if ((rc = launch_init_bf16(m, m->embed, (size_t)c.vocab * H, seed, id++))) return fail(rc);
    m->layers.resize(c.layers);
    for (uint32_t l = 0; l < c.layers; l++) {
        Layer &L = m->layers[l];
        if ((rc = m->alloc(&L.ln1, H)) || (rc = m->alloc(&L.qkv, (size_t)QKV * H)) ||
            (rc = m->alloc(&L.q_norm, D)) || (rc = m->alloc(&L.k_norm, D)) || (rc = m->alloc(&L.o, (size_t)H * QD)) ||
            (rc = m->alloc(&L.ln2, H)) || (rc = m->alloc(&L.gate_up, (size_t)2 * c.ffn * H)) ||
            (rc = m->alloc(&L.down, (size_t)H * c.ffn)) ||
            (rc = m->alloc(&L.k_cache, kv_rows * c.kv_heads * D)) ||
            (rc = m->alloc(&L.v_cache, kv_rows * c.kv_heads * D)))
            return fail(rc);
        // Weight order of decoder.rs:226-247: ln1, q, k, v, q_norm, k_norm, o, ln2, gate, up, down.
        if ((rc = launch_init_gain(m, L.ln1, H, seed, id++)) ||
            (rc = launch_init_bf16(m, L.qkv, (size_t)QD * H, seed, id++)) ||
            (rc = launch_init_bf16(m, L.qkv + (size_t)QD * H, (size_t)c.kv_heads * D * H, seed, id++)) ||
            (rc = launch_init_bf16(m, L.qkv + (size_t)(QD + c.kv_heads * D) * H, (size_t)c.kv_heads * D * H, seed,
                                   id++)) ||
            (rc = launch_init_gain(m, L.q_norm, D, seed, id++)) || (rc = launch_init_gain(m, L.k_norm, D, seed, id++)) ||
            (rc = launch_init_bf16(m, L.o, (size_t)H * QD, seed, id++)) ||
            (rc = launch_init_gain(m, L.ln2, H, seed, id++)) ||
            (rc = launch_init_bf16(m, L.gate_up, (size_t)c.ffn * H, seed, id++)) ||
            (rc = launch_init_bf16(m, L.gate_up + (size_t)c.ffn * H, (size_t)c.ffn * H, seed, id++)) ||
            (rc = launch_init_bf16(m, L.down, (size_t)H * c.ffn, seed, id++)))
            return fail(rc);
        e = hipMemsetAsync(L.k_cache, 0, kv_rows * c.kv_heads * D * 2, m->stream);
        if (e == hipSuccess) e = hipMemsetAsync(L.v_cache, 0, kv_rows * c.kv_heads * D * 2, m->stream);
        if (e != hipSuccess) return fail(ts::hip_status(e, "hipMemsetAsync"));
    }
    if ((rc = m->alloc(&m->norm, H)) || (rc = launch_init_gain(m, m->norm, H, seed, id++))) return fail(rc);
    const size_t R = c.max_prompt;
    if ((rc = m->alloc(&m->x, R * H)) || (rc = m->alloc(&m->xn, R * H)) || (rc = m->alloc(&m->qkv, R * QKV)) ||
        (rc = m->alloc(&m->q, R * QD)) || (rc = m->alloc(&m->attn, R * QD)) ||
        (rc = m->alloc(&m->h, R * c.ffn)) || (rc = m->alloc(&m->logits, (size_t)c.vocab)) ||
        (rc = m->alloc(&m->d_tok, 1)) || (rc = m->alloc(&m->d_pos, 1)) || (rc = m->alloc(&m->d_slot, 1)) ||
        (rc = m->alloc(&m->d_hist, (size_t)c.max_context + 1)) || (rc = m->alloc(&m->d_prompt, R)) ||
        (rc = m->alloc(&m->d_prompt_pos, R)) || (rc = m->alloc(&m->d_prompt_slot, R)) ||
        (rc = m->alloc(&m->d_table, m->kept_pages)) || (rc = m->alloc(&m->rope, (size_t)c.max_context * D)) ||
        (rc = m->alloc(&m->d_buffers, 2 * (size_t)c.layers)) || (rc = m->alloc(&m->d_copy, 1)) ||
        (rc = m->alloc(&m->d_key, 1)))
        return fail(rc);
    e = hipMemsetAsync(m->d_key, 0, 8, m->stream);
    if (e != hipSuccess) return fail(ts::hip_status(e, "hipMemsetAsync"));
    {
        std::vector<void *> bufs;
        for (const Layer &L : m->layers) { bufs.push_back(L.k_cache); bufs.push_back(L.v_cache); }
        e = hipMemcpyAsync(m->d_buffers, bufs.data(), bufs.size() * sizeof(void *), hipMemcpyHostToDevice, m->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
        if (e != hipSuccess) return fail(ts::hip_status(e, "buffer list upload"));
    }
    const ts_angles_args angles = {m->rope, c.max_context, D, c.theta};
    if ((rc = tessera_hip_rope_table(&angles, m->stream))) return fail(rc);
    m->ws_bytes = workspace_need(m);
    if (m->ws_bytes) {
        char *w = nullptr;
        if ((rc = m->alloc(&w, m->ws_bytes))) return fail(rc);
        m->ws = w;
        e = hipMemsetAsync(m->ws, 0, m->ws_bytes, m->stream);
        if (e != hipSuccess) return fail(ts::hip_status(e, "hipMemsetAsync"));
    }
    std::vector<uint32_t> zeros(R, 0), ramp(R);
    for (size_t i = 0; i < R; i++) ramp[i] = (uint32_t)i;
    e = hipMemcpyAsync(m->d_prompt_pos, ramp.data(), R * 4, hipMemcpyHostToDevice, m->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(m->d_prompt_slot, zeros.data(), R * 4, hipMemcpyHostToDevice, m->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(m->d_slot, zeros.data(), 4, hipMemcpyHostToDevice, m->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
    if (e != hipSuccess) return fail(ts::hip_status(e, "open upload"));
    m->pool = tessera_kv_new(m->total_pages, c.page);
    rc = ts::decode_step_supported(H, c.layers, c.heads, c.kv_heads, D, c.ffn, c.vocab, m->kept_pages);
    if (rc < 0) return fail(rc);
    if (rc == TS_OK) {
        if ((rc = ts::decode_step_groups(&m->groups))) return fail(rc);
        const size_t words = ts::decode_step_hand_words(H, c.layers, c.heads, c.kv_heads, c.ffn, m->groups);
        if ((rc = m->alloc(&m->hand, words)) || (rc = m->alloc(&m->d_error, 1))) return fail(rc);
        e = hipMemsetAsync(m->hand, 0, words * 8, m->stream);
        if (e == hipSuccess) e = hipMemsetAsync(m->d_error, 0, 4, m->stream);
        if (e != hipSuccess) return fail(ts::hip_status(e, "open: hand-off words"));
        // The step reads its own copy of the weights, laid out for its loads (made
        // once here, after the weights are written; the graph path reads the originals).
        m->packed.assign((size_t)c.layers * 4, nullptr);
        for (uint32_t l = 0; l < c.layers; l++) {
            const Layer &L = m->layers[l];
            const uint16_t *src[4] = {L.qkv, L.o, L.gate_up, L.down};
            for (uint32_t r = 0; r < 4; r++) {
                const size_t n = ts::decode_step_packed_elems(H, c.heads, c.kv_heads, c.ffn, c.vocab, m->groups, r);
                uint16_t *dst = nullptr;
                if ((rc = m->alloc(&dst, n)) ||
                    (rc = ts::decode_step_pack(src[r], dst, H, c.heads, c.kv_heads, c.ffn, c.vocab, m->groups, r,
                                               m->stream)))
                    return fail(rc);
                m->packed[(size_t)l * 4 + r] = dst;
            }
        }
        {
            const size_t n = ts::decode_step_packed_elems(H, c.heads, c.kv_heads, c.ffn, c.vocab, m->groups, 4);
            if ((rc = m->alloc(&m->lm_packed, n)) ||
                (rc = ts::decode_step_pack(m->embed, m->lm_packed, H, c.heads, c.kv_heads, c.ffn, c.vocab, m->groups,
                                           4, m->stream)))
                return fail(rc);
        }
        e = hipStreamSynchronize(m->stream);
        if (e != hipSuccess) return fail(ts::hip_status(e, "open: packed weights"));
        m->step_ok = m->use_step = true;
    }
    *out = m;
    return TS_OK;
}

extern "C" void tessera_qwen3_close(ts_qwen3 *m) {
    if (!m) return;
    // Teardown: errors here have no caller to report to; every resource is released regardless.
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    if (m->graph) (void)hipGraphExecDestroy(m->graph);
    for (void *p : m->allocs) (void)hipFree(p);
    if (m->ev0) (void)hipEventDestroy(m->ev0);
    if (m->ev1) (void)hipEventDestroy(m->ev1);
    if (m->stream) (void)hipStreamDestroy(m->stream);
    if (m->pool) tessera_kv_free(m->pool);
    delete m;
}

extern "C" int tessera_qwen3_weight(ts_qwen3 *m, const char *name, uint32_t layer, void **ptr, uint64_t *bytes,
                                    int32_t *dtype) {
    TS_REQUIRE(m && name && ptr && bytes && dtype, "qwen3_weight: null argument");
    const ts_qwen3_config &c = m->c;
    const uint64_t H = c.hidden, D = c.head_dim, QD = c.heads * D, QKV = (c.heads + 2 * c.kv_heads) * D;
    if (!strcmp(name, "embed")) { *ptr = m->embed; *bytes = c.vocab * H * 2; *dtype = TS_BF16; return TS_OK; }
    if (!strcmp(name, "norm")) { *ptr = m->norm; *bytes = H * 4; *dtype = TS_F32; return TS_OK; }
    TS_REQUIRE(layer < c.layers, "qwen3_weight: layer %u of %u", layer, c.layers);
    const Layer &L = m->layers[layer];
    struct { const char *n; void *p; uint64_t b; int32_t t; } all[] = {
        {"ln1", L.ln1, H * 4, TS_F32}, {"qkv", L.qkv, QKV * H * 2, TS_BF16}, {"q_norm", L.q_norm, D * 4, TS_F32},
        {"k_norm", L.k_norm, D * 4, TS_F32}, {"o", L.o, H * QD * 2, TS_BF16}, {"ln2", L.ln2, H * 4, TS_F32},
        {"gate_up", L.gate_up, 2 * c.ffn * H * 2, TS_BF16}, {"down", L.down, H * c.ffn * 2, TS_BF16},
        {"k_cache", L.k_cache, (uint64_t)m->total_pages * c.page * c.kv_heads * D * 2, TS_BF16},
        {"v_cache", L.v_cache, (uint64_t)m->total_pages * c.page * c.kv_heads * D * 2, TS_BF16}};
    for (auto &w : all)
        if (!strcmp(name, w.n)) { *ptr = w.p; *bytes = w.b; *dtype = w.t; return TS_OK; }
    return ts::fail(TS_ERR_ARG, "qwen3_weight: no weight named %s", name);
}

extern "C" int tessera_qwen3_read(ts_qwen3 *m, const char *name, uint32_t layer, void *host, uint64_t bytes) {
    void *ptr = nullptr;
    uint64_t have = 0;
    int32_t dtype = 0;
    TRY(tessera_qwen3_weight(m, name, layer, &ptr, &have, &dtype));
    TS_REQUIRE(host && bytes <= have, "qwen3_read: %llu bytes of %llu", (unsigned long long)bytes,
               (unsigned long long)have);
    hipError_t e = hipMemcpyAsync(host, ptr, bytes, hipMemcpyDeviceToHost, m->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
    if (e != hipSuccess) return ts::hip_status(e, "qwen3_read");
    return TS_OK;
}

namespace {

// The copy Pool::grow asked for, made in every layer's K and V before anything
// appends (engine/ir/kv/src/pool.rs:193-223).
int copy_pages(ts_qwen3 *m, const ts_kv_copy &cp) {
    hipError_t e = hipMemcpyAsync(m->d_copy, &cp, sizeof cp, hipMemcpyHostToDevice, m->stream);
    if (e != hipSuccess) return ts::hip_status(e, "page copy upload");
    ts_kv_copy_args a;
    memset(&a, 0, sizeof a);
    a.buffers = m->d_buffers; a.copies = m->d_copy; a.buffer_count = 2 * m->c.layers; a.copy_count = 1;
    a.page = m->c.page; a.row_bytes = m->c.kv_heads * m->c.head_dim * 2; a.pages = m->total_pages;
    return tessera_hip_kv_copy(&a, m->stream);
}

}  // namespace

extern "C" int tessera_qwen3_prefill(ts_qwen3 *m, const uint32_t *tokens, uint32_t count, uint32_t *next) {
    TS_REQUIRE(m && tokens && count >= 1, "qwen3_prefill: empty prompt");
    TS_REQUIRE(count <= m->c.max_prompt, "qwen3_prefill: %u tokens (at most %u)", count, m->c.max_prompt);
    for (uint32_t i = 0; i < count; i++)
        TS_REQUIRE(tokens[i] < m->c.vocab, "qwen3_prefill: token %u at %u is past the vocabulary", tokens[i], i);
    // A fresh run for the slot, grown to its worst case so the decode graph never
    // needs the table to change (lowest free pages first, pool.rs:359-372).
    if (m->have_run) tessera_kv_release(m->pool, m->run);
    int k = tessera_kv_reserve(m->pool, 0, count, m->c.max_context, &m->run);
    if (k != TS_KV_OK) return ts::fail(TS_ERR_ARG, "qwen3_prefill: page pool refused (%d)", k);
    m->have_run = true;
    ts_kv_copy cp;
    uint32_t ncp = 0;
    k = tessera_kv_grow(m->pool, m->run, m->c.max_context, &cp, &ncp);
    if (k != TS_KV_OK) return ts::fail(TS_ERR_ARG, "qwen3_prefill: page pool refused growth (%d)", k);
    if (ncp) TRY(copy_pages(m, cp));
    const uint32_t *pages = nullptr;
    uint32_t npages = 0;
    tessera_kv_pages(m->pool, m->run, &pages, &npages);
    hipError_t e = hipMemcpyAsync(m->d_table, pages, npages * 4, hipMemcpyHostToDevice, m->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(m->d_prompt, tokens, count * 4, hipMemcpyHostToDevice, m->stream);
    if (e != hipSuccess) return ts::hip_status(e, "prefill upload");
    const ts_qwen3_config &c = m->c;
    const ts_gather_args g = {m->embed, m->d_prompt, m->x, count, c.vocab, c.hidden, 0};
    TRY(tessera_hip_gather(&g, m->stream));
    TRY(run_layers(m, count, m->d_prompt_slot, m->d_prompt_pos, count - 1));
    TRY(head(m, count - 1));
    hipLaunchKernelGGL(start_kernel, dim3(1), dim3(1), 0, m->stream, m->d_key, m->d_tok, m->d_pos, m->d_hist, count,
                       c.vocab);
    TS_CHECK_LAUNCH("start");
    e = hipMemcpyAsync(next, m->d_tok, 4, hipMemcpyDeviceToHost, m->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
    if (e != hipSuccess) return ts::hip_status(e, "prefill");
    m->position = count;
    return TS_OK;
}

extern "C" int tessera_qwen3_decode(ts_qwen3 *m, uint32_t steps, uint32_t *tokens_out) {
    TS_REQUIRE(m && m->have_run, "qwen3_decode: prefill first");
    TS_REQUIRE(m->position + steps <= m->c.max_context,
               "qwen3_decode: %u steps from position %u pass the kept context %u", steps, m->position,
               m->c.max_context);
    hipError_t e;
    if (!m->ev0) {
        e = hipEventCreate(&m->ev0);
        if (e == hipSuccess) e = hipEventCreate(&m->ev1);
        if (e != hipSuccess) return ts::hip_status(e, "hipEventCreate");
    }
    const bool timed = steps > 0 && (m->use_step || m->graph || !m->use_graph);
    if (timed && (e = hipEventRecord(m->ev0, m->stream)) != hipSuccess) return ts::hip_status(e, "hipEventRecord");
    if (m->use_step && steps > 0) {
        TRY(launch_step(m, steps));
    } else if (m->use_graph && !m->graph && steps > 0) {
        hipGraph_t g = nullptr;
        e = hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal);
        if (e != hipSuccess) return ts::hip_status(e, "hipStreamBeginCapture");
        int rc = decode_step(m);
        e = hipStreamEndCapture(m->stream, &g);
        if (rc != TS_OK) {
            if (g) (void)hipGraphDestroy(g);
            return rc;
        }
        if (e != hipSuccess) return ts::hip_status(e, "hipStreamEndCapture");
        e = hipGraphInstantiate(&m->graph, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (e != hipSuccess) return ts::hip_status(e, "hipGraphInstantiate");
    }
    for (uint32_t i = 0; i < steps && !m->use_step; i++) {
        if (m->use_graph) {
            e = hipGraphLaunch(m->graph, m->stream);
            if (e != hipSuccess) return ts::hip_status(e, "hipGraphLaunch");
        } else {
            TRY(decode_step(m));
        }
    }
    if (timed && (e = hipEventRecord(m->ev1, m->stream)) != hipSuccess) return ts::hip_status(e, "hipEventRecord");
    const uint32_t first = m->position;
    m->position += steps;
    if (tokens_out && steps) {
        e = hipMemcpyAsync(tokens_out, m->d_hist + first + 1, steps * 4, hipMemcpyDeviceToHost, m->stream);
        if (e != hipSuccess) return ts::hip_status(e, "decode download");
    }
    e = hipStreamSynchronize(m->stream);
    if (e != hipSuccess) return ts::hip_status(e, "decode");
    m->decode_ms = -1.0f;
    if (timed && (e = hipEventElapsedTime(&m->decode_ms, m->ev0, m->ev1)) != hipSuccess)
        return ts::hip_status(e, "hipEventElapsedTime");
    if (m->use_step && steps > 0) {
        uint32_t err = 0;
        e = hipMemcpy(&err, m->d_error, 4, hipMemcpyDeviceToHost);
        if (e != hipSuccess) return ts::hip_status(e, "decode: error word");
        if (err) {
            // The grid left early: the step is not trusted again in this runner.
            m->use_step = m->step_ok = false;
            return ts::fail(TS_ERR_ARG, "qwen3_decode: a hand-off wait of the persistent step timed out");
        }
    }
    return TS_OK;
}

extern "C" int tessera_qwen3_logits(ts_qwen3 *m, float *host, uint64_t count) {
    TS_REQUIRE(m && host && count <= m->c.vocab, "qwen3_logits: bad arguments");
    hipError_t e = hipMemcpyAsync(host, m->logits, count * 4, hipMemcpyDeviceToHost, m->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
    if (e != hipSuccess) return ts::hip_status(e, "logits download");
    return TS_OK;
}

extern "C" int tessera_qwen3_set_token(ts_qwen3 *m, uint32_t token) {
    TS_REQUIRE(m && m->have_run, "qwen3_set_token: prefill first");
    TS_REQUIRE(token < m->c.vocab, "qwen3_set_token: token %u past the vocabulary (%u)", token, m->c.vocab);
    TS_REQUIRE(m->position <= m->c.max_context, "qwen3_set_token: context full");
    hipLaunchKernelGGL(set_token_kernel, dim3(1), dim3(1), 0, m->stream, m->d_tok, m->d_hist, m->position, token);
    TS_CHECK_LAUNCH("qwen3_set_token launch");
    return TS_OK;
}

extern "C" int tessera_qwen3_set_graph(ts_qwen3 *m, int on) {
    TS_REQUIRE(m, "qwen3_set_graph: null");
    m->use_graph = on != 0;
    return TS_OK;
}

extern "C" int tessera_qwen3_set_step(ts_qwen3 *m, int on) {
    TS_REQUIRE(m, "qwen3_set_step: null");
    TS_REQUIRE(!on || m->step_ok, "qwen3_set_step: this shape does not fit the persistent step");
    m->use_step = on != 0;
    return TS_OK;
}

extern "C" int tessera_qwen3_step_mode(ts_qwen3 *m) { return m && m->use_step ? 1 : 0; }

// Device time of the last decode call's steps (HIP events on the runner's stream
// around the persistent launch or the graph replays), ms; -1 when not timed
// (a first graph call also captures and instantiates the graph).
extern "C" float tessera_qwen3_decode_ms(ts_qwen3 *m) { return m ? m->decode_ms : -1.0f; }

// Debug: the persistent step records phase stamps into `marks` (device memory,
// groups * (layers + 2) * 10 words) on its next launches; NULL stops it.
extern "C" int tessera_qwen3_step_marks(ts_qwen3 *m, uint64_t *marks, uint32_t *groups) {
    TS_REQUIRE(m && groups, "qwen3_step_marks: null");
    m->step_marks = marks;
    *groups = m->groups;
    return TS_OK;
}

extern "C" void *tessera_qwen3_stream(ts_qwen3 *m) { return m ? (void *)m->stream : nullptr; }

extern "C" uint32_t tessera_qwen3_position(ts_qwen3 *m) { return m ? m->position : 0; }

extern "C" int tessera_qwen3_pages(ts_qwen3 *m, uint32_t *host, uint32_t count) {
    TS_REQUIRE(m && host && m->have_run, "qwen3_pages: prefill first");
    const uint32_t *pages = nullptr;
    uint32_t n = 0;
    tessera_kv_pages(m->pool, m->run, &pages, &n);
    TS_REQUIRE(count <= n, "qwen3_pages: %u of %u pages", count, n);
    memcpy(host, pages, count * 4);
    return TS_OK;
}
