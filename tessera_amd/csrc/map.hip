// Elementwise chains: the standalone map (rule "map") and the host check of every
// stage chain a product or map receives.
//
// The reference's Map launches one thread per element over a generated chain
// (engine/plan/lower/src/kernels/map.rs:29-35,187-260). Here one kernel serves every
// chain: each thread takes four consecutive elements, x read and out written with
// 16-byte accesses when aligned, the operands read by the chain itself (their four
// elements share a line). HBM-bound: 4 + 4 per operand + 4 bytes an element.
#include <algorithm>

#include "after.h"

namespace ts {

namespace {

constexpr uint32_t kMapThreads = 256;

__global__ __launch_bounds__(kMapThreads) void map_kernel(const float *x, float *out, uint32_t len, ts_after c,
                                                          int vec) {
    const uint32_t stride = gridDim.x * kMapThreads * 4;
    for (uint32_t i0 = (blockIdx.x * kMapThreads + threadIdx.x) * 4; i0 < len; i0 += stride) {
        float xs[4];
        if (vec && i0 + 4 <= len) {
            const f32x4 v = *(const f32x4 *)(x + i0);
            xs[0] = v[0]; xs[1] = v[1]; xs[2] = v[2]; xs[3] = v[3];
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++) xs[e] = i0 + e < len ? x[i0 + e] : 0.0f;
        }
        float r[4] = {xs[0], xs[1], xs[2], xs[3]};
        after_values<4, true>(c, r, [&](int e) { return (size_t)i0 + e; }, [&](int e) { return i0 + e < len; });
        if (vec && i0 + 4 <= len) {
            *(f32x4 *)(out + i0) = f32x4{r[0], r[1], r[2], r[3]};
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (i0 + e < len) out[i0 + e] = r[e];
        }
    }
}

}  // namespace

int after_check(const ts_after *c, bool product, const char *rule, ts_after *out) {
    *out = ts_after{};
    if (!c) return TS_OK;
    TS_REQUIRE(c->count <= TS_MAP_STAGES, "%s: %u stages (at most %d)", rule, c->count, TS_MAP_STAGES);
    uint32_t reads = 0;
    for (uint32_t s = 0; s < c->count; s++) {
        const ts_map_stage &st = c->stage[s];
        TS_REQUIRE(st.op >= TS_MAP_ADD && st.op <= TS_MAP_ACT, "%s: stage %u op %d", rule, s, st.op);
        TS_REQUIRE(st.op != TS_MAP_ACT || (st.act >= TS_ACT_GELU_TANH && st.act <= TS_ACT_TANH),
                   "%s: stage %u activation %d", rule, s, st.act);
        if (st.op == TS_MAP_ADD || st.op == TS_MAP_MUL) reads++;
    }
    TS_REQUIRE(reads <= TS_MAP_OPERANDS, "%s: %u operands (at most %d)", rule, reads, TS_MAP_OPERANDS);
    TS_REQUIRE(c->sum <= reads, "%s: sum is read %u of %u", rule, c->sum, reads + 1);
    for (uint32_t j = 0; j < reads; j++) {
        TS_REQUIRE(c->operand[j], "%s: operand %u is NULL", rule, j);
        TS_REQUIRE(!product || c->spans[j] == 0, "%s: operand %u repeats (span %u): a product's operands are "
                   "as long as its output", rule, j, c->spans[j]);
    }
    *out = *c;
    for (uint32_t j = reads; j < TS_MAP_OPERANDS; j++) {
        out->operand[j] = nullptr;
        out->spans[j] = 0;
    }
    return TS_OK;
}

int linear_after(const ts_linear_args *a, const char *rule, ts_after *out) {
    *out = ts_after{};
    if (!a->after) return TS_OK;
    TS_REQUIRE(!(a->stages & (TS_AFTER_ADD | TS_AFTER_ARGMAX)),
               "%s: a stage chain replaces TS_AFTER_ADD and cannot follow TS_AFTER_ARGMAX", rule);
    return after_check(a->after, true, rule, out);
}

}  // namespace ts

extern "C" int tessera_hip_map(const ts_map_args *a, void *stream) {
    TS_REQUIRE(a && a->x && a->out, "map: x and out are required");
    ts_after c;
    int rc = ts::after_check(&a->after, false, "map", &c);
    if (rc) return rc;
    if (a->len == 0) return TS_OK;
    bool vec = ts::aligned(a->x, 16) && ts::aligned(a->out, 16);
    uint32_t reads = 0;
    for (uint32_t s = 0; s < c.count; s++) reads += c.stage[s].op == TS_MAP_ADD || c.stage[s].op == TS_MAP_MUL;
    for (uint32_t j = 0; j < reads; j++) vec = vec && (c.spans[j] != 0 || ts::aligned(c.operand[j], 16));
    const uint32_t quads = (a->len + 3) / 4;
    const uint32_t groups = std::min<uint32_t>((quads + ts::kMapThreads - 1) / ts::kMapThreads, 4096u);
    hipLaunchKernelGGL(ts::map_kernel, dim3(groups), dim3(ts::kMapThreads), 0, (hipStream_t)stream, a->x, a->out,
                       a->len, c, vec ? 1 : 0);
    TS_CHECK_LAUNCH("map launch");
    return TS_OK;
}

namespace ts {
namespace {

// hi = bf16(w), lo = bf16(w - hi), both round to nearest even (NaN kept quiet).
__global__ __launch_bounds__(256) void pack_f32_kernel(const float *w, uint16_t *out, uint64_t count) {
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < count; i += (uint64_t)gridDim.x * 256) {
        const float v = w[i];
        const uint16_t hi = bf16_bits(v);
        out[i] = hi;
        out[count + i] = bf16_bits(v - bf16_float(hi));
    }
}

}  // namespace
}  // namespace ts

extern "C" int tessera_hip_pack_f32(const ts_pack_args *a, void *stream) {
    TS_REQUIRE(a && a->w && a->out, "pack_f32: null pointer");
    const uint64_t count = (uint64_t)a->n * a->k;
    if (count == 0) return TS_OK;
    const uint32_t groups = (uint32_t)std::min<uint64_t>((count + 255) / 256, 8192);
    hipLaunchKernelGGL(ts::pack_f32_kernel, dim3(groups), dim3(256), 0, (hipStream_t)stream, a->w,
                       (uint16_t *)a->out, count);
    TS_CHECK_LAUNCH("pack_f32 launch");
    return TS_OK;
}
