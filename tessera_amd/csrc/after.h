// The general stage chain a product's sum runs through before its store, and the
// standalone map over an input (ts_after in include/tessera_hip.h).
//
// The reference generates one kernel per chain (engine/plan/lower/src/kernels/map.rs:
// 125-185, stage_stmts and finish); here the chain is data: a ts_after passed by value
// in each kernel's parameters, read with compile-time indices only (unrolled stages,
// operands picked by selects), so it stays in scalar registers and never reaches
// scratch memory. Kernels call after_apply only when count > 0 (a uniform branch).
#pragma once

#include "common.h"

namespace ts {

// Stage arithmetic exactly as the interpreter evaluates it (engine/ir/interp/src/
// cpu.rs:8-29 act, :353-390 stage): every operation rounded on its own.
TS_DEV float act_value(int a, float x) {
#pragma clang fp contract(off)
    switch (a) {
    case TS_ACT_GELU_TANH: {
        const float inner = 0.7978846f * (x + 0.044715f * x * x * x);
        return 0.5f * x * (1.0f + tanhf(inner));
    }
    case TS_ACT_SILU: return x / (1.0f + expf(-x));
    case TS_ACT_SIGMOID: return 1.0f / (1.0f + expf(-x));
    case TS_ACT_RELU: return x > 0.0f ? x : 0.0f;  // NaN -> 0, as f32::max(NaN, 0)
    case TS_ACT_SOFTPLUS: return fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x)));
    case TS_ACT_EXP: return expf(x);
    default: return tanhf(x);
    }
}

// Operand j's element for output index `at` (SPANS: the operand may repeat).
template <bool SPANS>
TS_DEV float after_load(const ts_after &c, uint32_t j, size_t at) {
    const float *o = c.operand[j];
    if (!SPANS) return o[at];
    const uint32_t span = c.spans[j];
    return o[span == 0 ? at : span == 1 ? 0 : at % span];
}

// The chain over the E values one thread finishes. On entry v[e] holds value e's sum
// (after any SiLU pair and weight scale), on exit its finished value; at(e) is its
// output index and ok(e) whether it is stored (values that are not read nothing).
// The stages run one at a time over all E values (a loop over the stages, reading
// them from the kernel's parameters at run time), so each stage kind's code appears
// once per value: a chain costs no more code than its longest stage.
template <int E, bool SPANS, class At, class Ok>
TS_DEV void after_values(const ts_after &c, float (&v)[E], At at, Ok ok) {
#pragma clang fp contract(off)
    float sum[E];  // the sums, when the chain starts from an operand (sum != 0)
    if (c.sum != 0) {
#pragma unroll
        for (int e = 0; e < E; e++) {
            sum[e] = v[e];
            v[e] = ok(e) ? after_load<SPANS>(c, 0, at(e)) : 0.0f;
        }
    }
    uint32_t next = 1;  // the chain's next read
    for (uint32_t s = 0; s < c.count; s++) {
        const ts_map_stage st = c.stage[s];
        if (st.op == TS_MAP_ADD || st.op == TS_MAP_MUL) {
            const uint32_t i = next++;
            const bool is_sum = i == c.sum;
            const uint32_t j = i < c.sum ? i : i - 1;
            const bool add = st.op == TS_MAP_ADD;
#pragma unroll
            for (int e = 0; e < E; e++) {
                const float x = is_sum ? sum[e] : ok(e) ? after_load<SPANS>(c, j, at(e)) : 0.0f;
                v[e] = add ? v[e] + x : v[e] * x;
            }
        } else if (st.op == TS_MAP_SCALE) {
#pragma unroll
            for (int e = 0; e < E; e++) v[e] = v[e] * st.by;
        } else {
            switch (st.act) {
#define TS_ACT_CASE(A)                                                   \
    case A:                                                              \
        _Pragma("unroll") for (int e = 0; e < E; e++) v[e] = act_value(A, v[e]); \
        break;
            TS_ACT_CASE(TS_ACT_GELU_TANH)
            TS_ACT_CASE(TS_ACT_SILU)
            TS_ACT_CASE(TS_ACT_SIGMOID)
            TS_ACT_CASE(TS_ACT_RELU)
            TS_ACT_CASE(TS_ACT_SOFTPLUS)
            TS_ACT_CASE(TS_ACT_EXP)
            default: TS_ACT_CASE(TS_ACT_TANH)
#undef TS_ACT_CASE
            }
        }
    }
}

// One value (product kernels that finish one output at a time).
TS_DEV float after_apply(const ts_after &c, float sum, size_t at) {
    float v[1] = {sum};
    after_values<1, false>(c, v, [&](int) { return at; }, [](int) { return true; });
    return v[0];
}

// Host side: a chain's validity for a product (no repeating operands) or for map;
// the number of operands it reads. Fills `out` with an empty chain when `c` is NULL.
int after_check(const ts_after *c, bool product, const char *rule, ts_after *out);

}  // namespace ts
