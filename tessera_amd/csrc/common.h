// Shared device and host helpers for the gfx950 kernels behind libtessera_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/tessera_hip.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define TS_DEV __device__ __forceinline__


// ---------------------------------------------------------------------------
// Host-side error plumbing: a thread-local message, an int status code.
// ---------------------------------------------------------------------------
namespace ts {

int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_status(hipError_t e, const char *what);

#define TS_CHECK_LAUNCH(what)                                             \
    do {                                                                  \
        hipError_t _e = hipPeekAtLastError();                             \
        if (_e != hipSuccess) return ::ts::hip_status(_e, what);          \
    } while (0)

#define TS_REQUIRE(cond, ...)                                             \
    do {                                                                  \
        if (!(cond)) return ::ts::fail(TS_ERR_ARG, __VA_ARGS__);         \
    } while (0)

inline bool aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

// A product's stage chain (ts_linear_args.after), checked (map.hip): an empty chain
// when after is NULL; refused with TS_AFTER_ADD or TS_AFTER_ARGMAX, or with operands
// that repeat.
int linear_after(const ts_linear_args *a, const char *rule, ts_after *out);

// The vector-ALU product for m <= 4 rows (gemv.hip); arguments already checked.
int gemv_launch(const ts_linear_args *a, void *stream);

// Block-form weights (TS_Q8_0 .. TS_INT4_G128): codes a block, bytes a block, head
// bytes (blocks.hip); the m <= 4 decode product (blocks.hip) and the matrix-unit
// product for more rows (blockmat.hip), each checking its own arguments.
struct BlockShape {
    uint32_t block, bytes, head;
};
bool block_form(int32_t dtype);
BlockShape block_shape(int32_t dtype);
int block_check(const ts_linear_args *a, const char *rule);
int block_gemv_launch(const ts_linear_args *a, void *stream);
int block_tiled_launch(const ts_linear_args *a, void *stream);

// The 256x256 tiled kernel (tiled_big.hip): TS_OK when launched, 1 when the
// product is not its shape (bf16 x and w, no SiLU pair, enough tiles), else an error.
int tiled_big_launch(const ts_linear_args *a, void *stream);

// Rows of a picked product sorted by matrix (moe.hip), in the caller's workspace.
struct Route {
    uint32_t *row_start;   // [count + 2]: first sorted position per bucket (the last: out-of-range ids)
    uint32_t *tile_start;  // [count + 1]: first row tile per matrix
    uint32_t *perm;        // [rows]: row at each sorted position
};
size_t route_words(uint32_t rows, uint32_t count);
int route_launch(const uint32_t *ids, uint32_t rows, uint32_t first, uint32_t count, uint32_t tile_rows, void *ws,
                 Route *route, void *stream);
// Rows whose id is outside the set: their sum is 0, stored through the chain.
int zero_absent_launch(const Route &route, uint32_t count, void *out, uint32_t n, int out_bf16, const ts_after &after,
                       void *stream);

}  // namespace ts

// ---------------------------------------------------------------------------
// Narrow floats. bf16 narrowing is round-to-nearest-even with NaN kept quiet
// (the rule of engine/ir/graph/src/scalar.rs:20-44 for 8 exponent and 7
// mantissa bits; the bit form below gives the same code for every f32,
// subnormals and overflow to infinity included).
// ---------------------------------------------------------------------------
// f32 -> bf16, round to nearest even, on gfx950's conversion instruction
// (v_cvt_pk_bf16_f32); NaN becomes sign | 0x7fc0 through a select, not a branch (a
// branch per value made the exec-mask bookkeeping cost more than the work).
typedef __bf16 ts_bf16x2 __attribute__((ext_vector_type(2)));
typedef float ts_f32x2 __attribute__((ext_vector_type(2)));
TS_DEV uint32_t pack_bf16x2(float a, float b) {
    uint32_t r = __builtin_bit_cast(uint32_t, __builtin_convertvector(ts_f32x2{a, b}, ts_bf16x2));
    const uint32_t ua = __float_as_uint(a), ub = __float_as_uint(b);
    const uint32_t na = ((ua >> 16) & 0x8000u) | 0x7fc0u, nb = (ub & 0x80000000u) | 0x7fc00000u;
    r = (ua & 0x7fffffffu) > 0x7f800000u ? (r & 0xffff0000u) | na : r;
    r = (ub & 0x7fffffffu) > 0x7f800000u ? (r & 0x0000ffffu) | nb : r;
    return r;
}
TS_DEV uint16_t bf16_bits(float x) { return (uint16_t)(pack_bf16x2(x, 0.0f) & 0xffffu); }
TS_DEV float bf16_float(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
TS_DEV float bf16_round(float x) { return bf16_float(bf16_bits(x)); }

TS_DEV float lo_bf16(uint32_t v) { return __uint_as_float(v << 16); }
TS_DEV float hi_bf16(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

typedef float ts_f32x2_t __attribute__((ext_vector_type(2)));

// OCP e4m3 (e4m3fn) code -> f32 on gfx950's conversion (scale 1.0: exact, subnormals
// included); codes 0x7F / 0xFF give NaN, as the format defines (and the interpreter's
// widening does).
TS_DEV float e4m3_float(uint32_t c) { return __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(c, 1.0f, false)[0]; }

// Four e4m3 codes (byte order) -> four f32, the same conversion two at a time.
TS_DEV void e4m3x4_float(uint32_t w, float *f) {
    const ts_f32x2_t lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, 1.0f, false);
    const ts_f32x2_t hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, 1.0f, true);
    f[0] = lo[0]; f[1] = lo[1]; f[2] = hi[0]; f[3] = hi[1];
}

// Four e4m3 codes (one u32) -> two packed bf16 pairs (exact: 3 mantissa bits).
// Four e4m3 codes (OCP e4m3fn: bias 7, subnormals, NaN 0x7f/0xff) to four bf16, in
// byte order, with the gfx950 conversion (scale 1.0): every e4m3 value is exact in bf16.
TS_DEV u32x2 e4m3x4_to_bf16x4(uint32_t w) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
    const bf16x2_t hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true);
    return u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
}

// Four e4m3 codes to f32, in byte order (gfx950 v_cvt_pk_f32_fp8; exact).
TS_DEV void e4m3x4_to_f32(uint32_t w, float *f) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    const f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8(w, false), hi = __builtin_amdgcn_cvt_pk_f32_fp8(w, true);
    f[0] = lo[0]; f[1] = lo[1]; f[2] = hi[0]; f[3] = hi[1];
}

// The argmax key of entry n with value v, ordered as the pick (argmax_spans):
// larger values first, then lower indices; 0 (never the max) for NaN and -inf.
TS_DEV uint64_t argmax_key(float v, uint32_t n) {
    if (!(v > -__builtin_inff())) return 0;  // NaN or -inf
    const uint32_t f = __float_as_uint(v);
    const uint32_t ord = (f & 0x80000000u) ? ~f : (f | 0x80000000u);
    return ((uint64_t)ord << 32) | (uint32_t)~n;
}

// ---------------------------------------------------------------------------
// Wave64 reductions (DPP/permute via the compiler's __shfl_xor).
// ---------------------------------------------------------------------------
// DPP moves within a row of 16 lanes: quad_perm [1,0,3,2] (xor 1), quad_perm
// [2,3,0,1] (xor 2), row_half_mirror (lane i <-> 7-i of each 8), row_mirror
// (i <-> 15-i). After the four steps every lane of the row holds the row's
// total; each step is one VALU op with a DPP source, not an LDS round trip.
TS_DEV float dpp_f(float v, int ctrl_id) {
    const int x = __float_as_int(v);
    int r;
    switch (ctrl_id) {
    case 0: r = __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false); break;
    case 1: r = __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false); break;
    case 2: r = __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false); break;
    default: r = __builtin_amdgcn_update_dpp(0, x, 0x140, 0xF, 0xF, false); break;
    }
    return __int_as_float(r);
}

TS_DEV float row16_sum(float v) {
    v += dpp_f(v, 0);
    v += dpp_f(v, 1);
    v += dpp_f(v, 2);
    v += dpp_f(v, 3);
    return v;
}

TS_DEV float row16_max(float v) {
    v = fmaxf(v, dpp_f(v, 0));
    v = fmaxf(v, dpp_f(v, 1));
    v = fmaxf(v, dpp_f(v, 2));
    v = fmaxf(v, dpp_f(v, 3));
    return v;
}

// Whole-wave totals in every lane: rows by DPP, then two cross-row exchanges.
TS_DEV float wave_sum(float v) {
    v = row16_sum(v);
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

TS_DEV float wave_max(float v) {
    v = row16_max(v);
    v = fmaxf(v, __shfl_xor(v, 16, 64));
    v = fmaxf(v, __shfl_xor(v, 32, 64));
    return v;
}

// MFMA 16x16x32 bf16 -> f32. Operand lane layout (wave64): A lane l holds row
// l%16, eight k values of the k-group l/16; B lane l holds column l%16 and the
// same k-group; D lane l holds column l%16, rows 4*(l/16)+0..3.
TS_DEV f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// D = A * B^T + C on a 32 x 32 x 16 tile. A lane l: row l % 32, k 8 (l / 32) .. +7;
// B likewise by column; D lane l: column l % 32, rows 8 (r / 4) + 4 (l / 32) + r % 4.
TS_DEV f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) { return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0); }

// A group barrier that publishes LDS writes (lgkmcnt(0)) but leaves global loads in
// flight. __syncthreads() also fences global memory, which makes the compiler wait
// for every outstanding load (vmcnt(0)) first and drains any prefetch. The memory
// clobber keeps the compiler from moving LDS accesses across it.
TS_DEV void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

TS_DEV bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// In-kernel marks (the reference's TS_MARK ledger, engine/plan/run/src/marks.cuh):
// with TS_MARKS defined, TS_MARK(ledger, i) records the 100 MHz real-time clock
// for mark i of this group's first thread into ledger[group * 16 + i].
#ifdef TS_MARKS
#define TS_MARK(ledger, i)                                                                      \
    do {                                                                                        \
        if ((ledger) && threadIdx.x == 0) {                                                     \
            const uint32_t _g = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z); \
            (ledger)[_g * 16 + (i)] = __builtin_amdgcn_s_memrealtime();                         \
        }                                                                                       \
    } while (0)
#else
#define TS_MARK(ledger, i) \
    do {                   \
    } while (0)
#endif
