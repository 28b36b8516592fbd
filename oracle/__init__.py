"""TEST INFRASTRUCTURE ONLY: numpy bindings of the C restatement of tessera-interp.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
may import this package, and only as the checker. The product library
(``tessera_amd``) never imports it.

Each wrapper names the reference function it restates (paths relative to the
reference repository root).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i64 = C.c_int64

ACTS = {"gelu_tanh": 0, "silu": 1, "sigmoid": 2, "relu": 3, "softplus": 4, "exp": 5, "tanh": 6}
BIG = 1 << 62  # a mask window of "all keys"


def build() -> None:
    """Compiles interp.c into liboracle.so (gcc, no reference sources involved)."""
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    L = C.CDLL(LIB_PATH)
    sig = {
        "or_set_threads": (None, [C.c_int]),
        "or_threads_available": (C.c_int, []),
        "or_bf16_narrow": (C.c_uint16, [C.c_float]),
        "or_bf16_widen": (C.c_float, [C.c_uint16]),
        "or_bf16_widen_exact": (C.c_float, [C.c_uint16]),
        "or_e4m3_narrow": (C.c_uint8, [C.c_float]),
        "or_e4m3_widen": (C.c_float, [C.c_uint8]),
        "or_bf16_narrow_n": (None, [_f32p, _u16p, _i64]),
        "or_bf16_widen_n": (None, [_u16p, _f32p, _i64]),
        "or_e4m3_narrow_n": (None, [_f32p, _u8p, _i64]),
        "or_e4m3_widen_n": (None, [_u8p, _f32p, _i64]),
        "or_noise": (None, [C.POINTER(C.c_uint64), _f32p, _i64]),
        "or_acc_sum": (C.c_float, [C.c_int, _f32p, _i64]),
        "or_product": (None, [_i64, _i64, _i64, _f32p, _f32p, _f32p]),
        "or_product_bf16w": (None, [_i64, _i64, _i64, _f32p, _u16p, _f32p]),
        "or_product_e4m3w": (None, [_i64, _i64, _i64, _f32p, _u8p, _u16p, _f32p]),
        "or_product_picked_bf16w": (None, [_i64, _i64, _i64, _i64, _f32p, _u16p, _i64, _u32p, _i64, _f32p]),
        "or_act": (None, [C.c_int, _f32p, _i64]),
        "or_softmax": (None, [_f32p, _i64, _i64]),
        "or_rms_norm": (None, [_f32p, _i64, _i64, C.c_void_p, C.c_float]),
        "or_angle": (C.c_float, [_i64, _i64, _i64, C.c_float]),
        "or_rope": (None, [_f32p, _i64, _i64, _u32p, _i64, C.c_float, C.c_int, _i64]),
        "or_attend": (C.c_int, [_i64] * 7 + [C.c_float, _i64, _i64, C.c_int, _f32p, _f32p, _f32p, _f32p]),
        "or_paged_row": (C.c_uint64, [_u32p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32]),
        "or_attend_rows": (C.c_int, [_i64] * 5 + [C.c_float, _i64, _i64, _i64, _f32p, _f32p, _f32p,
                                                 _u32p, _u32p, C.c_void_p, C.c_uint32, C.c_uint32, _f32p]),
        "or_top_k": (None, [_f32p, _i64, _i64, _i64, _u32p]),
        "or_take": (None, [_f32p, _i64, _i64, _u32p, _i64, _f32p]),
        "or_gather": (None, [C.c_void_p, _i64, _i64, _u32p, _i64, _i64, C.c_void_p]),
        "or_mix": (None, [_f32p, _i64, _i64, _i64, C.c_void_p, _f32p]),
        "or_f16_narrow": (C.c_uint16, [C.c_float]),
        "or_f16_widen": (C.c_float, [C.c_uint16]),
        "or_e8m0_narrow": (C.c_uint8, [C.c_float]),
        "or_e8m0_widen": (C.c_float, [C.c_uint8]),
        "or_block_bytes": (C.c_int, [C.c_int]),
        "or_block_size": (C.c_int, [C.c_int]),
        "or_block_head": (C.c_int, [C.c_int]),
        "or_block_tensor_bytes": (_i64, [C.c_int, _i64]),
        "or_e2m1_narrow": (C.c_uint8, [C.c_float]),
        "or_e2m1_widen": (C.c_float, [C.c_uint8]),
        "or_block_pack": (None, [C.c_int, _f32p, _i64, _u8p]),
        "or_block_unpack": (C.c_float, [C.c_int, _u8p, _i64]),
        "or_block_unpack_n": (None, [C.c_int, _u8p, _i64, _i64, _f32p]),
        "or_block_dot": (C.c_float, [C.c_int, _f32p, _u8p, _i64, _i64]),
        "or_block_product": (None, [C.c_int, _i64, _i64, _i64, _f32p, _u8p, _f32p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def set_threads(n: int) -> None:
    lib().or_set_threads(int(n))


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u32(a):
    return np.ascontiguousarray(a, dtype=np.uint32)


# --- narrow floats: engine/ir/graph/src/scalar.rs:20-59 -------------------------

def bf16_narrow(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().or_bf16_narrow_n(x.reshape(-1), out.reshape(-1), x.size)
    return out


def bf16_widen(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().or_bf16_widen_n(b.reshape(-1), out.reshape(-1), b.size)
    return out


def bf16_round(x) -> np.ndarray:
    return bf16_widen(bf16_narrow(x))


def e4m3_narrow(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, np.uint8)
    lib().or_e4m3_narrow_n(x.reshape(-1), out.reshape(-1), x.size)
    return out


def e4m3_widen(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint8)
    out = np.empty(b.shape, np.float32)
    lib().or_e4m3_widen_n(b.reshape(-1), out.reshape(-1), b.size)
    return out


# --- engine/ir/testkit/src/noise.rs:5-10 ---------------------------------------

class Noise:
    """The reference's test LCG: values in [-1, 1)."""

    def __init__(self, seed: int):
        self.state = C.c_uint64(seed)

    def draw(self, n: int) -> np.ndarray:
        out = np.empty(n, np.float32)
        lib().or_noise(C.byref(self.state), out, n)
        return out


def acc_sum(values, acc: str = "f32") -> float:
    """Acc::sum (engine/ir/interp/src/round.rs:18-30)."""
    return lib().or_acc_sum({"f32": 0, "f16": 1, "bf16": 2}[acc], _f32(values), len(values))


# --- products: engine/ir/interp/src/cpu.rs:82-138 -------------------------------

def product(x, w) -> np.ndarray:
    """out = x @ w.T summed sequentially in f32; w f32 [N, K]."""
    x, w = _f32(x), _f32(w)
    m, k = x.shape
    n = w.shape[0]
    out = np.empty((m, n), np.float32)
    lib().or_product(m, n, k, x, w, out)
    return out


def product_bf16w(x, w_bits) -> np.ndarray:
    """product with w stored as bf16 bits [N, K] (widened per element)."""
    x = _f32(x)
    w_bits = np.ascontiguousarray(w_bits, dtype=np.uint16)
    m, k = x.shape
    n = w_bits.shape[0]
    out = np.empty((m, n), np.float32)
    lib().or_product_bf16w(m, n, k, x, w_bits, out)
    return out


def product_e4m3w(x, codes, scale_bits) -> np.ndarray:
    """product with w = e4m3(code) * bf16(scale[row]) (exlr8.rs:133-137 row dequant)."""
    x = _f32(x)
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    scale_bits = np.ascontiguousarray(scale_bits, dtype=np.uint16)
    m, k = x.shape
    n = codes.shape[0]
    out = np.empty((m, n), np.float32)
    lib().or_product_e4m3w(m, n, k, x, codes, scale_bits, out)
    return out


def product_picked_bf16w(x, table_bits, ids, first: int = 0) -> np.ndarray:
    """matmul_picked (cpu.rs:89-105): row b multiplies table[ids[b]-first]; x rows repeat."""
    x = _f32(x)
    table_bits = np.ascontiguousarray(table_bits, dtype=np.uint16)
    ids = _u32(ids).reshape(-1)
    m, k = x.shape
    experts, n, _ = table_bits.shape
    rows = max(m, ids.size)
    out = np.empty((rows, n), np.float32)
    lib().or_product_picked_bf16w(rows, m, n, k, x, table_bits, experts, ids, first, out)
    return out


# --- row stages: cpu.rs:8-59, 353-447 -----------------------------------------

def act(kind: str, x) -> np.ndarray:
    out = _f32(x).copy()
    lib().or_act(ACTS[kind], out.reshape(-1), out.size)
    return out


def chain(total, stages, operands=(), sum_at: int = 0, spans=None) -> np.ndarray:
    """A stage chain on `total` (a product's sum, or map's input): v = read 0, then each
    stage in order, each read operand `Add`/`Mul` the next one (kernels/map.rs:125-185
    stage_stmts / finish: read `sum_at` is `total`, the others the operands in order),
    every operation one f32 rounding as interp's Stage::Add/Mul/Scale/Act
    (cpu.rs:353-390; an operand with span s repeats, read at i % s, cpu.rs:362-366).
    stages: "add", "mul", ("scale", by), or an activation name."""
    total = _f32(total)
    flat = total.reshape(-1)
    n = flat.size
    spans = list(spans or [0] * len(operands))

    def read(i):
        if i == sum_at:
            return flat
        j = i if i < sum_at else i - 1
        o = _f32(operands[j]).reshape(-1)
        return o[np.arange(n) % spans[j]] if spans[j] else o

    v = read(0).copy()
    nxt = 1
    for st in stages:
        if st in ("add", "mul"):
            x = read(nxt)
            nxt += 1
            v = (v + x) if st == "add" else (v * x)
        elif isinstance(st, tuple) and st[0] == "scale":
            v = v * np.float32(st[1])
        else:
            v = act(st, v)
        v = v.astype(np.float32)
    return v.reshape(total.shape)


def softmax(x) -> np.ndarray:
    out = _f32(x).copy()
    w = out.shape[-1]
    lib().or_softmax(out.reshape(-1), out.size // w, w)
    return out


def rms_norm(x, g, eps: float) -> np.ndarray:
    out = _f32(x).copy()
    w = out.shape[-1]
    gp = None
    if g is not None:
        g = _f32(g)
        gp = g.ctypes.data
    lib().or_rms_norm(out.reshape(-1), out.size // w, w, gp, eps)
    return out


def angle(pos: int, j: int, width: int, theta: float) -> float:
    return lib().or_angle(pos, j, width, theta)


def rope(x, positions, theta: float, pairs: str = "halves", turned: int = -1) -> np.ndarray:
    """Rope over the last axis; one equal block of x per position."""
    out = _f32(x).copy()
    pos = _u32(positions).reshape(-1)
    lib().or_rope(out.reshape(-1), out.size, pos.size, pos, out.shape[-1], theta,
                  1 if pairs == "halves" else 0, turned)
    return out


# --- attention: cpu.rs:61-77, 141-225, 293-351 --------------------------------

def window(mask: str, n: int = 0):
    """Mask::window (engine/ir/graph/src/node.rs:174-181) as (back, ahead, causal)."""
    return {"causal": (BIG, 0, 1), "bidirectional": (BIG, BIG, 0),
            "within": (n, n, 0), "back": (n, 0, 1)}[mask]


def attend(q, k, v, scale: float, mask: str = "causal", n: int = 0) -> np.ndarray:
    q, k, v = _f32(q), _f32(k), _f32(v)
    seqs, ctx, heads, d = q.shape
    keys, kvh, dv = k.shape[1], k.shape[2], v.shape[3]
    back, ahead, causal = window(mask, n)
    out = np.empty((seqs, ctx, heads, dv), np.float32)
    rc = lib().or_attend(seqs, ctx, keys, heads, kvh, d, dv, scale, back, ahead, causal, q, k, v, out)
    if rc != 0:
        raise ValueError(f"{ctx} queries, {keys} keys")
    return out


def attend_rows(q, k_rows, v_rows, slots, positions, keys: int, scale: float,
                mask: str = "causal", n: int = 0, table=None, kept_pages: int = 0,
                page: int = 16) -> np.ndarray:
    """Ragged rows over kept K/V rows ([*, kv_heads, d]); dense (slot*keys + j) or paged."""
    q, k_rows, v_rows = _f32(q), _f32(k_rows), _f32(v_rows)
    rows, heads, d = q.shape
    kvh, dv = k_rows.shape[-2], v_rows.shape[-1]
    back, ahead, _ = window(mask, n)
    slots, positions = _u32(slots), _u32(positions)
    tp = None
    if table is not None:
        table = _u32(table)
        tp = table.ctypes.data
    out = np.empty((rows, heads, dv), np.float32)
    rc = lib().or_attend_rows(rows, heads, kvh, d, dv, scale, back, ahead, keys,
                              q, k_rows.reshape(-1), v_rows.reshape(-1), slots, positions,
                              tp, kept_pages, page, out)
    if rc != 0:
        raise ValueError("a row's position is past the keys")
    return out


def paged_row(table, kept_pages: int, page: int, slot: int, pos: int) -> int:
    return lib().or_paged_row(_u32(table), kept_pages, page, slot, pos)


# --- indices: run.rs:577-591, cpu.rs:450-525 -----------------------------------

def top_k(x, k: int) -> np.ndarray:
    x = _f32(x)
    width = x.shape[-1]
    rows = x.size // max(width, 1)
    ids = np.empty(x.shape[:-1] + (k,), np.uint32)
    lib().or_top_k(x.reshape(-1), rows, width, k, ids.reshape(-1))
    return ids


def take(x, ids) -> np.ndarray:
    x, ids = _f32(x), _u32(ids)
    width = x.shape[-1]
    rows = x.size // max(width, 1)
    out = np.empty(ids.shape, np.float32)
    lib().or_take(x.reshape(-1), rows, width, ids.reshape(-1), ids.size, out.reshape(-1))
    return out


def gather(table, ids, first: int = 0) -> np.ndarray:
    table = np.ascontiguousarray(table)
    ids = _u32(ids)
    rows = table.shape[0]
    row_bytes = table.nbytes // max(rows, 1)
    out = np.empty(ids.shape + table.shape[1:], table.dtype)
    lib().or_gather(table.ctypes.data, rows, row_bytes, ids.reshape(-1), ids.size, first, out.ctypes.data)
    return out


def mix(x, weights=None) -> np.ndarray:
    """mean over axis 1 of [outer, count, inner]; with weights [outer, count], Σ w·x."""
    x = _f32(x)
    outer, count = x.shape[0], x.shape[1]
    inner = x.size // max(outer * count, 1)
    out = np.empty((outer,) + x.shape[2:], np.float32)
    wp = None
    if weights is not None:
        weights = _f32(weights)
        wp = weights.ctypes.data
    lib().or_mix(x.reshape(-1), outer, count, inner, wp, out.reshape(-1))
    return out


# --- block forms: engine/ir/mem/src/block.rs:1-291 --------------------------------
# A packed tensor is [head] then its blocks in element order; a [n, k] matrix (k a
# multiple of the block) has row r's blocks from head + r k / B block bytes on.
BLOCK_FORMS = {"q8_0": 0, "mxfp8": 1, "int4_g32": 2, "q4_0": 3, "nvfp4": 4, "mxfp4": 5, "int4_g128": 6}


def block_bytes(form: str) -> int:
    """Bytes of one block (scale and codes)."""
    return lib().or_block_bytes(BLOCK_FORMS[form])


def block_size(form: str) -> int:
    return lib().or_block_size(BLOCK_FORMS[form])


def block_head(form: str) -> int:
    return lib().or_block_head(BLOCK_FORMS[form])


def block_pack(form: str, data) -> np.ndarray:
    """Packs data (any shape, flattened in C order) as one tensor: uint8 [bytes(n)]."""
    d = _f32(np.ravel(data))
    out = np.zeros(lib().or_block_tensor_bytes(BLOCK_FORMS[form], d.size), np.uint8)
    lib().or_block_pack(BLOCK_FORMS[form], d, d.size, out)
    return out


def block_unpack(form: str, tensor: np.ndarray, count: int, first: int = 0) -> np.ndarray:
    """Elements first .. first + count of a packed tensor."""
    b = np.ascontiguousarray(tensor, dtype=np.uint8)
    out = np.empty(count, np.float32)
    lib().or_block_unpack_n(BLOCK_FORMS[form], b, first, count, out)
    return out


def block_dot(form: str, x, tensor, at: int = 0) -> float:
    """Block::dot: x against the tensor's elements from `at` (a block start) on."""
    x = _f32(x)
    return lib().or_block_dot(BLOCK_FORMS[form], x, np.ascontiguousarray(tensor, dtype=np.uint8), at, x.size)


def block_product(form: str, x, wb, n: int) -> np.ndarray:
    """out[m, r] = dot(x[m], the packed [n, k] tensor from element r k), per output."""
    x = _f32(np.atleast_2d(x))
    wb = np.ascontiguousarray(wb, dtype=np.uint8)
    m, k = x.shape
    out = np.empty((m, n), np.float32)
    lib().or_block_product(BLOCK_FORMS[form], m, n, k, x, wb.reshape(-1), out)
    return out
