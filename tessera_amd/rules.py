"""Host-side mirror of the reference's lowering-rule kernels, over torch device tensors.

Each function is named for the reference rule whose kernel it launches
(``tiled``, ``lanes``, ``linear``, ``attend_rows``, ``flash_rows``, ``rms_norm``,
``rope``, ``argmax``, ``top_k``, ``gather``) and takes the same operands in the
same order as that rule's Launch (reads, epilogue operands, output, counts:
engine/plan/lower/src/abi.rs:148-153, product.rs:70-76, rule.rs:92-110).
torch only provides device memory and the current stream; every computation is
a call into libtessera_hip.so through ``tessera_amd.abi``. Errors raise
``abi.HipError`` with the library's message.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import abi

_DT = {torch.float32: abi.TS_F32, torch.bfloat16: abi.TS_BF16, torch.uint8: abi.TS_E4M3,
       torch.float8_e4m3fn: abi.TS_E4M3}


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


class Workspace:
    """Caller-owned scratch for split-K / split-KV partials: grown on demand, zeroed
    once when (re)allocated (the kernels return their counters to zero)."""

    def __init__(self, device="cuda"):
        self.device = device
        self.buf = None

    def get(self, nbytes: int):
        if nbytes == 0:
            return None, 0
        if self.buf is None or self.buf.numel() < nbytes:
            self.buf = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=self.device)
        return C.c_void_p(self.buf.data_ptr()), self.buf.numel()


_ws = {}


def workspace(device) -> Workspace:
    key = str(device)
    if key not in _ws:
        _ws[key] = Workspace(device)
    return _ws[key]


BLOCK_FORMS = {"q8_0": abi.TS_Q8_0, "mxfp8": abi.TS_MXFP8, "int4_g32": abi.TS_INT4_G32, "q4_0": abi.TS_Q4_0,
               "nvfp4": abi.TS_NVFP4, "mxfp4": abi.TS_MXFP4, "int4_g128": abi.TS_INT4_G128}


def chain(stages, operands=(), *, sum_at=0, spans=None):
    """A stage chain (ts_after) for a product's epilogue or for map(): `stages` in order,
    each "add", "mul", ("scale", by) or an activation name ("gelu_tanh", "silu",
    "sigmoid", "relu", "softplus", "exp", "tanh"); `operands` the f32 tensors the Add /
    Mul stages read, in order; `sum_at` which of the chain's reads is the sum (or map's
    input). engine/plan/lower/src/kernels/map.rs:40-59,125-185. The tensors must stay
    alive until the call has been enqueued (the struct holds their addresses)."""
    c = abi.After()
    if len(stages) > abi.TS_MAP_STAGES or len(operands) > abi.TS_MAP_OPERANDS:
        raise ValueError(f"at most {abi.TS_MAP_STAGES} stages and {abi.TS_MAP_OPERANDS} operands")
    for i, st in enumerate(stages):
        if st == "add":
            c.stage[i].op = abi.TS_MAP_ADD
        elif st == "mul":
            c.stage[i].op = abi.TS_MAP_MUL
        elif isinstance(st, tuple) and st[0] == "scale":
            c.stage[i].op, c.stage[i].by = abi.TS_MAP_SCALE, float(st[1])
        else:
            c.stage[i].op, c.stage[i].act = abi.TS_MAP_ACT, abi.ACTS[st]
    for j, t in enumerate(operands):
        if t.dtype != torch.float32:
            raise ValueError("chain operands are f32")
        c.operand[j] = t.data_ptr()
        c.spans[j] = (spans or [0] * len(operands))[j]
    c.count, c.sum = len(stages), sum_at
    c._keep = list(operands)
    return c


def linear_args(x, w, out, *, w_scale=None, gain=None, a0=None, stages=0, eps=1e-6, w_form=None):
    m, k = x.shape
    n = out.shape[1]
    a = abi.LinearArgs()
    a.x, a.w, a.w_scale, a.gain, a.a0, a.out = (_ptr(x), _ptr(w), _ptr(w_scale), _ptr(gain), _ptr(a0),
                                                _ptr(out))
    a.m, a.n, a.k = m, n, k
    a.x_dtype, a.out_dtype = _DT[x.dtype], _DT[out.dtype]
    # Block forms: w is the packed tensor (uint8: head, then each row's blocks).
    a.w_dtype = (abi.TS_F32_PARTS if w_form == "f32_parts" else BLOCK_FORMS[w_form]) if w_form is not None \
        else _DT[w.dtype]
    a.stages, a.eps = stages, eps
    return a


def _linear(fn: str, x, w, *, out=None, out_dtype=torch.float32, w_scale=None, gain=None, a0=None,
            silu_mul=False, eps=1e-6, w_form=None, rows=None, after=None):
    """rows: the weight rows of a packed block-form tensor (w is then flat bytes).
    after: a chain() run on each sum before the store."""
    m = x.shape[0]
    wr = rows if w_form is not None and w_form != "f32_parts" else w.shape[0]
    if wr is None:
        raise ValueError("a block-form weight tensor needs rows=")
    n = wr // 2 if silu_mul or w_form == "f32_parts" else wr
    if out is None:
        out = torch.empty((m, n), dtype=out_dtype, device=x.device)
    stages = (abi.TS_AFTER_ADD if a0 is not None else 0) | (abi.TS_AFTER_SILU_MUL if silu_mul else 0) | \
        (abi.TS_BEFORE_RMS_NORM if gain is not None else 0)
    a = linear_args(x, w, out, w_scale=w_scale, gain=gain, a0=a0, stages=stages, eps=eps, w_form=w_form)
    if after is not None:
        a.after = C.addressof(after)
    lib = abi.load()
    need = getattr(lib, fn + "_workspace")(C.byref(a)) if hasattr(lib, fn + "_workspace") else 0
    a.workspace, a.workspace_bytes = workspace(x.device).get(need)
    abi.call(fn, C.byref(a), _stream())
    return out


def pack_f32(w):
    """f32 weights [n, k] to the TS_F32_PARTS layout ([2n, k] bf16: high parts, then
    low parts), once at load; pass the result with w_form="f32_parts"."""
    n, k = w.shape
    out = torch.empty((2 * n, k), dtype=torch.bfloat16, device=w.device)
    abi.call("tessera_hip_pack_f32", C.byref(abi.PackArgs(_ptr(w), _ptr(out), n, k)), _stream())
    return out


def linear(x, w, **kw):
    """tiled or lanes by row count (the cost select between the two rules)."""
    return _linear("tessera_hip_linear", x, w, **kw)


def lanes(x, w, **kw):
    """Few-row product (rule "lanes"/"thin"): m <= 64."""
    return _linear("tessera_hip_lanes", x, w, **kw)


def tiled(x, w, **kw):
    """Matrix-unit product (rule "tiled")."""
    return _linear("tessera_hip_tiled", x, w, **kw)


def picked(x, w, ids, *, n=None, repeat=1, first=0, offset=0, silu_mul=False, w_scale=None, out=None,
           out_dtype=torch.float32, after=None):
    """Rule "picked": row r multiplies matrix ids[r] - first of the set w [count, stride, k]
    (rows offset..offset+n, or the gate/up pair with silu_mul); x row r // repeat."""
    count, stride, k = w.shape
    rows = ids.numel()
    if n is None:
        n = (stride - offset) // 2 if silu_mul else stride - offset
    if out is None:
        out = torch.empty((rows, n), dtype=out_dtype, device=x.device)
    a = abi.PickedArgs()
    a.x, a.w, a.w_scale, a.ids, a.out = _ptr(x), _ptr(w), _ptr(w_scale), _ptr(ids), _ptr(out)
    a.rows, a.n, a.k, a.count, a.stride, a.offset, a.repeat, a.first = rows, n, k, count, stride, offset, repeat, first
    a.x_dtype, a.w_dtype, a.out_dtype = _DT[x.dtype], _DT[w.dtype], _DT[out.dtype]
    a.stages = abi.TS_AFTER_SILU_MUL if silu_mul else 0
    if after is not None:
        a.after = C.addressof(after)
    need = abi.load().tessera_hip_picked_workspace(C.byref(a))
    a.workspace, a.workspace_bytes = workspace(x.device).get(need)
    abi.call("tessera_hip_picked", C.byref(a), _stream())
    return out


def map(x, stages, operands=(), *, sum_at=0, spans=None, out=None):
    """Rule "map": out = chain(x) elementwise over f32 x (map.rs:60-65,187-260)."""
    if out is None:
        out = torch.empty_like(x)
    a = abi.MapArgs()
    a.x, a.out, a.len = _ptr(x), _ptr(out), x.numel()
    a.after = chain(stages, operands, sum_at=sum_at, spans=spans)
    abi.call("tessera_hip_map", C.byref(a), _stream())
    return out


def take(x, ids, out=None):
    rows, width = x.shape
    picks = ids.shape[-1]
    if out is None:
        out = torch.empty(ids.shape, dtype=torch.float32, device=x.device)
    abi.call("tessera_hip_take", C.byref(abi.TakeArgs(_ptr(x), _ptr(ids), _ptr(out), rows, width, picks)), _stream())
    return out


def softmax(x, out=None):
    width = x.shape[-1]
    rows = x.numel() // width
    if out is None:
        out = torch.empty_like(x)
    abi.call("tessera_hip_softmax", C.byref(abi.SoftmaxArgs(_ptr(x), _ptr(out), rows, width)), _stream())
    return out


def mix(x, weights=None, out=None):
    """Weighted sum over axis 1 of x [outer, count, inner] (mean without weights)."""
    outer, count = x.shape[0], x.shape[1]
    inner = x.numel() // (outer * count)
    if out is None:
        out = torch.empty((outer,) + tuple(x.shape[2:]), dtype=torch.float32, device=x.device)
    abi.call("tessera_hip_mix", C.byref(abi.MixArgs(_ptr(x), _ptr(weights), _ptr(out), outer, count, inner)),
             _stream())
    return out


def moe_layer(h, router, w_in, w_out, *, top=8, shared_in=None, shared_out=None, inner_dtype=torch.bfloat16,
              scores=None):
    """One MoE MLP as the reference composes it (engine/models/src/decoder.rs:73-84):
    scores = h . router^T; ids = top_k(scores); gates = softmax(take(scores, ids));
    inner = silu(h . gate_e) * (h . up_e) per pick; y = mix(inner . out_e, gates);
    plus the shared expert's SwiGLU when given. `scores` given: the router product is
    skipped (router may be None). Returns (y, ids, gates)."""
    tokens = h.shape[0]
    if scores is None:
        scores = linear(h, router)
    ids = top_k(scores, top)
    gates = softmax(take(scores, ids))
    ffn = w_out.shape[2]
    inner = picked(h, w_in, ids, n=ffn, repeat=top, silu_mul=True, out_dtype=inner_dtype)
    y_picks = picked(inner, w_out, ids, out_dtype=torch.float32)
    y = mix(y_picks.view(tokens, top, -1), gates)
    if shared_in is not None:
        s_inner = linear(h, shared_in, silu_mul=True, out_dtype=inner_dtype)
        y = linear(s_inner, shared_out, a0=y, out=y)
    return y, ids, gates


def rows_args(q, k, v, out, slots, positions, *, keys, scale, table=None, kept_pages=0, page=16,
              back=abi.U32_MAX, max_position=None, status=None):
    rows, heads, width = q.shape
    a = abi.RowsArgs()
    a.q, a.k, a.v, a.out = _ptr(q), _ptr(k), _ptr(v), _ptr(out)
    a.slots, a.positions, a.kept_table = _ptr(slots), _ptr(positions), _ptr(table)
    a.rows, a.keys, a.heads, a.kv_heads, a.width = rows, keys, heads, k.shape[-2], width
    a.back, a.kept_pages, a.page, a.scale = back, kept_pages, page, scale
    a.q_dtype, a.kv_dtype, a.out_dtype = _DT[q.dtype], _DT[k.dtype], _DT[out.dtype]
    if max_position is None:
        max_position = int(positions.max().item()) if rows else 0
    a.max_position = max_position
    a.status = _ptr(status)  # int32 device word: TS_STATUS_* bits of refused rows
    return a


def attend_rows(q, k, v, slots, positions, *, keys, scale, table=None, kept_pages=0, page=16,
                back=abi.U32_MAX, max_position=None, out=None, status=None):
    """Decode rows over kept K/V (rule "attend"/attend_rows; split-KV)."""
    if out is None:
        out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    a = rows_args(q, k, v, out, slots, positions, keys=keys, scale=scale, table=table,
                  kept_pages=kept_pages, page=page, back=back, max_position=max_position, status=status)
    need = abi.load().tessera_hip_attend_rows_workspace(C.byref(a))
    a.workspace, a.workspace_bytes = workspace(q.device).get(need)
    abi.call("tessera_hip_attend_rows", C.byref(a), _stream())
    return out


def rope_table(positions, theta, width=128, device="cuda"):
    """(cos, sin) of every (position, pair) angle (the "angles" stage)."""
    t = torch.empty((positions, width // 2, 2), dtype=torch.float32, device=device)
    abi.call("tessera_hip_rope_table", C.byref(abi.AnglesArgs(_ptr(t), positions, width, theta)), _stream())
    return t


def attend_step(qkv, q_gain, k_gain, k, v, slots, positions, *, heads, keys, scale, eps, theta, table=None,
                kept_pages=0, page=16, back=abi.U32_MAX, max_position=None, out=None, angles=None):
    """Fused decode step: q/k RmsNorm + RoPE from raw product rows, append, attend."""
    rows = qkv.shape[0]
    if angles is None:
        angles = rope_table(keys, theta, device=qkv.device)
    if out is None:
        out = torch.empty((rows, heads, 128), dtype=torch.float32, device=qkv.device)
    qshape = torch.empty((rows, heads, 128), device=qkv.device)  # shape carrier only
    a = rows_args(qshape, k, v, out, slots, positions, keys=keys, scale=scale, table=table,
                  kept_pages=kept_pages, page=page, back=back, max_position=max_position)
    need = abi.load().tessera_hip_attend_rows_workspace(C.byref(a))
    a.workspace, a.workspace_bytes = workspace(qkv.device).get(need)
    st = abi.StepArgs(a, _ptr(qkv), _ptr(q_gain), _ptr(k_gain), _ptr(angles), angles.shape[0], eps)
    abi.call("tessera_hip_attend_step", C.byref(st), _stream())
    return out


def flash_rows(q, k, v, slots, positions, *, keys, scale, table=None, kept_pages=0, page=16,
               back=abi.U32_MAX, max_position=None, out=None, status=None):
    """Prefill rows over kept K/V (rule "flash"/flash_rows); rows may be packed ragged.
    max_position (an upper bound on positions) defaults to their maximum (a host read:
    pass it when capturing a graph)."""
    if out is None:
        out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    a = rows_args(q, k, v, out, slots, positions, keys=keys, scale=scale, table=table,
                  kept_pages=kept_pages, page=page, back=back, max_position=max_position, status=status)
    abi.call("tessera_hip_flash_rows", C.byref(a), _stream())
    return out


MASKS = {"causal": lambda n: (abi.U32_MAX, 0, 1), "bidirectional": lambda n: (abi.U32_MAX, abi.U32_MAX, 0),
         "within": lambda n: (n, n, 0), "back": lambda n: (n, 0, 1)}


def flash(q, k, v, *, scale, mask="causal", n=0, out=None):
    """Rule "flash" on whole sequences: q [seqs, rows, heads, 128] (f32 or bf16), k / v
    [seqs, keys, kv_heads, 128] bf16, any mask of engine/ir/graph/src/node.rs:162-181
    ("causal", "bidirectional", "within" n, "back" n)."""
    seqs, rows, heads, width = q.shape
    keys, kvh = k.shape[1], k.shape[2]
    if out is None:
        out = torch.empty((seqs, rows, heads, width), dtype=torch.float32, device=q.device)
    back, ahead, causal = MASKS[mask](n)
    a = abi.FlashArgs(_ptr(q), _ptr(k), _ptr(v), _ptr(out), seqs, rows, keys, heads, kvh, width, back, ahead,
                      causal, scale, _DT[q.dtype], _DT[k.dtype], _DT[out.dtype])
    abi.call("tessera_hip_flash", C.byref(a), _stream())
    return out


def rms_norm(x, gain, eps, out=None):
    rows, width = x.reshape(-1, x.shape[-1]).shape
    if out is None:
        out = torch.empty_like(x)
    abi.call("tessera_hip_rms_norm", C.byref(abi.NormArgs(_ptr(x), _ptr(gain), _ptr(out), rows, width, eps)),
             _stream())
    return out


def rope(x, positions, theta, halves=True):
    """In place on x [rows, heads, width]."""
    rows, heads, width = x.shape
    a = abi.RopeArgs(_ptr(x), _ptr(positions), rows, heads, width, theta, 1 if halves else 0)
    abi.call("tessera_hip_rope", C.byref(a), _stream())
    return x


def qk_norm_rope_append(qkv, q_gain, k_gain, q_out, k_cache, v_cache, slots, positions, *, heads,
                        kv_heads, keys, eps, theta, table=None, kept_pages=0, page=16):
    rows = qkv.shape[0]
    a = abi.QkArgs(_ptr(qkv), _ptr(q_gain), _ptr(k_gain), _ptr(q_out), _ptr(k_cache), _ptr(v_cache),
                   _ptr(slots), _ptr(positions), _ptr(table), rows, heads, kv_heads, 128, keys, kept_pages,
                   page, eps, theta)
    abi.call("tessera_hip_qk_norm_rope_append", C.byref(a), _stream())
    return q_out


def gather(table, ids, first=0, out=None):
    count = ids.numel()
    rows, width = table.shape
    if out is None:
        out = torch.empty((count, width), dtype=torch.float32, device=table.device)
    a = abi.GatherArgs(_ptr(table), _ptr(ids), _ptr(out), count, rows, width, first)
    abi.call("tessera_hip_gather", C.byref(a), _stream())
    return out


def argmax(x, ids=None):
    rows, width = x.shape
    if ids is None:
        ids = torch.empty(rows, dtype=torch.int32, device=x.device)
    a = abi.ArgmaxArgs(_ptr(x), _ptr(ids), None, 0, rows, width)
    a.workspace, a.workspace_bytes = workspace(x.device).get(abi.load().tessera_hip_argmax_workspace(C.byref(a)))
    abi.call("tessera_hip_argmax", C.byref(a), _stream())
    return ids


def linear_argmax(x, w, *, gain=None, eps=1e-6, keys=None):
    """The few-row product with the greedy pick folded in (TS_AFTER_ARGMAX): (logits,
    ids). `keys` (int64 [m], zero) may be passed to reuse; it is zero again after."""
    m, n = x.shape[0], w.shape[0]
    out = torch.empty((m, n), dtype=torch.float32, device=x.device)
    if keys is None:
        keys = torch.zeros(m, dtype=torch.int64, device=x.device)
    stages = abi.TS_AFTER_ARGMAX | (abi.TS_BEFORE_RMS_NORM if gain is not None else 0)
    a = linear_args(x, w, out, gain=gain, stages=stages, eps=eps)
    a.workspace, a.workspace_bytes = _ptr(keys), keys.numel() * 8
    abi.call("tessera_hip_lanes", C.byref(a), _stream())
    ids = torch.empty(m, dtype=torch.int32, device=x.device)
    abi.call("tessera_hip_argmax_keys", C.byref(abi.KeysArgs(_ptr(keys), _ptr(ids), m, n)), _stream())
    return out, ids


def top_k(x, k, ids=None):
    rows, width = x.shape
    if ids is None:
        ids = torch.empty((rows, k), dtype=torch.int32, device=x.device)
    abi.call("tessera_hip_top_k", C.byref(abi.TopKArgs(_ptr(x), _ptr(ids), rows, width, k)), _stream())
    return ids
