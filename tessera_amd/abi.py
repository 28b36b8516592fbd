"""ctypes binding of libtessera_hip.so: the C ABI declared in include/tessera_hip.h.

This plays the part of the reference's ``tessera_dl::library!`` struct
(engine/gpu/dl/src/lib.rs:66) that engine/gpu/gpukit/src/rocm/hip.rs:48-94 uses to
bind libamdhip64: one table of typed function pointers, resolved once. Loading fails
loudly when the library has not been built; there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("TESSERA_HIP_LIB") or os.path.join(HERE, "libtessera_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "tessera_hip.h")

TS_OK = 0
TS_ERR_ARG = -1
TS_ERR_ARCH = -2
TS_ERR_WORKSPACE = -3

TS_STATUS_POSITION = 1  # ts_rows_args.status: a row's position was refused

TS_F32, TS_BF16, TS_E4M3, TS_U32 = 0, 1, 2, 3
TS_Q8_0, TS_MXFP8, TS_INT4_G32, TS_Q4_0 = 4, 5, 6, 7  # block forms (engine/ir/mem/src/block.rs:251-291)
TS_NVFP4, TS_MXFP4, TS_INT4_G128 = 8, 9, 10
TS_F32_PARTS = 11  # f32 weights as tessera_hip_pack_f32 lays them out

TS_AFTER_ADD = 1
TS_AFTER_SILU_MUL = 2
TS_BEFORE_RMS_NORM = 4
TS_AFTER_ARGMAX = 8

U32_MAX = 0xFFFFFFFF

# Stage chains (ts_after): stage ops and activations.
TS_MAP_STAGES, TS_MAP_OPERANDS = 8, 4
TS_MAP_ADD, TS_MAP_MUL, TS_MAP_SCALE, TS_MAP_ACT = 0, 1, 2, 3
ACTS = {"gelu_tanh": 0, "silu": 1, "sigmoid": 2, "relu": 3, "softplus": 4, "exp": 5, "tanh": 6}


class MapStage(C.Structure):
    """ts_map_stage (include/tessera_hip.h)."""
    _fields_ = [("op", C.c_int32), ("act", C.c_int32), ("by", C.c_float)]


class After(C.Structure):
    """ts_after (include/tessera_hip.h): a stage chain and its operands."""
    _fields_ = [("operand", C.c_void_p * TS_MAP_OPERANDS), ("spans", C.c_uint32 * TS_MAP_OPERANDS),
                ("count", C.c_uint32), ("sum", C.c_uint32), ("stage", MapStage * TS_MAP_STAGES)]


class MapArgs(C.Structure):
    """ts_map_args (include/tessera_hip.h)."""
    _fields_ = [("x", C.c_void_p), ("out", C.c_void_p), ("len", C.c_uint32), ("after", After)]


class LinearArgs(C.Structure):
    """ts_linear_args (include/tessera_hip.h)."""
    _fields_ = [
        ("x", C.c_void_p), ("w", C.c_void_p), ("w_scale", C.c_void_p), ("gain", C.c_void_p),
        ("a0", C.c_void_p), ("out", C.c_void_p), ("workspace", C.c_void_p),
        ("workspace_bytes", C.c_size_t),
        ("m", C.c_uint32), ("n", C.c_uint32), ("k", C.c_uint32),
        ("x_dtype", C.c_int32), ("w_dtype", C.c_int32), ("out_dtype", C.c_int32),
        ("stages", C.c_uint32), ("eps", C.c_float), ("after", C.c_void_p),
    ]


class RowsArgs(C.Structure):
    """ts_rows_args (include/tessera_hip.h)."""
    _fields_ = [
        ("q", C.c_void_p), ("k", C.c_void_p), ("v", C.c_void_p), ("out", C.c_void_p),
        ("slots", C.c_void_p), ("positions", C.c_void_p), ("kept_table", C.c_void_p),
        ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
        ("rows", C.c_uint32), ("keys", C.c_uint32), ("heads", C.c_uint32), ("kv_heads", C.c_uint32),
        ("width", C.c_uint32), ("back", C.c_uint32), ("kept_pages", C.c_uint32), ("page", C.c_uint32),
        ("scale", C.c_float), ("q_dtype", C.c_int32), ("kv_dtype", C.c_int32), ("out_dtype", C.c_int32),
        ("max_position", C.c_uint32), ("status", C.c_void_p),
    ]


class PickedArgs(C.Structure):
    """ts_picked_args (include/tessera_hip.h)."""
    _fields_ = [
        ("x", C.c_void_p), ("w", C.c_void_p), ("w_scale", C.c_void_p), ("ids", C.c_void_p),
        ("out", C.c_void_p), ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
        ("rows", C.c_uint32), ("n", C.c_uint32), ("k", C.c_uint32), ("count", C.c_uint32),
        ("stride", C.c_uint32), ("offset", C.c_uint32), ("repeat", C.c_uint32), ("first", C.c_uint32),
        ("x_dtype", C.c_int32), ("w_dtype", C.c_int32), ("out_dtype", C.c_int32), ("stages", C.c_uint32),
        ("after", C.c_void_p),
    ]


def _args(name, doc, fields):
    """A ctypes Structure for one of the row stages' argument structs."""
    return type(name, (C.Structure,), {"__doc__": doc + " (include/tessera_hip.h).", "_fields_": fields})


_v, _u, _f = C.c_void_p, C.c_uint32, C.c_float
NormArgs = _args("NormArgs", "ts_norm_args", [
    ("x", _v), ("gain", _v), ("out", _v), ("rows", _u), ("width", _u), ("eps", _f)])
RopeArgs = _args("RopeArgs", "ts_rope_args", [
    ("x", _v), ("positions", _v), ("rows", _u), ("heads", _u), ("width", _u), ("theta", _f),
    ("halves", C.c_int32)])
AnglesArgs = _args("AnglesArgs", "ts_angles_args", [
    ("table", _v), ("positions", _u), ("width", _u), ("theta", _f)])
QkArgs = _args("QkArgs", "ts_qk_args", [
    ("qkv", _v), ("q_gain", _v), ("k_gain", _v), ("q_out", _v), ("k_cache", _v), ("v_cache", _v),
    ("slots", _v), ("positions", _v), ("kept_table", _v), ("rows", _u), ("heads", _u),
    ("kv_heads", _u), ("width", _u), ("keys", _u), ("kept_pages", _u), ("page", _u),
    ("eps", _f), ("theta", _f)])
GatherArgs = _args("GatherArgs", "ts_gather_args", [
    ("table", _v), ("ids", _v), ("out", _v), ("count", _u), ("table_rows", _u), ("width", _u),
    ("first", _u)])
TakeArgs = _args("TakeArgs", "ts_take_args", [
    ("x", _v), ("ids", _v), ("out", _v), ("rows", _u), ("width", _u), ("picks", _u)])
SoftmaxArgs = _args("SoftmaxArgs", "ts_softmax_args", [
    ("x", _v), ("out", _v), ("rows", _u), ("width", _u)])
MixArgs = _args("MixArgs", "ts_mix_args", [
    ("x", _v), ("weights", _v), ("out", _v), ("outer", _u), ("count", _u), ("inner", _u)])
ArgmaxArgs = _args("ArgmaxArgs", "ts_argmax_args", [
    ("x", _v), ("ids", _v), ("workspace", _v), ("workspace_bytes", C.c_size_t), ("rows", _u),
    ("width", _u)])
KeysArgs = _args("KeysArgs", "ts_keys_args", [
    ("keys", _v), ("ids", _v), ("rows", _u), ("width", _u)])
TopKArgs = _args("TopKArgs", "ts_top_k_args", [
    ("x", _v), ("ids", _v), ("rows", _u), ("width", _u), ("k", _u)])
PackArgs = _args("PackArgs", "ts_pack_args", [("w", _v), ("out", _v), ("n", _u), ("k", _u)])
FlashArgs = _args("FlashArgs", "ts_flash_args", [
    ("q", _v), ("k", _v), ("v", _v), ("out", _v), ("seqs", _u), ("rows", _u), ("keys", _u), ("heads", _u),
    ("kv_heads", _u), ("width", _u), ("back", _u), ("ahead", _u), ("causal", C.c_int32), ("scale", _f),
    ("q_dtype", C.c_int32), ("kv_dtype", C.c_int32), ("out_dtype", C.c_int32)])
StepArgs = _args("StepArgs", "ts_step_args", [
    ("rows", RowsArgs), ("qkv", _v), ("q_gain", _v), ("k_gain", _v), ("rope_table", _v),
    ("rope_rows", _u), ("eps", _f)])


_P = C.c_void_p
_U = C.c_uint32
_LA = C.POINTER(LinearArgs)
_RA = C.POINTER(RowsArgs)
_PA = C.POINTER(PickedArgs)

SIGNATURES = {
    "tessera_hip_init": (C.c_int, []),
    "tessera_hip_last_error": (C.c_char_p, []),
    "tessera_hip_abi_version": (C.c_int, []),
    "tessera_hip_linear": (C.c_int, [_LA, _P]),
    "tessera_hip_linear_workspace": (C.c_size_t, [_LA]),
    "tessera_hip_lanes": (C.c_int, [_LA, _P]),
    "tessera_hip_lanes_workspace": (C.c_size_t, [_LA]),
    "tessera_hip_tiled": (C.c_int, [_LA, _P]),
    "tessera_hip_picked": (C.c_int, [_PA, _P]),
    "tessera_hip_picked_workspace": (C.c_size_t, [_PA]),
    "tessera_hip_take": (C.c_int, [C.POINTER(TakeArgs), _P]),
    "tessera_hip_softmax": (C.c_int, [C.POINTER(SoftmaxArgs), _P]),
    "tessera_hip_mix": (C.c_int, [C.POINTER(MixArgs), _P]),
    "tessera_hip_attend_rows": (C.c_int, [_RA, _P]),
    "tessera_hip_attend_rows_workspace": (C.c_size_t, [_RA]),
    "tessera_hip_attend_rows_noalloc": (C.c_int, [_RA, _P]),
    "tessera_hip_attend_rows_noalloc_limit": (C.c_size_t, []),
    "tessera_hip_flash_rows": (C.c_int, [_RA, _P]),
    "tessera_hip_attend_step": (C.c_int, [C.POINTER(StepArgs), _P]),
    "tessera_hip_rope_table": (C.c_int, [C.POINTER(AnglesArgs), _P]),
    "tessera_hip_rms_norm": (C.c_int, [C.POINTER(NormArgs), _P]),
    "tessera_hip_rope": (C.c_int, [C.POINTER(RopeArgs), _P]),
    "tessera_hip_qk_norm_rope_append": (C.c_int, [C.POINTER(QkArgs), _P]),
    "tessera_hip_gather": (C.c_int, [C.POINTER(GatherArgs), _P]),
    "tessera_hip_argmax": (C.c_int, [C.POINTER(ArgmaxArgs), _P]),
    "tessera_hip_argmax_workspace": (C.c_size_t, [C.POINTER(ArgmaxArgs)]),
    "tessera_hip_argmax_keys": (C.c_int, [C.POINTER(KeysArgs), _P]),
    "tessera_hip_top_k": (C.c_int, [C.POINTER(TopKArgs), _P]),
    "tessera_hip_map": (C.c_int, [C.POINTER(MapArgs), _P]),
    "tessera_hip_flash": (C.c_int, [C.POINTER(FlashArgs), _P]),
    "tessera_hip_pack_f32": (C.c_int, [C.POINTER(PackArgs), _P]),
}


class HipError(RuntimeError):
    def __init__(self, code: int, what: str, message: str):
        super().__init__(f"{what} returned {code}: {message}")
        self.code = code


_lib = None


def load():
    """The resolved library. Raises if it is missing: there is no CPU fallback."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build() first")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _header_text(header=None) -> str:
    paths = [header] if header else sorted(
        os.path.join(os.path.dirname(HEADER), f) for f in os.listdir(os.path.dirname(HEADER)) if f.endswith(".h"))
    return re.sub(r"/\*.*?\*/", "", "".join(open(p).read() for p in paths), flags=re.S)


def declared_functions(header=None) -> list[str]:
    """Every function the public headers declare (checked against the exports)."""
    return sorted(set(re.findall(r"\b(tessera_\w+)\s*\(", _header_text(header))))


def declared_arity(header=None) -> dict[str, int]:
    """Parameter count of each prototype in the public headers."""
    out = {}
    for name, params in re.findall(r"\b(tessera_\w+)\s*\(([^)]*)\)\s*;", _header_text(header)):
        params = params.strip()
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def check(code: int, what: str) -> None:
    if code != TS_OK:
        raise HipError(code, what, load().tessera_hip_last_error().decode())


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args), name)
