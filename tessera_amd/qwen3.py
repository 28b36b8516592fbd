"""ctypes binding of the Qwen3 runner (include/tessera_run.h)."""
from __future__ import annotations

import ctypes as C
import re

import numpy as np

from . import abi


class Config(C.Structure):
    _fields_ = [("vocab", C.c_uint32), ("hidden", C.c_uint32), ("layers", C.c_uint32), ("heads", C.c_uint32),
                ("kv_heads", C.c_uint32), ("head_dim", C.c_uint32), ("ffn", C.c_uint32), ("eps", C.c_float),
                ("theta", C.c_float), ("max_context", C.c_uint32), ("page", C.c_uint32),
                ("max_prompt", C.c_uint32)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


_P = C.c_void_p
SIGNATURES = {
    "tessera_qwen3_default_config": (None, [C.POINTER(Config)]),
    "tessera_qwen3_open": (C.c_int, [C.POINTER(Config), C.c_uint64, C.POINTER(_P)]),
    "tessera_qwen3_close": (None, [_P]),
    "tessera_qwen3_weight": (C.c_int, [_P, C.c_char_p, C.c_uint32, C.POINTER(_P), C.POINTER(C.c_uint64),
                                       C.POINTER(C.c_int32)]),
    "tessera_qwen3_read": (C.c_int, [_P, C.c_char_p, C.c_uint32, _P, C.c_uint64]),
    "tessera_qwen3_prefill": (C.c_int, [_P, _P, C.c_uint32, C.POINTER(C.c_uint32)]),
    "tessera_qwen3_decode": (C.c_int, [_P, C.c_uint32, _P]),
    "tessera_qwen3_logits": (C.c_int, [_P, _P, C.c_uint64]),
    "tessera_qwen3_set_token": (C.c_int, [_P, C.c_uint32]),
    "tessera_qwen3_set_graph": (C.c_int, [_P, C.c_int]),
    "tessera_qwen3_set_step": (C.c_int, [_P, C.c_int]),
    "tessera_qwen3_step_mode": (C.c_int, [_P]),
    "tessera_qwen3_decode_ms": (C.c_float, [_P]),
    "tessera_qwen3_step_marks": (C.c_int, [_P, _P, C.POINTER(C.c_uint32)]),
    "tessera_qwen3_stream": (_P, [_P]),
    "tessera_qwen3_position": (C.c_uint32, [_P]),
    "tessera_qwen3_pages": (C.c_int, [_P, _P, C.c_uint32]),
}

_bound = False


def lib():
    global _bound
    L = abi.load()
    if not _bound:
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _bound = True
    return L


def default_config(**over) -> Config:
    c = Config()
    lib().tessera_qwen3_default_config(C.byref(c))
    for k, v in over.items():
        setattr(c, k, v)
    return c


class Qwen3:
    """A Qwen3-shaped decoder on one GPU: seeded weights, paged kept rows, greedy decode."""

    def __init__(self, config: Config | None = None, seed: int = 0):
        self.L = lib()
        self.config = config or default_config()
        h = _P()
        abi.check(self.L.tessera_qwen3_open(C.byref(self.config), seed, C.byref(h)), "tessera_qwen3_open")
        self.h = h

    def close(self):
        if self.h:
            self.L.tessera_qwen3_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def read(self, name: str, layer: int = 0) -> np.ndarray:
        ptr, nbytes, dtype = _P(), C.c_uint64(), C.c_int32()
        abi.check(self.L.tessera_qwen3_weight(self.h, name.encode(), layer, C.byref(ptr), C.byref(nbytes),
                                              C.byref(dtype)), "tessera_qwen3_weight")
        out = np.empty(nbytes.value // (2 if dtype.value == abi.TS_BF16 else 4),
                       np.uint16 if dtype.value == abi.TS_BF16 else np.float32)
        abi.check(self.L.tessera_qwen3_read(self.h, name.encode(), layer, out.ctypes.data, nbytes.value),
                  "tessera_qwen3_read")
        return out

    def prefill(self, tokens) -> int:
        t = np.ascontiguousarray(tokens, np.uint32)
        nxt = C.c_uint32()
        abi.check(self.L.tessera_qwen3_prefill(self.h, t.ctypes.data, len(t), C.byref(nxt)), "tessera_qwen3_prefill")
        return nxt.value

    def decode(self, steps: int, want_tokens: bool = True):
        out = np.empty(steps, np.uint32) if want_tokens else None
        abi.check(self.L.tessera_qwen3_decode(self.h, steps, out.ctypes.data if want_tokens else None),
                  "tessera_qwen3_decode")
        return out

    def set_token(self, token: int):
        """The next decode step reads `token` instead of the previous greedy pick."""
        abi.check(self.L.tessera_qwen3_set_token(self.h, int(token)), "tessera_qwen3_set_token")

    def logits(self) -> np.ndarray:
        out = np.empty(self.config.vocab, np.float32)
        abi.check(self.L.tessera_qwen3_logits(self.h, out.ctypes.data, out.size), "tessera_qwen3_logits")
        return out

    def set_graph(self, on: bool):
        abi.check(self.L.tessera_qwen3_set_graph(self.h, 1 if on else 0), "tessera_qwen3_set_graph")

    def set_step(self, on: bool):
        """True: decode as one persistent launch per call; False: the graph of kernels."""
        abi.check(self.L.tessera_qwen3_set_step(self.h, 1 if on else 0), "tessera_qwen3_set_step")

    @property
    def decode_ms(self) -> float:
        """Device time of the last decode call's steps (HIP events), ms; -1 if untimed."""
        return float(self.L.tessera_qwen3_decode_ms(self.h))

    @property
    def step_mode(self) -> bool:
        return bool(self.L.tessera_qwen3_step_mode(self.h))

    @property
    def position(self) -> int:
        return self.L.tessera_qwen3_position(self.h)

    def pages(self, count: int):
        out = np.empty(count, np.uint32)
        abi.check(self.L.tessera_qwen3_pages(self.h, out.ctypes.data, count), "tessera_qwen3_pages")
        return out
