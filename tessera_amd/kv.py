"""ctypes binding of the page pool (include/tessera_kv.h), with the reference's
method names: Pool.reserve / fork / grow / truncate / retain / adopt / release
(engine/ir/kv/src/pool.rs). Refusals raise PoolError carrying the reference's
error name and payload."""
from __future__ import annotations

import ctypes as C

from . import abi

OK, NO_ROOM, PAST_WORST, PAST_SOURCE, LIVE, RETAINED, UNKNOWN = range(7)
NAMES = {NO_ROOM: "NoRoom", PAST_WORST: "PastWorst", PAST_SOURCE: "PastSource", LIVE: "Live",
         RETAINED: "Retained", UNKNOWN: "Unknown"}


class RunId(C.Structure):
    _fields_ = [("at", C.c_uint32), ("generation", C.c_uint32)]

    def key(self):
        return (self.at, self.generation)

    def __eq__(self, other):
        return isinstance(other, RunId) and self.key() == other.key()

    def __hash__(self):
        return hash(self.key())

    def __repr__(self):
        return f"RunId{self.key()}"


class PageCopy(C.Structure):
    _fields_ = [("from_", C.c_uint32), ("to", C.c_uint32), ("rows", C.c_uint64)]

    def tuple(self):
        return (self.from_, self.to, self.rows)


class CopyArgs(C.Structure):
    """ts_kv_copy_args (include/tessera_kv.h)."""
    _fields_ = [("buffers", C.c_void_p), ("copies", C.c_void_p), ("buffer_count", C.c_uint32),
                ("copy_count", C.c_uint32), ("page", C.c_uint32), ("row_bytes", C.c_uint32),
                ("pages", C.c_uint32), ("status", C.c_void_p)]


STATUS_COPY = 2  # TS_KV_STATUS_COPY


class Stats(C.Structure):
    _fields_ = [("size", C.c_uint64), ("active", C.c_uint64), ("worst", C.c_uint64),
                ("live_runs", C.c_uint64), ("kept_runs", C.c_uint64)]


class PoolError(Exception):
    def __init__(self, code, value=None, value2=None):
        self.code, self.value, self.value2 = code, value, value2
        super().__init__(f"{NAMES.get(code, code)}({value}, {value2})")

    def name(self):
        return NAMES[self.code]


_P = C.c_void_p
_R = RunId
SIGNATURES = {
    "tessera_kv_new": (_P, [C.c_uint32, C.c_uint32]),
    "tessera_kv_free": (None, [_P]),
    "tessera_kv_reserve": (C.c_int, [_P, C.c_uint64, C.c_uint64, C.c_uint64, C.POINTER(_R)]),
    "tessera_kv_fork": (C.c_int, [_P, _R, C.c_uint64, C.c_uint64, C.POINTER(_R)]),
    "tessera_kv_grow": (C.c_int, [_P, _R, C.c_uint64, C.POINTER(PageCopy), C.POINTER(C.c_uint32)]),
    "tessera_kv_truncate": (C.c_int, [_P, _R, C.c_uint64]),
    "tessera_kv_retain": (C.c_int, [_P, _R]),
    "tessera_kv_adopt": (C.c_int, [_P, _R, C.c_uint64, C.c_uint64, C.POINTER(_R)]),
    "tessera_kv_release": (C.c_int, [_P, _R]),
    "tessera_kv_pages": (C.c_int, [_P, _R, C.POINTER(C.POINTER(C.c_uint32)), C.POINTER(C.c_uint32)]),
    "tessera_kv_rows": (C.c_int, [_P, _R, C.POINTER(C.c_uint64)]),
    "tessera_kv_tag": (C.c_int, [_P, _R, C.POINTER(C.c_uint64)]),
    "tessera_kv_spare": (C.c_uint64, [_P]),
    "tessera_kv_promised": (C.c_uint64, [_P]),
    "tessera_kv_get_stats": (None, [_P, C.POINTER(Stats)]),
    "tessera_kv_digest": (C.c_uint64, [_P]),
    "tessera_kv_consistent": (C.c_int, [_P]),
    "tessera_kv_error_value": (C.c_uint64, [_P]),
    "tessera_kv_error_value2": (C.c_uint64, [_P]),
    "tessera_hip_kv_copy": (C.c_int, [C.POINTER(CopyArgs), _P]),
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


class Pool:
    """Pages of `page` rows each, shared by runs of kept rows."""

    def __init__(self, pages: int, page: int):
        self._l = lib()
        self._p = self._l.tessera_kv_new(pages, page)
        if not self._p:
            raise ValueError("page must be > 0")

    def __del__(self):
        if getattr(self, "_p", None):
            self._l.tessera_kv_free(self._p)
            self._p = None

    def _ok(self, code):
        if code != OK:
            v = self._l.tessera_kv_error_value(self._p)
            v2 = self._l.tessera_kv_error_value2(self._p)
            raise PoolError(code, v if code in (NO_ROOM, PAST_WORST, PAST_SOURCE) else None,
                            v2 if code == PAST_WORST else None)

    def reserve(self, tag, rows, worst) -> RunId:
        out = RunId()
        self._ok(self._l.tessera_kv_reserve(self._p, tag, rows, worst, C.byref(out)))
        return out

    def fork(self, source, rows, worst) -> RunId:
        out = RunId()
        self._ok(self._l.tessera_kv_fork(self._p, source, rows, worst, C.byref(out)))
        return out

    def grow(self, run, rows):
        cp, n = PageCopy(), C.c_uint32(0)
        self._ok(self._l.tessera_kv_grow(self._p, run, rows, C.byref(cp), C.byref(n)))
        return [cp.tuple()] if n.value else []

    def truncate(self, run, rows):
        self._ok(self._l.tessera_kv_truncate(self._p, run, rows))

    def retain(self, run):
        self._ok(self._l.tessera_kv_retain(self._p, run))

    def adopt(self, run, rows, worst) -> RunId:
        out = RunId()
        self._ok(self._l.tessera_kv_adopt(self._p, run, rows, worst, C.byref(out)))
        return out

    def release(self, run):
        self._ok(self._l.tessera_kv_release(self._p, run))

    def pages(self, run):
        ptr, n = C.POINTER(C.c_uint32)(), C.c_uint32(0)
        self._ok(self._l.tessera_kv_pages(self._p, run, C.byref(ptr), C.byref(n)))
        return [ptr[i] for i in range(n.value)]

    def rows(self, run):
        v = C.c_uint64(0)
        self._ok(self._l.tessera_kv_rows(self._p, run, C.byref(v)))
        return v.value

    def spare(self):
        return self._l.tessera_kv_spare(self._p)

    def stats(self) -> Stats:
        s = Stats()
        self._l.tessera_kv_get_stats(self._p, C.byref(s))
        return s

    def digest(self):
        return self._l.tessera_kv_digest(self._p)

    def consistent(self):
        return bool(self._l.tessera_kv_consistent(self._p))


def copy_pages(buffers, copies, *, page, pages, status=None, check=True):
    """Makes Pool.grow's copies on the device in every kept-row buffer (torch tensors
    [pages * page, ...], e.g. K and V of each layer), in stream order before the
    launch that appends. copies: [(from, to, rows), ...]. check=False leaves the
    overlap check to the device (which skips such copies and reports them)."""
    import torch
    if not copies:
        return
    # The copies of one call run at once: no page may be one copy's target and another
    # copy's source or target (the device skips and reports such pairs too).
    for i, (f, t, _) in enumerate(copies if check else ()):
        for j, (f2, t2, _) in enumerate(copies):
            if i != j and (t == t2 or t == f2):
                raise ValueError(f"copies {i} and {j} overlap: page {t} is written by one and read or written "
                                 "by the other")
    dev = buffers[0].device
    ptrs = torch.tensor([b.data_ptr() for b in buffers], dtype=torch.int64).to(dev)
    raw = torch.tensor([[f, t, r & 0xFFFFFFFF, r >> 32] for f, t, r in copies], dtype=torch.int64)
    cps = raw.to(torch.int32).to(dev)  # ts_kv_copy: u32 from, u32 to, u64 rows (little endian)
    a = CopyArgs()
    a.buffers, a.copies = ptrs.data_ptr(), cps.data_ptr()
    a.buffer_count, a.copy_count, a.page, a.pages = len(buffers), len(copies), page, pages
    a.row_bytes = buffers[0][0].numel() * buffers[0].element_size()
    a.status = status.data_ptr() if status is not None else None
    rc = lib().tessera_hip_kv_copy(C.byref(a), C.c_void_p(torch.cuda.current_stream().cuda_stream))
    abi.check(rc, "tessera_hip_kv_copy")
