"""tessera_hip_attend_rows_noalloc (partials in a fixed device array, no workspace,
no allocation) against tessera_hip_attend_rows with a caller's workspace: the same
kernels on the same inputs, so the outputs are bit-identical. Two calls in a row,
the second with a smaller input (fewer rows, shorter contexts), both split across
partitions so the fixed array carries partials; then a launch past the limit is
refused before anything runs."""
import ctypes as C
import math

import numpy as np
import pytest

from tests.helpers import bf16_bits_normal, rng, to_dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _case(seed, ctxs, heads=16, kvh=8, page=16):
    r = rng(seed)
    kept_pages = max(math.ceil(c / page) for c in ctxs)
    total = len(ctxs) * kept_pages
    table = r.permutation(total).astype(np.int32)
    kb, _ = bf16_bits_normal(r, (total * page, kvh, 128))
    vb, _ = bf16_bits_normal(r, (total * page, kvh, 128))
    q = r.standard_normal((len(ctxs), heads, 128)).astype(np.float32)
    dev = dict(q=to_dev(q, torch), k=to_dev(kb, torch), v=to_dev(vb, torch),
               slots=torch.arange(len(ctxs), dtype=torch.int32, device="cuda"),
               pos=torch.tensor([c - 1 for c in ctxs], dtype=torch.int32, device="cuda"),
               table=torch.from_numpy(table).cuda())
    return dev, kept_pages, page, max(ctxs) - 1


def _both(seed, ctxs):
    from tessera_amd import abi
    from tessera_amd import rules as R
    d, kept_pages, page, mp = _case(seed, ctxs)
    kw = dict(keys=kept_pages * page, scale=1 / math.sqrt(128), table=d["table"], kept_pages=kept_pages,
              page=page, max_position=mp)
    want = R.attend_rows(d["q"], d["k"], d["v"], d["slots"], d["pos"], **kw)
    out = torch.full_like(d["q"], float("nan"))
    a = R.rows_args(d["q"], d["k"], d["v"], out, d["slots"], d["pos"], **kw)
    lib = abi.load()
    assert lib.tessera_hip_attend_rows_workspace(C.byref(a)) > 0  # the split path: partials exist
    abi.call("tessera_hip_attend_rows_noalloc", C.byref(a), C.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int32), want.view(torch.int32))


def test_noalloc_matches_attend_rows_twice():
    print("noalloc: 32 rows, ctx U[512, 8192]", flush=True)
    _both(2, rng(2).integers(512, 8193, 32).tolist())
    print("noalloc: 5 rows, ctx U[300, 3000]", flush=True)
    _both(3, rng(3).integers(300, 3001, 5).tolist())


def test_noalloc_refuses_past_limit():
    from tessera_amd import abi
    from tessera_amd import rules as R
    lib = abi.load()
    limit = lib.tessera_hip_attend_rows_noalloc_limit()
    assert limit == 16 << 20
    a = abi.RowsArgs()
    q = torch.zeros((512, 16, 128), device="cuda")
    kv = torch.zeros((16, 8, 128), device="cuda", dtype=torch.bfloat16)
    ids = torch.zeros(512, dtype=torch.int32, device="cuda")
    a = R.rows_args(q, kv, kv, q, ids, ids, keys=8192, scale=0.1, max_position=8191)
    assert lib.tessera_hip_attend_rows_workspace(C.byref(a)) > limit
    rc = lib.tessera_hip_attend_rows_noalloc(C.byref(a), None)
    assert rc == abi.TS_ERR_WORKSPACE and b"fixed scratch" in lib.tessera_hip_last_error()
