"""Copy-on-write of a shared partial page, end to end on the device.

The scenario of the reference's pool test `shared_writes_copy`
(engine/ir/kv/src/pool_test.rs:20-41) at the kept-row shape of the decoder (16-row
pages, 8 kv heads x 128 bf16): run a holds 40 rows (two whole pages and a partial
third), run b forks it at 40 rows, b grows to 41 and receives a PageCopy of the 8
written rows of the shared last page; the copy runs on the device
(tessera_hip_kv_copy), a grows with no copy, then one fused attend_step launch appends
each run's row 40 and attends over rows 0..40 of its own run.

Checked against the interpreter's Store::append semantics (engine/ir/interp/src/
run.rs:122-198: each run keeps its own rows, appended at its own positions): every
kept row read through each run's table row is bit-identical to that run's dense
store (the new k row within one bf16 step: device vs host angle), and the outputs
match the oracle's attend_rows over the dense stores within 2e-4.
"""
import math

import numpy as np
import pytest

import oracle as O
from tests.helpers import bf16_bits_normal, from_dev, rng, to_dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def test_fork_grow_copy_append_attend():
    from tessera_amd import kv
    from tessera_amd import rules as R
    page, kvh, heads, D, worst = 16, 8, 16, 128, 100
    pool = kv.Pool(32, page)
    a = pool.reserve(0, 40, worst)
    b = pool.fork(a, 40, worst)
    first, second, last = pool.pages(a)
    assert pool.pages(b) == [first, second, last]

    r = rng(404)
    total = 32 * page
    kb, kf = bf16_bits_normal(r, (total, kvh, D))
    vb, vf = bf16_bits_normal(r, (total, kvh, D))
    K, V = to_dev(kb, torch), to_dev(vb, torch)

    copies = pool.grow(b, 41)
    assert len(copies) == 1
    frm, to, rows = copies[0]
    assert (frm, rows) == (last, 8) and to not in (first, second, last)
    assert pool.pages(b) == [first, second, to]
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    kv.copy_pages([K, V], copies, page=page, pages=32, status=status)
    assert pool.grow(a, 41) == []
    assert pool.consistent()

    kept_pages = math.ceil(worst / page)
    table = np.zeros((2, kept_pages), np.uint32)
    table[0, :3] = pool.pages(a)
    table[1, :3] = pool.pages(b)
    keys = kept_pages * page

    # Each run's dense store (Store::append): rows 0..39 are a's written rows.
    def rows_of(pages_, n):
        return np.array([pages_[p // page] * page + p % page for p in range(n)])
    src = rows_of([first, second, last], 40)
    dense_k = np.zeros((2 * keys, kvh, D), np.float32)
    dense_v = np.zeros((2 * keys, kvh, D), np.float32)
    for s_ in range(2):
        dense_k[s_ * keys: s_ * keys + 40] = kf[src]
        dense_v[s_ * keys: s_ * keys + 40] = vf[src]

    qkv = r.standard_normal((2, (heads + 2 * kvh) * D)).astype(np.float32)
    qg = (1 + 0.05 * r.standard_normal(D)).astype(np.float32)
    kg = (1 + 0.05 * r.standard_normal(D)).astype(np.float32)
    slots = np.array([0, 1], np.uint32)
    pos = np.array([40, 40], np.uint32)
    s = 1 / math.sqrt(D)
    got = from_dev(R.attend_step(to_dev(qkv, torch), to_dev(qg, torch), to_dev(kg, torch), K, V,
                                 to_dev(slots, torch, torch.int32), to_dev(pos, torch, torch.int32),
                                 heads=heads, keys=keys, scale=s, eps=1e-6, theta=1e6,
                                 table=to_dev(table, torch, torch.int32), kept_pages=kept_pages, page=page))
    torch.cuda.synchronize()
    assert int(status.item()) == 0

    q = O.rope(O.rms_norm(qkv[:, : heads * D].reshape(2, heads, D), qg, 1e-6), pos, 1e6)
    k_new = O.rope(O.rms_norm(qkv[:, heads * D:(heads + kvh) * D].reshape(2, kvh, D), kg, 1e-6), pos, 1e6)
    v_new = qkv[:, (heads + kvh) * D:].reshape(2, kvh, D)
    for s_ in range(2):
        dense_k[s_ * keys + 40] = O.bf16_round(k_new[s_])
        dense_v[s_ * keys + 40] = O.bf16_round(v_new[s_])
    want = O.attend_rows(q, dense_k, dense_v, slots, pos, keys, s)
    np.testing.assert_allclose(got, want, atol=2e-4, rtol=0)

    # Kept rows through each run's table row, against its dense store.
    K_after, V_after = from_dev(K), from_dev(V)
    for s_, pages_ in enumerate([pool.pages(a), pool.pages(b)]):
        at = rows_of(pages_, 41)
        assert np.array_equal(V_after[at], dense_v[s_ * keys: s_ * keys + 41]), s_
        assert np.array_equal(K_after[at[:40]], dense_k[s_ * keys: s_ * keys + 40]), s_
        np.testing.assert_allclose(K_after[at[40]], dense_k[s_ * keys + 40], rtol=2 ** -7, atol=1e-6)
    # The copy wrote only the 8 written rows of the new page; a's page kept its rows.
    assert np.array_equal(K_after[to * page + 8 + 1: to * page + 16], kf[to * page + 9: to * page + 16])


def test_copy_refuses_bad_pages():
    """Copies naming a page past the buffers, more rows than a page, or a page onto
    itself are skipped and reported (TS_KV_STATUS_COPY); a good copy in the same call
    still runs; every kernel exits normally."""
    from tessera_amd import kv
    page = 16
    K = torch.arange(8 * page * 256, dtype=torch.int32, device="cuda").view(8 * page, 256)
    before = K.clone()
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    kv.copy_pages([K], [(1, 9, 4), (2, 3, 17), (4, 4, 2), (5, 6, 3)], page=page, pages=8, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == kv.STATUS_COPY
    want = before.clone()
    want[6 * page: 6 * page + 3] = before[5 * page: 5 * page + 3]
    assert torch.equal(K, want)


def test_copy_skips_overlapping_pages():
    """Copies of one call run at once: a copy whose target another copy reads or writes
    is skipped on the device with its partner, and reported; an unrelated copy runs."""
    from tessera_amd import kv
    page = 16
    K = torch.arange(8 * page * 256, dtype=torch.int32, device="cuda").view(8 * page, 256)
    before = K.clone()
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    kv.copy_pages([K], [(1, 2, 4), (2, 3, 4), (5, 6, 3)], page=page, pages=8, status=status, check=False)
    torch.cuda.synchronize()
    assert int(status.item()) == kv.STATUS_COPY
    want = before.clone()
    want[6 * page: 6 * page + 3] = before[5 * page: 5 * page + 3]
    assert torch.equal(K, want)
