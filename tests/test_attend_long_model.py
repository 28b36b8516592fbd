"""A CPU model of attend_long_kernel's address arithmetic (tessera_amd/csrc/attention.hip),
run over the C3 decode inputs (32 rows, contexts U[512, 8192] seed 2, 16 q / 8 kv heads,
16-row pages in a shuffled table) at the split the library picks (groups of 2 waves) and
at every pinned iteration count 1..32, for groups of 2 waves and of 8 (the earlier form):
every page-table read, LDS table index, kept-row load, partial write and merge read must
land inside its buffer.

This guards the conclusion that the long-context kernel's accesses are in bounds for
every iteration count (one such pinned count once ran on a GPU together with a
workspace overrun in another kernel, since fixed). The model restates the kernel's
index formulas line by line; the workspace size comes from the library's own query.
"""
import ctypes as C

import numpy as np

LONG_WAVES, LONG_PAGES, LONG_SPAN = 2, 1024, 2048  # waves a group as built
G_STRIDE = 130  # floats of one (max, sum, 128 acc) partial


def c3_decode_case():
    r = np.random.default_rng(2)
    ctxs = r.integers(512, 8193, 32)
    page, kv_heads, heads = 16, 8, 16
    kept_pages = int(np.ceil(ctxs.max() / page))
    total = 32 * kept_pages
    table = np.random.default_rng(2).permutation(total).astype(np.uint32)
    return dict(pos=(ctxs - 1).astype(np.int64), slots=np.arange(32), page=page, kv_heads=kv_heads, heads=heads,
                kept_pages=kept_pages, keys=kept_pages * page, table=table, total_rows=total * page)


def library_split_iters(span):
    """split() of attention.hip for the long kernel: iters = clamp(span / (16 * 2 * 32), 1, 32)."""
    return max(1, min(32, span // (16 * LONG_WAVES * 32)))


def model(case, iters, workspace_floats, waves=LONG_WAVES):
    pos, slots = case["pos"], case["slots"]
    shift = int(np.log2(case["page"]))
    pmask = case["page"] - 1
    kvh_n, G = case["kv_heads"], case["heads"] // case["kv_heads"]
    kept_pages, table, total_rows = case["kept_pages"], case["table"], case["total_rows"]
    span = int(pos.max()) + 1
    span_keys = waves * 32 * iters
    parts = (span + span_keys - 1) // span_keys
    rows = len(pos)
    # the merge reads every partition of every (row, kv head)
    assert rows * kvh_n * parts * G * G_STRIDE <= workspace_floats
    for r in range(rows):
        p_, slot = int(pos[r]), int(slots[r])
        frm = 0  # back = all
        for part in range(parts):
            g0, g1 = part * span_keys, part * span_keys + span_keys
            for kvh in range(kvh_n):
                gi = r * kvh_n + kvh
                mine = (gi * parts + part) * G * G_STRIDE
                assert 0 <= mine and mine + G * G_STRIDE <= workspace_floats
            if g0 > p_ or g1 <= frm:
                continue  # an empty partial: written above, nothing loaded
            p0 = g0 >> shift
            np_ = min((min(g1, p_ + 1) - 1) >> shift, kept_pages - 1) - p0 + 1
            assert 1 <= np_ <= LONG_PAGES
            assert slot * kept_pages + p0 + np_ - 1 < table.size  # the table rows copied to LDS
            stab = table[slot * kept_pages + p0: slot * kept_pages + p0 + np_].astype(np.int64)
            for wave in range(waves):
                w0 = g0 + wave * 32 * iters
                kb = w0 + 16 * np.arange(2 * iters)  # every block the prefetch loop loads
                kbc = np.minimum(kb, p_) & ~15
                si = (kbc >> shift) - p0
                assert si.min() >= 0 and si.max() < np_, (r, part, wave)
                row0 = (stab[si] << shift) | (kbc & pmask)
                # K: key min(col, 15); V: key min(4 j + grp, 15) -> rows row0 .. row0 + 15 of one page
                assert row0.min() >= 0 and (row0 + 15).max() < total_rows
                assert np.all((row0 & pmask) == 0)  # a 16-key block never crosses a page
    return parts


def test_attend_long_accesses_in_bounds_at_every_iteration_count():
    from tessera_amd import abi
    case = c3_decode_case()
    lib = abi.load()
    a = abi.RowsArgs()
    a.rows, a.heads, a.kv_heads, a.width = 32, case["heads"], case["kv_heads"], 128
    a.max_position = int(case["pos"].max())
    span = a.max_position + 1
    assert span > LONG_SPAN  # the C3 decode shape takes the long kernel
    query = lib.tessera_hip_attend_rows_workspace(C.byref(a)) // 4
    # the library's own split
    model(case, library_split_iters(span), query)
    # every pinned iteration count, with a workspace sized for that count's partitions,
    # for groups of 2 waves and of 8
    for waves in (LONG_WAVES, 8):
        for iters in range(1, 33):
            parts = (span + waves * 32 * iters - 1) // (waves * 32 * iters)
            need = 32 * case["kv_heads"] * parts * (case["heads"] // case["kv_heads"]) * G_STRIDE
            assert model(case, iters, need, waves) == parts


def test_model_catches_an_overrun():
    """The model is not vacuous: one float short of the merge's partials fails."""
    import pytest
    case = c3_decode_case()
    span = int(case["pos"].max()) + 1
    parts = (span + LONG_WAVES * 32 * 2 - 1) // (LONG_WAVES * 32 * 2)
    need = 32 * case["kv_heads"] * parts * 2 * G_STRIDE
    with pytest.raises(AssertionError):
        model(case, 2, need - 1)
