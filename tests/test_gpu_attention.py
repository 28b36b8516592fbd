"""Parity of the attention kernels with the oracle's attend_rows over paged K/V.

K/V are stored bf16 in the kept rows; the oracle reads the same bf16 values widened.
Tolerance: |got - want| <= 2e-4 (outputs are convex combinations of N(0,1) V rows;
q is carried in two exact bf16 parts, P in two parts for the prefill kernel, and
the rest is f32 in another summation order).
"""
import math

import numpy as np
import pytest

import oracle as O
from tests.helpers import bf16_bits_normal, from_dev, rng, to_dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
ATOL = 2e-4


def paged_case(seed, ctxs, heads=16, kv_heads=8, page=16, pos=None):
    """Kept rows for len(ctxs) slots in shuffled pages, one query row per slot at
    ctx-1 (decode) unless `pos` gives each row's (slot, position)."""
    r = rng(seed)
    slots_n = len(ctxs)
    kept_pages = max(math.ceil(c / page) for c in ctxs)
    total = slots_n * kept_pages
    table = r.permutation(total).astype(np.uint32)  # seeded shuffle of every page
    kb, kf = bf16_bits_normal(r, (total * page, kv_heads, 128))
    vb, vf = bf16_bits_normal(r, (total * page, kv_heads, 128))
    if pos is None:
        slots = np.arange(slots_n, dtype=np.uint32)
        positions = np.array([c - 1 for c in ctxs], np.uint32)
    else:
        slots, positions = (np.array(a, np.uint32) for a in pos)
    q = r.standard_normal((len(slots), heads, 128)).astype(np.float32)
    return dict(q=q, kb=kb, kf=kf, vb=vb, vf=vf, table=table, slots=slots, positions=positions,
                kept_pages=kept_pages, page=page, keys=kept_pages * page)


def run(kernel, c, scale, back=0xFFFFFFFF):
    from tessera_amd import rules as R
    fn = R.attend_rows if kernel == "attend" else R.flash_rows
    return from_dev(fn(to_dev(c["q"], torch), to_dev(c["kb"], torch), to_dev(c["vb"], torch),
                       to_dev(c["slots"], torch, torch.int32), to_dev(c["positions"], torch, torch.int32),
                       keys=c["keys"], scale=scale, table=to_dev(c["table"], torch, torch.int32),
                       kept_pages=c["kept_pages"], page=c["page"], back=back))


def want(c, scale, mask="causal", n=0):
    return O.attend_rows(c["q"], c["kf"], c["vf"], c["slots"], c["positions"], c["keys"], scale,
                         mask=mask, n=n, table=c["table"], kept_pages=c["kept_pages"], page=c["page"])


@pytest.mark.parametrize("ctxs", [[1], [17, 5, 33], [144], [512, 1000, 2049], [8192, 600]])
def test_decode_rows_paged(ctxs):
    c = paged_case(len(ctxs) * 100 + ctxs[0], ctxs)
    s = 1 / math.sqrt(128)
    np.testing.assert_allclose(run("attend", c, s), want(c, s), atol=ATOL, rtol=0)


def test_decode_rows_c3_sample():
    """C3 decode shape on a subset of rows: contexts U[512, 8192] (seed 2)."""
    ctxs = rng(2).integers(512, 8193, 8).tolist()
    c = paged_case(2, ctxs)
    s = 1 / math.sqrt(128)
    np.testing.assert_allclose(run("attend", c, s), want(c, s), atol=ATOL, rtol=0)


def test_decode_rows_c3_full():
    """The whole C3 decode shape: 32 rows, contexts U[512, 8192] (seed 2, as the bench
    draws them), 16 q / 8 kv heads, shuffled 16-row pages."""
    ctxs = rng(2).integers(512, 8193, 32).tolist()
    c = paged_case(2, ctxs)
    s = 1 / math.sqrt(128)
    np.testing.assert_allclose(run("attend", c, s), want(c, s), atol=ATOL, rtol=0)


@pytest.mark.parametrize("heads,kv_heads", [(4, 4), (32, 8), (16, 1)])
def test_decode_gqa_groups(heads, kv_heads):
    c = paged_case(9 + heads, [300, 70], heads=heads, kv_heads=kv_heads)
    np.testing.assert_allclose(run("attend", c, 0.1), want(c, 0.1), atol=ATOL, rtol=0)


def test_decode_window():
    c = paged_case(77, [400, 90])
    got = run("attend", c, 0.2, back=31)
    np.testing.assert_allclose(got, want(c, 0.2, "back", 31), atol=ATOL, rtol=0)


def test_decode_many_rows_per_slot():
    """Rows of one slot at several positions (a verify/prefill-like batch)."""
    c = paged_case(5, [100], pos=([0, 0, 0, 0], [0, 15, 16, 99]))
    np.testing.assert_allclose(run("attend", c, 0.3), want(c, 0.3), atol=ATOL, rtol=0)


@pytest.mark.parametrize("lens", [[1], [64], [100], [130, 70], [2048], [64, 64, 64], [10, 64, 5]])
def test_prefill_flash_rows(lens):
    """Prefill: each slot's rows at positions 0..len-1, slots padded to 64-row blocks
    apart (a 64-row block never crosses a slot)."""
    slots, positions = [], []
    for s, n in enumerate(lens):
        slots += [s] * n
        positions += list(range(n))
        pad = (-n) % 64
        if s + 1 < len(lens) and pad:
            # fill with the same slot's last position again so blocks stay in one slot
            slots += [s] * pad
            positions += [n - 1] * pad
    c = paged_case(sum(lens), lens, pos=(slots, positions))
    s = 1 / math.sqrt(128)
    np.testing.assert_allclose(run("flash", c, s), want(c, s), atol=ATOL, rtol=0)


@pytest.mark.parametrize("lens", [[130, 70], [2048]])
def test_prefill_flash_rows_bf16_q(lens):
    """bf16 q (the C3 prefill form): q single-part on the matrix unit, P rounded once
    to bf16. The oracle reads the same bf16 q widened; the one P rounding bounds the
    error by 2^-8 * max|v| per output (about 0.017 here); these cases stay within
    4e-3, which the test holds them to."""
    from tessera_amd import rules as R
    slots, positions = [], []
    for s_, n in enumerate(lens):
        slots += [s_] * n
        positions += list(range(n))
        pad = (-n) % 64
        if s_ + 1 < len(lens) and pad:
            slots += [s_] * pad
            positions += [n - 1] * pad
    c = paged_case(sum(lens) + 1, lens, pos=(slots, positions))
    qb = O.bf16_narrow(c["q"])
    c["q"] = O.bf16_widen(qb)
    s = 1 / math.sqrt(128)
    got = from_dev(R.flash_rows(to_dev(qb, torch), to_dev(c["kb"], torch), to_dev(c["vb"], torch),
                                to_dev(c["slots"], torch, torch.int32), to_dev(c["positions"], torch, torch.int32),
                                keys=c["keys"], scale=s, table=to_dev(c["table"], torch, torch.int32),
                                kept_pages=c["kept_pages"], page=c["page"]))
    np.testing.assert_allclose(got, want(c, s), atol=4e-3, rtol=0)


@pytest.mark.parametrize("scale", [-1 / math.sqrt(128), 0.0, 0.3])
@pytest.mark.parametrize("bf16_q", [False, True])
def test_prefill_flash_rows_scale_sign(scale, bf16_q):
    """Negative, zero and large scales: the kernel folds the scale's sign into q and
    takes a maximum of raw scores, so a wrong sign fold picks the smallest score as
    the reference point (and overflows p) and a zero scale must give the plain mean
    of the window's V rows."""
    from tessera_amd import rules as R
    lens = [130, 70]
    slots, positions = [], []
    for s_, n in enumerate(lens):
        slots += [s_] * n
        positions += list(range(n))
        pad = (-n) % 64
        if s_ + 1 < len(lens) and pad:
            slots += [s_] * pad
            positions += [n - 1] * pad
    c = paged_case(7, lens, pos=(slots, positions))
    q = c["q"]
    if bf16_q:
        q = O.bf16_narrow(c["q"])
        c["q"] = O.bf16_widen(q)
    got = from_dev(R.flash_rows(to_dev(q, torch), to_dev(c["kb"], torch), to_dev(c["vb"], torch),
                                to_dev(c["slots"], torch, torch.int32), to_dev(c["positions"], torch, torch.int32),
                                keys=c["keys"], scale=scale, table=to_dev(c["table"], torch, torch.int32),
                                kept_pages=c["kept_pages"], page=c["page"]))
    # bf16 q: P is rounded once to bf16 (8 significant bits: relative 2^-8), so each
    # output, a p-weighted mean of V rows, is off by at most 2^-8 * max|v|.
    atol = 2.0 ** -8 * float(np.abs(c["vf"]).max()) if bf16_q else ATOL
    np.testing.assert_allclose(got, want(c, scale), atol=atol, rtol=0)


@pytest.mark.parametrize("heads,kv_heads", [(8, 2), (4, 4), (6, 2)])
def test_prefill_flash_window_and_gqa(heads, kv_heads):
    """A window of 40 keys; q heads per kv head 4 (groups of 8 waves over two heads),
    1 and 3 (groups of 4 waves over one head)."""
    c = paged_case(8, [200], heads=heads, kv_heads=kv_heads, pos=([0] * 200, list(range(200))))
    np.testing.assert_allclose(run("flash", c, 0.25, back=40), want(c, 0.25, "back", 40), atol=ATOL, rtol=0)


@pytest.mark.parametrize("ctx", [1, 16, 17, 150, 3000])
def test_attend_step_fused(ctx):
    """q/k RmsNorm + Halves RoPE + append + attend in one launch, against the oracle's
    chain (rms_norm per head, rope, bf16 kept rows, attend_rows)."""
    from tessera_amd import rules as R
    c = paged_case(ctx, [ctx], pos=([0], [ctx - 1]))
    r = rng(ctx + 5)
    heads, kvh = 16, 8
    qkv = r.standard_normal((1, (heads + 2 * kvh) * 128)).astype(np.float32)
    qg = (1 + 0.05 * r.standard_normal(128)).astype(np.float32)
    kg = (1 + 0.05 * r.standard_normal(128)).astype(np.float32)
    kd, vd = to_dev(c["kb"], torch), to_dev(c["vb"], torch)
    s = 1 / math.sqrt(128)
    got = from_dev(R.attend_step(to_dev(qkv, torch), to_dev(qg, torch), to_dev(kg, torch), kd, vd,
                                 to_dev(c["slots"], torch, torch.int32), to_dev(c["positions"], torch, torch.int32),
                                 heads=heads, keys=c["keys"], scale=s, eps=1e-6, theta=1e6,
                                 table=to_dev(c["table"], torch, torch.int32), kept_pages=c["kept_pages"],
                                 page=c["page"]))
    pos = np.array([ctx - 1], np.uint32)
    q = O.rope(O.rms_norm(qkv[:, : heads * 128].reshape(1, heads, 128), qg, 1e-6), pos, 1e6)
    k = O.rope(O.rms_norm(qkv[:, heads * 128:(heads + kvh) * 128].reshape(1, kvh, 128), kg, 1e-6), pos, 1e6)
    v = qkv[:, (heads + kvh) * 128:].reshape(1, kvh, 128)
    row = O.paged_row(c["table"], c["kept_pages"], c["page"], 0, ctx - 1)
    kf, vf = c["kf"].copy(), c["vf"].copy()
    kf[row], vf[row] = O.bf16_round(k[0]), O.bf16_round(v[0])
    want = O.attend_rows(q, kf, vf, [0], pos, c["keys"], s, table=c["table"], kept_pages=c["kept_pages"],
                         page=c["page"])
    np.testing.assert_allclose(got, want, atol=ATOL, rtol=0)
    # The new rows landed in the kept rows, bf16: v exactly, k within one bf16 step
    # (device powf/sincosf against the host's for the rotation angle).
    assert np.array_equal(from_dev(vd)[row], vf[row])
    np.testing.assert_allclose(from_dev(kd)[row], kf[row], rtol=2 ** -7, atol=1e-6)


def _packed(lens):
    """Prompts packed back to back with no padding (the lowered Launch layout): rows
    of slot s at positions 0..len-1, then the next slot's rows at once."""
    slots, positions = [], []
    for s_, n in enumerate(lens):
        slots += [s_] * n
        positions += list(range(n))
    return slots, positions


@pytest.mark.parametrize("lens", [[70, 130, 5], [3] * 45, [1, 2, 200, 1, 64, 63], [127, 129]])
def test_prefill_flash_rows_packed(lens):
    """Ragged prompts back to back: 128-row groups hold rows of several slots (up to 43
    in one group for [3] * 45); each group makes one pass per distinct slot."""
    c = paged_case(sum(lens) + 7, lens, pos=_packed(lens))
    s = 1 / math.sqrt(128)
    np.testing.assert_allclose(run("flash", c, s), want(c, s), atol=ATOL, rtol=0)


@pytest.mark.parametrize("prompts", [200, 262])
def test_prefill_flash_rows_many_groups(prompts):
    """Hundreds of ragged prompts packed back to back (lengths 100..156): 200 prompts
    give ~200 128-row groups that the kernel ranks by their key spans and runs widest
    first; 262 give more groups than it ranks (256), which run in launch order. Every
    row is checked against the oracle (2 q heads over 1 kv head keep it small)."""
    lens = [100 + (i * 37) % 57 for i in range(prompts)]
    assert (sum(lens) + 127) // 128 > 256 if prompts == 262 else (sum(lens) + 127) // 128 <= 256
    c = paged_case(prompts, lens, heads=2, kv_heads=1, pos=_packed(lens))
    s = 1 / math.sqrt(128)
    np.testing.assert_allclose(run("flash", c, s), want(c, s), atol=ATOL, rtol=0)


def test_prefill_flash_rows_interleaved_slots():
    """Rows of two slots interleaved row by row (slots not in runs), a window of 50."""
    n = 150
    slots = [i % 2 for i in range(2 * n)]
    positions = [i // 2 for i in range(2 * n)]
    c = paged_case(31, [n, n], pos=(slots, positions))
    np.testing.assert_allclose(run("flash", c, 0.2, back=50), want(c, 0.2, "back", 50), atol=ATOL, rtol=0)


def test_prefill_flash_rows_packed_bf16_q():
    """The packed layout on the bf16-q form (atol 4e-3: P rounded once to bf16)."""
    from tessera_amd import rules as R
    lens = [70, 130, 5]
    c = paged_case(99, lens, pos=_packed(lens))
    qb = O.bf16_narrow(c["q"])
    c["q"] = O.bf16_widen(qb)
    s = 1 / math.sqrt(128)
    got = from_dev(R.flash_rows(to_dev(qb, torch), to_dev(c["kb"], torch), to_dev(c["vb"], torch),
                                to_dev(c["slots"], torch, torch.int32), to_dev(c["positions"], torch, torch.int32),
                                keys=c["keys"], scale=s, table=to_dev(c["table"], torch, torch.int32),
                                kept_pages=c["kept_pages"], page=c["page"]))
    np.testing.assert_allclose(got, want(c, s), atol=4e-3, rtol=0)


@pytest.mark.parametrize("kernel,ctxs", [("attend", [300, 40]), ("attend", [3000, 600]), ("flash", [200, 90])])
def test_refused_positions(kernel, ctxs):
    """A row whose position the slot cannot hold (>= keys) or beyond the stated
    max_position is refused on the device, as the interpreter refuses a read at >= keys
    (engine/ir/interp/src/cpu.rs:323-327): it loads nothing, its outputs are NaN and the
    status word gets TS_STATUS_POSITION; the other rows are unchanged. [3000, 600] runs
    the split path (partials merged by a second kernel); every kernel exits normally."""
    from tessera_amd import abi
    from tessera_amd import rules as R
    if kernel == "attend":
        pos = ([0, 1, 0, 1], [ctxs[0] - 1, ctxs[1] - 1, 0, 0])
    else:
        pos = ([0] * ctxs[0] + [1] * ctxs[1], list(range(ctxs[0])) + list(range(ctxs[1])))
    c = paged_case(55 + ctxs[0], ctxs, pos=pos)
    s = 1 / math.sqrt(128)
    good = want(c, s)
    bad_rows = [2, 3] if kernel == "attend" else [5, ctxs[0] + 3]
    positions = c["positions"].copy()
    positions[bad_rows[0]] = c["keys"]            # the slot cannot hold it
    positions[bad_rows[1]] = c["keys"] + 1000     # past the slot's table row too
    mp = int(c["positions"].max())
    fn = R.attend_rows if kernel == "attend" else R.flash_rows
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    got = from_dev(fn(to_dev(c["q"], torch), to_dev(c["kb"], torch), to_dev(c["vb"], torch),
                      to_dev(c["slots"], torch, torch.int32), to_dev(positions, torch, torch.int32),
                      keys=c["keys"], scale=s, table=to_dev(c["table"], torch, torch.int32),
                      kept_pages=c["kept_pages"], page=c["page"], max_position=mp, status=status))
    torch.cuda.synchronize()
    assert int(status.item()) == abi.TS_STATUS_POSITION
    keep = np.setdiff1d(np.arange(len(positions)), bad_rows)
    np.testing.assert_allclose(got[keep], good[keep], atol=ATOL, rtol=0)
    assert np.all(np.isnan(got[bad_rows]))
    # In range, the word stays clear.
    status.zero_()
    fn(to_dev(c["q"], torch), to_dev(c["kb"], torch), to_dev(c["vb"], torch),
       to_dev(c["slots"], torch, torch.int32), to_dev(c["positions"], torch, torch.int32),
       keys=c["keys"], scale=s, table=to_dev(c["table"], torch, torch.int32),
       kept_pages=c["kept_pages"], page=c["page"], max_position=mp, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0


def test_refused_beyond_max_position():
    """A row past the launch's stated max_position (which sized the key split) is
    refused rather than read with part of its keys dropped."""
    from tessera_amd import abi
    from tessera_amd import rules as R
    c = paged_case(61, [500, 500])
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    got = from_dev(R.attend_rows(to_dev(c["q"], torch), to_dev(c["kb"], torch), to_dev(c["vb"], torch),
                                 to_dev(c["slots"], torch, torch.int32), to_dev(c["positions"], torch, torch.int32),
                                 keys=c["keys"], scale=0.1, table=to_dev(c["table"], torch, torch.int32),
                                 kept_pages=c["kept_pages"], page=c["page"], max_position=200, status=status))
    torch.cuda.synchronize()
    assert int(status.item()) == abi.TS_STATUS_POSITION
    assert np.all(np.isnan(got))


def test_prefill_c3_full():
    """The whole C3 prefill shape as benchmarked: 4 slots x 2048 causal rows (8192 rows
    packed back to back), bf16 q, 16 q / 8 kv heads, shuffled 16-row pages, one
    launch; the oracle on 24 sampled rows of each slot (first and last positions, the
    page and 128-row group edges, random ones). Tolerance as the bf16-q case: 4e-3."""
    from tessera_amd import rules as R
    lens = [2048] * 4
    slots = np.repeat(np.arange(4), 2048).astype(np.uint32)
    positions = np.tile(np.arange(2048), 4).astype(np.uint32)
    c = paged_case(3, lens, pos=(slots, positions))
    qb = O.bf16_narrow(c["q"])
    s = 1 / math.sqrt(128)
    got = from_dev(R.flash_rows(to_dev(qb, torch), to_dev(c["kb"], torch), to_dev(c["vb"], torch),
                                to_dev(c["slots"], torch, torch.int32), to_dev(c["positions"], torch, torch.int32),
                                keys=c["keys"], scale=s, table=to_dev(c["table"], torch, torch.int32),
                                kept_pages=c["kept_pages"], page=c["page"]))
    r = rng(33)
    pick = []
    for sl in range(4):
        base = sl * 2048
        fixed = [0, 1, 15, 16, 127, 128, 1023, 1024, 2046, 2047]
        pick += [base + p for p in fixed] + list(base + r.choice(2048, 14, replace=False))
    pick = np.array(sorted(set(pick)))
    sub = dict(c, q=O.bf16_widen(qb[pick]), slots=c["slots"][pick], positions=c["positions"][pick])
    np.testing.assert_allclose(got[pick], want(sub, s), atol=4e-3, rtol=0)


# attention_test.rs:44-60 flash_matches_cpu: (seqs, rows, keys) and the five masks.
FLASH_CASES = [(1, 1, 1), (1, 1, 38), (2, 7, 7), (1, 33, 33), (2, 70, 93), (1, 128, 128), (2, 300, 300),
               (1, 40, 20)]
FLASH_MASKS = [("causal", 0), ("bidirectional", 0), ("within", 5), ("within", 40), ("back", 5)]


@pytest.mark.parametrize("mask,n", FLASH_MASKS)
@pytest.mark.parametrize("heads,kv_heads", [(2, 2), (16, 8)])
def test_flash_whole_sequences_every_mask(mask, n, heads, kv_heads):
    """Whole-sequence flash (tessera_hip_flash) against the oracle's attend over the
    reference test's cases, f32 q, bf16 K/V. More rows than keys (1, 40, 20) is
    refused for the causal masks, as interp refuses it; for the others the rows start
    at position 0 and rows past every key's window write zeros."""
    from tessera_amd import abi, rules as R
    s = 1 / math.sqrt(128)
    for seqs, rows, keys in FLASH_CASES:
        r = rng(seqs * 1000 + rows * 10 + keys + heads)
        q = r.standard_normal((seqs, rows, heads, 128)).astype(np.float32)
        kb, kf = bf16_bits_normal(r, (seqs, keys, kv_heads, 128))
        vb, vf = bf16_bits_normal(r, (seqs, keys, kv_heads, 128))
        if keys < rows and mask in ("causal", "back"):
            with pytest.raises(abi.HipError, match="causal mask"):
                R.flash(to_dev(q, torch), to_dev(kb, torch), to_dev(vb, torch), scale=s, mask=mask, n=n)
            continue
        got = from_dev(R.flash(to_dev(q, torch), to_dev(kb, torch), to_dev(vb, torch), scale=s, mask=mask, n=n))
        want = O.attend(q, kf, vf, s, mask, n)
        np.testing.assert_allclose(got, want, atol=ATOL, rtol=0, err_msg=f"{(seqs, rows, keys)}")


def test_flash_bf16_q_within_window():
    """bf16 q (P once in bf16: 4e-3 as the ragged bf16-q case), a window both ways, 2
    sequences of 1000 rows over 1200 keys."""
    from tessera_amd import rules as R
    r = rng(77)
    s = 1 / math.sqrt(128)
    qb, qf = bf16_bits_normal(r, (2, 1000, 16, 128))
    kb, kf = bf16_bits_normal(r, (2, 1200, 8, 128))
    vb, vf = bf16_bits_normal(r, (2, 1200, 8, 128))
    got = from_dev(R.flash(to_dev(qb, torch), to_dev(kb, torch), to_dev(vb, torch), scale=s, mask="within", n=100))
    np.testing.assert_allclose(got, O.attend(qf, kf, vf, s, "within", 100), atol=4e-3, rtol=0)
