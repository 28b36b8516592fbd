"""Parity of the row-stage and index kernels with the oracle.

Floating point: RmsNorm and RoPE within 1e-5 relative to max|x| (different sum
order; device sin/cos/pow within a few ulp). Indices: bit-exact.
"""
import math

import numpy as np
import pytest

import oracle as O
from tests.helpers import bf16_bits_normal, from_dev, rng, to_dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def R():
    from tessera_amd import rules
    return rules


def test_rms_norm():
    r = rng(1)
    x = r.standard_normal((5, 1024)).astype(np.float32)
    g = (1 + 0.02 * r.standard_normal(1024)).astype(np.float32)
    got = from_dev(R().rms_norm(to_dev(x, torch), to_dev(g, torch), 1e-6))
    np.testing.assert_allclose(got, O.rms_norm(x, g, 1e-6), rtol=1e-5, atol=1e-6)
    # rms_divides_rows (cpu_test.rs:130-146) at a width of 4.
    x = np.array([[1, -3, 5, -1], [2, 0, 0, -2]], np.float32)
    w = np.array([1, 2, -1, 0.5], np.float32)
    got = from_dev(R().rms_norm(to_dev(x, torch), to_dev(w, torch), 7.0))
    np.testing.assert_allclose(got.reshape(-1), [0.25, -1.5, -1.25, -0.125, 2 / 3, 0, 0, -1 / 3], rtol=1e-6)


@pytest.mark.parametrize("halves", [True, False])
def test_rope(halves):
    # rope_both_pairs (cpu_test.rs:116-128): positions 0 and 3, theta 4, width 4.
    x = (np.arange(16, dtype=np.float32) - 5.5).reshape(2, 2, 4)
    xd = to_dev(x, torch)
    R().rope(xd, to_dev(np.array([0, 3], np.uint32), torch, torch.int32), 4.0, halves)
    want = O.rope(x, [0, 3], 4.0, "halves" if halves else "adjacent")
    np.testing.assert_allclose(from_dev(xd), want, rtol=1e-6, atol=1e-6)
    # Qwen3 shape: theta 1e6, positions up to 8191.
    r = rng(2)
    x = r.standard_normal((6, 16, 128)).astype(np.float32)
    pos = np.array([0, 1, 127, 128, 4000, 8191], np.uint32)
    xd = to_dev(x, torch)
    R().rope(xd, to_dev(pos, torch, torch.int32), 1e6, halves)
    want = O.rope(x, pos, 1e6, "halves" if halves else "adjacent")
    np.testing.assert_allclose(from_dev(xd), want, atol=2e-3 * np.abs(x).max(), rtol=0)


def test_qk_norm_rope_append():
    """Per-head RmsNorm, Halves RoPE, then k/v rows written bf16 into paged kept rows."""
    r = rng(3)
    rows, heads, kvh, page = 3, 16, 8, 16
    qkv = r.standard_normal((rows, (heads + 2 * kvh) * 128)).astype(np.float32)
    qg = (1 + 0.02 * r.standard_normal(128)).astype(np.float32)
    kg = (1 + 0.02 * r.standard_normal(128)).astype(np.float32)
    slots = np.array([0, 1, 1], np.uint32)
    positions = np.array([5, 0, 17], np.uint32)
    kept_pages = 2
    table = np.array([3, 1, 0, 2], np.uint32)
    kc = torch.zeros((4 * page, kvh, 128), dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    qo = torch.empty((rows, heads, 128), device="cuda")
    R().qk_norm_rope_append(to_dev(qkv, torch), to_dev(qg, torch), to_dev(kg, torch), qo, kc, vc,
                            to_dev(slots, torch, torch.int32), to_dev(positions, torch, torch.int32),
                            heads=heads, kv_heads=kvh, keys=32, eps=1e-6, theta=1e6,
                            table=to_dev(table, torch, torch.int32), kept_pages=kept_pages, page=page)
    q = qkv[:, : heads * 128].reshape(rows, heads, 128)
    k = qkv[:, heads * 128:(heads + kvh) * 128].reshape(rows, kvh, 128)
    v = qkv[:, (heads + kvh) * 128:].reshape(rows, kvh, 128)
    wq = O.rope(O.rms_norm(q, qg, 1e-6), positions, 1e6)
    wk = O.rope(O.rms_norm(k, kg, 1e-6), positions, 1e6)
    np.testing.assert_allclose(from_dev(qo), wq, atol=1e-4, rtol=0)
    kcn, vcn = from_dev(kc), from_dev(vc)
    for i in range(rows):
        row = O.paged_row(table, kept_pages, page, int(slots[i]), int(positions[i]))
        # bf16 storage: within one bf16 rounding of the oracle's f32 value.
        np.testing.assert_allclose(kcn[row], wk[i], rtol=2 ** -8, atol=1e-6)
        assert np.array_equal(kcn[row], O.bf16_round(kcn[row]))
        assert np.array_equal(vcn[row], O.bf16_round(v[i]))


def test_gather_rows():
    # gather_rows (cpu_test.rs:199-211) on a bf16 table: repeats, both ends, past the end.
    table = np.array([[1, 2], [3, 4], [5, 6], [7, 8]], np.float32)
    tb = O.bf16_narrow(table)
    got = from_dev(R().gather(to_dev(tb, torch), to_dev(np.array([3, 0, 3, 4], np.uint32), torch, torch.int32)))
    np.testing.assert_array_equal(got.reshape(-1), [7, 8, 1, 2, 7, 8, 0, 0])
    r = rng(4)
    tb, tf = bf16_bits_normal(r, (1000, 1024))
    ids = r.integers(0, 1000, 7).astype(np.uint32)
    got = from_dev(R().gather(to_dev(tb, torch), to_dev(ids, torch, torch.int32)))
    assert np.array_equal(got, O.gather(tf, ids))


def test_argmax_bit_exact():
    # top_k(1) contract (run.rs:577-591): first index of the max, NaN/-inf skipped.
    r = rng(5)
    x = r.standard_normal((3, 151936)).astype(np.float32)
    x[1, 1000] = x[1, 90000] = 50.0           # a tie: lower index wins
    x[2, :] = -np.inf
    x[2, 7] = np.nan
    x[2, 151935] = -1.0
    got = from_dev(R().argmax(to_dev(x, torch)))
    want = O.top_k(x, 1).reshape(-1)
    assert got.tolist() == want.astype(np.int64).tolist()
    allbad = np.full((1, 9000), -np.inf, np.float32)
    assert from_dev(R().argmax(to_dev(allbad, torch))).tolist() == [9000]


def test_top_k_routing_bit_exact():
    """C5 routing: top-8 of 128 per row, plus the run_test.rs:55-66 tie cases."""
    inf, nan = np.inf, np.nan
    x = np.array([2, 7, 7, -1, -inf, 3, nan, -inf, -0.0, 0.0, -0.0, inf], np.float32).reshape(3, 4)
    got = from_dev(R().top_k(to_dev(x, torch), 3))
    assert got.reshape(-1).tolist() == [1, 2, 0, 1, 4, 4, 3, 0, 1]
    r = rng(3)
    logits = r.standard_normal((4096, 128)).astype(np.float32)
    logits[::7, 5] = logits[::7, 9]  # exact ties
    got = from_dev(R().top_k(to_dev(logits, torch), 8))
    assert np.array_equal(got.astype(np.uint32), O.top_k(logits, 8))


def test_rope_table_matches_angles():
    """The angle table against the oracle's angle (cpu.rs:32-34) at Qwen3's theta."""
    t = from_dev(R().rope_table(200, 1e6)).reshape(200, 64, 2)
    for pos in (0, 1, 77, 199):
        for j in (0, 1, 31, 63):
            ang = O.angle(pos, j, 128, 1e6)
            assert abs(t[pos, j, 0] - math.cos(ang)) < 2e-6 and abs(t[pos, j, 1] - math.sin(ang)) < 2e-6


@pytest.mark.parametrize("m", [1, 2, 4])
def test_argmax_fused_into_the_product(m):
    """TS_AFTER_ARGMAX: the pick folded into the lm_head product equals argmax over the
    logits the same launch wrote (first index of the max; NaN and -inf skipped), with
    two identical weight rows (a tie), a NaN row and a -inf row; the keys are zero again
    after, so a second call reuses them."""
    n, k = 151936, 1024
    r = rng(40 + m)
    wbits, _ = bf16_bits_normal(r, (n, k), 0.02)
    wbits[90000] = wbits[1000] = O.bf16_narrow(np.full(k, 0.5, np.float32))  # large and equal
    wbits[5] = O.bf16_narrow(np.full(k, np.nan, np.float32))
    wbits[6] = O.bf16_narrow(np.full(k, -np.inf, np.float32))
    x = np.abs(r.standard_normal((m, k))).astype(np.float32)
    g = (1.0 + 0.1 * r.standard_normal(k)).astype(np.float32)
    keys = torch.zeros(m, dtype=torch.int64, device="cuda")
    for _ in range(2):
        logits, ids = R().linear_argmax(to_dev(x, torch), to_dev(wbits, torch), gain=to_dev(g, torch), keys=keys)
        lg = from_dev(logits)
        assert np.isnan(lg[:, 5]).all() and np.isneginf(lg[:, 6]).all()
        assert from_dev(ids).tolist() == O.top_k(lg, 1).reshape(-1).astype(np.int64).tolist() == [1000] * m
        assert from_dev(keys).tolist() == [0] * m


def test_argmax_fused_nothing_finite():
    k = 256
    w = O.bf16_narrow(np.full((300, k), -np.inf, np.float32))
    x = np.ones((1, k), np.float32)
    logits, ids = R().linear_argmax(to_dev(x, torch), to_dev(w, torch))
    assert np.isneginf(from_dev(logits)).all() and from_dev(ids).tolist() == [300]
