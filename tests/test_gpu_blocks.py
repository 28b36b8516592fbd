"""Block-form weights (the seven forms of engine/ir/mem/src/block.rs:251-291).

  * m <= 4 (the decode product): bit-exact against the oracle's restatement of
    Block::dot (block.rs:202-217), since every rounding step is the reference's (same
    f32 activations).
  * m > 4 (the matrix unit): against the CPU product over the form's decoded weights
    (tiled_test.rs:58-121: the reference compares with the interpreter run on the
    round-tripped weights), within the analytic bound of tests/helpers.product_bound
    with the block path's extra roundings (one scale multiply and one add per block,
    the head): lane = 2 k / B + 8.
"""
import numpy as np
import pytest

import oracle as O
from helpers import assert_within, from_dev, product_bound, rng, to_dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

FORMS = list(O.BLOCK_FORMS)


def _case(form, m, n, k, seed, x_bf16=False):
    r = rng(seed)
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    wb = O.block_pack(form, w)
    x = r.standard_normal((m, k)).astype(np.float32)
    if x_bf16:
        xb = O.bf16_narrow(x)
        return O.bf16_widen(xb), xb, wb
    return x, x, wb


def _dev(wb):
    return torch.from_numpy(wb).cuda()


@pytest.mark.parametrize("form", FORMS)
@pytest.mark.parametrize("m,n,k", [(1, 2048, 1024), (2, 300, 3072), (2, 100, 1024), (1, 37, 4096), (3, 37, 8192), (3, 37, 1024), (4, 1024, 512),
                                   (1, 151936, 1024)])
def test_block_product_bit_exact(form, m, n, k):
    from tessera_amd import rules as R
    print(f"block gemv {form} m={m} n={n} k={k}", flush=True)
    xf, xd, wb = _case(form, m, n, k, n + k + m)
    want = O.block_product(form, xf, wb, n)
    got = from_dev(R.lanes(to_dev(xd, torch), _dev(wb), w_form=form, rows=n))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("form", FORMS)
def test_block_product_bf16_rows_add_and_bf16_out(form):
    from tessera_amd import rules as R
    m, n, k = 2, 1000, 2048
    xf, xd, wb = _case(form, m, n, k, 7, x_bf16=True)
    res = rng(8).standard_normal((m, n)).astype(np.float32)
    want = O.block_product(form, xf, wb, n)
    got = from_dev(R.linear(to_dev(xd, torch), _dev(wb), w_form=form, rows=n, a0=to_dev(res, torch)))
    assert np.array_equal(got, want + res)
    got16 = from_dev(R.linear(to_dev(xd, torch), _dev(wb), w_form=form, rows=n, out_dtype=torch.bfloat16))
    assert np.array_equal(got16, O.bf16_widen(O.bf16_narrow(want)))


@pytest.mark.parametrize("k", [1024, 8192])
def test_block_product_e4m3_nan_codes(k):
    """e4m3 0x7F / 0xFF are NaN (e4m3fn; the interpreter's widening): a hand-placed
    NaN code (mxfp8) or block scale (nvfp4) makes exactly its row NaN, as in the
    oracle, on the short-row (k 1024) and the long-row (k 8192) forms."""
    from tessera_amd import rules as R
    n, m = 40, 2
    for form, bb, head, at in (("mxfp8", 33, 0, 1 + 5), ("nvfp4", 9, 4, 0)):
        xf, xd, wb = _case(form, m, n, k, 11)
        wb = wb.copy()
        nb = k // O.block_size(form)
        for row, blk, code in ((3, 2, 0x7F), (17, nb - 1, 0xFF)):
            wb[head + (row * nb + blk) * bb + at] = code
        want = O.block_product(form, xf, wb, n)
        assert np.isnan(want[:, 3]).all() and np.isnan(want[:, 17]).all()
        got = from_dev(R.lanes(to_dev(xd, torch), _dev(wb), w_form=form, rows=n))
        np.testing.assert_array_equal(got, want)


def _lane(form, k):
    return 2 * k / O.block_size(form) + 8


# tiles_match_cpu sizes that fit the forms' k alignment, and wider ones.
MAT = [(5, 96, 512), (37, 50, 1024), (64, 64, 512), (300, 200, 1024), (256, 512, 2048)]


@pytest.mark.parametrize("form", FORMS)
@pytest.mark.parametrize("m,n,k", MAT)
def test_block_matrix_rows(form, m, n, k):
    """tiled with block weights, f32 rows (two bf16 parts) and bf16 rows."""
    from tessera_amd import rules as R
    print(f"block tiled {form} m={m} n={n} k={k}", flush=True)
    xf, _, wb = _case(form, m, n, k, 3 * m + n + k)
    wdec = O.block_unpack(form, wb, n * k).reshape(n, k)
    want = O.product(xf, wdec)
    got = from_dev(R.tiled(to_dev(xf, torch), _dev(wb), w_form=form, rows=n))
    assert_within(got, want, product_bound(xf, wdec, x_bits=16, parts=2, lane=_lane(form, k)))
    xb = O.bf16_narrow(xf)
    xw = O.bf16_widen(xb)
    want_b = O.product(xw, wdec)
    got_b = from_dev(R.linear(to_dev(xb, torch), _dev(wb), w_form=form, rows=n))
    assert_within(got_b, want_b, product_bound(xw, wdec, lane=_lane(form, k)))


@pytest.mark.parametrize("form", ["q8_0", "nvfp4", "int4_g128"])
def test_block_matrix_silu_pair_add_and_bf16_out(form):
    """The fused stages with block weights (m = 70: the matrix unit): silu(gate) * up
    over 2n rows, and on the plain product bf16 output (one more rounding: 2^-8 of the
    value) and the residual add."""
    from tessera_amd import rules as R
    m, n, k = 70, 96, 1024
    r = rng(11)
    w = (r.standard_normal((2 * n, k)) * 0.05).astype(np.float32)
    wb = O.block_pack(form, w)
    wdec = O.block_unpack(form, wb, 2 * n * k).reshape(2 * n, k)
    xb = O.bf16_narrow(r.standard_normal((m, k)).astype(np.float32))
    x = O.bf16_widen(xb)
    g, u = O.product(x, wdec[:n]), O.product(x, wdec[n:])
    want = g / (1.0 + np.exp(-g.astype(np.float64))) * u
    got = from_dev(R.linear(to_dev(xb, torch), _dev(wb), w_form=form, rows=2 * n, silu_mul=True))
    bg = product_bound(x, wdec[:n], lane=_lane(form, k))
    bu = product_bound(x, wdec[n:], lane=_lane(form, k))
    # silu(g) u moves by at most |d silu/dg| |u| bg + |silu(g)| bu, |d silu/dg| <= 1.1
    sg = np.abs(g / (1.0 + np.exp(-g.astype(np.float64))))
    assert_within(got, want, 1.1 * np.abs(u) * bg + sg * bu + 1e-6 * np.abs(want))
    res = r.standard_normal((m, 2 * n)).astype(np.float32)
    got16 = from_dev(R.linear(to_dev(xb, torch), _dev(wb), w_form=form, rows=2 * n, out_dtype=torch.bfloat16))
    full = O.product(x, wdec)
    assert_within(got16, full, product_bound(x, wdec, lane=_lane(form, k)) + np.abs(full) * 2.0 ** -8)
    got_add = from_dev(R.linear(to_dev(xb, torch), _dev(wb), w_form=form, rows=2 * n, a0=to_dev(res, torch)))
    assert_within(got_add, full + res, product_bound(x, wdec, lane=_lane(form, k) + 1) + np.abs(res) * 2.0 ** -24)


def test_block_form_k_alignment_refused():
    from tessera_amd import rules as R
    xf, xd, wb = _case("int4_g128", 8, 64, 256, 1)
    with pytest.raises(Exception, match="multiple of 512"):
        R.linear(to_dev(xd, torch), _dev(wb), w_form="int4_g128", rows=64)
