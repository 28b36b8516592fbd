"""Block-form weights (q8_0, mxfp8, int4_g32) on the decode product, against the
oracle's restatement of Block::dot (engine/ir/mem/src/block.rs:202-219): bit-exact,
since every rounding step is the reference's (same f32 activations)."""
import numpy as np
import pytest

import oracle as O
from helpers import from_dev, rng, to_dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _case(form, m, n, k, seed, x_bf16=False):
    r = rng(seed)
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    wb = O.block_pack(form, w)
    x = r.standard_normal((m, k)).astype(np.float32)
    if x_bf16:
        xb = O.bf16_narrow(x)
        return O.bf16_widen(xb), xb, wb
    return x, x, wb


@pytest.mark.parametrize("form", ["q8_0", "mxfp8", "int4_g32", "q4_0"])
@pytest.mark.parametrize("m,n,k", [(1, 2048, 1024), (2, 300, 3072), (3, 37, 8192), (4, 1024, 128), (1, 151936, 1024)])
def test_block_product_bit_exact(form, m, n, k):
    from tessera_amd import rules as R
    xf, xd, wb = _case(form, m, n, k, n + k + m)
    want = O.block_product(form, xf, wb)
    got = from_dev(R.lanes(to_dev(xd, torch), torch.from_numpy(wb).cuda(), w_form=form))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("form", ["q8_0", "mxfp8", "int4_g32", "q4_0"])
def test_block_product_bf16_rows_add_and_bf16_out(form):
    from tessera_amd import rules as R
    m, n, k = 2, 1000, 2048
    xf, xd, wb = _case(form, m, n, k, 7, x_bf16=True)
    res = rng(8).standard_normal((m, n)).astype(np.float32)
    want = O.block_product(form, xf, wb)
    got = from_dev(R.linear(to_dev(xd, torch), torch.from_numpy(wb).cuda(), w_form=form, a0=to_dev(res, torch)))
    assert np.array_equal(got, want + res)
    got16 = from_dev(R.linear(to_dev(xd, torch), torch.from_numpy(wb).cuda(), w_form=form,
                              out_dtype=torch.bfloat16))
    assert np.array_equal(got16, O.bf16_widen(O.bf16_narrow(want)))


def test_block_form_refuses_matrix_rows():
    from tessera_amd import abi, rules as R
    xf, xd, wb = _case("q8_0", 8, 64, 256, 1)
    with pytest.raises(Exception, match="outside 1..4"):
        R.lanes(to_dev(xd, torch), torch.from_numpy(wb).cuda(), w_form="q8_0")
