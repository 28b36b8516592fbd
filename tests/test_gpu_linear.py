"""Parity of the linear kernels (lanes, tiled) with the oracle's product.

Tolerances (stated per test):
  * f32 out: per element within the analytic bound of tests/helpers.product_bound,
    the reference's Terms::matmul (engine/plan/codegen/src/numerics.rs:150-175,
    asserted by tiled_test.rs:104-114) with this unit's precision: exact weights,
    f32 rows as two bf16 parts (16 bits), bf16 rows exact, at most k / 32 + 16
    accumulator roundings (doubled) of 2^-21, and the bound below a tenth of the
    outputs.
  * bf16 out adds one bf16 rounding: max-rel <= 2e-2 (BASELINE tolerance).
"""
import numpy as np
import pytest

import oracle as O
from tests.helpers import linear_bound, bf16_bits_normal, from_dev, max_rel, rng, to_dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _bound(x, w):
    return linear_bound(x, w)


def _rules():
    from tessera_amd import rules
    return rules


def _check(got, want, bound):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.all(err <= bound), f"max err {err.max()} vs bound at argmax {bound.reshape(-1)[err.argmax()]}"


# tiles_match_cpu sizes (engine/rules/linear/tests/tiled_test.rs:58-71) plus decode rows.
SHAPES = [(1, 3, 4), (37, 50, 72), (64, 64, 64), (600, 40, 512), (256, 512, 1024),
          (1, 2048, 1024), (4, 1024, 3072), (16, 6144, 1024), (3, 100, 200)]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_linear_f32_rows_bf16_weights(m, n, k):
    R = _rules()
    r = rng(29 + m + n + k)
    x = r.standard_normal((m, k)).astype(np.float32)
    wb, wf = bf16_bits_normal(r, (n, k), 0.02)
    want = O.product_bf16w(x, wb)
    got = from_dev(R.linear(to_dev(x, torch), to_dev(wb, torch)))
    _check(got, want, _bound(x, wf))


@pytest.mark.parametrize("m", [1, 4, 16, 128])
@pytest.mark.parametrize("k,n", [(1024, 2048), (1024, 1024), (2048, 1024), (1024, 6144), (3072, 1024)])
def test_linear_bf16_sweep_shapes(m, k, n):
    """C2: N(0,1) bf16 x and w, f32 accumulate, bf16 and f32 out."""
    R = _rules()
    r = rng(m * 7 + k + n)
    xb, xf = bf16_bits_normal(r, (m, k))
    wb, wf = bf16_bits_normal(r, (n, k))
    want = O.product_bf16w(xf, wb)
    got = from_dev(R.linear(to_dev(xb, torch), to_dev(wb, torch)))
    _check(got, want, _bound(xf, wf))
    got16 = from_dev(R.linear(to_dev(xb, torch), to_dev(wb, torch), out_dtype=torch.bfloat16))
    assert max_rel(got16, want) <= 2e-2


@pytest.fixture(scope="module")
def lm_head_case():
    r = rng(2153)
    k, n = 1024, 151936
    wb = O.bf16_narrow(r.standard_normal((n, k)).astype(np.float32))
    return wb, to_dev(wb, torch)


@pytest.mark.parametrize("m", [1, 4, 16, 128])
def test_linear_bf16_sweep_lm_head(m, lm_head_case):
    """C2 lm_head 1024 x 151936 at the few-row sizes, bf16 x and w: the whole product
    launched as benchmarked, f32 and bf16 out, checked on column slices (first,
    middle, the ragged end) against the oracle."""
    R = _rules()
    wb, wd = lm_head_case
    n = wb.shape[0]
    r = rng(2154 + m)
    xb, xf = bf16_bits_normal(r, (m, 1024))
    xd = to_dev(xb, torch)
    got32 = R.linear(xd, wd)
    got16 = R.linear(xd, wd, out_dtype=torch.bfloat16)
    for lo, hi in [(0, 700), (75000, 75500), (n - 600, n)]:
        w = np.ascontiguousarray(wb[lo:hi])
        want = O.product_bf16w(xf, w)
        _check(from_dev(got32[:, lo:hi].contiguous()), want, _bound(xf, O.bf16_widen(w)))
        assert max_rel(from_dev(got16[:, lo:hi].contiguous()), want) <= 2e-2


@pytest.mark.parametrize("m,n,k", [(2048, 8192, 256), (2000, 7777, 192), (2000, 7777, 136), (1300, 12300, 64),
                                   (4096, 16384, 128), (2048, 20000, 1024)])
def test_tiled_256_tiles(m, n, k):
    """Products with enough 256x256 tiles take the big-tile kernel (bf16 x and w, k a
    multiple of 64): one tile per CU, ragged edges, several tiles per CU (4096 x 16384;
    2048 x 20000 mixes whole tiles with a ragged last column of tiles); k 136 takes
    the 128x128 kernel. Each product runs with an added operand, to f32 and to
    bf16."""
    R = _rules()
    O.set_threads(O.lib().or_threads_available())
    r = rng(m + n + k)
    xb, xf = bf16_bits_normal(r, (m, k))
    wb, wf = bf16_bits_normal(r, (n, k))
    want = O.product_bf16w(xf, wb)
    O.set_threads(1)
    res = r.standard_normal((m, n)).astype(np.float32)
    got = from_dev(R.linear(to_dev(xb, torch), to_dev(wb, torch), a0=to_dev(res, torch)))
    _check(got, want + res, _bound(xf, wf) + 1e-5)
    got32 = from_dev(R.linear(to_dev(xb, torch), to_dev(wb, torch)))
    _check(got32, want, _bound(xf, wf))
    got16 = from_dev(R.linear(to_dev(xb, torch), to_dev(wb, torch), out_dtype=torch.bfloat16))
    assert max_rel(got16, want) <= 2e-2
    # Same sums, one rounding: the bf16 output is the f32 output rounded to nearest
    # even, element for element (pins where each value lands in the bf16 epilogue).
    assert np.array_equal(got16, O.bf16_widen(O.bf16_narrow(got32)))


def test_lanes_and_tiled_agree_at_16_rows():
    R = _rules()
    r = rng(5)
    x = r.standard_normal((16, 512)).astype(np.float32)
    wb, wf = bf16_bits_normal(r, (300, 512), 0.05)
    a = from_dev(R.lanes(to_dev(x, torch), to_dev(wb, torch)))
    b = from_dev(R.tiled(to_dev(x, torch), to_dev(wb, torch)))
    _check(a, b, _bound(x, wf))


@pytest.mark.parametrize("m", [1, 5, 40, 100, 300])
def test_fused_stages(m):
    """RmsNorm before (lanes only), SiLU*up and the residual add after."""
    R = _rules()
    r = rng(11 + m)
    k, n = 256, 96
    x = r.standard_normal((m, k)).astype(np.float32)
    g = (1.0 + 0.02 * r.standard_normal(k)).astype(np.float32)
    wb, wf = bf16_bits_normal(r, (2 * n, k), 0.05)
    res = r.standard_normal((m, n)).astype(np.float32)
    # silu(gate) * up, then + residual (engine/models/src/shared.rs:375-378; map.rs:93-96)
    gu = O.product_bf16w(x, wb)
    want = O.act("silu", gu[:, :n]) * gu[:, n:] + res
    got = from_dev(R.linear(to_dev(x, torch), to_dev(wb, torch), silu_mul=True, a0=to_dev(res, torch)))
    # First-order error of silu(g)*u: |silu'| <= 1.1, |silu(g)| <= |g|.
    b = _bound(x, wf)
    _check(got, want, 1.1 * b[:, :n] * np.abs(gu[:, n:]) + np.abs(gu[:, :n]) * b[:, n:] + 1e-5)
    if m <= 16:
        xn = O.rms_norm(x, g, 1e-6)
        want2 = O.product_bf16w(xn, wb[:n])
        got2 = from_dev(R.linear(to_dev(x, torch), to_dev(wb[:n], torch), gain=to_dev(g, torch), eps=1e-6))
        _check(got2, want2, 2 * _bound(xn, wf[:n]))


def test_residual_in_place():
    R = _rules()
    r = rng(3)
    x = r.standard_normal((1, 1024)).astype(np.float32)
    wb, wf = bf16_bits_normal(r, (1024, 1024), 0.02)
    h = r.standard_normal((1, 1024)).astype(np.float32)
    hd = to_dev(h, torch)
    R.linear(to_dev(x, torch), to_dev(wb, torch), a0=hd, out=hd)
    _check(from_dev(hd), O.product_bf16w(x, wb) + h, _bound(x, wf) + 1e-6)


def _quantize(r, n, k):
    """C4 weights: N(0,0.02) rows, scale = absmax/448 as bf16, codes = e4m3(w/s)."""
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    s_bits = O.bf16_narrow((np.abs(w).max(1) / 448.0).astype(np.float32))
    s = O.bf16_widen(s_bits)
    codes = O.e4m3_narrow(w / s[:, None])
    return codes, s_bits


@pytest.mark.parametrize("m", [1, 8, 64])
def test_e4m3_weights(m):
    R = _rules()
    r = rng(40 + m)
    k, n = 1024, 512
    codes, s_bits = _quantize(r, n, k)
    xb, xf = bf16_bits_normal(r, (m, k))
    want = O.product_e4m3w(xf, codes, s_bits)
    wdeq = O.e4m3_widen(codes) * O.bf16_widen(s_bits)[:, None]
    got = from_dev(R.linear(to_dev(xb, torch), to_dev(codes, torch), w_scale=to_dev(s_bits, torch)))
    _check(got, want, _bound(xf, wdeq))


def test_argument_errors_raise():
    R = _rules()
    from tessera_amd import abi
    x = torch.zeros((65, 64), device="cuda")
    w = torch.zeros((8, 64), device="cuda", dtype=torch.bfloat16)
    with pytest.raises(abi.HipError) as e:
        R.lanes(x, w)
    assert e.value.code == abi.TS_ERR_ARG and "m=65" in str(e.value)


@pytest.mark.parametrize("m", [1, 8, 80])
def test_e4m3_decode_every_code(m):
    """Every e4m3 code through the product paths (vector ALU m=1, few-row MFMA m=8,
    tiled m=80): row n holds code n everywhere, scale 1.0, x = one-hot at k=0, so
    out[:, n] is the decoded code itself; bit-exact against the oracle's e4m3 widen
    (scalar.rs), NaN for 0x7f/0xff (-0 compares equal to the +0 a sum from 0 gives)."""
    R = _rules()
    k = 64
    codes = np.repeat(np.arange(256, dtype=np.uint8)[:, None], k, axis=1)
    scale = O.bf16_narrow(np.ones(256, np.float32))
    x = np.zeros((m, k), np.float32)
    x[:, 0] = 1.0
    got = from_dev(R.linear(to_dev(x, torch), to_dev(codes, torch), w_scale=to_dev(scale, torch)))
    want = O.e4m3_widen(np.arange(256, dtype=np.uint8))
    for row in got:
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(row), nan)
        assert np.array_equal(row[~nan], want[~nan].astype(np.float32))


def test_silu_pair_big_tiles():
    """SiLU pair + residual on the 128x128 tiled kernel (enough tiles: 2048 x 4096)."""
    R = _rules()
    O.set_threads(O.lib().or_threads_available())
    r = rng(21)
    m, k, n = 2048, 64, 4096
    x = r.standard_normal((m, k)).astype(np.float32)
    wb, wf = bf16_bits_normal(r, (2 * n, k), 0.05)
    res = r.standard_normal((m, n)).astype(np.float32)
    gu = O.product_bf16w(x, wb)
    O.set_threads(1)
    want = O.act("silu", gu[:, :n]) * gu[:, n:] + res
    got = from_dev(R.linear(to_dev(x, torch), to_dev(wb, torch), silu_mul=True, a0=to_dev(res, torch)))
    b = _bound(x, wf)
    _check(got, want, 1.1 * b[:, :n] * np.abs(gu[:, n:]) + np.abs(gu[:, :n]) * b[:, n:] + 1e-5)


def test_bf16_output_rounding_matches_oracle():
    """The device's f32 -> bf16 rounding (every bf16 store) is the reference's RNE
    (scalar.rs): out = x * 1.0 through a 4-row product with bf16 output, over random
    values of every exponent, exact ties, denormals, values next to overflow, +-inf,
    NaN and +-0; bit-exact (NaN compared as NaN; -0 becomes +0 because the product's
    sum starts at +0, as the reference's Acc does)."""
    R = _rules()
    r = rng(123)
    bits = r.integers(0, 2 ** 32, 4000, dtype=np.uint64).astype(np.uint32)
    ties = (r.integers(0, 2 ** 16, 200, dtype=np.uint64).astype(np.uint32) << 16) | 0x8000
    special = np.array([0x00000001, 0x00008000, 0x0000ffff, 0x007fffff, 0x00800000, 0x7f7f8000, 0x7f7fffff,
                        0x7f800000, 0xff800000, 0x7fc00001, 0xffa00000, 0x80000000, 0x00000000, 0x3f808000,
                        0x3f818000], np.uint32)
    vals = np.concatenate([bits, ties, special]).view(np.float32)
    vals = np.concatenate([vals, np.zeros((-len(vals)) % 4, np.float32)])
    w = np.zeros((1, 8), np.uint16)
    w[0, 0] = O.bf16_narrow(np.array([1.0], np.float32))[0]
    wd = to_dev(w, torch)
    got = []
    for i in range(0, len(vals), 4):
        x = np.zeros((4, 8), np.float32)
        x[:, 0] = vals[i:i + 4]
        out = R.linear(to_dev(x, torch), wd, out_dtype=torch.bfloat16)
        got.append(out.view(torch.int16).cpu().numpy().view(np.uint16)[:, 0])
    got = np.concatenate(got)
    want = O.bf16_narrow(vals)
    want[vals == 0] = 0  # +0 + (-0 * 1) = +0
    nan = np.isnan(vals)
    bad = np.nonzero((got != want) & ~nan)[0]
    assert bad.size == 0, "x bits / got / want: " + ", ".join(
        f"{vals[i:i + 1].view(np.uint32)[0]:08x}/{got[i]:04x}/{want[i]:04x}" for i in bad[:12]) + f" ({bad.size} differ)"
    assert np.all((got[nan] & 0x7fff) > 0x7f80)


@pytest.mark.parametrize("m,n,k", SHAPES + [(128, 1024, 1024), (2048, 1024, 256)])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_linear_f32_weights(m, n, k, xdt):
    """f32 weights (tiles_match_cpu iterates every float form, engine/rules/linear/tests/
    common/mod.rs:67-75): packed once into two bf16 parts (tessera_hip_pack_f32, checked
    bit for bit here), then the product of every kernel family against the oracle's
    f32 product, within the analytic bound with ew = |w| 2^-16 and four part products
    per output."""
    R = _rules()
    r = rng(300 + m + n + k)
    w = (r.standard_normal((n, k)) * 0.05).astype(np.float32)
    wd = to_dev(w, torch)
    packed = R.pack_f32(wd)
    hi = O.bf16_narrow(w)
    lo = O.bf16_narrow(w - O.bf16_widen(hi))
    assert np.array_equal(packed.view(torch.int16).cpu().numpy().view(np.uint16), np.concatenate([hi, lo]))
    if xdt == "f32":
        x = r.standard_normal((m, k)).astype(np.float32)
        xd = to_dev(x, torch)
    else:
        xb, x = bf16_bits_normal(r, (m, k))
        xd = to_dev(xb, torch)
    if m * n * k > 1 << 28:
        O.set_threads(O.lib().or_threads_available())
    want = O.product(x, w)
    O.set_threads(1)
    got = from_dev(R.linear(xd, packed, w_form="f32_parts"))
    from tests.helpers import product_bound
    bound = product_bound(x, w, x_bits=16 if xdt == "f32" else None, parts=4, w_bits=16, lane=9)
    _check(got, want, bound)
