"""Parity at the benchmarked shapes themselves: the C4 fp8-weight products
(Llama-3-8B-like, M in {1, 8, 64}) and the C2 bf16 projections at M = 2048,
each against the oracle's product on the same seeded inputs.

These are the exact kernel plans the benchmark times: the 4-wave gemv with its LDS
cross-wave sum (14336 -> 4096 at m = 1), the few-row MFMA kernel with 16 k splits and
the ordered finish (4096 -> 1024 at m = 8 and 64), and the 256x256 / 128x128 tile
kernels at M = 2048 (the lm_head checked on column slices of the full product).

Tolerance: f32 out per element within the analytic bound of
tests/helpers.product_bound (the reference's Terms::matmul with this unit's precision:
exact bf16/e4m3 operands, f32 accumulation); bf16 out additionally: max-rel <= 2e-2
and equal to the f32 output rounded to nearest even.
"""
import numpy as np
import pytest

import oracle as O
from tests.helpers import linear_bound, bf16_bits_normal, from_dev, max_rel, rng, to_dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _rules():
    from tessera_amd import rules
    return rules


def _bound(x, w):
    return linear_bound(x, w)


def _check(got, want, bound):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.all(err <= bound), f"max err {err.max()} vs bound at argmax {bound.reshape(-1)[err.argmax()]}"


@pytest.fixture(autouse=True)
def _oracle_threads():
    O.set_threads(O.lib().or_threads_available())
    yield
    O.set_threads(1)


def _quantize(r, n, k):
    """C4 weights: N(0,0.02) rows, scale = absmax/448 rounded to bf16, codes = e4m3(w/s)."""
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    s_bits = O.bf16_narrow((np.abs(w).max(1) / 448.0).astype(np.float32))
    codes = O.e4m3_narrow(w / O.bf16_widen(s_bits)[:, None])
    return codes, s_bits


# C4 shapes (K -> N): q/o 4096->4096, k/v 4096->1024, gate/up 4096->14336, down 14336->4096.
C4 = [("q_o", 4096, 4096), ("k_v", 4096, 1024), ("gate_up", 4096, 14336), ("down", 14336, 4096)]


@pytest.mark.parametrize("m", [1, 8, 64])
@pytest.mark.parametrize("name,k,n", C4)
def test_c4_e4m3_shapes(name, k, n, m):
    R = _rules()
    r = rng(1000 + k + n + m)
    codes, s_bits = _quantize(r, n, k)
    xb, xf = bf16_bits_normal(r, (m, k))
    want = O.product_e4m3w(xf, codes, s_bits)
    wdeq = O.e4m3_widen(codes) * O.bf16_widen(s_bits)[:, None]
    print(f"C4 {name} m={m} k={k} n={n}", flush=True)
    cd, sd = to_dev(codes, torch), to_dev(s_bits, torch)
    got = from_dev(R.linear(to_dev(xb, torch), cd, w_scale=sd))
    _check(got, want, _bound(xf, wdeq))
    got16 = from_dev(R.linear(to_dev(xb, torch), cd, w_scale=sd, out_dtype=torch.bfloat16))
    assert max_rel(got16, want) <= 2e-2


# C2 projection shapes (K x N) at M = 2048, the benchmark's prefill sweep.
C2 = [("q", 1024, 2048), ("kv", 1024, 2048), ("k", 1024, 1024), ("o", 2048, 1024), ("gate_up", 1024, 6144),
      ("down", 3072, 1024)]


@pytest.mark.parametrize("name,k,n", C2)
def test_c2_m2048_shapes(name, k, n):
    R = _rules()
    m = 2048
    r = rng(2000 + k + n)
    xb, xf = bf16_bits_normal(r, (m, k))
    wb, wf = bf16_bits_normal(r, (n, k))
    print(f"C2 {name} m={m} k={k} n={n}", flush=True)
    want = O.product_bf16w(xf, wb)
    xd, wd = to_dev(xb, torch), to_dev(wb, torch)
    got32 = from_dev(R.linear(xd, wd))
    _check(got32, want, _bound(xf, wf))
    got16 = from_dev(R.linear(xd, wd, out_dtype=torch.bfloat16))
    assert max_rel(got16, want) <= 2e-2
    assert np.array_equal(got16, O.bf16_widen(O.bf16_narrow(got32)))


def test_c2_m2048_lm_head_slices():
    """The full 2048 x 151936 x 1024 product with bf16 output (the benchmarked launch),
    checked on three column slices: the first tiles, a middle run and the ragged end
    (151936 = 593 * 256 + 128)."""
    R = _rules()
    m, k, n = 2048, 1024, 151936
    r = rng(2151)
    xb, xf = bf16_bits_normal(r, (m, k))
    wb = O.bf16_narrow(r.standard_normal((n, k)).astype(np.float32))
    print("C2 lm_head m=2048 k=1024 n=151936", flush=True)
    got = R.linear(to_dev(xb, torch), to_dev(wb, torch), out_dtype=torch.bfloat16)
    for lo, hi in [(0, 1024), (75000, 75700), (n - 900, n)]:
        want = O.product_bf16w(xf, np.ascontiguousarray(wb[lo:hi]))
        g = from_dev(got[:, lo:hi].contiguous())
        assert max_rel(g, want) <= 2e-2, (lo, hi)
        # bf16 of a sum within the f32 bound: one rounding on top of that bound.
        _check(g, want, _bound(xf, O.bf16_widen(wb[lo:hi])) + np.abs(want) * 2.0 ** -8)


def test_graph_lm_head_gemv():
    """The graph path's lm_head launch: one f32 row through the fused RmsNorm with the
    final norm's gain, against the 151936 x 1024 tied embedding (bf16), f32 logits."""
    R = _rules()
    r = rng(2152)
    k, n = 1024, 151936
    x = r.standard_normal((1, k)).astype(np.float32)
    g = (1.0 + 0.02 * r.standard_normal(k)).astype(np.float32)
    wb, wf = bf16_bits_normal(r, (n, k), 0.02)
    xn = O.rms_norm(x, g, 1e-6)
    want = O.product_bf16w(xn, wb)
    got = from_dev(R.linear(to_dev(x, torch), to_dev(wb, torch), gain=to_dev(g, torch), eps=1e-6))
    _check(got, want, 2 * _bound(xn, wf))
