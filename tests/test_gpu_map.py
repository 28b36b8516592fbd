"""Stage chains (the reference's MapStage / Map / Finished, engine/plan/lower/src/
kernels/map.rs:40-185): the standalone map and chains fused into every product kernel,
against the oracle's chain (oracle.chain: interp's Stage::Add / Mul / Scale / Act,
engine/ir/interp/src/cpu.rs:8-29,353-390).

Tolerances (stated per test):
  * activations and map chains: within 4 units in the last place of the oracle's
    value per stage (the device's expf / tanhf / log1pf against glibc's; the other
    operations are the same single f32 roundings), NaN where the oracle gives NaN;
  * chains fused into a product: the product's analytic bound (tests/helpers.
    product_bound) carried through the chain — Add keeps it, Mul and Scale multiply it
    by |operand|, an activation by its largest slope over the interval — plus 4 units
    in the last place per stage.
"""
import numpy as np
import pytest

import oracle as O
from tests.helpers import bf16_bits_normal, from_dev, linear_bound, product_bound, rng, to_dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

ACTS = ["gelu_tanh", "silu", "sigmoid", "relu", "softplus", "exp", "tanh"]
ULP = 2.0 ** -23


def _rules():
    from tessera_amd import rules
    return rules


def ulps_close(got, want, per=4, scale=None):
    """|got - want| <= per ulps of `scale` (default |want|: the largest value the
    computation passes through; NaN where want is NaN; inf equal)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = np.abs(want) if scale is None else np.maximum(np.abs(want), np.abs(np.asarray(scale, np.float64)))
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan), "NaN where the oracle has none (or the reverse)"
    inf = np.isinf(want)
    assert np.array_equal(got[inf], want[inf])
    ok = ~nan & ~inf
    tol = per * ULP * np.maximum(scale[ok], 2.0 ** -126)
    err = np.abs(got[ok] - want[ok])
    bad = np.nonzero(err > tol)[0]
    assert bad.size == 0, f"{bad.size} values off, e.g. got {got[ok][bad[0]]:.9e} want {want[ok][bad[0]]:.9e}"


def stage_scale(x, stages, ops=(), sum_at=0, spans=None):
    """The largest |value| each element passes through in the chain (its input and
    every stage's result): an f32 step loses at most a few ulps of that."""
    big = np.abs(np.asarray(x, np.float64))
    for i in range(1, len(stages) + 1):
        v = O.chain(x, stages[:i], ops, sum_at, spans)
        big = np.maximum(big, np.nan_to_num(np.abs(v.astype(np.float64)), posinf=0))
    return big


def test_act_values_known_answers():
    """cpu_test.rs:173-196 act_values through the device map, one activation a stage."""
    R = _rules()
    x = torch.tensor([-2.0, 0.0, 1.0, 3.0], device="cuda")
    want = {
        "relu": [0, 0, 1, 3],
        "sigmoid": [0.11920292, 0.5, 0.7310586, 0.9525741],
        "silu": [-0.23840584, 0, 0.7310586, 2.8577224],
        "gelu_tanh": [-0.0454023, 0, 0.841192, 2.9963626],
        "softplus": [0.126928, float(np.log(2)), 1.3132617, 3.0485874],
        "exp": [0.13533528, 1, float(np.e), 20.085537],
        "tanh": [-0.9640276, 0, 0.7615942, 0.995055],
    }
    for a, w in want.items():
        got = from_dev(R.map(x, [a]))
        np.testing.assert_allclose(got, np.array(w, np.float32), rtol=1e-6, atol=1e-7, err_msg=a)


@pytest.mark.parametrize("act", ACTS)
def test_each_activation_against_the_oracle(act):
    """A dense grid over [-30, 30], tiny and huge magnitudes, +-0, +-inf and NaN."""
    R = _rules()
    r = rng(ACTS.index(act))
    x = np.concatenate([np.linspace(-30, 30, 60001, dtype=np.float32), r.standard_normal(4000).astype(np.float32),
                        np.array([0.0, -0.0, 1e-30, -1e-30, 1e-8, -1e-8, 88.0, -88.0, 100.0, -100.0, 1e30, -1e30,
                                  np.inf, -np.inf, np.nan], np.float32)])
    got = from_dev(R.map(to_dev(x, torch), [act]))
    # gelu's 1 + tanh(.) cancels for negative x: its error is an ulp of 0.5 |x|
    ulps_close(got, O.act(act, x), scale=np.abs(x) if act == "gelu_tanh" else None)


CHAINS = [
    (["add"], 1, 0, None),
    (["mul", "silu"], 1, 0, None),
    ([("scale", 0.0883883476), "add", "tanh"], 1, 0, None),
    (["add", "mul", "gelu_tanh"], 2, 1, None),           # the input enters second
    (["mul", "add", "softplus", ("scale", -1.5)], 2, 2, None),  # the input enters last
    (["add", "sigmoid", "mul", "exp", "relu"], 2, 0, [7, 1]),   # a repeating row and a scalar
    ([], 0, 0, None),                                     # a copy
]


@pytest.mark.parametrize("stages,nops,sum_at,spans", CHAINS)
def test_map_chains(stages, nops, sum_at, spans):
    R = _rules()
    r = rng(len(stages) * 10 + nops)
    n = 5003  # not a multiple of 4: the scalar tail
    x = r.standard_normal(n).astype(np.float32)
    ops = [r.standard_normal(n if not spans else max(spans[j], 1)).astype(np.float32) for j in range(nops)]
    got = from_dev(R.map(to_dev(x, torch), stages, [to_dev(o, torch) for o in ops], sum_at=sum_at, spans=spans))
    want = O.chain(x, stages, ops, sum_at, spans)
    ulps_close(got, want, per=4 * max(len(stages), 1), scale=stage_scale(x, stages, ops, sum_at, spans))


def test_map_in_place_and_q_prescale():
    """out aliasing x, and the q pre-scale the reference emits before flash
    (Map Scale(1/sqrt(d)), engine/rules/attention/src/lib.rs:22-31): one rounding."""
    R = _rules()
    q = rng(3).standard_normal((7, 16, 128)).astype(np.float32)
    d = to_dev(q, torch)
    s = np.float32(1 / np.sqrt(128))
    R.map(d, [("scale", float(s))], out=d)
    assert np.array_equal(from_dev(d), q * s)


def _act_slope(act, lo, hi):
    """Largest |act'| over [lo, hi] (elementwise), generously: global bounds, exp local."""
    return {"gelu_tanh": 1.13, "silu": 1.1, "sigmoid": 0.25, "relu": 1.0, "softplus": 1.0, "tanh": 1.0}.get(act) \
        if act != "exp" else np.exp(np.maximum(lo, hi))


def chain_bound(total, bound, stages, operands, sum_at):
    """The product's error bound carried through the chain (first order, generous), plus
    4 ulps of each stage's value."""
    flat = np.asarray(total, np.float64).reshape(-1)
    e = np.asarray(bound, np.float64).reshape(-1)
    ops = [np.asarray(o, np.float64).reshape(-1) for o in operands]

    def read(i):
        return (flat, True) if i == sum_at else (ops[i if i < sum_at else i - 1], False)

    v, is_sum = read(0)
    v = v.copy()
    err = e.copy() if is_sum else np.zeros_like(flat)
    nxt = 1
    for st in stages:
        if st in ("add", "mul"):
            x, xs = read(nxt)
            nxt += 1
            if st == "add":
                err = err + (e if xs else 0)
                v = v + x
            else:
                err = err * np.abs(x) + (np.abs(v) * e if xs else 0) + (err * e if xs else 0)
                v = v * x
        elif isinstance(st, tuple):
            err = err * abs(st[1])
            v = v * st[1]
        else:
            err = err * _act_slope(st, v - err, v + err)
            v_in = np.abs(v)
            v = O.act(st, v.astype(np.float32)).astype(np.float64)
            err = err + 4 * ULP * v_in  # an activation's steps: ulps of its input (gelu cancels)
        err = err + 4 * ULP * np.abs(v) + 1e-30
    return err.reshape(np.shape(total))


def _check_fused(got, sums, bound, stages, ops, sum_at):
    want = O.chain(sums, stages, ops, sum_at)
    b = chain_bound(sums, bound, stages, ops, sum_at)
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= b), f"max err {err.max():.3e}, bound there {b.reshape(-1)[err.argmax()]:.3e}"


FUSED = [(["add", "silu"], 1, 0), (["mul", ("scale", 0.5), "gelu_tanh"], 1, 0), (["add", "mul", "tanh"], 2, 1)]


@pytest.mark.parametrize("m,n,k,xdt", [
    (1, 300, 256, "f32"),      # the vector-ALU few-row kernel
    (4, 1024, 512, "bf16"),
    (8, 96, 256, "f32"),       # few rows on the matrix unit, one split
    (40, 200, 4096, "bf16"),   # k split across groups: the ordered finish runs the chain
    (64, 64, 1024, "f32"),
    (300, 136, 192, "f32"),    # register-staged tiles (f32 rows)
    (600, 1024, 256, "bf16"),  # pipelined tiles
    (2048, 8192, 256, "bf16"),  # a shape the 256x256 kernel would take without a chain
])
@pytest.mark.parametrize("chain_i", range(len(FUSED)))
def test_chain_fused_into_products(m, n, k, xdt, chain_i):
    R = _rules()
    stages, nops, sum_at = FUSED[chain_i]
    r = rng(m + n + k + chain_i)
    if xdt == "f32":
        x = r.standard_normal((m, k)).astype(np.float32)
        xd = to_dev(x, torch)
    else:
        xb, x = bf16_bits_normal(r, (m, k))
        xd = to_dev(xb, torch)
    wb, wf = bf16_bits_normal(r, (n, k), 0.05)
    ops = [r.standard_normal((m, n)).astype(np.float32) for _ in range(nops)]
    if m > 256:
        O.set_threads(O.lib().or_threads_available())
    sums = O.product_bf16w(x, wb)
    O.set_threads(1)
    bound = linear_bound(x, wf)
    c = R.chain(stages, [to_dev(o, torch) for o in ops], sum_at=sum_at)
    got = from_dev(R.linear(xd, to_dev(wb, torch), after=c))
    _check_fused(got, sums, bound, stages, ops, sum_at)
    if m in (4, 600):  # bf16 out: the chain runs before the rounding
        got16 = from_dev(R.linear(xd, to_dev(wb, torch), after=c, out_dtype=torch.bfloat16))
        want = O.chain(sums, stages, ops, sum_at)
        assert np.array_equal(got16, O.bf16_widen(O.bf16_narrow(got.astype(np.float32)))) or \
            np.max(np.abs(got16 - want)) <= np.max(np.abs(want)) * 2e-2


@pytest.mark.parametrize("m", [1, 8, 100])
def test_chain_with_silu_pair_and_e4m3(m):
    """The chain runs on silu(gate) * up, and on e4m3 products after the row scale."""
    R = _rules()
    r = rng(70 + m)
    k, n = 256, 64
    x = r.standard_normal((m, k)).astype(np.float32)
    wb, wf = bf16_bits_normal(r, (2 * n, k), 0.05)
    op = r.standard_normal((m, n)).astype(np.float32)
    stages = ["mul", ("scale", 2.0)]
    c = R.chain(stages, [to_dev(op, torch)])
    got = from_dev(R.linear(to_dev(x, torch), to_dev(wb, torch), silu_mul=True, after=c))
    gu = O.product_bf16w(x, wb)
    inner = O.act("silu", gu[:, :n]) * gu[:, n:]
    b = linear_bound(x, wf)
    ib = 1.1 * b[:, :n] * np.abs(gu[:, n:]) + np.abs(gu[:, :n]) * b[:, n:] + 1e-6
    _check_fused(got, inner, ib, stages, [op], 0)
    # e4m3 weights with a per-row scale
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    s_bits = O.bf16_narrow((np.abs(w).max(1) / 448.0).astype(np.float32))
    codes = O.e4m3_narrow(w / O.bf16_widen(s_bits)[:, None])
    wdeq = O.e4m3_widen(codes) * O.bf16_widen(s_bits)[:, None]
    stages = ["relu", "add"]
    c = R.chain(stages, [to_dev(op, torch)])
    got = from_dev(R.linear(to_dev(x, torch), to_dev(codes, torch), w_scale=to_dev(s_bits, torch), after=c))
    _check_fused(got, O.product_e4m3w(x, codes, s_bits), linear_bound(x, wdeq), stages, [op], 0)


@pytest.mark.parametrize("m", [1, 8])
def test_chain_on_block_forms(m):
    """Block-form weights (q8_0): the decode product (m <= 4, bit-exact sums) and the
    matrix-unit form, each with a chain."""
    R = _rules()
    r = rng(90 + m)
    k, n = 256, 96
    x = r.standard_normal((m, k)).astype(np.float32)
    w = (r.standard_normal((n, k)) * 0.05).astype(np.float32)
    packed = O.block_pack("q8_0", w)
    op = r.standard_normal((m, n)).astype(np.float32)
    stages = ["add", "sigmoid"]
    c = R.chain(stages, [to_dev(op, torch)])
    got = from_dev(R.linear(to_dev(x, torch), torch.from_numpy(packed).cuda(), w_form="q8_0", rows=n, after=c))
    if m <= 4:  # Block::dot's sums, bit for bit
        sums, bound = O.block_product("q8_0", x, packed, n), 0.0
    else:
        wdeq = O.block_unpack("q8_0", packed, n * k).reshape(n, k)
        sums = O.product(x, wdeq)
        bound = product_bound(x, wdeq, x_bits=16, parts=2, lane=2 * k / 32 + 8)
    _check_fused(got, sums, np.broadcast_to(bound, sums.shape), stages, [op], 0)


def test_chain_on_picked_rows():
    """Picked products (MoE experts) with a chain; rows whose id is outside the set
    store the chain of a zero sum."""
    R = _rules()
    r = rng(5)
    count, k, n, rows = 6, 128, 64, 300
    tb, tf = bf16_bits_normal(r, (count, n, k), 0.05)
    xb, x = bf16_bits_normal(r, (rows, k))
    ids = r.integers(0, count + 2, size=rows).astype(np.uint32)
    op = r.standard_normal((rows, n)).astype(np.float32)
    stages = ["add", "softplus"]
    c = R.chain(stages, [to_dev(op, torch)])
    got = from_dev(R.picked(to_dev(xb, torch), to_dev(tb, torch), to_dev(ids.astype(np.int32), torch), after=c))
    sums = O.product_picked_bf16w(x, tb, ids, 0)
    bound = np.zeros_like(sums)
    for i in range(rows):
        if ids[i] < count:
            bound[i] = linear_bound(x[i:i + 1], tf[ids[i]])[0]
    _check_fused(got, sums, bound, stages, [op], 0)


def test_chain_refusals():
    R = _rules()
    from tessera_amd import abi
    x = torch.zeros((4, 64), device="cuda")
    w = torch.zeros((8, 64), device="cuda", dtype=torch.bfloat16)
    a0 = torch.zeros((4, 8), device="cuda")
    with pytest.raises(abi.HipError, match="replaces TS_AFTER_ADD"):
        R.linear(x, w, a0=a0, after=R.chain(["add"], [a0]))
    with pytest.raises(abi.HipError, match="repeats"):
        R.linear(x, w, after=R.chain(["add"], [a0], spans=[8]))
