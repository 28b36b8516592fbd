"""Pins the oracle (the C restatement of tessera-interp) before anything trusts it.

Each test transcribes a known answer from the reference's own tests (cited), a closed
form, or a brute force chosen so a plausible slip (dropped term, wrong sign or index,
transposed operand) fails it.
"""
import math

import numpy as np
import pytest

import oracle as O


def close(got, want, tol=1e-5):
    got = np.asarray(got, np.float32).reshape(-1)
    want = np.asarray(want, np.float32).reshape(-1)
    assert got.shape == want.shape
    bound = tol * np.maximum(np.abs(want), 1.0)
    assert np.all(np.abs(got - want) <= bound), (got, want)


# --- narrow floats: engine/ir/graph/src/scalar.rs ------------------------------

def test_bf16_all_codes_round_trip():
    codes = np.arange(1 << 16, dtype=np.uint16)
    f = O.bf16_widen(codes)
    exact = np.array([O.lib().or_bf16_widen_exact(int(c)) for c in codes[::97]], np.float32)
    ok = ~np.isnan(f[::97])
    assert np.array_equal(f[::97][ok], exact[ok]) and np.all(np.isnan(exact[~ok]))
    back = O.bf16_narrow(f)
    nan = np.isnan(f)
    assert np.array_equal(back[~nan], codes[~nan])
    # The bit pattern is the top half of the f32 for every non-NaN code.
    assert np.array_equal(f[~nan].view(np.uint32) >> 16, codes[~nan].astype(np.uint32))


def test_bf16_rne_ties_and_overflow():
    one = np.float32(1.0)
    ulp = np.float32(2.0 ** -7)
    # Halfway between 1 and 1+ulp rounds to even (1); halfway above 1+ulp rounds up.
    assert O.bf16_widen(O.bf16_narrow(one + ulp / 2)) == one
    assert O.bf16_widen(O.bf16_narrow(one + ulp + ulp / 2)) == one + 2 * ulp
    assert O.bf16_widen(O.bf16_narrow(one + ulp / 2 + ulp / 64)) == one + ulp
    # Past the largest finite bf16 rounds to inf; NaN stays NaN (quiet code 0x7FC0).
    big = np.float32(3.4028235e38)
    assert O.bf16_narrow(big) == 0x7F80
    assert O.bf16_narrow(np.float32("nan")) == 0x7FC0
    assert O.bf16_narrow(-0.0) == 0x8000
    # The smallest subnormal and its half (ties to zero, even).
    sub = np.float32(2.0 ** -133)
    assert O.bf16_narrow(sub) == 1 and O.bf16_narrow(sub / 2) == 0
    assert O.bf16_narrow(sub * 1.5) == 2  # 1.5 ties to even 2


def test_e4m3_codes_and_saturation():
    codes = np.arange(256, dtype=np.uint8)
    f = O.e4m3_widen(codes)
    nan = np.isnan(f)
    assert list(codes[nan]) == [0x7F, 0xFF]
    assert np.array_equal(O.e4m3_narrow(f[~nan]), codes[~nan])
    assert f[0x7E] == 448.0 and f[0x08] == 2.0 ** -6 and f[0x01] == 2.0 ** -9
    # Saturation: anything past 448 (including inf) narrows to the top code.
    for x in (449.0, 500.0, 1e9, float("inf")):
        assert O.e4m3_narrow(np.float32(x)) == 0x7E
        assert O.e4m3_narrow(np.float32(-x)) == 0xFE
    assert O.e4m3_narrow(np.float32("nan")) == 0x7F
    # RNE: 464 lies halfway between 448 (mantissa 110) and 480 (past the top): even, 448.
    assert O.e4m3_narrow(np.float32(464.0)) == 0x7E
    # 1.0625 is halfway between 1 and 1.125: ties to even 1.0.
    assert O.e4m3_widen(O.e4m3_narrow(np.float32(1.0625))) == 1.0
    assert O.e4m3_widen(O.e4m3_narrow(np.float32(1.1875))) == 1.25
    # Every value rounds to the nearest representable (brute force on a grid).
    fin = np.sort(f[~nan & (f >= 0)])
    xs = np.linspace(0, 448, 4001, dtype=np.float32)
    got = O.e4m3_widen(O.e4m3_narrow(xs))
    d = np.abs(xs[:, None] - fin[None, :]).min(1)
    assert np.all(np.abs(got - xs) <= d + 1e-7)


# --- Noise: engine/ir/testkit/src/noise.rs --------------------------------------

def test_noise_closed_form():
    n = O.Noise(29)
    got = n.draw(5)
    s = 29
    want = []
    for _ in range(5):
        s = (s * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        want.append(np.float32((s >> 40) / float(1 << 23)) - np.float32(1.0))
    assert np.array_equal(got, np.array(want, np.float32))
    assert np.all(got >= -1) and np.all(got < 1)


# --- Acc: round_test.rs sums_round; interp_test.rs accumulators_follow_numerics ---

def test_accumulators():
    xs = [2048.0, 1.0, 1.0, 1.0]
    assert O.acc_sum(xs, "f32") == 2051.0
    assert O.acc_sum(xs, "bf16") == 2048.0
    assert O.acc_sum(xs, "f16") == 2048.0


# --- product: cpu.rs:82-138 ------------------------------------------------------

@pytest.mark.parametrize("m,n,k", [(1, 3, 4), (37, 50, 72), (64, 64, 64)])
def test_product_matches_f64(m, n, k):
    # tiled_test.rs:58-71 shapes; x·wᵀ, not x·w: a transposed operand fails here.
    noise = O.Noise(29)
    x = noise.draw(m * k).reshape(m, k)
    w = noise.draw(n * k).reshape(n, k)
    got = O.product(x, w)
    want = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.max(np.abs(got - want)) < 1e-5 * k
    # Sequential f32 order, restated element by element on a few outputs.
    for r, c in [(0, 0), (m - 1, n - 1)]:
        s = np.float32(0)
        for i in range(k):
            s = np.float32(s + np.float32(x[r, i] * w[c, i]))
        assert got[r, c] == s


def test_product_integer_exact_and_bf16():
    rng = np.random.default_rng(0)
    x = rng.integers(-8, 8, (5, 33)).astype(np.float32)
    w = rng.integers(-8, 8, (7, 33)).astype(np.float32)
    want = (x.astype(np.int64) @ w.astype(np.int64).T).astype(np.float32)
    assert np.array_equal(O.product(x, w), want)
    assert np.array_equal(O.product_bf16w(x, O.bf16_narrow(w)), want)


def test_product_e4m3_and_picked():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 16)).astype(np.float32)
    codes = rng.integers(0, 256, (5, 16)).astype(np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x10  # no NaN codes
    scale = O.bf16_narrow(rng.uniform(0.5, 2, 5).astype(np.float32))
    w = O.e4m3_widen(codes) * O.bf16_widen(scale)[:, None]
    got = O.product_e4m3w(x, codes, scale)
    close(got, x.astype(np.float64) @ w.astype(np.float64).T, 1e-5)
    # picked: rows pick their expert; ids outside the table read zeros.
    table = O.bf16_narrow(rng.standard_normal((3, 4, 16)).astype(np.float32))
    ids = np.array([2, 0, 5, 1], np.uint32)
    xp = rng.standard_normal((4, 16)).astype(np.float32)
    out = O.product_picked_bf16w(xp, table, ids)
    tf = O.bf16_widen(table)
    for r, e in enumerate(ids):
        want = np.zeros(4) if e >= 3 else tf[e].astype(np.float64) @ xp[r]
        close(out[r], want, 1e-5)
    # repeat: 2 x rows shared by 4 picks (8 picks per token in the MoE layout).
    out2 = O.product_picked_bf16w(xp[:2], table, ids)
    close(out2[1], tf[0].astype(np.float64) @ xp[0], 1e-5)
    close(out2[3], tf[1].astype(np.float64) @ xp[1], 1e-5)


# --- stages: cpu_test.rs ----------------------------------------------------------

def test_rope_both_pairs():
    # cpu_test.rs:116-128 with `turned` at 56-88: positions 0 and 3, theta 4, width 4.
    x = (np.arange(16, dtype=np.float32) - 5.5).reshape(2, 2, 4)
    s0, c0 = math.sin(3.0), math.cos(3.0)
    s1, c1 = math.sin(1.5), math.cos(1.5)
    for pairs in ("adjacent", "halves"):
        want = list(x.reshape(-1)[:8])
        for r in x.reshape(-1)[8:].reshape(2, 4):
            a, b, c, d = r
            if pairs == "adjacent":
                want += [a * c0 - b * s0, a * s0 + b * c0, c * c1 - d * s1, c * s1 + d * c1]
            else:
                want += [a * c0 - c * s0, b * c1 - d * s1, a * s0 + c * c0, b * s1 + d * c1]
        close(O.rope(x, [0, 3], 4.0, pairs), want)
    assert abs(O.angle(3, 1, 4, 4.0) - 1.5) < 1e-7


def test_rms_divides_rows():
    # cpu_test.rs:130-146: mean squares 9 and 2 plus eps 7 -> roots 4 and 3.
    x = np.array([[1, -3, 5, -1], [2, 0, 0, -2]], np.float32)
    w = np.array([1, 2, -1, 0.5], np.float32)
    close(O.rms_norm(x, None, 7.0), [0.25, -0.75, 1.25, -0.25, 2 / 3, 0, 0, -2 / 3])
    close(O.rms_norm(x, w, 7.0), [0.25, -1.5, -1.25, -0.125, 2 / 3, 0, 0, -1 / 3])


def test_softmax_rows():
    # cpu_test.rs:161-171.
    x = np.array([0, math.log(2), math.log(3), math.log(4), 500, 500, -np.inf, 500], np.float32)
    close(O.softmax(x.reshape(2, 4)), [0.1, 0.2, 0.3, 0.4, 1 / 3, 1 / 3, 0, 1 / 3])


def test_act_values():
    # cpu_test.rs:173-197.
    x = np.array([-2, 0, 1, 3], np.float32)
    close(O.act("relu", x), [0, 0, 1, 3])
    close(O.act("sigmoid", x), [0.11920292, 0.5, 0.7310586, 0.9525741])
    close(O.act("silu", x), [-0.23840584, 0, 0.7310586, 2.8577224])
    close(O.act("gelu_tanh", x), [-0.0454023, 0, 0.841192, 2.9963626])
    close(O.act("softplus", x), [0.126928, math.log(2), 1.3132617, 3.0485874])
    close(O.act("exp", x), [0.13533528, 1, math.e, 20.085537])
    close(O.act("tanh", x), [-0.9640276, 0, 0.7615942, 0.995055])


def test_gather_rows():
    # cpu_test.rs:199-211: repeats, both ends, one row past the table reads zeros.
    table = np.array([[1, 2], [3, 4], [5, 6], [7, 8]], np.float32)
    close(O.gather(table, [3, 0, 3]), [7, 8, 1, 2, 7, 8])
    close(O.gather(table, [4, 1]), [0, 0, 3, 4])
    bits = O.bf16_narrow(table)
    assert np.array_equal(O.gather(bits, [2]), bits[2:3])


def test_mean_each_axis_and_mix():
    # cpu_test.rs:213-220 over axis 1 of [2,3,2]: 6a+2b+c means.
    x = np.arange(12, dtype=np.float32).reshape(2, 3, 2)
    close(O.mix(x), [2, 3, 8, 9])
    w = np.array([[1, 0, 0], [0.5, 0.25, 0.25]], np.float32)
    close(O.mix(x, w), [0, 1, 0.5 * 6 + 0.25 * 8 + 0.25 * 10, 0.5 * 7 + 0.25 * 9 + 0.25 * 11])


def test_top_k_ties():
    # run_test.rs:55-66: NaN skipped, 0.0 ties -0.0, ties keep the lower index,
    # spare slots hold the width.
    inf, nan = np.inf, np.nan
    x = np.array([2, 7, 7, -1, -inf, 3, nan, -inf, -0.0, 0.0, -0.0, inf], np.float32).reshape(3, 4)
    assert O.top_k(x, 3).reshape(-1).tolist() == [1, 2, 0, 1, 4, 4, 3, 0, 1]


def test_top_k_brute_force():
    rng = np.random.default_rng(3)
    x = rng.integers(-4, 4, (50, 37)).astype(np.float32)  # many ties
    x[rng.random(x.shape) < 0.1] = -np.inf
    got = O.top_k(x, 8)
    for r in range(50):
        order = sorted([i for i in range(37) if x[r, i] > -np.inf], key=lambda i: (-x[r, i], i))
        order = (order + [37] * 8)[:8]
        assert got[r].tolist() == order


def test_take():
    x = np.arange(8, dtype=np.float32).reshape(2, 4)
    close(O.take(x, np.array([[3, 0], [1, 9]], np.uint32)), [3, 0, 5, 0])


# --- attention: interp_test.rs ---------------------------------------------------

def test_window_edges():
    # interp_test.rs:294-302: zero queries average the keys within one position.
    v = np.array([[float(1 << t), -t] for t in range(4)], np.float32).reshape(1, 4, 1, 2)
    want = [1.5, -0.5, 7 / 3, -1, 14 / 3, -2, 6, -2.5]
    q = np.zeros((1, 4, 1, 2), np.float32)
    close(O.attend(q, v, v, 1.0, "within", 1), want)
    close(O.attend(q[:, :1], v, v, 1.0, "within", 1), want[6:])


def _rows_over(positions):
    ln3 = math.log(3)
    k = [0, ln3, 0, 0, ln3, 0, 0, 0, 99, 99, 99, 99] + [9] * 12
    v = [4, -8, 0, 2, 8, 4, 4, 0, 99, 99, 99, 99, -1, 2, 3, -3, 50, 50, 50, 50, 60, 60, 60, 60]
    q = np.array([1, 0, 0, 1] * 4, np.float32).reshape(2, 4, 2)
    k = np.array(k, np.float32).reshape(2 * 3, 2, 2)
    v = np.array(v, np.float32).reshape(2 * 3, 2, 2)
    return O.attend_rows(q, k, v, [1, 0], positions, 3, 1.0)


def test_rows_read_slots():
    # interp_test.rs:304-312: row 0 (slot 1, position 0) sees one key; row 1 weighs two.
    want = [-1, 2, -1, 2, 3, -3, 3, -3, 7, 1, 5, -5, 2, 1, 2, 1]
    close(_rows_over([0, 1]), want)
    with pytest.raises(ValueError):
        _rows_over([0, 3])


def test_rows_paged_equals_dense():
    # The same kept rows laid out in 2-row pages under a reversed table read the same.
    rng = np.random.default_rng(5)
    slots_n, keys, kvh, d = 3, 8, 2, 4
    dense_k = rng.standard_normal((slots_n * keys, kvh, d)).astype(np.float32)
    dense_v = rng.standard_normal((slots_n * keys, kvh, d)).astype(np.float32)
    page = 2
    kept_pages = keys // page
    total = slots_n * kept_pages
    table = np.arange(total, dtype=np.uint32)[::-1].copy()
    paged_k = np.zeros_like(dense_k)
    paged_v = np.zeros_like(dense_v)
    for s in range(slots_n):
        for p in range(keys):
            row = O.paged_row(table, kept_pages, page, s, p)
            assert row == (table[s * kept_pages + p // page] * page) | (p % page)
            paged_k[row] = dense_k[s * keys + p]
            paged_v[row] = dense_v[s * keys + p]
    q = rng.standard_normal((4, 4, d)).astype(np.float32)
    slots, pos = [2, 0, 1, 2], [7, 3, 0, 5]
    a = O.attend_rows(q, dense_k, dense_v, slots, pos, keys, 0.5)
    b = O.attend_rows(q, paged_k, paged_v, slots, pos, keys, 0.5, table=table,
                      kept_pages=kept_pages, page=page)
    assert np.array_equal(a, b)


def test_attend_invariants():
    rng = np.random.default_rng(7)
    q = rng.standard_normal((2, 4, 2, 3)).astype(np.float32)
    k = rng.standard_normal((2, 4, 1, 3)).astype(np.float32)
    v = rng.standard_normal((2, 4, 1, 3)).astype(np.float32)
    out = O.attend(q, k, v, 0.5, "causal")
    # causal_first_row: the first query sees one key: its output is that value row.
    close(out[:, 0, 0], v[:, 0, 0])
    close(out[:, 0, 1], v[:, 0, 0])
    # decode_sees_past_keys: a lone last query is the same causal or bidirectional.
    a = O.attend(q[:, :1], k, v, 0.5, "causal")
    b = O.attend(q[:, :1], k, v, 0.5, "bidirectional")
    assert np.array_equal(a, b)
    # Uniform scores (zero query) give the mean of the values seen.
    z = O.attend(np.zeros_like(q), k, v, 0.5, "causal")
    for t in range(4):
        close(z[:, t, 0], v[:, : t + 1, 0].mean(1), 1e-5)
    # Fewer keys than queries is refused under a causal mask.
    with pytest.raises(ValueError):
        O.attend(q, k[:, :2], v[:, :2], 0.5, "causal")
    # GQA: heads h read kv head h // (heads / kv_heads); against an f64 softmax.
    qq = rng.standard_normal((1, 3, 4, 5)).astype(np.float32)
    kk = rng.standard_normal((1, 3, 2, 5)).astype(np.float32)
    vv = rng.standard_normal((1, 3, 2, 5)).astype(np.float32)
    got = O.attend(qq, kk, vv, 0.3, "causal")
    for t in range(3):
        for h in range(4):
            s = np.array([qq[0, t, h] @ kk[0, j, h // 2] * 0.3 for j in range(t + 1)], np.float64)
            p = np.exp(s - s.max()); p /= p.sum()
            close(got[0, t, h], p @ vv[0, : t + 1, h // 2].astype(np.float64), 1e-5)


def test_threads_bit_identical():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((3, 300)).astype(np.float32)
    w = O.bf16_narrow(rng.standard_normal((257, 300)).astype(np.float32))
    O.set_threads(1)
    a = O.product_bf16w(x, w)
    O.set_threads(4)
    b = O.product_bf16w(x, w)
    O.set_threads(1)
    assert np.array_equal(a, b)


def test_act_against_closed_forms():
    """Every activation of the oracle (cpu.rs:8-29) against its formula in float64 on a
    dense grid: within 4e-7 relative (the f32 rounding of each step) plus 1e-37."""
    x = np.concatenate([np.linspace(-20, 20, 8001), [0.0, 1e-6, -1e-6, 50.0, -50.0]]).astype(np.float32)
    d = x.astype(np.float64)
    forms = {
        "gelu_tanh": 0.5 * d * (1 + np.tanh(0.7978846 * (d + 0.044715 * d ** 3))),
        "silu": d / (1 + np.exp(-d)),
        "sigmoid": 1 / (1 + np.exp(-d)),
        "relu": np.maximum(d, 0),
        "softplus": np.maximum(d, 0) + np.log1p(np.exp(-np.abs(d))),
        "exp": np.exp(d),
        "tanh": np.tanh(d),
    }
    for a, want in forms.items():
        got = O.act(a, x).astype(np.float64)
        # gelu's inner sum cancels near x = 0 only where the result is tiny
        tol = 1e-6 * np.abs(want) + 1e-37 + (1e-7 if a == "gelu_tanh" else 0)
        assert np.all(np.abs(got - want) <= tol), a


def test_chain_known_answers():
    """The chain's read order (kernels/map.rs:125-185): read `sum_at` is the input, the
    others the operands in order; each stage one f32 rounding (cpu.rs:353-390)."""
    x = np.array([1.0, 2.0], np.float32)
    a = np.array([3.0, 4.0], np.float32)
    b = np.array([0.5, -1.0], np.float32)
    # v = x; v = v + a; v = v * b; v = v * 2
    close(O.chain(x, ["add", "mul", ("scale", 2.0)], [a, b], 0), [4.0, -12.0])
    # the input read second: v = a; v = v + x; v = v * b
    close(O.chain(x, ["add", "mul"], [a, b], 1), [2.0, -6.0])
    # the input read last: v = a; v = v * b; v = v + x
    close(O.chain(x, ["mul", "add"], [a, b], 2), [2.5, -2.0])
    # spans: a row of 2 repeating, and a scalar
    r = np.array([10.0, 20.0], np.float32)
    close(O.chain(np.arange(4, dtype=np.float32), ["add", "mul"], [r, np.array([3.0], np.float32)], 0, [2, 1]),
          [30.0, 63.0, 36.0, 69.0])
    # each stage rounds: (1 + 2^-24) + 2^-24 = 1 twice over in f32, not 1 + 2^-23
    tiny = np.float32(2.0 ** -24)
    assert O.chain(np.array([1.0], np.float32), ["add", "add"], [np.array([tiny]), np.array([tiny])])[0] == 1.0
    close(O.chain(np.array([-2.0, 3.0], np.float32), ["relu", "exp"]), [1.0, float(np.exp(np.float32(3.0)))])
