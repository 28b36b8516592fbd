"""Parity of the MoE pieces (picked products, take, softmax, mix, the whole layer)
with the oracle.

Tolerances (stated per test):
  * picked, f32 out: within the analytic bound of tests/helpers.product_bound (the
    reference's Terms::matmul, engine/plan/codegen/src/numerics.rs:150-175, with the
    matrix unit's accumulation and the two-bf16-part f32 rows), as for the linear
    kernels. Rows with an id outside the set must be exactly zero.
  * take, mix: bit-exact (same order, products rounded before each add).
  * softmax: |got - want| <= 2e-7 per entry (device expf vs glibc expf ulps).
  * the layer: routing ids bit-exact against the oracle's top_k of the device's own
    scores; gates within 2e-6; output max-rel <= 2e-2 (bf16 tolerance; the device
    keeps silu(g)*u in bf16 between the two expert products).
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


def _picked_want(x, table_bits, ids, repeat, first, offset, n, silu):
    """Oracle picked product (matmul_picked, cpu.rs:89-105) on rows offset.. of each
    matrix; with silu the gate rows offset..offset+n and up rows offset+n..offset+2n."""
    sub = table_bits[:, offset:offset + (2 * n if silu else n)]
    xs = np.repeat(x, repeat, axis=0)[: ids.size]
    full = O.product_picked_bf16w(xs, np.ascontiguousarray(sub), ids, first)
    if not silu:
        return full, None
    g, u = full[:, :n], full[:, n:]
    return O.act("silu", g) * u, (g, u)


@pytest.mark.parametrize("rows,count,k,n,repeat,first,xdt", [
    (1, 3, 64, 40, 1, 0, "f32"),
    (300, 16, 256, 96, 1, 0, "f32"),
    (600, 16, 128, 130, 4, 2, "bf16"),   # ids below `first` and past the set read zeros
    (2000, 64, 64, 64, 8, 0, "bf16"),
    (1000, 330, 64, 32, 1, 0, "bf16"),  # more matrices than the one-pass routing scan takes
    (700, 8, 128, 192, 2, 0, "bf16"),    # columns in whole 192-wide tiles: the 128 x 192 form
])
def test_picked_matches_oracle(rows, count, k, n, repeat, first, xdt):
    R = _rules()
    r = rng(rows + count + k)
    stride, offset = n + 8, 5
    table_bits, table = bf16_bits_normal(r, (count, stride, k), 0.05)
    ids = r.integers(0, count + first + 3, size=rows).astype(np.uint32)
    tokens = (rows + repeat - 1) // repeat
    if xdt == "f32":
        x = r.standard_normal((tokens, k)).astype(np.float32)
        xd = to_dev(x, torch)
    else:
        xb, x = bf16_bits_normal(r, (tokens, k))
        xd = to_dev(xb, torch)
    want, _ = _picked_want(x, table_bits, ids, repeat, first, offset, n, False)
    got = from_dev(R.picked(xd, to_dev(table_bits, torch), to_dev(ids.astype(np.int32), torch), n=n, repeat=repeat,
                            first=first, offset=offset))
    xs = np.repeat(x, repeat, axis=0)[:rows]
    for i in range(rows):  # per row: its own matrix's bound, exact zeros outside the set
        e = int(ids[i]) - first
        if e < 0 or e >= count:
            assert np.all(got[i] == 0.0)
        else:
            b = _bound(xs[i:i + 1], table[e, offset:offset + n])[0]
            assert np.all(np.abs(got[i] - want[i]) <= b), f"row {i} expert {e}"


def test_picked_many_rows():
    """Past 32768 rows the routing scan takes its general path; every row within its
    matrix's bound, in one vectorized check per matrix."""
    R = _rules()
    r = rng(41)
    rows, count, k, n = 40000, 3, 64, 16
    table_bits, table = bf16_bits_normal(r, (count, n, k), 0.05)
    xb, x = bf16_bits_normal(r, (rows, k))
    ids = r.integers(0, count, size=rows).astype(np.uint32)
    want = O.product_picked_bf16w(x, table_bits, ids, 0)
    got = from_dev(R.picked(to_dev(xb, torch), to_dev(table_bits, torch), to_dev(ids.astype(np.int32), torch)))
    for e in range(count):
        sel = ids == e
        assert np.all(np.abs(got[sel] - want[sel]) <= _bound(x[sel], table[e])), f"matrix {e}"


def test_picked_silu_pair_bf16_out():
    """The fused gate/up pair (silu(g) * u), bf16 out: max-rel <= 2e-2."""
    R = _rules()
    r = rng(77)
    count, ffn, k, tokens, top = 8, 96, 256, 200, 4
    table_bits, _ = bf16_bits_normal(r, (count, 2 * ffn, k), 0.05)
    xb, x = bf16_bits_normal(r, (tokens, k))
    ids = r.integers(0, count, size=tokens * top).astype(np.uint32)
    want, _ = _picked_want(x, table_bits, ids, top, 0, 0, ffn, True)
    got = from_dev(R.picked(to_dev(xb, torch), to_dev(table_bits, torch), to_dev(ids.astype(np.int32), torch), n=ffn,
                            repeat=top, silu_mul=True, out_dtype=torch.bfloat16))
    assert max_rel(got, want) <= 2e-2


def test_picked_is_stable_under_permuted_rows():
    """Routing is a stable sort: moving rows between matrices or reordering them
    moves the outputs with them, bit-identically (each row's product is computed
    by the same tile code whatever its neighbours)."""
    R = _rules()
    r = rng(5)
    count, k, n, rows = 12, 128, 64, 512
    table_bits, _ = bf16_bits_normal(r, (count, n, k), 0.05)
    xb, _ = bf16_bits_normal(r, (rows, k))
    ids = r.integers(0, count, size=rows).astype(np.uint32)
    a = from_dev(R.picked(to_dev(xb, torch), to_dev(table_bits, torch), to_dev(ids.astype(np.int32), torch)))
    # every row alone (rows = 1 per launch) gives the same bits as in the batch
    for i in [0, 1, 77, rows - 1]:
        one = from_dev(R.picked(to_dev(xb[i:i + 1], torch), to_dev(table_bits, torch),
                                to_dev(ids[i:i + 1].astype(np.int32), torch)))
        assert np.array_equal(one[0], a[i])


def test_take_softmax_mix():
    R = _rules()
    r = rng(9)
    rows, width, picks, inner = 257, 128, 8, 96
    x = r.standard_normal((rows, width)).astype(np.float32)
    ids = r.integers(0, width + 4, size=(rows, picks)).astype(np.uint32)  # some out of range
    got_t = from_dev(R.take(to_dev(x, torch), to_dev(ids.astype(np.int32), torch)))
    assert np.array_equal(got_t, O.take(x, ids))
    g = x[:, :picks].copy()
    got_s = from_dev(R.softmax(to_dev(g, torch)))
    assert np.max(np.abs(got_s - O.softmax(g))) <= 2e-7
    y = r.standard_normal((rows, picks, inner)).astype(np.float32)
    w = O.softmax(g)
    assert np.array_equal(from_dev(R.mix(to_dev(y, torch), to_dev(w, torch))), O.mix(y, w))
    assert np.array_equal(from_dev(R.mix(to_dev(y, torch))), O.mix(y))
    y5 = r.standard_normal((rows, picks, 5)).astype(np.float32)  # inner not a multiple of 4
    assert np.array_equal(from_dev(R.mix(to_dev(y5, torch), to_dev(w, torch))), O.mix(y5, w))
    # cpu_test.rs:161 softmax_rows
    rows2 = np.array([[1, 2, 3, 4], [0, 0, -np.inf, 0]], np.float32)
    want2 = np.array([[0.0320586, 0.0871443, 0.2368828, 0.6439143], [1 / 3, 1 / 3, 0, 1 / 3]], np.float32)
    assert np.allclose(from_dev(R.softmax(to_dev(rows2, torch))), want2, atol=1e-6)


@pytest.mark.parametrize("tokens,hidden,experts,top,ffn", [(384, 256, 16, 4, 128), (1024, 1024, 128, 8, 512),
                                                         (512, 512, 32, 4, 192)])  # gate/up in 128 x 192 tiles
def test_moe_layer_matches_oracle(tokens, hidden, experts, top, ffn):
    """One MoE MLP (decoder.rs:73-84) plus a shared expert: a small shape, and C5's
    128 experts top-8 at 1024 tokens (hidden and FFN narrowed so the oracle is quick)."""
    R = _rules()
    r = rng(31)
    hb, h = bf16_bits_normal(r, (tokens, hidden))
    router_b, _ = bf16_bits_normal(r, (experts, hidden), 0.2)
    win_b, _ = bf16_bits_normal(r, (experts, 2 * ffn, hidden), 0.05)
    wout_b, _ = bf16_bits_normal(r, (experts, hidden, ffn), 0.05)
    sin_b, _ = bf16_bits_normal(r, (2 * ffn, hidden), 0.05)
    sout_b, _ = bf16_bits_normal(r, (hidden, ffn), 0.05)
    y, ids, gates = R.moe_layer(to_dev(hb, torch), to_dev(router_b, torch), to_dev(win_b, torch),
                                to_dev(wout_b, torch), top=top, shared_in=to_dev(sin_b, torch),
                                shared_out=to_dev(sout_b, torch))
    torch.cuda.synchronize()
    scores = from_dev(R.linear(to_dev(hb, torch), to_dev(router_b, torch)))
    ids_np = from_dev(ids).astype(np.uint32)
    # routing: bit-exact top_k of the device's scores
    assert np.array_equal(ids_np, O.top_k(scores, top))
    want_gates = O.softmax(O.take(scores, ids_np))
    assert np.max(np.abs(from_dev(gates) - want_gates)) <= 2e-6
    # the rest through the oracle with the same picks
    flat = ids_np.reshape(-1)
    inner, _ = _picked_want(h, win_b, flat, top, 0, 0, ffn, True)
    y_picks = O.product_picked_bf16w(inner, wout_b, flat, 0)
    want = O.mix(y_picks.reshape(tokens, top, hidden), want_gates)
    s_gu = O.product_bf16w(h, sin_b)
    s_inner = O.act("silu", s_gu[:, :ffn]) * s_gu[:, ffn:]
    want = want + O.product_bf16w(s_inner, sout_b)
    assert max_rel(from_dev(y), want) <= 2e-2


def test_moe_layer_c5_full_shape():
    """C5 as benchmarked: 4096 tokens, hidden 4096, 128 experts top-8, FFN 1536, one
    shared expert, the gate logits given as scores (N(0,1) f32, seed 3) and the weights
    drawn as the bench draws them. Routing ids bit-exact on every row against the
    oracle's top_k; the stable sort's permutation (read from the routing workspace of
    a picked launch with the same ids) bit-exact against a stable argsort by expert;
    gates within 2e-6; the layer's output within max-rel 2e-2 of the oracle on 64
    sampled tokens, which together pick at least 100 experts."""
    R = _rules()
    O.set_threads(O.lib().or_threads_available())
    tokens, hidden, experts, top, ffn = 4096, 4096, 128, 8, 1536
    g = torch.Generator(device="cuda").manual_seed(3)
    logits = torch.randn((tokens, experts), device="cuda", generator=g)
    h = torch.randn((tokens, hidden), device="cuda", generator=g).to(torch.bfloat16)
    w_in = torch.empty((experts, 2 * ffn, hidden), device="cuda", dtype=torch.bfloat16)
    w_out = torch.empty((experts, hidden, ffn), device="cuda", dtype=torch.bfloat16)
    for e in range(experts):
        w_in[e] = (torch.randn((2 * ffn, hidden), device="cuda", generator=g) * 0.02).to(torch.bfloat16)
        w_out[e] = (torch.randn((hidden, ffn), device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    s_in = (torch.randn((2 * ffn, hidden), device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    s_out = (torch.randn((hidden, ffn), device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    print("C5 full shape", flush=True)
    y, ids, gates = R.moe_layer(h, None, w_in, w_out, top=top, shared_in=s_in, shared_out=s_out, scores=logits)
    torch.cuda.synchronize()
    scores = from_dev(logits)
    ids_np = from_dev(ids).astype(np.uint32)
    assert np.array_equal(ids_np, O.top_k(scores, top))
    want_gates = O.softmax(O.take(scores, ids_np))
    assert np.max(np.abs(from_dev(gates) - want_gates)) <= 2e-6
    # the permutation: a picked launch over the same ids leaves its routing in the workspace
    flat = ids_np.reshape(-1)
    R.picked(h, w_in, ids, n=16, repeat=top)
    torch.cuda.synchronize()
    words = R.workspace(h.device).buf.view(torch.int32).cpu().numpy().view(np.uint32)
    rows, B = flat.size, experts + 1
    chunks = (rows + 255) // 256
    row_start = words[chunks * B: chunks * B + B + 1]
    perm = words[chunks * B + (B + 1) + (experts + 1):][:rows]
    assert np.array_equal(perm, np.argsort(flat, kind="stable").astype(np.uint32))
    assert np.array_equal(row_start[:B], np.searchsorted(np.sort(flat), np.arange(B)).astype(np.uint32))
    assert row_start[B] == rows
    # the output on sampled tokens, through the oracle with the same picks
    sample = np.sort(rng(64).choice(tokens, 64, replace=False))
    assert len(set(ids_np[sample].reshape(-1).tolist())) >= 100
    hb = h.view(torch.int16).cpu().numpy().view(np.uint16)[sample]
    hx = O.bf16_widen(hb)
    bits = lambda t: t.view(torch.int16).cpu().numpy().view(np.uint16)
    want = np.zeros((len(sample), hidden), np.float32)
    y_picks = np.zeros((len(sample), top, hidden), np.float32)
    for e in np.unique(ids_np[sample]):
        ti, pi = np.nonzero(ids_np[sample] == e)
        gu = O.product_bf16w(hx[ti], bits(w_in[e]))
        inner = O.act("silu", gu[:, :ffn]) * gu[:, ffn:]
        y_picks[ti, pi] = O.product_bf16w(inner, bits(w_out[e]))
    want = O.mix(y_picks, want_gates[sample])
    s_gu = O.product_bf16w(hx, bits(s_in))
    want = want + O.product_bf16w(O.act("silu", s_gu[:, :ffn]) * s_gu[:, ffn:], bits(s_out))
    assert max_rel(from_dev(y)[sample], want) <= 2e-2
    O.set_threads(1)
