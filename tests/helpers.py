"""Shared test helpers: seeded inputs, bf16/e4m3 bits via the oracle, tolerances."""
import numpy as np

import oracle as O


def rng(seed):
    return np.random.default_rng(seed)


def bf16_bits_normal(r, shape, std=1.0):
    """N(0, std) values rounded to bf16 (RNE): (bits uint16, widened f32)."""
    bits = O.bf16_narrow((r.standard_normal(shape) * std).astype(np.float32))
    return bits, O.bf16_widen(bits)


def to_dev(a, torch, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if a.dtype == np.uint16:
        t = t.view(torch.int16).view(torch.bfloat16)
    return t.to("cuda") if dtype is None else t.to("cuda", dtype)


def from_dev(t):
    import torch
    if t.dtype == torch.bfloat16:
        return O.bf16_widen(t.view(torch.int16).cpu().numpy().view(np.uint16))
    return t.float().cpu().numpy() if t.dtype != torch.int32 else t.cpu().numpy()


def product_bound(x, w, *, x_bits=None, parts=1, lane=8, w_bits=None):
    """Per-output error bound of a matrix-unit product x @ w^T, after the reference's
    Terms::matmul (engine/plan/codegen/src/numerics.rs:150-175):
        sum_i |x_i| ew_i + |w_i| ex_i + |x_i| |w_i| (tile acc_error + lane 2^-24).
    For this build's kernels: weights enter the unit exactly (bf16, e4m3 and every
    block code are bf16 values), so ew = 0; bf16 rows are exact (ex = 0) and f32 rows
    enter as two bf16 parts, 16 significant bits (ex = |x| 2^-16, parts = 2). Each
    output sees at most k / 32 accumulating v_mfma_f32_16x16x32_bf16 per part plus up
    to 16 split-K partial adds; the count is doubled for headroom (tile = (k / 16 + 16)
    parts), each costing the reference's HIP accumulator error 2^-21 (22 bits,
    truncating: numerics.rs:47-52). `lane` counts f32 roundings outside the unit
    (scale multiplies, block adds, the epilogue). f32 weights enter as two bf16 parts
    (w_bits = 16: ew = |w| 2^-16)."""
    ax = np.abs(np.atleast_2d(x)).astype(np.float64)
    aw = np.abs(np.atleast_2d(w)).astype(np.float64)
    k = ax.shape[1]
    tile = (k / 16 + 16) * parts
    adds = tile * 2.0 ** -21 + lane * 2.0 ** -24
    bound = (ax @ aw.T) * adds
    if x_bits is not None:
        bound += (ax * 2.0 ** -x_bits) @ aw.T
    if w_bits is not None:  # weights held to w_bits significant bits (f32 weights as two bf16 parts)
        bound += ax @ (aw * 2.0 ** -w_bits).T
    return bound


def linear_bound(x, w, lane=8):
    """product_bound for the linear kernels' operands: rows whose values are all bf16
    enter exactly; other f32 rows as two bf16 parts."""
    x = np.asarray(x, np.float32)
    exact = np.array_equal(O.bf16_round(x), x)
    return product_bound(x, w, x_bits=None if exact else 16, parts=1 if exact else 2, lane=lane)


def assert_within(got, want, bound):
    """|got - want| <= bound per element, and the bound says something: below a tenth
    of the largest output (tiled_test.rs:104-114)."""
    err = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))
    assert np.all(err <= bound), f"max err {err.max():.3e}, bound there {bound.reshape(-1)[err.argmax()]:.3e}"
    most = float(np.max(np.abs(want)))
    assert float(np.max(bound)) < most / 10, f"bound {np.max(bound):.3e} against outputs of {most:.3e}"


def max_rel(got, want):
    """max |got - want| / max |want| (the reference parity suite's `off`)."""
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


def cosine(a, b):
    a = a.astype(np.float64).reshape(-1)
    b = b.astype(np.float64).reshape(-1)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def host_weights(model):
    from oracle.qwen3 import from_runner
    return from_runner(model)


def greedy_agrees(token, want_logits, tol):
    """The device's greedy token matches the oracle's, or the oracle's top two are
    within `tol` of each other (a near-tie that summation order may flip)."""
    best = int(np.argmax(want_logits))
    if token == best:
        return True
    return float(want_logits[best] - want_logits[token]) <= tol
