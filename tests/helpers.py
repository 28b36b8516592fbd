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
