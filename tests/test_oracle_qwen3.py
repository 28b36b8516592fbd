"""The oracle's Qwen3 decoder composition (oracle/qwen3.py) against what the
mathematics fixes, on the CPU.

The reference's golden Qwen3 logits are not available, so the composition is pinned
by cases whose answer does not go through the composition's own code:
* the parameter count of the runner's default shape is Qwen3-0.6B's 596,049,920
  (tools/parity/tests/qwen3/mod.rs:16 in the reference);
* at position 0 a row attends only to itself, so each head's attention output is its
  kv head's v row (softmax over one key is 1): the whole step reduces to products,
  norms and SwiGLU, computed here in float64 straight from the weights;
* with the o and down weights zero every block is the identity on the residual
  stream: the logits are the tied unembedding of the final-normed embedding row,
  whatever the attention does;
* a prompt prefilled in one call and the same prompt fed one token at a time give the
  same last logits (kept rows appended at their positions, causal masking).
* RoPE after the per-head norm makes attention depend on relative positions only: the
  same prompt placed at positions s..s+n-1 gives the logits of positions 0..n-1, which
  fails for the rotation and the norm swapped or a row rotated by the wrong position.
A dropped residual, a norm on the wrong tensor, a wrong GQA head map or a transposed
product fails one of them.
"""
import math

import numpy as np

import oracle as O
from oracle.qwen3 import Qwen3, Weights


def tiny(seed, layers=2, vocab=50, hidden=32, heads=4, kv_heads=2, head_dim=8, ffn=48, zero_o_down=False):
    r = np.random.default_rng(seed)
    cfg = dict(vocab=vocab, hidden=hidden, layers=layers, heads=heads, kv_heads=kv_heads, head_dim=head_dim,
               ffn=ffn, eps=1e-6, theta=1e4, max_context=16)
    bits = lambda shape, s=0.3: O.bf16_narrow(r.standard_normal(shape).astype(np.float32) * s)
    gain = lambda n: (1.0 + 0.1 * r.standard_normal(n)).astype(np.float32)
    w = Weights(cfg)
    w.embed = bits((vocab, hidden), 1.0)
    w.norm = gain(hidden)
    QD, QKV = heads * head_dim, (heads + 2 * kv_heads) * head_dim
    for _ in range(layers):
        o = bits((hidden, QD))
        down = bits((hidden, ffn))
        if zero_o_down:
            o[:] = 0
            down[:] = 0
        w.layers.append(dict(ln1=gain(hidden), ln2=gain(hidden), q_norm=gain(head_dim), k_norm=gain(head_dim),
                             qkv=bits((QKV, hidden)), o=o, gate_up=bits((2 * ffn, hidden)), down=down))
    return w


def f64(bits):
    return O.bf16_widen(bits).astype(np.float64)


def rms64(x, g, eps):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * g


def test_default_shape_is_qwen3_0_6b():
    from tessera_amd.qwen3 import default_config
    c = default_config()
    H, D, F, V, L = c.hidden, c.head_dim, c.ffn, c.vocab, c.layers
    per_layer = 2 * H + (c.heads + 2 * c.kv_heads) * D * H + 2 * D + H * c.heads * D + 2 * F * H + H * F
    assert V * H + L * per_layer + H == 596_049_920
    assert (L, H, c.heads, c.kv_heads, D, F, V) == (28, 1024, 16, 8, 128, 3072, 151936)


def test_position_zero_reduces_to_products():
    w = tiny(1)
    c = w.cfg
    D, Hq, Hkv, F, eps = c["head_dim"], c["heads"], c["kv_heads"], c["ffn"], c["eps"]
    tok = 7
    got = Qwen3(w).forward([tok], [0])
    x = f64(w.embed[tok])
    for L in w.layers:
        h = rms64(x, L["ln1"], eps)
        qkv = f64(L["qkv"]) @ h
        v = qkv[(Hq + Hkv) * D:].reshape(Hkv, D)
        v = O.bf16_widen(O.bf16_narrow(v.astype(np.float32))).astype(np.float64)  # kept rows are bf16
        att = np.concatenate([v[h_ // (Hq // Hkv)] for h_ in range(Hq)])           # q head h reads kv head h / G
        x = x + f64(L["o"]) @ att
        h2 = rms64(x, L["ln2"], eps)
        gu = f64(L["gate_up"]) @ h2
        g, u = gu[:F], gu[F:]
        x = x + f64(L["down"]) @ (g / (1 + np.exp(-g)) * u)
    want = f64(w.embed) @ rms64(x, w.norm, eps)
    assert np.max(np.abs(got - want)) <= 1e-4 * np.max(np.abs(want))


def test_identity_blocks_leave_the_embedding():
    w = tiny(2, zero_o_down=True)
    eps = w.cfg["eps"]
    toks = [3, 11, 40, 5]
    got = Qwen3(w).forward(toks, np.arange(len(toks)))
    want = f64(w.embed) @ rms64(f64(w.embed[toks[-1]]), w.norm, eps)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))


def test_prefill_equals_token_by_token():
    w = tiny(3)
    toks = [4, 9, 33, 1, 17]
    a = Qwen3(w).forward(toks, np.arange(len(toks)))
    m = Qwen3(w)
    for i, t in enumerate(toks):
        b = m.forward([t], [i])
    # Same sequential sums per row either way: bit-identical.
    assert np.array_equal(a, b)
    # And the last token does depend on the earlier ones (the causal rows are read).
    c = Qwen3(w).forward([toks[-1]], [0])
    assert not np.allclose(a, c)


class RopeFirst(Qwen3):
    """The composition with the rotation and the per-head norm swapped (a plausible
    mistake the shift test must catch)."""

    def norm_rope(self, t, gain, positions):
        c = self.c
        return O.rms_norm(O.rope(t, positions, c["theta"], "halves"), gain, c["eps"])


def shifted_logits(cls, w, toks, shift, keep=None):
    m = cls(w)
    m.origin = shift
    if keep is not None:
        m.keep = keep
    return m.forward(toks, shift + np.arange(len(toks)))


def test_rope_after_norm_is_shift_invariant():
    """RoPE makes q.k depend on the positions' difference only, so the same prompt
    placed at positions s..s+n-1 (the slot's keys starting at s) gives the logits of
    positions 0..n-1 — up to the bf16 rounding of the kept k rows, whose rotated values
    differ with the absolute position. This pins the q/k norm -> RoPE order and the
    position each row is rotated by (engine/models/src/shared.rs:109-145) at positions
    > 0, with non-uniform q_norm / k_norm gains (a norm after the rotation breaks the
    invariance; so does a row rotated by the wrong position)."""
    w = tiny(4)
    for L in w.layers:
        L["q_norm"] = (1.0 + 0.5 * np.random.default_rng(5).standard_normal(L["q_norm"].size)).astype(np.float32)
        L["k_norm"] = (1.0 + 0.5 * np.random.default_rng(6).standard_normal(L["k_norm"].size)).astype(np.float32)
    w.cfg["max_context"] = 64
    toks = [4, 9, 33, 1, 17, 26, 8]
    exact = lambda a: a
    base = shifted_logits(Qwen3, w, toks, 0, exact)
    scale = np.abs(base).max()
    for s in (1, 13, 40):
        # f32 kept rows: equal up to f32 rounding of the rotations
        d = np.abs(shifted_logits(Qwen3, w, toks, s, exact) - base).max() / scale
        assert d <= 1e-5, (s, d)
        # bf16 kept rows (the device's format): the rounding of rotated k moves with s
        b16 = shifted_logits(Qwen3, w, toks, 0)
        d = np.abs(shifted_logits(Qwen3, w, toks, s) - b16).max() / np.abs(b16).max()
        assert d <= 2e-2, (s, d)
    # The swapped composition is not invariant: it moves by far more than either bound.
    rb = shifted_logits(RopeFirst, w, toks, 0, exact)
    for s in (1, 13, 40):
        d = np.abs(shifted_logits(RopeFirst, w, toks, s, exact) - rb).max() / np.abs(rb).max()
        assert d > 0.1, (s, d)

    class OffByOne(Qwen3):
        """q of the last row rotated one position too far."""

        def norm_rope(self, t, gain, positions):
            last = (np.arange(len(positions)) == len(positions) - 1) & (t.shape[1] == self.c["heads"])
            return super().norm_rope(t, gain, positions + last.astype(np.uint32))

    ob = shifted_logits(OffByOne, w, toks, 0, exact)
    assert np.abs(ob - base).max() / scale > 1e-2
