"""TEST INFRASTRUCTURE ONLY: the Qwen3 decoder step composed from the oracle's ops.

Follows engine/models/src/decoder.rs:327-391 (trunk, attention) and
engine/models/src/shared.rs:109-145,375-378 (q/k RmsNorm per head, then Halves
RoPE; SwiGLU) as tessera-interp evaluates them: every product is the oracle's
sequential f32 dot over bf16 weights, every stage the oracle's restatement.
One format change at the boundary, as on the device: kept K/V rows are stored as
bf16, so appended rows are rounded to bf16 before attention reads them.
"""
from __future__ import annotations

import math

import numpy as np

import oracle as O


class Weights:
    """Host copies: bf16 bits for matrices, f32 for RmsNorm gains."""

    def __init__(self, cfg: dict):
        self.cfg = cfg
        self.embed = None
        self.norm = None
        self.layers = []


class Qwen3:
    def __init__(self, w: Weights):
        self.w = w
        c = w.cfg
        self.c = c
        self.kv = [dict(k=np.zeros((c["max_context"], c["kv_heads"], c["head_dim"]), np.float32),
                        v=np.zeros((c["max_context"], c["kv_heads"], c["head_dim"]), np.float32))
                   for _ in range(c["layers"])]
        # Kept rows below `origin` are not part of the slot (0: the slot starts at position 0).
        # Rotations use the absolute positions; attention reads keys origin..pos.
        self.origin = 0
        # Format of the kept rows: bf16, as the device stores them.
        self.keep = O.bf16_round

    def norm_rope(self, t, gain, positions):
        """Per-head RmsNorm, then Halves RoPE at the rows' positions
        (engine/models/src/shared.rs:109-145: q_norm/k_norm precede the rotation)."""
        c = self.c
        return O.rope(O.rms_norm(t, gain, c["eps"]), positions, c["theta"], "halves")

    def forward(self, tokens, positions) -> np.ndarray:
        """Rows of one slot at `positions`; returns the last row's logits."""
        c, w = self.c, self.w
        H, D, Hq, Hkv = c["hidden"], c["head_dim"], c["heads"], c["kv_heads"]
        eps, theta = c["eps"], c["theta"]
        tokens = np.asarray(tokens, np.uint32)
        positions = np.asarray(positions, np.uint32)
        rows = len(tokens)
        x = O.bf16_widen(O.gather(w.embed, tokens))                      # Model::embed (Gather)
        scale = 1.0 / math.sqrt(D)
        for li, L in enumerate(w.layers):
            h = O.rms_norm(x, L["ln1"], eps)                                # x.rms_norm(ln1)
            qkv = O.product_bf16w(h, L["qkv"])                              # q, k, v products
            q = qkv[:, : Hq * D].reshape(rows, Hq, D)
            k = qkv[:, Hq * D:(Hq + Hkv) * D].reshape(rows, Hkv, D)
            v = qkv[:, (Hq + Hkv) * D:].reshape(rows, Hkv, D)
            q = self.norm_rope(q, L["q_norm"], positions)
            k = self.norm_rope(k, L["k_norm"], positions)
            kv = self.kv[li]
            kv["k"][positions] = self.keep(k)                            # Append (bf16 kept rows)
            kv["v"][positions] = self.keep(v)
            o0 = self.origin                                                # first kept row of the slot
            attn = O.attend_rows(q, kv["k"][o0:], kv["v"][o0:], np.zeros(rows, np.uint32), positions - o0,
                                 c["max_context"] - o0, scale)              # attend_rows, causal
            x = O.product_bf16w(attn.reshape(rows, Hq * D), L["o"]) + x    # o, then .add(x)
            h = O.rms_norm(x, L["ln2"], eps)
            gu = O.product_bf16w(h, L["gate_up"])
            F = c["ffn"]
            inner = O.act("silu", gu[:, :F]) * gu[:, F:]                    # silu(gate) * up
            x = O.product_bf16w(inner, L["down"]) + x
        last = O.rms_norm(x[-1:], w.norm, eps)                              # final RmsNorm
        return O.product_bf16w(last, w.embed)[0]                           # tied unembed


def from_runner(model) -> Weights:
    """A runner's weights copied to host in the oracle model's layout."""
    c = model.config
    H, D = c.hidden, c.head_dim
    w = Weights(c.as_dict())
    w.embed = model.read("embed").reshape(c.vocab, H)
    w.norm = model.read("norm")
    QKV = (c.heads + 2 * c.kv_heads) * D
    for l in range(c.layers):
        w.layers.append(dict(
            ln1=model.read("ln1", l), ln2=model.read("ln2", l), q_norm=model.read("q_norm", l),
            k_norm=model.read("k_norm", l), qkv=model.read("qkv", l).reshape(QKV, H),
            o=model.read("o", l).reshape(H, c.heads * D), gate_up=model.read("gate_up", l).reshape(2 * c.ffn, H),
            down=model.read("down", l).reshape(H, c.ffn)))
    return w
