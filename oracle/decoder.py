"""CPU decoder forward -- TEST INFRASTRUCTURE ONLY (see the package header).

The layer order of the reference GPU runtime, restated from its stage
functions (each pinned in oracle.h):
  run_layer, src/gpu_llm/mod.rs:2056-2350 (one decode token) and
  run_batch_layer, src/gpu_llm/prefill.rs:897-1061 (a prompt chunk):
    x = embed(ids)                                    llm_embed  gpu_llm.cl:24-33
    per layer:
      h = rmsnorm(x, input_norm)                      llm_rmsnorm :72-98
      q, k, v = h.Wq^T, h.Wk^T, h.Wv^T                tv_hip_matrix_multiply
      q, k = rope(q), rope(k) at the token positions  llm_rope :102-146
      K/V cache += (k, v)                             mod.rs:2103-2136
      a = attention(q, K, V) causal                   llm_prefill_qk/softmax/pv :462-541
      x = x + a.Wo^T                                  llm_add :214-222
      h = rmsnorm(x, post_norm)
      x = x + swiglu(h.Wg^T, h.Wu^T).Wd^T             llm_swiglu :225-237
    logits = rmsnorm(x_last, final_norm).Wlm^T; token = argmax  llm_argmax :239-270
pin: the composition is checked in tests/test_oracle.py against closed forms
that a wrong wiring breaks: with every projection zero the residual stream is
the embedding and the logits are lm_head . rmsnorm(embedding); a one-token
prompt attends only to itself, so its attention output is V of the mapped
kv head exactly.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List

import numpy as np

from . import (add_bf16, argmax_bf16, embed_rows, gpu_reference_attention, matmul_bf16,
               rmsnorm_gpu, rope_gpu, swiglu)

LAYER_TENSORS = ("input_norm", "q", "k", "v", "o", "post_norm", "gate", "up", "down")


@dataclass
class Spec:
    layers: int
    hidden: int
    q_heads: int
    kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    rms_eps: float = 1e-5
    rope_theta: float = 500000.0
    llama3: int = 0
    rope_params: tuple = (1.0, 1.0, 2.0, 1.0)  # factor, low, high, original_max


@dataclass
class Session:
    keys: List[np.ndarray] = field(default_factory=list)    # per layer [T][KVH*D] bits
    values: List[np.ndarray] = field(default_factory=list)

    @property
    def tokens(self) -> int:
        return self.keys[0].shape[0] if self.keys else 0


class DecoderOracle:
    """Weights: dict of uint16 BF16 bit arrays keyed as the runner's ("embed",
    "final_norm", "lm_head", "layers.{l}.{name}"), laid out [out][in]."""

    def __init__(self, spec: Spec, weights: Dict[str, np.ndarray]):
        self.s = spec
        self.w = weights
        self.sessions: Dict[int, Session] = {}
        # Planted-mistake switches, off by default: tests turn them on to show
        # that a model-level tolerance separates plausible wiring errors.
        self.rope_shift = 0          # RoPE at position + rope_shift
        self.kv_head_reversed = False  # attend with the kv heads in reverse order

    def reset(self, seq: int) -> None:
        self.sessions[seq] = Session([np.zeros((0, self.s.kv_heads * self.s.head_dim), np.uint16)
                                      for _ in range(self.s.layers)],
                                     [np.zeros((0, self.s.kv_heads * self.s.head_dim), np.uint16)
                                      for _ in range(self.s.layers)])

    def _layer(self, l: int, x: np.ndarray, n: int, start: int, sess: Session) -> np.ndarray:
        s, w = self.s, self.w
        qd, kvd = s.q_heads * s.head_dim, s.kv_heads * s.head_dim
        g = lambda name: w[f"layers.{l}.{name}"]  # noqa: E731
        h = rmsnorm_gpu(x, g("input_norm"), n, s.hidden, s.rms_eps)
        q = matmul_bf16(g("q"), h, s.hidden, qd, n)
        k = matmul_bf16(g("k"), h, s.hidden, kvd, n)
        v = matmul_bf16(g("v"), h, s.hidden, kvd, n)
        pos = start + self.rope_shift
        q = rope_gpu(q, n, s.q_heads, s.head_dim, pos, s.rope_theta, s.llama3, *s.rope_params)
        k = rope_gpu(k, n, s.kv_heads, s.head_dim, pos, s.rope_theta, s.llama3, *s.rope_params)
        sess.keys[l] = np.concatenate([sess.keys[l], k.reshape(n, kvd)])
        sess.values[l] = np.concatenate([sess.values[l], v.reshape(n, kvd)])
        keys, values = sess.keys[l], sess.values[l]
        if self.kv_head_reversed:
            t = keys.shape[0]
            keys = keys.reshape(t, s.kv_heads, s.head_dim)[:, ::-1].reshape(t, kvd)
            values = values.reshape(t, s.kv_heads, s.head_dim)[:, ::-1].reshape(t, kvd)
        a = gpu_reference_attention(q, keys, values, s.q_heads, s.kv_heads, s.head_dim, n, start)
        x = add_bf16(x, matmul_bf16(g("o"), a, qd, s.hidden, n))
        h = rmsnorm_gpu(x, g("post_norm"), n, s.hidden, s.rms_eps)
        act = swiglu(matmul_bf16(g("gate"), h, s.hidden, s.intermediate, n),
                     matmul_bf16(g("up"), h, s.hidden, s.intermediate, n))
        return add_bf16(x, matmul_bf16(g("down"), act, s.intermediate, s.hidden, n))

    def hidden_rows(self, seq: int, ids) -> np.ndarray:
        """Appends `ids` to slot `seq` and returns the final residual rows."""
        if seq not in self.sessions:
            self.reset(seq)
        sess = self.sessions[seq]
        n, start = len(ids), sess.tokens
        x = embed_rows(self.w["embed"], ids, self.s.hidden).reshape(-1)
        for l in range(self.s.layers):
            x = self._layer(l, x, n, start, sess)
        return x.reshape(n, self.s.hidden)

    def logits(self, rows: np.ndarray) -> np.ndarray:
        s = self.s
        r = rows.shape[0]
        h = rmsnorm_gpu(rows.reshape(-1), self.w["final_norm"], r, s.hidden, s.rms_eps)
        return matmul_bf16(self.w["lm_head"], h, s.hidden, s.vocab, r).reshape(r, s.vocab)

    def prefill(self, seq: int, prompt) -> tuple:
        """(logits bits [vocab], greedy token) after the prompt; slot restarts."""
        self.reset(seq)
        x = self.hidden_rows(seq, list(prompt))
        lg = self.logits(x[-1:])
        return lg[0], int(argmax_bf16(lg, 1, self.s.vocab)[0])

    def step(self, seq: int, token: int) -> tuple:
        x = self.hidden_rows(seq, [token])
        lg = self.logits(x)
        return lg[0], int(argmax_bf16(lg, 1, self.s.vocab)[0])


def random_weights(spec: Spec, rng: np.random.Generator, scale: float = 0.08) -> Dict[str, np.ndarray]:
    """Seeded BF16 weights of the runner's layout: norms near 1, projections
    N(0, scale^2), embedding N(0, 1)."""
    from . import write_bf16

    def normal(shape, sc):
        return write_bf16(rng.standard_normal(shape, dtype=np.float32) * np.float32(sc)).reshape(shape)

    s = spec
    qd, kvd = s.q_heads * s.head_dim, s.kv_heads * s.head_dim
    w = {"embed": normal((s.vocab, s.hidden), 1.0),
         "final_norm": write_bf16(1.0 + 0.1 * rng.standard_normal(s.hidden, dtype=np.float32)),
         "lm_head": normal((s.vocab, s.hidden), scale)}
    shapes = {"q": (qd, s.hidden), "k": (kvd, s.hidden), "v": (kvd, s.hidden), "o": (s.hidden, qd),
              "gate": (s.intermediate, s.hidden), "up": (s.intermediate, s.hidden),
              "down": (s.hidden, s.intermediate)}
    for l in range(s.layers):
        for name in LAYER_TENSORS:
            if name.endswith("norm"):
                w[f"layers.{l}.{name}"] = write_bf16(1.0 + 0.1 * rng.standard_normal(s.hidden, dtype=np.float32))
            else:
                w[f"layers.{l}.{name}"] = normal(shapes[name], scale)
    return w
