"""TinyLLaMA attention-path layers on the `bten` op surface.

The layer classes keep the reference's constructor arguments and call
sequence (mygrad/llama/llama_layers.py:13-191), so code written against the
reference layers runs on this build:

* ``RMSNorm.__call__``          -> ``x.rmsnorm(weight, eps)``            (:25-26)
* ``RotaryEmbedding.__call__``  -> ``x.rope(offset, head_dim, theta)``   (:40-42)
* ``GroupedQueryAttention``     -> the sequence of :154-186.

``GroupedQueryAttention`` has three modes:

``"fused_head"`` (default) computes the reference's attention: one causal
softmax over the full hidden width, ``softmax(0.125 * Q_rope @ K_rep^T) @ V_rep``
(every head shares one probability matrix), in one launch
(``bten.fused_head_attention``: no K_rep / V_rep and no S x S matrices).
``"fused_head_ops"`` runs the same chain op by op as the reference does
(``repeat_kv`` on the device instead of the reference's host round trip,
:105-138; then matmul, scale, softmax, matmul).

``"per_head"`` is grouped-query attention with one softmax per query head
(query head h reads KV head h // (H/Hkv)), computed by the fused
``bten.gqa_prefill`` kernel.

Weights are ``bten.TensorF`` of the reference's shapes (x @ W layout:
``q_proj`` [hidden, hidden], ``k_proj``/``v_proj`` [hidden, Hkv*D], ``o_proj``
[hidden, hidden]); ``load_weights`` replaces them after construction, as the
reference's ``load_checkpoint`` does (llama_model.py:200-215).
"""
from __future__ import annotations

import math

import numpy as np

import bten


def _tensor(a: np.ndarray, is_cuda: bool = True) -> "bten.TensorF":
    a = np.ascontiguousarray(a, dtype=np.float32)
    t = bten.TensorF(a.shape[0], a.shape[1], is_cuda)
    t.copy_from_numpy(a)
    return t


class RMSNorm:
    """y = x / sqrt(mean(x^2) + eps) * weight, weight initialised to ones."""

    def __init__(self, hidden_size: int, eps: float = 1e-6, is_cuda: bool = True):
        self.hidden_size = hidden_size
        self.eps = eps
        self.is_cuda = is_cuda
        self.weight = _tensor(np.ones((1, hidden_size), np.float32), is_cuda)

    def __call__(self, x):
        return x.rmsnorm(self.weight, self.eps)

    def parameters(self):
        return [self.weight]


class RotaryEmbedding:
    """Interleaved-pair rotary embedding applied per head_dim block."""

    def __init__(self, dim: int, max_position_embeddings: int = 2048, base: float = 10000.0):
        self.dim = dim
        self.max_position_embeddings = max_position_embeddings
        self.base = base

    def __call__(self, x, position_offset: int = 0):
        return x.rope(position_offset, self.dim, self.base)


class GroupedQueryAttention:
    """Attention of one TinyLLaMA layer on `bten` tensors (rows = tokens)."""

    def __init__(self, config, is_cuda: bool = True, mode: str = "fused_head",
                 seed: int | None = None, init_std: float | None = None):
        if mode not in ("fused_head", "fused_head_ops", "per_head"):
            raise ValueError("mode must be 'fused_head', 'fused_head_ops' or 'per_head'")
        self.config = config
        self.is_cuda = is_cuda
        self.mode = mode
        self.num_heads = config.num_attention_heads
        self.num_kv_heads = config.num_key_value_heads
        self.hidden_size = config.hidden_size
        self.head_dim = self.hidden_size // self.num_heads
        self.rotary_emb = RotaryEmbedding(self.head_dim, config.max_position_embeddings,
                                          config.rope_theta)
        self.scale = 1.0 / math.sqrt(self.head_dim)
        rng = np.random.default_rng(seed)
        kv = self.num_kv_heads * self.head_dim

        def init(i, o):
            std = math.sqrt(2.0 / (i + o)) if init_std is None else init_std
            return _tensor(rng.standard_normal((i, o)).astype(np.float32) * std, is_cuda)

        self.q_proj = init(self.hidden_size, self.hidden_size)
        self.k_proj = init(self.hidden_size, kv)
        self.v_proj = init(self.hidden_size, kv)
        self.o_proj = init(self.hidden_size, self.hidden_size)

    def load_weights(self, wq, wk, wv, wo):
        self.q_proj, self.k_proj = _tensor(wq, self.is_cuda), _tensor(wk, self.is_cuda)
        self.v_proj, self.o_proj = _tensor(wv, self.is_cuda), _tensor(wo, self.is_cuda)

    def __call__(self, hidden_states, position_offset: int = 0, use_causal_mask: bool = True):
        query = hidden_states @ self.q_proj
        key = hidden_states @ self.k_proj
        value = hidden_states @ self.v_proj
        query = self.rotary_emb(query, position_offset)
        key = self.rotary_emb(key, position_offset)
        if self.mode == "per_head":
            attn_output = bten.gqa_prefill(query, key, value, 1, self.num_heads,
                                           self.num_kv_heads, self.head_dim, self.scale,
                                           use_causal_mask, position_offset)
        elif self.mode == "fused_head":
            attn_output = bten.fused_head_attention(query, key, value, self.num_heads,
                                                    self.num_kv_heads, self.head_dim, self.scale,
                                                    use_causal_mask, position_offset)
        else:
            n_rep = self.num_heads // self.num_kv_heads
            if n_rep > 1:
                key = bten.repeat_kv(key, n_rep, self.head_dim)
                value = bten.repeat_kv(value, n_rep, self.head_dim)
            attn_scores = query @ key.T
            attn_scores = attn_scores * self.scale
            attn_probs = attn_scores.softmax(use_causal_mask, position_offset)
            attn_output = attn_probs @ value
        return attn_output @ self.o_proj

    def parameters(self):
        return [self.q_proj, self.k_proj, self.v_proj, self.o_proj]
