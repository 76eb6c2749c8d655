"""TinyLLaMA-1.1B forward with a KV cache, built on the attention path.

Drives config 4: 22 layers, hidden 2048, 32/4 GQA heads, head_dim 64,
SwiGLU 5632, vocab 32000, RMSNorm, RoPE theta 10000, fp32, random weights;
a prompt prefill followed by greedy decode steps.

The decoder layer follows the reference (src/llama/llama_layers.hpp:241-272,
src/llama/llama_model.hpp:52-80): x -> RMSNorm -> GQA -> +x -> RMSNorm ->
SwiGLU MLP -> +x, final RMSNorm, lm_head.  Each residual add runs fused with
the RMSNorm that follows it (bn_add_rmsnorm), and the SwiGLU activation
silu(gate) * up is one kernel (bn_silu_mul).  The reference keeps no KV cache
(llama_model.py:135-141 reruns the prefix); this driver keeps one per layer
([1, max_len, Hkv, 64]) and decodes the new token with the split-K decode
kernel.  Per-head GQA semantics (query head h reads KV head h // 8).

RMSNorm (plain and fused with the residual add), RoPE, prefill attention,
decode attention and the SwiGLU activation run on the HIP kernels through the
C ABI (bnhip).  The Q, K and V projections are one GEMM against the
concatenated weight [hidden, (H + 2*Hkv)*64]; attention reads Q, K and V as
column slices of its output.  Projection weights are stored output-major
([out, in] row-major, so each output's weights are contiguous); the model
holds them as the transposed [in, out] views, so x @ W reads as in the
reference.  Decode steps (rows <= SMALL_ROWS) run every projection -- QKV, O,
the concatenated gate/up, down and lm_head -- on bn_linear_rope's
output-major few-rows kernel (one pass over each weight, no k split), with
the Q/K rotation fused into the QKV projection; the prompt runs the library
GEMM (torch) and rotates the Q and K columns in place in one bn_rope launch.  The embedding gather is a torch GPU
operation.  The config's metric is the device time of the attention
(prefill and decode), standalone RoPE (the prompt's bn_rope) and RMSNorm
kernels; the decode steps' QKV projection, which carries their rotation in
its epilogue, is logged as its own kind (qkv_rope) and reported beside the
metric, not in it.  ``path_ms`` accumulates hip-event time around the logged
kernel launches (an upper bound on their device time; the rocprofv3 kernel
trace gives the exact per-kernel durations).
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass

import torch

import bnhip


@dataclass
class TinyLlamaConfig:
    vocab_size: int = 32000
    hidden_size: int = 2048
    intermediate_size: int = 5632
    num_hidden_layers: int = 22
    num_attention_heads: int = 32
    num_key_value_heads: int = 4
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0

    @property
    def head_dim(self):
        return self.hidden_size // self.num_attention_heads


class TinyLlama:
    # Rows up to which the projections run on bn_linear_rope's output-major
    # few-rows kernel (one pass over the weights, the QKV rotation in its
    # epilogue; it takes up to 4 rows).  Longer prompts take the library GEMM
    # and a separate RoPE launch: at 512 rows hipBLASLt's fp32 GEMM plus
    # bn_rope (45 + 4 us) beats the hand-written tiled kernel (66 us).
    SMALL_ROWS = 4

    def __init__(self, cfg: TinyLlamaConfig, max_len: int, seed: int = 1, std: float = 0.02,
                 dtype=torch.float32, out_major: bool = True):
        """out_major: projection weights stored [out, in] (default; decode steps
        take the output-major few-rows kernel) or [in, out] row-major (the
        split-k few-rows kernel); the same values either way."""
        if dtype != torch.float32:
            raise ValueError("config 4 is fp32")
        self.cfg = cfg
        self.max_len = max_len
        self.out_major = out_major
        g = torch.Generator(device="cuda").manual_seed(seed)
        h, kv, inter = cfg.hidden_size, cfg.num_key_value_heads * cfg.head_dim, cfg.intermediate_size

        def w(*shape):
            return torch.randn(shape, generator=g, device="cuda") * std

        def laid_out(m):
            # [in, out] values stored [out, in] (out_major); the model keeps the [in, out] view
            return m.t().contiguous().t() if out_major else m

        self.embed = w(cfg.vocab_size, h)
        self.layers = []
        for _ in range(cfg.num_hidden_layers):
            wq, wk, wv = w(h, h), w(h, kv), w(h, kv)
            wo = w(h, h)
            wg, wu = w(h, inter), w(h, inter)
            self.layers.append(dict(
                ln1=torch.ones((1, h), device="cuda"),
                wqkv=laid_out(torch.cat([wq, wk, wv], dim=1)), wo=laid_out(wo),
                ln2=torch.ones((1, h), device="cuda"), wgu=laid_out(torch.cat([wg, wu], dim=1)),
                wd=laid_out(w(inter, h)),
                k_cache=torch.zeros((1, max_len, cfg.num_key_value_heads, cfg.head_dim), device="cuda"),
                v_cache=torch.zeros((1, max_len, cfg.num_key_value_heads, cfg.head_dim), device="cuda")))
        self.ln_f = torch.ones((1, h), device="cuda")
        self.lm_head = laid_out(w(h, cfg.vocab_size))
        self.length = 0
        self.ws = bnhip.decode_workspace(1, max_len, cfg.num_attention_heads, cfg.head_dim)
        # row-major few-rows projections: split-k partial sums of the largest one
        shapes = [(h, h + 2 * kv), (h, h), (h, 2 * inter), (inter, h), (h, cfg.vocab_size)]
        n_ws = 0 if out_major else max(bnhip.lib().bn_linear_rope_workspace_size(0, self.SMALL_ROWS, n, k)
                                       for k, n in shapes)
        self.lin_ws = torch.empty(max(n_ws // 4, 1), device="cuda") if n_ws else None
        self.path_ms = 0.0
        self.timing = False
        self.trace = None  # list of (kernel, inputs, output, kw) when set
        # trace only the launches of the layers / positions this selects
        # (callable (layer, first position of the rows) -> bool; None: all)
        self.trace_select = None
        self._where = (0, 0)
        # list of (kind, launch, algorithmic work) when set; work is bytes for
        # the HBM-bound kinds and flops for prefill attention
        self.path_log = None

    # ------------------------------------------------------------ path kernels
    def _timed(self, fn, kind, work=0):
        """Runs a path-kernel launch; with path_log set (a list), also keeps
        (kind, fn, work) so the launches can be replayed from a captured graph
        and priced against their roofline."""
        if self.path_log is not None:
            self.path_log.append((kind, fn, work))
        if not self.timing:
            return fn()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        out = fn()
        e.record()
        self._events.append((s, e))
        return out

    def _tracing(self):
        return self.trace is not None and (self.trace_select is None or
                                           self.trace_select(*self._where))

    def _record(self, name, inputs, out, **kw):
        if self._tracing():
            torch.cuda.synchronize()
            kw = dict(kw, layer=self._where[0], pos0=self._where[1])
            self.trace.append((name, [t.detach().cpu().numpy().copy() for t in inputs],
                               out.detach().cpu().numpy().copy(), kw))

    def rmsnorm(self, x, weight):
        y = torch.empty_like(x)

        def run():
            bnhip.call("bn_rmsnorm", C.byref(bnhip.view(x)), C.byref(bnhip.view(weight)),
                       C.byref(bnhip.view(y)), self.cfg.rms_norm_eps, bnhip.stream_of())
        self._timed(run, "rmsnorm", 4 * (2 * x.numel() + weight.numel()))  # x in, y out
        self._record("rmsnorm", [x, weight], y, eps=self.cfg.rms_norm_eps)
        return y

    def add_rmsnorm(self, hdn, delta, weight):
        """hdn += delta in place; returns (hdn, RMSNorm(hdn) * weight)."""
        before = hdn.clone() if self._tracing() else None
        y = torch.empty_like(hdn)

        def run():
            bnhip.call("bn_add_rmsnorm", C.byref(bnhip.view(hdn)), C.byref(bnhip.view(delta)),
                       C.byref(bnhip.view(weight)), C.byref(bnhip.view(hdn)), C.byref(bnhip.view(y)),
                       self.cfg.rms_norm_eps, bnhip.stream_of())
        self._timed(run, "rmsnorm", 4 * (4 * hdn.numel() + weight.numel()))  # h, delta in; h, y out
        if self._tracing():
            self._record("add_rmsnorm", [before, delta, weight], torch.stack([hdn, y]),
                         eps=self.cfg.rms_norm_eps)
        return hdn, y

    def silu_mul(self, gate, up):
        out = torch.empty_like(gate)
        bnhip.call("bn_silu_mul", C.byref(bnhip.view(gate)), C.byref(bnhip.view(up)),
                   C.byref(bnhip.view(out)), bnhip.stream_of())
        return out

    def rope_(self, x, offset):
        """RoPE in place on a (possibly strided) [rows, heads*64] view."""
        before = x.clone() if self._tracing() else None

        def run():
            bnhip.call("bn_rope", C.byref(bnhip.view(x)), C.byref(bnhip.view(x)), offset,
                       self.cfg.head_dim, self.cfg.rope_theta, bnhip.stream_of())
        self._timed(run, "rope", 4 * 2 * x.numel())  # read and written in place
        self._record("rope", [before] if before is not None else [], x, offset=offset,
                     head_dim=self.cfg.head_dim, theta=self.cfg.rope_theta)
        return x

    def linear(self, x, w, rope_cols=0, pos0=0):
        """x @ w on the few-rows projection kernel; RoPE at positions pos0.. on
        the first rope_cols columns (the Q and K heads of the fused QKV)."""
        y = torch.empty((x.shape[0], w.shape[1]), device="cuda")

        def run():
            bnhip.linear_rope(x, w, y, rope_cols=rope_cols, position_offset=pos0,
                              head_dim=self.cfg.head_dim, theta=self.cfg.rope_theta,
                              workspace=self.lin_ws)
        if rope_cols:
            # carries the RoPE of the step; work = the projection's bytes
            self._timed(run, "qkv_rope", 4 * (x.numel() + w.numel() + y.numel()))
            self._record("linear_rope", [x, w], y, rope_cols=rope_cols, offset=pos0,
                         head_dim=self.cfg.head_dim, theta=self.cfg.rope_theta)
        else:
            run()
        return y

    def prefill_attention(self, q, k, v):
        cfg = self.cfg
        S = q.shape[0]
        q4 = q.view(1, S, cfg.num_attention_heads, cfg.head_dim)
        k4 = k.view(1, S, cfg.num_key_value_heads, cfg.head_dim)
        v4 = v.view(1, S, cfg.num_key_value_heads, cfg.head_dim)
        # causal QK^T and PV MACs x 2
        flops = 4 * cfg.num_attention_heads * cfg.head_dim * S * (S + 1) // 2
        o = self._timed(lambda: bnhip.gqa_prefill(q4, k4, v4, scale=1.0 / math.sqrt(cfg.head_dim)),
                        "prefill_attention", flops)
        self._record("prefill", [q4, k4, v4], o)
        return o.view(S, cfg.hidden_size)

    def decode_attention(self, q, layer, length):
        cfg = self.cfg
        q3 = q.view(1, cfg.num_attention_heads, cfg.head_dim)
        lens = torch.tensor([length], dtype=torch.int32, device="cuda")
        o = self._timed(lambda: bnhip.gqa_decode(q3, layer["k_cache"], layer["v_cache"], lens,
                                                 scale=1.0 / math.sqrt(cfg.head_dim),
                                                 workspace=self.ws), "decode_attention",
                        # fp32 K and V rows of the cached positions, q in, o out
                        4 * (2 * length * cfg.num_key_value_heads * cfg.head_dim +
                             2 * cfg.num_attention_heads * cfg.head_dim))
        self._record("decode", [q3, layer["k_cache"][:, :length], layer["v_cache"][:, :length]], o,
                     length=length)
        return o.view(1, cfg.hidden_size)

    # ------------------------------------------------------------ model
    def _attention(self, x, L, pos0):
        """Attention of one layer on the normalised rows x; returns o @ W_o."""
        cfg = self.cfg
        n = x.shape[0]
        hq, hk = cfg.hidden_size, cfg.num_key_value_heads * cfg.head_dim
        few = n <= self.SMALL_ROWS
        if few:                                   # [n, hq + 2*hk], Q and K rotated
            qkv = self.linear(x, L["wqkv"], hq + hk, pos0)
        else:
            qkv = x @ L["wqkv"]
            self.rope_(qkv[:, :hq + hk], pos0)    # Q and K columns, one launch
        q, k, v = qkv[:, :hq], qkv[:, hq:hq + hk], qkv[:, hq + hk:]
        L["k_cache"][0, pos0:pos0 + n] = k.view(n, cfg.num_key_value_heads, cfg.head_dim)
        L["v_cache"][0, pos0:pos0 + n] = v.view(n, cfg.num_key_value_heads, cfg.head_dim)
        if pos0 == 0:
            o = self.prefill_attention(q, k, v)
        else:
            o = self.decode_attention(q, L, pos0 + 1)
        return self.linear(o, L["wo"]) if few else o @ L["wo"]

    def _forward(self, hdn, pos0):
        """Decoder layers over rows hdn (positions pos0..); returns the final
        norm of every row.  Each residual add is fused with the RMSNorm that
        follows it (the next layer's input norm, or the final norm)."""
        self._where = (0, pos0)
        x = self.rmsnorm(hdn, self.layers[0]["ln1"])
        for i, L in enumerate(self.layers):
            self._where = (i, pos0)  # launches below belong to layer i
            hdn, x = self.add_rmsnorm(hdn, self._attention(x, L, pos0), L["ln2"])
            inter = self.cfg.intermediate_size
            if x.shape[0] <= self.SMALL_ROWS:
                gu = self.linear(x, L["wgu"])
                mlp = self.linear(self.silu_mul(gu[:, :inter], gu[:, inter:]), L["wd"])
            else:
                gu = x @ L["wgu"]
                mlp = self.silu_mul(gu[:, :inter], gu[:, inter:]) @ L["wd"]
            nxt = self.layers[i + 1]["ln1"] if i + 1 < len(self.layers) else self.ln_f
            hdn, x = self.add_rmsnorm(hdn, mlp, nxt)
        return x

    def prefill(self, ids: torch.Tensor) -> torch.Tensor:
        """Process the prompt (positions 0..S-1); returns last-row logits."""
        assert self.length == 0 and ids.numel() <= self.max_len
        xf = self._forward(self.embed[ids], 0)
        self.length = ids.numel()
        return xf[-1:] @ self.lm_head

    def step(self, token: torch.Tensor) -> torch.Tensor:
        """Append one token at position `length`; returns its logits."""
        assert self.length < self.max_len
        xf = self._forward(self.embed[token.view(1)], self.length)
        self.length += 1
        return self.linear(xf, self.lm_head)

    def generate(self, ids: torch.Tensor, new_tokens: int, time_path: bool = False):
        """Greedy decode; returns the generated ids and the path-kernel ms."""
        self.timing, self._events, self.path_ms = time_path, [], 0.0
        logits = self.prefill(ids)
        out = []
        for _ in range(new_tokens):
            tok = torch.argmax(logits[-1])
            out.append(tok)
            logits = self.step(tok)
        self.last_logits = logits  # of the last token fed (position length - 1)
        torch.cuda.synchronize()
        if time_path:
            self.path_ms = sum(s.elapsed_time(e) for s, e in self._events)
        self.timing = False
        return torch.stack(out), self.path_ms

    # ------------------------------------------------------- native decoding
    def native_config(self) -> bnhip.BnLlamaConfig:
        cfg = self.cfg
        return bnhip.BnLlamaConfig(cfg.num_hidden_layers, cfg.hidden_size, cfg.num_attention_heads,
                                   cfg.num_key_value_heads, cfg.intermediate_size, cfg.vocab_size,
                                   self.max_len, cfg.rms_norm_eps, cfg.rope_theta,
                                   int(self.out_major))

    def generate_native(self, ids: torch.Tensor, new_tokens: int):
        """Greedy decode with the decode loop in native code: the prompt runs
        through prefill(), then one bn_llama_decode call runs every decode
        step (embedding gather, layers, lm_head, argmax) on the current
        stream with no host round trip.  Same kernels in the same order as
        generate(), so the tokens and the KV caches match it exactly."""
        logits = self.prefill(ids)
        t0 = int(torch.argmax(logits[-1]))
        out = torch.empty(new_tokens + 1, dtype=torch.int32, device="cuda")
        out[0] = t0
        if new_tokens > 0:                        # out[1 + t] = argmax after step t
            self.decode_native(t0, new_tokens, out[1:])
        return out[:new_tokens].long()

    def decode_native(self, first_token: int, n_tokens: int, tokens_out: torch.Tensor):
        """n_tokens decode steps from position `length`: step t feeds
        first_token (t = 0) or the token step t-1 chose (tokens_out[t-1]) and
        writes its own argmax to tokens_out[t]."""
        cfg = self.cfg
        c = self.native_config()
        layers = (bnhip.BnLlamaLayer * cfg.num_hidden_layers)(*[
            bnhip.BnLlamaLayer(L["ln1"].data_ptr(), L["wqkv"].data_ptr(), L["wo"].data_ptr(),
                               L["ln2"].data_ptr(), L["wgu"].data_ptr(), L["wd"].data_ptr(),
                               L["k_cache"].data_ptr(), L["v_cache"].data_ptr())
            for L in self.layers])
        if not hasattr(self, "native_ws"):
            n = bnhip.lib().bn_llama_decode_workspace_size(C.byref(c))
            self.native_ws = torch.empty(max(n // 4, 1), device="cuda")
        assert tokens_out.dtype == torch.int32 and tokens_out.is_cuda and tokens_out.numel() >= n_tokens
        bnhip.call("bn_llama_decode", C.byref(c), self.embed.data_ptr(), self.ln_f.data_ptr(),
                   self.lm_head.data_ptr(), layers, first_token, self.length, n_tokens,
                   tokens_out.data_ptr(), self.native_ws.data_ptr(), self.native_ws.numel() * 4,
                   torch.cuda.current_stream().cuda_stream)
        self.length += n_tokens
