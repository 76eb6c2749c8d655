"""ctypes front-end of the CPU oracle (oracle/bn_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of bench.py, always as the checker / baseline.  The
product (``bten`` and ``libbnhip.so``) never imports this module.

All arrays are numpy float32 (int32 for lengths).  Functions take and return
dense row-major arrays; strided views are exercised through ``view()``.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libbn_oracle.so")
_lib = None


class OrView(C.Structure):
    _fields_ = [("p", C.POINTER(C.c_float)), ("offset", C.c_int64),
                ("h", C.c_int32), ("w", C.c_int32),
                ("stride_h", C.c_int32), ("stride_w", C.c_int32)]


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "all"], cwd=_HERE,
                       check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        V = OrView
        fp, ip = C.POINTER(C.c_float), C.POINTER(C.c_int32)
        i64 = C.c_int64
        L.or_rmsnorm.argtypes = [V, V, V, C.c_float]
        L.or_rmsnorm_backward.argtypes = [V, V, V, V, V, C.c_float]
        L.or_rope_freq.argtypes = [C.c_int, C.c_int, C.c_float]
        L.or_rope_freq.restype = C.c_float
        L.or_rope.argtypes = [V, V, C.c_int, C.c_int, C.c_float]
        L.or_rope_backward.argtypes = [V, V, C.c_int, C.c_int, C.c_float]
        L.or_rmsnorm_rope.argtypes = [V, V, V, C.c_float, C.c_int, C.c_int, C.c_float]
        L.or_softmax.argtypes = [V, V, C.c_int, C.c_int]
        L.or_softmax_backward.argtypes = [V, V, V]
        L.or_matmul.argtypes = [V, V, V]
        L.or_scale.argtypes = [V, C.c_float, V]
        L.or_repeat_kv.argtypes = [V, V, C.c_int, C.c_int]
        L.or_gqa_prefill.argtypes = [fp, fp, fp, fp] + [C.c_int] * 6 + [i64] * 6 + \
            [C.c_float, C.c_int, C.c_int, fp]
        L.or_gqa_decode.argtypes = [fp, fp, fp, ip, fp] + [C.c_int] * 5 + [C.c_float, fp]
        L.or_gqa_layer_scratch.argtypes = [C.c_int] * 4
        L.or_gqa_layer_scratch.restype = i64
        L.or_gqa_layer.argtypes = [fp, C.c_int, C.c_int, C.c_int, C.c_int, fp, fp, fp, fp,
                                   C.c_float, C.c_int, C.c_int, fp, fp]
        _lib = L
    return _lib


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a


def _ptr(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def view(a: np.ndarray, offset=0, h=None, w=None, stride_h=None, stride_w=1) -> OrView:
    """Strided view over a float32 buffer (kept alive by the caller)."""
    assert a.dtype == np.float32 and a.flags.c_contiguous
    if a.ndim == 1:
        a2w = a.shape[0]
    else:
        a2w = a.shape[-1]
    h = a.shape[0] if h is None else h
    w = a2w if w is None else w
    stride_h = a2w if stride_h is None else stride_h
    return OrView(_ptr(a), offset, h, w, stride_h, stride_w)


def _v(a):
    return view(a)


def rmsnorm(x, weight, eps=1e-6):
    x, weight = _f32(x), _f32(weight).reshape(1, -1)
    y = np.empty_like(x)
    lib().or_rmsnorm(_v(x), _v(weight), _v(y), eps)
    return y


def rmsnorm_backward(x, weight, dy, eps=1e-6):
    x, weight, dy = _f32(x), _f32(weight).reshape(1, -1), _f32(dy)
    dx = np.empty_like(x)
    dw = np.empty_like(weight)
    lib().or_rmsnorm_backward(_v(x), _v(weight), _v(dy), _v(dx), _v(dw), eps)
    return dx, dw


def add_rmsnorm(x, delta, weight, eps=1e-6):
    """Decoder-layer residual add then RMSNorm (llama_layers.hpp:241-272):
    h = x + delta elementwise in fp32 (op_add, op_elemwise.cuh:77-88 shape),
    y = rmsnorm(h) as op_rmsnorm computes it.  Returns (h, y)."""
    h = (_f32(x) + _f32(delta)).astype(np.float32)
    return h, rmsnorm(h, weight, eps)


def silu_mul(gate, up):
    """SwiGLU activation: SiLUFunc g / (1 + exp(-g)) (op_silu.cuh:8-14) on the
    gate, then the elementwise product with up (op_multiply), fp32."""
    g = _f32(gate)
    with np.errstate(over="ignore"):
        s = g / (np.float32(1) + np.exp(-g))
    return (s * _f32(up)).astype(np.float32)


def rope_freq(pair, head_dim, theta):
    return lib().or_rope_freq(pair, head_dim, theta)


def rope(x, position_offset=0, head_dim=64, theta=10000.0):
    x = _f32(x)
    y = np.empty_like(x)
    lib().or_rope(_v(x), _v(y), position_offset, head_dim, theta)
    return y


def rope_backward(dy, position_offset=0, head_dim=64, theta=10000.0):
    dy = _f32(dy)
    dx = np.empty_like(dy)
    lib().or_rope_backward(_v(dy), _v(dx), position_offset, head_dim, theta)
    return dx


def rmsnorm_rope(x, weight, eps=1e-6, position_offset=0, head_dim=64, theta=10000.0):
    x, weight = _f32(x), _f32(weight).reshape(1, -1)
    y = np.empty_like(x)
    lib().or_rmsnorm_rope(_v(x), _v(weight), _v(y), eps, position_offset, head_dim, theta)
    return y


def softmax(x, causal=False, seq_offset=0):
    x = _f32(x)
    y = np.empty_like(x)
    lib().or_softmax(_v(x), _v(y), int(causal), seq_offset)
    return y


def softmax_backward(y, dy):
    y, dy = _f32(y), _f32(dy)
    dx = np.empty_like(y)
    lib().or_softmax_backward(_v(y), _v(dy), _v(dx))
    return dx


def matmul(a, b):
    a, b = _f32(a), _f32(b)
    c = np.empty((a.shape[0], b.shape[1]), np.float32)
    lib().or_matmul(_v(a), _v(b), _v(c))
    return c


def linear_rope(x, w, rope_cols=0, position_offset=0, head_dim=64, theta=10000.0):
    """The Q/K/V projection followed by RoPE on its Q and K columns
    (llama_layers.hpp:72-81): y = x @ w -- op_mm (op_mm.cuh:23-36), here in
    fp64 and rounded to float32 -- then op_rope (or_rope, op_rope.cuh:55-99)
    on columns [0, rope_cols) at position position_offset + row.  Returns
    float32 [M, N]."""
    y = (np.asarray(x, np.float64) @ np.asarray(w, np.float64)).astype(np.float32)
    if rope_cols:
        y[:, :rope_cols] = rope(y[:, :rope_cols], position_offset, head_dim, theta)
    return y


def matmul_views(a: OrView, b: OrView, c: OrView):
    lib().or_matmul(a, b, c)


def scale(x, c):
    x = _f32(x)
    y = np.empty_like(x)
    lib().or_scale(_v(x), c, _v(y))
    return y


def repeat_kv(kv, head_dim, n_rep):
    kv = _f32(kv)
    out = np.empty((kv.shape[0], kv.shape[1] * n_rep), np.float32)
    lib().or_repeat_kv(_v(kv), _v(out), head_dim, n_rep)
    return out


def fused_head_attention(q, k, v, head_dim, n_rep, scale_c, causal=True, seq_offset=0):
    """The reference's fused-head chain (llama_layers.hpp:87-109) on the
    oracle's own ops: repeat_kv (:87-89), q @ k_rep^T (:96-98), * scale (:101),
    softmax(causal, seq_offset) (:105), @ v_rep (:108-109).  q [Sq, H*D],
    k/v [Sk, Hkv*D] float32 -> [Sq, H*D]."""
    k, v = _f32(k), _f32(v)
    kr = repeat_kv(k, head_dim, n_rep) if n_rep > 1 else k
    vr = repeat_kv(v, head_dim, n_rep) if n_rep > 1 else v
    s = scale(matmul(q, np.ascontiguousarray(kr.T)), scale_c)
    return matmul(softmax(s, causal, seq_offset), vr)


def gqa_prefill(q, k, v, scale, causal=True, seq_offset=0):
    """q [B,Sq,H,D], k/v [B,Skv,Hkv,D] float32 -> o [B,Sq,H,D]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, Sq, H, D = q.shape
    _, Skv, Hkv, _ = k.shape
    o = np.empty_like(q)
    scratch = np.empty(2 * Sq * Skv + 1, np.float32)
    lib().or_gqa_prefill(_ptr(q), _ptr(k), _ptr(v), _ptr(o), B, Sq, Skv, H, Hkv, D,
                         Sq * H * D, H * D, Skv * Hkv * D, Hkv * D, Sq * H * D, H * D,
                         scale, int(causal), seq_offset, _ptr(scratch))
    return o


def gqa_decode(q, k_cache, v_cache, seq_lens, scale):
    """q [B,H,D], caches [B,Lmax,Hkv,D], seq_lens [B] -> o [B,H,D]."""
    q, k_cache, v_cache = _f32(q), _f32(k_cache), _f32(v_cache)
    lens = np.ascontiguousarray(seq_lens, dtype=np.int32)
    B, H, D = q.shape
    _, Lmax, Hkv, _ = k_cache.shape
    o = np.empty_like(q)
    scratch = np.empty(2 * Lmax + 1, np.float32)
    lib().or_gqa_decode(_ptr(q), _ptr(k_cache), _ptr(v_cache),
                        lens.ctypes.data_as(C.POINTER(C.c_int32)), _ptr(o), B, Lmax, H,
                        Hkv, D, scale, _ptr(scratch))
    return o


def _visible(Sq, Skv, causal, seq_offset):
    """Mask of visible keys: key j for query row i iff j <= i + seq_offset
    (op_softmax.cuh:89-99) and j < Skv."""
    i = np.arange(Sq)[:, None]
    j = np.arange(Skv)[None, :]
    return (j <= i + seq_offset) if causal else np.ones((Sq, Skv), bool)


def gqa_prefill_lse(q, k, scale, causal=True, seq_offset=0):
    """Row log-sum-exp (natural log) of the scaled, masked scores per query head:
    lse[b, h, i] = log sum_{visible j} exp(scale * q_i . k_j), fp64; -inf for a
    row with no visible key.  Returns float64 [B, H, Sq]."""
    q, k = np.asarray(q, np.float64), np.asarray(k, np.float64)
    B, Sq, H, D = q.shape
    _, Skv, Hkv, _ = k.shape
    G = H // Hkv
    vis = _visible(Sq, Skv, causal, seq_offset)
    out = np.empty((B, H, Sq))
    for b in range(B):
        for h in range(H):
            s = scale * q[b, :, h] @ k[b, :, h // G].T
            s = np.where(vis, s, -np.inf)
            m = s.max(1, keepdims=True)
            mf = np.where(np.isfinite(m), m, 0.0)
            with np.errstate(divide="ignore"):
                out[b, h] = (mf + np.log(np.exp(s - mf).sum(1, keepdims=True)))[:, 0]
    return out


def gqa_prefill_backward(q, k, v, do, scale, causal=True, seq_offset=0):
    """Gradients of o = gqa_prefill(q, k, v) for the upstream gradient do,
    composed per query head h (KV head g = h // (H/Hkv)) from the backward of
    the reference chain's primitives: S = Q_h K_g^T, P = softmax(scale*S,
    causal, seq_offset); dP = dO_h V_g^T and dV_g += P^T dO_h (op_mm's
    backward); dS = P * (dP - rowsum(P * dP)) (op_softmax_backward,
    op_softmax.cuh:182-246); dQ_h = scale dS K_g, dK_g += scale dS^T Q_h (the
    scale, op_elemwise.cuh:436-451); repeat_kv's backward sums the G query
    heads of a KV head (llama_layers.hpp:159-163).  fp64; returns float32
    (dq, dk, dv) shaped like (q, k, v).  Rows with no visible key have P = 0."""
    q, k, v, do = (np.asarray(a, np.float64) for a in (q, k, v, do))
    B, Sq, H, D = q.shape
    _, Skv, Hkv, _ = k.shape
    G = H // Hkv
    vis = _visible(Sq, Skv, causal, seq_offset)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    for b in range(B):
        for h in range(H):
            g = h // G
            s = scale * q[b, :, h] @ k[b, :, g].T
            s = np.where(vis, s, -np.inf)
            m = s.max(1, keepdims=True)
            m = np.where(np.isfinite(m), m, 0.0)
            e = np.where(vis, np.exp(s - m), 0.0)
            tot = e.sum(1, keepdims=True)
            p = np.divide(e, tot, out=np.zeros_like(e), where=tot > 0)
            dp = do[b, :, h] @ v[b, :, g].T
            ds = p * (dp - (p * dp).sum(1, keepdims=True))
            dq[b, :, h] = scale * ds @ k[b, :, g]
            dk[b, :, g] += scale * ds.T @ q[b, :, h]
            dv[b, :, g] += p.T @ do[b, :, h]
    return dq.astype(np.float32), dk.astype(np.float32), dv.astype(np.float32)


def gqa_prefill_backward_from_residuals(q, k, v, o, lse, do, scale, causal=True, seq_offset=0,
                                        with_condition=False):
    """The same gradients as gqa_prefill_backward, computed from the forward's
    residuals (o and the natural-log row log-sum-exp lse [B,H,Sq]) as a
    flash-style backward does: P = exp(scale*Q_h K_g^T - lse) on the visible
    keys, and D = rowsum(dO_h * O_h) in place of rowsum(P * dP) -- equal
    because O_h = P V_g.  No reference counterpart (the reference keeps P);
    with exact o and lse it equals the chain form, which pins it.  fp64 on
    the given o and lse (which may carry bf16 rounding); float32 results.
    with_condition also returns the sums of absolute products behind each
    output element (scale |dS| |K|, scale |dS|^T |Q|, P^T |dO|): the factor
    that a rounding of the dot products' operands is multiplied by."""
    q, k, v, o, do = (np.asarray(a, np.float64) for a in (q, k, v, o, do))
    lse = np.asarray(lse, np.float64)
    B, Sq, H, D = q.shape
    _, Skv, Hkv, _ = k.shape
    G = H // Hkv
    vis = _visible(Sq, Skv, causal, seq_offset)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    mq, mk, mv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    for b in range(B):
        for h in range(H):
            g = h // G
            ok = vis & np.isfinite(lse[b, h])[:, None]
            with np.errstate(invalid="ignore", over="ignore"):
                p = np.where(ok, np.exp(scale * q[b, :, h] @ k[b, :, g].T - lse[b, h][:, None]), 0.0)
            dp = do[b, :, h] @ v[b, :, g].T
            ds = p * (dp - (do[b, :, h] * o[b, :, h]).sum(1, keepdims=True))
            dq[b, :, h] = scale * ds @ k[b, :, g]
            dk[b, :, g] += scale * ds.T @ q[b, :, h]
            dv[b, :, g] += p.T @ do[b, :, h]
            if with_condition:
                mq[b, :, h] = scale * np.abs(ds) @ np.abs(k[b, :, g])
                mk[b, :, g] += scale * np.abs(ds).T @ np.abs(q[b, :, h])
                mv[b, :, g] += p.T @ np.abs(do[b, :, h])
    grads = dq.astype(np.float32), dk.astype(np.float32), dv.astype(np.float32)
    return (grads, (mq, mk, mv)) if with_condition else grads


def gqa_layer(x, wq, wk, wv, wo, n_heads, n_kv_heads, theta=10000.0,
              position_offset=0, per_head=False):
    x = _f32(x)
    S, hidden = x.shape
    out = np.empty_like(x)
    n = lib().or_gqa_layer_scratch(S, hidden, n_heads, n_kv_heads)
    scratch = np.empty(n, np.float32)
    lib().or_gqa_layer(_ptr(x), S, hidden, n_heads, n_kv_heads, _ptr(_f32(wq)),
                       _ptr(_f32(wk)), _ptr(_f32(wv)), _ptr(_f32(wo)), theta,
                       position_offset, int(per_head), _ptr(out), _ptr(scratch))
    return out
