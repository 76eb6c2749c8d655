"""ctypes binding of libbnhip.so's C ABI (include/bn_hip.h).

This is the reference-side binding a Python caller would use without the
``bten`` module: plain pointers and sizes in, a status code out, errors raised
as ``RuntimeError`` carrying ``bn_last_error()``.  Device buffers can come
from anything that hands out a device pointer (torch tensors here: torch is
only the allocator and stream provider).

There is no fallback: if libbnhip.so is missing, ``lib()`` raises.
"""
from __future__ import annotations

import ctypes as C
import math
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libbnhip.so")
HEADER = os.path.join(os.path.dirname(_HERE), "include", "bn_hip.h")

BN_OK, BN_ERR_INVALID_ARG, BN_ERR_SHAPE, BN_ERR_UNSUPPORTED = 0, 1, 2, 3
BN_ERR_HIP, BN_ERR_OOM, BN_ERR_NOT_DEVICE = 4, 5, 6
BN_F32, BN_BF16, BN_U32 = 0, 1, 2
BN_ADD, BN_SUB, BN_MUL, BN_EQ = 0, 1, 2, 3
BN_RELU, BN_SILU, BN_ADD_SCALAR, BN_MUL_SCALAR = 0, 1, 2, 3


class BnView(C.Structure):
    _fields_ = [("data", C.c_void_p), ("offset", C.c_int64), ("h", C.c_int32),
                ("w", C.c_int32), ("stride_h", C.c_int32), ("stride_w", C.c_int32),
                ("dtype", C.c_int32), ("on_device", C.c_int32)]


class BnPoolStats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("bytes_in_use", "peak_bytes_in_use",
                                          "bytes_reserved", "n_allocs", "n_frees", "n_live")]


class BnLlamaConfig(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layers", "hidden", "n_heads", "n_kv_heads",
                                       "intermediate", "vocab", "max_len")] + \
               [("rms_eps", C.c_float), ("rope_theta", C.c_float), ("weights_out_major", C.c_int)]


class BnLlamaLayer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("ln1", "wqkv", "wo", "ln2", "wgu", "wd",
                                          "k_cache", "v_cache")]


class BnError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(msg)
        self.status = status


_lib = None


def declared_symbols(header: str = HEADER):
    """Names of every function the public header declares."""
    text = open(header).read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char \*)\s*(bn_\w+)\(", text, re.M)))


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"libbnhip.so not built ({LIB_PATH}); run __graft_entry__.build()")
    try:  # share torch's HIP runtime when torch is present (one runtime per process)
        import torch  # noqa: F401
    except ImportError:
        pass
    L = C.CDLL(LIB_PATH)
    vp, V = C.c_void_p, C.POINTER(BnView)
    i, f, i64, sz = C.c_int, C.c_float, C.c_int64, C.c_size_t
    sig = {
        "bn_abi_version": ([], i), "bn_last_error": ([], C.c_char_p),
        "bn_init": ([i], i), "bn_device_count": ([C.POINTER(C.c_int)], i),
        "bn_stream_create": ([C.POINTER(vp)], i), "bn_stream_destroy": ([vp], i),
        "bn_stream_synchronize": ([vp], i), "bn_device_synchronize": ([], i),
        "bn_alloc": ([C.POINTER(vp), sz, vp], i), "bn_free": ([vp, vp], i),
        "bn_pool_get_stats": ([C.POINTER(BnPoolStats)], i), "bn_pool_reset_peak": ([], i),
        "bn_pool_trim": ([sz], i), "bn_pool_set_limit": ([sz], i),
        "bn_memcpy": ([vp, vp, sz, i, vp], i),
        "bn_rmsnorm": ([V, V, V, f, vp], i),
        "bn_rmsnorm_backward": ([V, V, V, V, V, f, vp], i),
        "bn_rope": ([V, V, i, i, f, vp], i), "bn_rope_backward": ([V, V, i, i, f, vp], i),
        "bn_rmsnorm_rope": ([V, V, V, f, i, i, f, vp], i),
        "bn_add_rmsnorm": ([V, V, V, V, V, f, vp], i), "bn_silu_mul": ([V, V, V, vp], i),
        "bn_softmax": ([V, V, i, i, vp], i), "bn_softmax_backward": ([V, V, V, vp], i),
        "bn_matmul": ([V, V, V, vp], i), "bn_repeat_kv": ([V, V, i, i, vp], i),
        "bn_fused_head_attention": ([V, V, V, V, i, i, i, f, i, i, vp], i),
        "bn_binary": ([i, V, V, V, vp], i), "bn_unary": ([i, V, f, V, vp], i),
        "bn_unary_backward": ([i, V, V, V, vp], i), "bn_fill": ([V, C.c_double, vp], i),
        "bn_sum": ([V, V, i, vp], i), "bn_argmax": ([V, V, vp], i), "bn_copy": ([V, V, vp], i),
        "bn_fill_uniform": ([V, f, f, C.c_uint64, vp], i),
        "bn_embedding": ([V, vp, i, V, vp], i),
        "bn_mem_get_info": ([C.POINTER(sz), C.POINTER(sz)], i),
        "bn_gqa_prefill": ([i, vp, vp, vp, vp] + [i] * 6 + [i64] * 6 + [f, i, i, vp], i),
        "bn_gqa_prefill_lse": ([i, vp, vp, vp, vp, vp] + [i] * 6 + [i64] * 6 + [f, i, i, vp], i),
        "bn_gqa_prefill_backward_workspace_size": ([i] * 7, sz),
        "bn_linear_rope_workspace_size": ([i] * 4, sz),
        "bn_linear_rope": ([V, V, V, i, i, i, f, vp, sz, vp], i),
        "bn_gqa_prefill_backward": ([i] + [vp] * 9 + [i] * 6 + [i64] * 6 + [f, i, i, vp, sz, vp], i),
        "bn_llama_decode_workspace_size": ([C.POINTER(BnLlamaConfig)], sz),
        "bn_llama_decode": ([C.POINTER(BnLlamaConfig), vp, vp, vp, C.POINTER(BnLlamaLayer),
                             i, i, i, vp, vp, sz, vp], i),
        "bn_gqa_decode_workspace_size": ([i, i, i, i], sz),
        "bn_gqa_decode": ([i, vp, vp, vp, vp, vp] + [i] * 5 + [f, vp, sz, vp], i),
        "bn_gqa_decode_noalloc": ([i, vp, vp, vp, vp, vp] + [i] * 5 + [f, vp], i),
        "bn_gqa_decode_strided": ([i, vp, vp, vp, vp, vp] + [i] * 5 + [i64] * 3 + [f, vp, sz, vp], i),
        "bn_gqa_decode_planned_workspace_size": ([i, i, i, i, i], sz),
        "bn_gqa_decode_planned": ([i, vp, vp, vp, vp, vp, vp] + [i] * 5 + [f, vp, sz, vp], i),
        "bn_gqa_decode_planned_strided": ([i, vp, vp, vp, vp, vp, vp] + [i] * 5 + [i64] * 3 +
                                          [f, vp, sz, vp], i),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return L


def check(status: int):
    if status != BN_OK:
        raise BnError(status, lib().bn_last_error().decode())


def call(name: str, *args):
    """Call a status-returning entry point; raise BnError on failure."""
    check(getattr(lib(), name)(*args))


def status_of(name: str, *args):
    """Call an entry point and return (status, message) without raising."""
    st = getattr(lib(), name)(*args)
    return st, (lib().bn_last_error().decode() if st else "")


# --------------------------------------------------------------- torch glue
def _torch_dtype_code(t):
    import torch
    return {torch.float32: BN_F32, torch.bfloat16: BN_BF16, torch.int32: BN_U32}[t.dtype]


def view(t, on_device=None) -> BnView:
    """bn_view of a 2-D torch tensor (any strides)."""
    assert t.dim() == 2
    dev = t.is_cuda if on_device is None else on_device
    return BnView(t.data_ptr(), 0, t.shape[0], t.shape[1], t.stride(0), t.stride(1),
                  _torch_dtype_code(t), int(dev))


def host_view(h, w, dtype=BN_F32, stride_h=None, stride_w=1, data=0x1000) -> BnView:
    """A host-memory view for validation tests (never dereferenced)."""
    return BnView(data, 0, h, w, w if stride_h is None else stride_h, stride_w, dtype, 0)


def stream_of(torch_stream=None):
    import torch
    s = torch.cuda.current_stream() if torch_stream is None else torch_stream
    return C.c_void_p(s.cuda_stream)


def gqa_prefill(q, k, v, o=None, scale=None, causal=True, seq_offset=0, stream=None):
    """q [B,Sq,H,D], k/v [B,Skv,Hkv,D] torch (f32 or bf16, rows contiguous)."""
    B, Sq, H, D = q.shape
    _, Skv, Hkv, _ = k.shape
    if o is None:
        import torch
        o = torch.empty_like(q)
    sc = 1.0 / math.sqrt(D) if scale is None else scale
    assert k.stride(1) == v.stride(1) and k.stride(0) == v.stride(0)
    call("bn_gqa_prefill", _torch_dtype_code(q), q.data_ptr(), k.data_ptr(), v.data_ptr(),
         o.data_ptr(), B, Sq, Skv, H, Hkv, D, q.stride(0), q.stride(1), k.stride(0),
         k.stride(1), o.stride(0), o.stride(1), sc, int(causal), seq_offset, stream_of(stream))
    return o


def fused_head_attention(q, k, v, n_heads, n_kv_heads, head_dim=64, o=None, scale=None,
                         causal=True, seq_offset=0, stream=None):
    """The fused-head chain in one launch: q [Sq, H*D], k/v [Sk, Hkv*D] fp32
    torch 2-D views -> o [Sq, H*D]."""
    if o is None:
        import torch
        o = torch.empty((q.shape[0], n_heads * head_dim), device=q.device, dtype=q.dtype)
    sc = 1.0 / math.sqrt(head_dim) if scale is None else scale
    call("bn_fused_head_attention", C.byref(view(q)), C.byref(view(k)), C.byref(view(v)),
         C.byref(view(o)), n_heads, n_kv_heads, head_dim, sc, int(causal), seq_offset,
         stream_of(stream))
    return o


def add_rmsnorm(x, delta, weight, eps, h=None, y=None, stream=None):
    """(h, y): h = x + delta, y = RMSNorm(h) * weight; h may be x (in place)."""
    import torch
    h = torch.empty_like(x) if h is None else h
    y = torch.empty_like(x) if y is None else y
    call("bn_add_rmsnorm", C.byref(view(x)), C.byref(view(delta)), C.byref(view(weight)),
         C.byref(view(h)), C.byref(view(y)), eps, stream_of(stream))
    return h, y


def silu_mul(gate, up, out=None, stream=None):
    """silu(gate) * up (SwiGLU activation)."""
    import torch
    out = torch.empty_like(gate) if out is None else out
    call("bn_silu_mul", C.byref(view(gate)), C.byref(view(up)), C.byref(view(out)), stream_of(stream))
    return out


def gqa_prefill_lse(q, k, v, o=None, lse=None, scale=None, causal=True, seq_offset=0, stream=None):
    """gqa_prefill that also returns lse [B, H, Sq] fp32 (natural-log row
    log-sum-exp of scale * q.k over the visible keys)."""
    import torch
    B, Sq, H, D = q.shape
    _, Skv, Hkv, _ = k.shape
    o = torch.empty_like(q) if o is None else o
    lse = torch.empty((B, H, Sq), device=q.device, dtype=torch.float32) if lse is None else lse
    sc = 1.0 / math.sqrt(D) if scale is None else scale
    assert k.stride(1) == v.stride(1) and k.stride(0) == v.stride(0) and lse.is_contiguous()
    call("bn_gqa_prefill_lse", _torch_dtype_code(q), q.data_ptr(), k.data_ptr(), v.data_ptr(),
         o.data_ptr(), lse.data_ptr(), B, Sq, Skv, H, Hkv, D, q.stride(0), q.stride(1),
         k.stride(0), k.stride(1), o.stride(0), o.stride(1), sc, int(causal), seq_offset,
         stream_of(stream))
    return o, lse


def gqa_prefill_backward(q, k, v, o, dout, lse, scale=None, causal=True, seq_offset=0,
                         dq=None, dk=None, dv=None, workspace=None, stream=None):
    """(dq, dk, dv) of gqa_prefill (bf16): o and lse from gqa_prefill_lse,
    dout the gradient of o.  dq shares q's strides, dk/dv share k's."""
    import torch
    B, Sq, H, D = q.shape
    _, Skv, Hkv, _ = k.shape
    dq = torch.empty_like(q) if dq is None else dq
    dk = torch.empty_like(k) if dk is None else dk
    dv = torch.empty_like(k) if dv is None else dv
    sc = 1.0 / math.sqrt(D) if scale is None else scale
    assert k.stride()[:2] == v.stride()[:2] == dk.stride()[:2] == dv.stride()[:2]
    assert q.stride()[:2] == dq.stride()[:2] and o.stride()[:2] == dout.stride()[:2]
    assert lse.is_contiguous() and lse.dtype == torch.float32
    ws, wsb = (None, 0) if workspace is None else (workspace.data_ptr(), workspace.numel() * workspace.element_size())
    call("bn_gqa_prefill_backward", _torch_dtype_code(q), q.data_ptr(), k.data_ptr(), v.data_ptr(),
         o.data_ptr(), dout.data_ptr(), lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
         B, Sq, Skv, H, Hkv, D, q.stride(0), q.stride(1), k.stride(0), k.stride(1), o.stride(0),
         o.stride(1), sc, int(causal), seq_offset, ws, wsb, stream_of(stream))
    return dq, dk, dv


def linear_rope(x, w, y=None, rope_cols=0, position_offset=0, head_dim=64, theta=10000.0,
                workspace=None, stream=None):
    """y = x @ w with RoPE on columns [0, rope_cols) (2-D torch, f32 or bf16)."""
    import torch
    y = torch.empty((x.shape[0], w.shape[1]), dtype=x.dtype, device=x.device) if y is None else y
    ws, wsb = (None, 0) if workspace is None else (workspace.data_ptr(), workspace.numel() * workspace.element_size())
    call("bn_linear_rope", C.byref(view(x)), C.byref(view(w)), C.byref(view(y)), rope_cols,
         position_offset, head_dim, theta, ws, wsb, stream_of(stream))
    return y


def gqa_decode(q, k_cache, v_cache, seq_lens, o=None, scale=None, workspace=None, stream=None):
    """q [B,H,D] and o contiguous, caches [B,Lmax,Hkv,D], seq_lens int32 [B]
    (device).  Contiguous caches take bn_gqa_decode; any other layout whose
    key rows are contiguous (e.g. the head-major storage
    ``torch.empty(B, Hkv, Lmax, D).transpose(1, 2)``) takes
    bn_gqa_decode_strided with the caches' strides (K and V alike)."""
    import torch
    B, H, D = q.shape
    _, Lmax, Hkv, _ = k_cache.shape
    if o is None:
        o = torch.empty_like(q)
    if not (q.is_contiguous() and o.is_contiguous()):
        raise ValueError("gqa_decode: q and o must be contiguous [B, H, D]")
    if tuple(v_cache.shape) != tuple(k_cache.shape) or v_cache.stride() != k_cache.stride():
        raise ValueError("gqa_decode: k_cache and v_cache must have the same shape and strides")
    sc = 1.0 / math.sqrt(D) if scale is None else scale
    ws_ptr, ws_bytes = (None, 0) if workspace is None else (workspace.data_ptr(),
                                                            workspace.numel() * workspace.element_size())
    if k_cache.is_contiguous():
        call("bn_gqa_decode", _torch_dtype_code(q), q.data_ptr(), k_cache.data_ptr(),
             v_cache.data_ptr(), seq_lens.data_ptr(), o.data_ptr(), B, Lmax, H, Hkv, D, sc,
             ws_ptr, ws_bytes, stream_of(stream))
        return o
    if k_cache.stride(3) != 1:
        raise ValueError("gqa_decode: cache key rows must be contiguous (stride 1 along head_dim)")
    call("bn_gqa_decode_strided", _torch_dtype_code(q), q.data_ptr(), k_cache.data_ptr(),
         v_cache.data_ptr(), seq_lens.data_ptr(), o.data_ptr(), B, Lmax, H, Hkv, D,
         k_cache.stride(0), k_cache.stride(2), k_cache.stride(1), sc, ws_ptr, ws_bytes,
         stream_of(stream))
    return o


def gqa_decode_planned(q, k_cache, v_cache, seq_lens, h_seq_lens, o=None, scale=None,
                       workspace=None, stream=None):
    """gqa_decode with the lengths also on the host (h_seq_lens: a sequence of
    ints, the values of the device tensor seq_lens): equal shares of the
    batch's tiles per compute unit when the lengths are ragged.  Caches as
    for gqa_decode: contiguous, or any layout with contiguous key rows
    (bn_gqa_decode_planned_strided)."""
    import numpy as np
    import torch
    B, H, D = q.shape
    _, Lmax, Hkv, _ = k_cache.shape
    if o is None:
        o = torch.empty_like(q)
    sc = 1.0 / math.sqrt(D) if scale is None else scale
    if not (q.is_contiguous() and o.is_contiguous()):
        raise ValueError("gqa_decode_planned: q and o must be contiguous [B, H, D]")
    if tuple(v_cache.shape) != tuple(k_cache.shape) or v_cache.stride() != k_cache.stride():
        raise ValueError("gqa_decode_planned: k_cache and v_cache must have the same shape and strides")
    hl = np.ascontiguousarray(np.asarray(h_seq_lens, dtype=np.int32))
    assert hl.shape == (B,)
    ws_ptr, ws_bytes = (None, 0) if workspace is None else (workspace.data_ptr(),
                                                            workspace.numel() * workspace.element_size())
    if k_cache.is_contiguous():
        call("bn_gqa_decode_planned", _torch_dtype_code(q), q.data_ptr(), k_cache.data_ptr(),
             v_cache.data_ptr(), seq_lens.data_ptr(), hl.ctypes.data, o.data_ptr(), B, Lmax, H, Hkv,
             D, sc, ws_ptr, ws_bytes, stream_of(stream))
        return o
    if k_cache.stride(3) != 1:
        raise ValueError("gqa_decode_planned: cache key rows must be contiguous (stride 1 along head_dim)")
    call("bn_gqa_decode_planned_strided", _torch_dtype_code(q), q.data_ptr(), k_cache.data_ptr(),
         v_cache.data_ptr(), seq_lens.data_ptr(), hl.ctypes.data, o.data_ptr(), B, Lmax, H, Hkv, D,
         k_cache.stride(0), k_cache.stride(2), k_cache.stride(1), sc, ws_ptr, ws_bytes,
         stream_of(stream))
    return o


def decode_workspace(B, Lmax, H, D=64):
    import torch
    n = lib().bn_gqa_decode_workspace_size(B, Lmax, H, D)
    return torch.empty(max(n, 4), dtype=torch.uint8, device="cuda")
