"""C-ABI checks that need no GPU: the library loads, exports every symbol the
public header declares, and rejects malformed requests during host-side
validation (before anything could be launched) with the reference's error
stems and the documented status codes."""
import ctypes as C

import pytest

import bnhip as B


def test_library_exports_every_declared_symbol():
    L = B.lib()
    names = B.declared_symbols()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    assert L.bn_abi_version() == 1


def st(name, *args):
    return B.status_of(name, *args)


def V(*a, **k):
    return C.byref(B.host_view(*a, **k))


def test_rmsnorm_validation_order_matches_reference():
    # shape errors first (op_rmsnorm.cuh:142-147), then the device (:148-150)
    s, m = st("bn_rmsnorm", V(4, 64), V(1, 32), V(4, 64), 1e-6, None)
    assert s == B.BN_ERR_SHAPE and m == "RMSNorm: weight shape must be (1, hidden_dim)"
    s, m = st("bn_rmsnorm", V(4, 64), V(1, 64), V(4, 63), 1e-6, None)
    assert s == B.BN_ERR_SHAPE and m == "RMSNorm: input/output shape mismatch"
    s, m = st("bn_rmsnorm", V(4, 64), V(1, 64), V(4, 64), 1e-6, None)
    assert s == B.BN_ERR_NOT_DEVICE and m == "RMSNorm: only GPU implementation available"


def test_rope_validation():
    s, m = st("bn_rope", V(4, 96), V(4, 96), 0, 64, 1e4, None)
    assert s == B.BN_ERR_SHAPE and m == "RoPE: hidden_dim must be divisible by head_dim"
    s, m = st("bn_rope", V(4, 64), V(3, 64), 0, 64, 1e4, None)
    assert s == B.BN_ERR_SHAPE and m == "RoPE: input/output shape mismatch"
    s, m = st("bn_rope", V(4, 63), V(4, 63), 0, 63, 1e4, None)
    assert s == B.BN_ERR_SHAPE  # odd head_dim has no pairs
    s, m = st("bn_rope", V(4, 64), V(4, 64), 0, 64, 1e4, None)
    assert s == B.BN_ERR_NOT_DEVICE and m == "RoPE: only GPU implementation available"
    s, _ = st("bn_rmsnorm_rope", V(4, 64), V(1, 64), V(4, 64), 1e-6, 0, 48, 1e4, None)
    assert s == B.BN_ERR_SHAPE


def test_softmax_and_matmul_validation():
    s, m = st("bn_softmax", V(4, 64), V(4, 65), 1, 0, None)
    assert s == B.BN_ERR_SHAPE and m == "Softmax: input/output shape mismatch"
    s, m = st("bn_softmax", V(4, 64), V(4, 64), 1, 0, None)
    assert s == B.BN_ERR_NOT_DEVICE and m == "Softmax: only GPU implementation available"
    s, m = st("bn_matmul", V(4, 8), V(9, 3), V(4, 3), None)
    assert s == B.BN_ERR_SHAPE and m.startswith("a,b,out tensor shape mismatch")
    s, m = st("bn_matmul", V(4, 8), V(8, 3), V(4, 3), None)
    assert s == B.BN_ERR_NOT_DEVICE


def test_dtype_and_null_checks():
    s, _ = st("bn_rmsnorm", None, V(1, 64), V(4, 64), 1e-6, None)
    assert s == B.BN_ERR_INVALID_ARG
    s, _ = st("bn_matmul", V(4, 8, dtype=B.BN_BF16), V(8, 3), V(4, 3), None)
    assert s == B.BN_ERR_UNSUPPORTED
    s, _ = st("bn_rmsnorm", V(4, 64, dtype=B.BN_BF16), V(1, 64), V(4, 64), 1e-6, None)
    assert s == B.BN_ERR_UNSUPPORTED
    s, _ = st("bn_binary", 9, V(2, 2), V(2, 2), V(2, 2), None)
    assert s == B.BN_ERR_INVALID_ARG
    s, m = st("bn_binary", B.BN_ADD, V(2, 3), V(3, 2), V(2, 3), None)
    assert s == B.BN_ERR_SHAPE and m == "a,b shape mismatch"


def prefill_args(**kw):
    a = dict(dtype=B.BN_BF16, q=0x1000, k=0x2000, v=0x3000, o=0x4000, batch=4, seq_q=2048,
             seq_kv=2048, H=32, Hkv=4, D=64, qbs=2048 * 2048, qrs=2048, kvbs=2048 * 256,
             kvrs=256, obs=2048 * 2048, ors=2048, scale=0.125, causal=1, off=0)
    a.update(kw)
    return (a["dtype"], a["q"], a["k"], a["v"], a["o"], a["batch"], a["seq_q"], a["seq_kv"],
            a["H"], a["Hkv"], a["D"], a["qbs"], a["qrs"], a["kvbs"], a["kvrs"], a["obs"],
            a["ors"], a["scale"], a["causal"], a["off"], None)


@pytest.mark.parametrize("kw,status", [
    (dict(H=30), B.BN_ERR_SHAPE),               # H % Hkv != 0
    (dict(Hkv=0), B.BN_ERR_SHAPE),
    (dict(D=128), B.BN_ERR_UNSUPPORTED),
    (dict(dtype=B.BN_U32), B.BN_ERR_UNSUPPORTED),
    (dict(seq_q=-1), B.BN_ERR_SHAPE),
    (dict(qrs=1024), B.BN_ERR_SHAPE),           # row stride < H*D
    (dict(kvbs=100), B.BN_ERR_SHAPE),           # batch stride < S*row stride
    (dict(q=0x1004), B.BN_ERR_UNSUPPORTED),     # misaligned
    (dict(kvrs=260, kvbs=2048 * 264), B.BN_ERR_UNSUPPORTED),  # stride not 16-byte multiple
    (dict(q=0), B.BN_ERR_INVALID_ARG),
    (dict(scale=-1.0), B.BN_ERR_INVALID_ARG),
    (dict(scale=float("nan")), B.BN_ERR_INVALID_ARG),
    (dict(seq_kv=8, kvrs=1 << 24, kvbs=8 << 24), B.BN_ERR_UNSUPPORTED),  # bf16 K/V stride >= 2^24
])
def test_prefill_validation(kw, status):
    s, m = st("bn_gqa_prefill", *prefill_args(**kw))
    assert s == status, m
    assert m.startswith("GQA prefill:")


def test_prefill_empty_is_noop():
    assert st("bn_gqa_prefill", *prefill_args(batch=0))[0] == B.BN_OK
    assert st("bn_gqa_prefill", *prefill_args(seq_q=0))[0] == B.BN_OK


@pytest.mark.parametrize("kw,status", [
    (dict(H=24), B.BN_ERR_UNSUPPORTED),   # 6 heads per KV head
    (dict(H=30), B.BN_ERR_SHAPE),
    (dict(D=32), B.BN_ERR_UNSUPPORTED),
    (dict(L=0), B.BN_ERR_SHAPE),
    (dict(lens=0), B.BN_ERR_INVALID_ARG),
    (dict(q=0x1008), B.BN_ERR_UNSUPPORTED),
    (dict(ws=0x9000, wsb=16), B.BN_ERR_INVALID_ARG),  # workspace too small
])
def test_decode_validation(kw, status):
    a = dict(dt=B.BN_BF16, q=0x1000, k=0x2000, v=0x3000, lens=0x5000, o=0x4000, B=64,
             L=4096, H=32, Hkv=4, D=64, sc=0.125, ws=None, wsb=0)
    a.update(kw)
    s, m = st("bn_gqa_decode", a["dt"], a["q"], a["k"], a["v"], a["lens"], a["o"], a["B"],
              a["L"], a["H"], a["Hkv"], a["D"], a["sc"], a["ws"], a["wsb"], None)
    assert s == status, m
    assert m.startswith("GQA decode:")


@pytest.mark.parametrize("kw,status", [
    (dict(H=24), B.BN_ERR_UNSUPPORTED),
    (dict(D=32), B.BN_ERR_UNSUPPORTED),
    (dict(lens=0), B.BN_ERR_INVALID_ARG),
    (dict(q=0x1008), B.BN_ERR_UNSUPPORTED),
])
def test_decode_noalloc_validation(kw, status):
    # the no-allocation variant validates exactly as bn_gqa_decode does
    a = dict(dt=B.BN_BF16, q=0x1000, k=0x2000, v=0x3000, lens=0x5000, o=0x4000, B=64,
             L=4096, H=32, Hkv=4, D=64, sc=0.125)
    a.update(kw)
    s, m = st("bn_gqa_decode_noalloc", a["dt"], a["q"], a["k"], a["v"], a["lens"], a["o"],
              a["B"], a["L"], a["H"], a["Hkv"], a["D"], a["sc"], None)
    assert s == status, m
    assert m.startswith("GQA decode (no allocation):")


@pytest.mark.parametrize("kw,status", [
    (dict(bs=0), B.BN_ERR_INVALID_ARG),
    (dict(hs=-64), B.BN_ERR_INVALID_ARG),
    (dict(rs=60), B.BN_ERR_INVALID_ARG),                    # rows not 16-byte aligned (bf16)
    (dict(dt=B.BN_F32, rs=66), B.BN_ERR_INVALID_ARG),       # nor in fp32
    (dict(hs=1 << 41), B.BN_ERR_INVALID_ARG),
    (dict(H=24), B.BN_ERR_UNSUPPORTED),                     # the shape checks of bn_gqa_decode
    (dict(lens=0), B.BN_ERR_INVALID_ARG),
    (dict(ws=0x9000, wsb=16), B.BN_ERR_INVALID_ARG),
])
def test_decode_strided_validation(kw, status):
    # head-major [64, 4, 4096, 64] strides unless changed; fake pointers, no GPU
    a = dict(dt=B.BN_BF16, q=0x1000, k=0x2000, v=0x3000, lens=0x5000, o=0x4000, B=64,
             L=4096, H=32, Hkv=4, D=64, bs=4 * 4096 * 64, hs=4096 * 64, rs=64, sc=0.125,
             ws=None, wsb=0)
    a.update(kw)
    s, m = st("bn_gqa_decode_strided", a["dt"], a["q"], a["k"], a["v"], a["lens"], a["o"],
              a["B"], a["L"], a["H"], a["Hkv"], a["D"], a["bs"], a["hs"], a["rs"], a["sc"],
              a["ws"], a["wsb"], None)
    assert s == status, m
    assert m.startswith("GQA decode (strided):"), m


def test_decode_strided_fp32_alignment():
    """fp32 rows need 4-element strides, bf16 rows 8: a stride of 4 passes the
    fp32 check and fails the bf16 one (the fp32 call then stops at the NULL
    lengths, before any device work)."""
    args = lambda dt: (dt, 0x1000, 0x2000, 0x3000, 0, 0x4000, 1, 256, 8, 1, 64, 4 * 256, 4, 64,
                       0.125, None, 0, None)
    s, m = st("bn_gqa_decode_strided", *args(B.BN_BF16))
    assert s == B.BN_ERR_INVALID_ARG and "multiples of 8 elements" in m, m
    s, m = st("bn_gqa_decode_strided", *args(B.BN_F32))
    assert s == B.BN_ERR_INVALID_ARG and "NULL pointer" in m, m


@pytest.mark.parametrize("kw,status,stem", [
    (dict(hl=0), B.BN_ERR_INVALID_ARG, "GQA decode (planned): NULL host lengths"),
    (dict(ws=0x9000, wsb=16), B.BN_ERR_INVALID_ARG, "GQA decode (planned): workspace of 16 bytes"),
    (dict(H=24), B.BN_ERR_UNSUPPORTED, "GQA decode: "),   # every other check is bn_gqa_decode's
    (dict(lens=0), B.BN_ERR_INVALID_ARG, "GQA decode: "),
    (dict(q=0x1008), B.BN_ERR_UNSUPPORTED, "GQA decode: "),
])
def test_decode_planned_validation(kw, status, stem):
    a = dict(dt=B.BN_BF16, q=0x1000, k=0x2000, v=0x3000, lens=0x5000, hl=0x6000, o=0x4000, B=64,
             L=4096, H=32, Hkv=4, D=64, sc=0.125, ws=None, wsb=0)
    a.update(kw)
    s, m = st("bn_gqa_decode_planned", a["dt"], a["q"], a["k"], a["v"], a["lens"], a["hl"], a["o"],
              a["B"], a["L"], a["H"], a["Hkv"], a["D"], a["sc"], a["ws"], a["wsb"], None)
    assert s == status, m
    assert m.startswith(stem), m


def test_decode_planned_strided_validation():
    # bad strides leave the plan and fail in bn_gqa_decode_strided's checks (fake pointers)
    args = (B.BN_BF16, 0x1000, 0x2000, 0x3000, 0x5000, 0x6000, 0x4000, 64, 4096, 32, 4, 64,
            4 * 4096 * 64, 4096 * 64, 60, 0.125, None, 0, None)
    s, m = st("bn_gqa_decode_planned_strided", *args)
    assert s == B.BN_ERR_INVALID_ARG and m.startswith("GQA decode (strided): cache strides"), m
    s, m = st("bn_gqa_decode_planned_strided", *args[:5], 0, *args[6:])
    assert s == B.BN_ERR_INVALID_ARG and m == "GQA decode (planned): NULL host lengths", m


def test_decode_planned_workspace_size():
    L = B.lib()
    # config 3: the unplanned fallback's partials exceed the plan's records
    assert L.bn_gqa_decode_planned_workspace_size(64, 4096, 32, 4, 64) == \
        L.bn_gqa_decode_workspace_size(64, 4096, 32, 64)
    # short caches: the records are larger -- (64*4 + 256) parts, each 8 heads x 64
    # acc words plus 8 m and 8 l words, 8-byte epoch-tagged
    assert L.bn_gqa_decode_planned_workspace_size(64, 128, 32, 4, 64) == (64 * 4 + 256) * (8 * 64 + 16) * 8
    assert L.bn_gqa_decode_planned_workspace_size(64, 128, 32, 4, 32) == 0
    assert L.bn_gqa_decode_planned_workspace_size(64, 128, 30, 4, 64) == 0


def test_decode_noalloc_refuses_partials_above_scratch():
    """fp32 split path: 16 sequences of 2^20 keys in 1024-key chunks need
    16*32*1024*66*4 bytes of partials, above the 32 MiB array; the refusal
    happens on the host before any device call (fake pointers, no GPU)."""
    s, m = st("bn_gqa_decode_noalloc", B.BN_F32, 0x1000, 0x2000, 0x3000, 0x5000, 0x4000,
              16, 1 << 20, 32, 4, 64, 0.125, None)
    assert s == B.BN_ERR_UNSUPPORTED, m
    assert m == ("GQA decode (no allocation): the call needs 138412032 bytes of chunk "
                 "partials, above the 33554432-byte scratch"), m
    assert 16 * 32 * 1024 * 66 * 4 == 138412032


def test_decode_workspace_size():
    L = B.lib()
    n = L.bn_gqa_decode_workspace_size(64, 4096, 32, 64)
    assert n == 64 * 32 * 32 * 66 * 4
    assert L.bn_gqa_decode_workspace_size(64, 4096, 32, 128) == 0
    # short caches (at most 1024 keys, at most 256 sequence x query-head
    # pairs: the fp32 short-cache split) keep at least 4 split records per pair
    assert L.bn_gqa_decode_workspace_size(1, 256, 32, 64) == 1 * 32 * 4 * 66 * 4
    assert L.bn_gqa_decode_workspace_size(1, 640, 32, 64) == 1 * 32 * 5 * 66 * 4
    assert L.bn_gqa_decode_workspace_size(4, 1024, 64, 64) == 4 * 64 * 8 * 66 * 4
    assert L.bn_gqa_decode_workspace_size(1, 1025, 32, 64) == 1 * 32 * 9 * 66 * 4
    assert L.bn_gqa_decode_workspace_size(9, 256, 32, 64) == 9 * 32 * 2 * 66 * 4


def test_pool_bookkeeping_without_device():
    s = B.BnPoolStats()
    B.call("bn_pool_get_stats", C.byref(s))
    assert s.n_live == s.n_allocs - s.n_frees
    # freeing a pointer the pool never handed out is an argument error
    code, msg = st("bn_free", C.c_void_p(0x1234), None)
    assert code == B.BN_ERR_INVALID_ARG and "not allocated" in msg
    assert st("bn_free", None, None)[0] == B.BN_OK
    assert st("bn_memcpy", None, C.c_void_p(8), 8, 0, None)[0] == B.BN_ERR_INVALID_ARG
    assert st("bn_memcpy", C.c_void_p(8), C.c_void_p(8), 8, 7, None)[0] == B.BN_ERR_INVALID_ARG


def backward_args(**kw):
    a = dict(dtype=B.BN_BF16, q=0x1000, k=0x2000, v=0x3000, o=0x4000, do=0x5000, lse=0x6000,
             dq=0x7000, dk=0x8000, dv=0x9000, batch=4, seq_q=2048, seq_kv=2048, H=32, Hkv=4,
             D=64, qbs=2048 * 2048, qrs=2048, kvbs=2048 * 256, kvrs=256, obs=2048 * 2048,
             ors=2048, scale=0.125, causal=1, off=0, ws=None, wsb=0)
    a.update(kw)
    return tuple(a[n] for n in ("dtype", "q", "k", "v", "o", "do", "lse", "dq", "dk", "dv",
                                "batch", "seq_q", "seq_kv", "H", "Hkv", "D", "qbs", "qrs",
                                "kvbs", "kvrs", "obs", "ors", "scale", "causal", "off", "ws",
                                "wsb")) + (None,)


@pytest.mark.parametrize("kw,status", [
    (dict(dtype=B.BN_F32), B.BN_ERR_UNSUPPORTED),
    (dict(H=30), B.BN_ERR_SHAPE),
    (dict(D=128), B.BN_ERR_UNSUPPORTED),
    (dict(seq_kv=-1), B.BN_ERR_SHAPE),
    (dict(ors=1024), B.BN_ERR_SHAPE),
    (dict(kvbs=100), B.BN_ERR_SHAPE),
    (dict(dk=0x8008), B.BN_ERR_UNSUPPORTED),
    (dict(lse=0x6002), B.BN_ERR_UNSUPPORTED),
    (dict(lse=0), B.BN_ERR_INVALID_ARG),
    (dict(do=0), B.BN_ERR_INVALID_ARG),
    (dict(scale=0.0), B.BN_ERR_INVALID_ARG),
    (dict(ws=0xA000, wsb=4 * 32 * 2048 * 4 - 4), B.BN_ERR_INVALID_ARG),  # workspace too small
])
def test_prefill_backward_validation(kw, status):
    s, m = st("bn_gqa_prefill_backward", *backward_args(**kw))
    assert s == status, m
    assert m.startswith("GQA prefill backward:")


def test_prefill_backward_workspace_size_and_empty():
    L = B.lib()
    # config 2, causal: D (fp32 per query row) + fp32 dK/dV partials of 4
    # two-head chunks (one-head chunks would pass 0.5 byte per 1000 flops)
    assert L.bn_gqa_prefill_backward_workspace_size(4, 2048, 2048, 32, 4, 64, 1) == \
        4 * 32 * 2048 * 4 + 4 * 4 * 4 * 2 * 2048 * 64 * 4
    # non-causal: 512 workgroups are enough, 4-head chunks
    assert L.bn_gqa_prefill_backward_workspace_size(4, 2048, 2048, 32, 4, 64, 0) == \
        4 * 32 * 2048 * 4 + 4 * 4 * 2 * 2 * 2048 * 64 * 4
    # one query head per KV head: no partials; D rounded up to 256 bytes
    assert L.bn_gqa_prefill_backward_workspace_size(1, 100, 100, 8, 8, 64, 1) == 3328
    assert L.bn_gqa_prefill_backward_workspace_size(0, 2048, 2048, 32, 4, 64, 1) == 0
    assert L.bn_gqa_prefill_backward_workspace_size(4, 2048, 2048, 32, 4, 128, 1) == 0
    assert st("bn_gqa_prefill_backward", *backward_args(batch=0))[0] == B.BN_OK
    assert st("bn_gqa_prefill_backward", *backward_args(seq_q=0, seq_kv=0))[0] == B.BN_OK


def test_prefill_lse_validation():
    args = list(prefill_args())
    s, m = st("bn_gqa_prefill_lse", *args[:5], None, *args[5:])
    assert s == B.BN_ERR_INVALID_ARG and m.startswith("GQA prefill:")
    s, m = st("bn_gqa_prefill_lse", *args[:5], 0x6002, *args[5:])
    assert s == B.BN_ERR_UNSUPPORTED


def test_linear_rope_validation():
    F, H = B.BN_F32, B.BN_BF16
    ok = (V(4, 64), V(64, 128), V(4, 128))
    s, m = st("bn_linear_rope", V(4, 64), V(32, 128), V(4, 128), 0, 0, 64, 1e4, None, 0, None)
    assert s == B.BN_ERR_SHAPE and m.startswith("Linear: shape mismatch")
    s, m = st("bn_linear_rope", V(4, 64), V(64, 128, dtype=H), V(4, 128), 0, 0, 64, 1e4, None, 0, None)
    assert s == B.BN_ERR_UNSUPPORTED and "one dtype" in m
    s, m = st("bn_linear_rope", *ok, 96, 0, 64, 1e4, None, 0, None)
    assert s == B.BN_ERR_SHAPE and "rope_cols" in m
    s, m = st("bn_linear_rope", *ok, 256, 0, 64, 1e4, None, 0, None)
    assert s == B.BN_ERR_SHAPE
    s, m = st("bn_linear_rope", *ok, 64, 0, 63, 1e4, None, 0, None)
    assert s == B.BN_ERR_SHAPE and "head_dim" in m
    s, m = st("bn_linear_rope", V(4, 64, stride_w=2, stride_h=128), V(64, 128), V(4, 128), 0, 0, 64,
              1e4, None, 0, None)
    assert s == B.BN_ERR_UNSUPPORTED and "contiguous" in m
    s, m = st("bn_linear_rope", V(4, 66), V(66, 128), V(4, 128), 0, 0, 64, 1e4, None, 0, None)
    assert s == B.BN_ERR_UNSUPPORTED  # k not a multiple of 16 bytes
    s, m = st("bn_linear_rope", *ok, 64, 0, 64, 1e4, None, 0, None)
    assert s == B.BN_ERR_NOT_DEVICE and m == "Linear: only GPU implementation available"


def test_linear_rope_output_major_validation():
    # w viewed [k, n] with stride_h 1: the output-major few-rows kernel; its
    # limits are checked before the device
    wt = lambda k, n, sw=None: V(k, n, stride_h=1, stride_w=k if sw is None else sw)
    # fp32 with more than 4 rows takes the many-rows matrix-core kernel (only
    # the device is missing here); bf16 stays within the few-rows kernel
    s, m = st("bn_linear_rope", V(5, 256), wt(256, 128), V(5, 128), 0, 0, 64, 1e4, None, 0, None)
    assert s == B.BN_ERR_NOT_DEVICE, m
    bw = lambda k, n: V(k, n, dtype=B.BN_BF16, stride_h=1, stride_w=k)
    s, m = st("bn_linear_rope", V(5, 256, dtype=B.BN_BF16), bw(256, 128), V(5, 128, dtype=B.BN_BF16), 0, 0,
              64, 1e4, None, 0, None)
    assert s == B.BN_ERR_UNSUPPORTED and "at most 4 rows" in m
    s, m = st("bn_linear_rope", V(1, 256), wt(256, 127), V(1, 127), 0, 0, 64, 1e4, None, 0, None)
    assert s == B.BN_ERR_UNSUPPORTED and "even output width" in m
    # y is stored one element at a time: a row stride that is not a multiple
    # of 16 bytes passes the layout checks (host views stop at the device check)
    s, m = st("bn_linear_rope", V(2, 256), wt(256, 126), V(2, 126), 0, 0, 64, 1e4, None, 0, None)
    assert s == B.BN_ERR_NOT_DEVICE
    s, m = st("bn_linear_rope", V(1, 256), wt(256, 128, 258), V(1, 128), 0, 0, 64, 1e4, None, 0, None)
    assert s == B.BN_ERR_UNSUPPORTED  # stride between outputs not a multiple of 16 bytes
    s, m = st("bn_linear_rope", V(2, 16384), wt(16384, 64), V(2, 64), 0, 0, 64, 1e4, None, 0, None)
    assert s == B.BN_ERR_UNSUPPORTED and "staged x elements" in m
    # three rows run the four-row instance: 4 x 4608 staged elements exceed the
    # budget although 3 x 4608 would not; one and two rows of 4608 fit
    s, m = st("bn_linear_rope", V(3, 4608), wt(4608, 64), V(3, 64), 0, 0, 64, 1e4, None, 0, None)
    assert s == B.BN_ERR_UNSUPPORTED and "staged x elements" in m
    s, m = st("bn_linear_rope", V(2, 4608), wt(4608, 64), V(2, 64), 0, 0, 64, 1e4, None, 0, None)
    assert s == B.BN_ERR_NOT_DEVICE
    s, m = st("bn_linear_rope", V(4, 256), wt(256, 128), V(4, 128), 64, 3, 64, 1e4, None, 0, None)
    assert s == B.BN_ERR_NOT_DEVICE and m == "Linear: only GPU implementation available"


def test_linear_rope_workspace_size():
    L = B.lib()
    # config 4 decode step (few rows): 10 strips of 256 columns x 32 slabs of 64 rows
    assert L.bn_linear_rope_workspace_size(B.BN_F32, 1, 2560, 2048) == 32 * 2560 * 4
    # bf16: 5 strips of 512 columns x 64 slabs of 32 rows
    assert L.bn_linear_rope_workspace_size(B.BN_BF16, 4, 2560, 2048) == 64 * 4 * 2560 * 4
    # 512 rows: 320 tiles, k split three ways (960 workgroups fit 1024 slots)
    assert L.bn_linear_rope_workspace_size(B.BN_F32, 512, 2560, 2048) == 3 * 512 * 2560 * 4
    assert L.bn_linear_rope_workspace_size(B.BN_BF16, 512, 2560, 2048) == 3 * 512 * 2560 * 4
    # enough tiles: no split
    assert L.bn_linear_rope_workspace_size(B.BN_F32, 4096, 4096, 2048) == 0
    assert L.bn_linear_rope_workspace_size(B.BN_U32, 4, 4, 4) == 0


def llama_cfg(**kw):
    d = dict(n_layers=22, hidden=2048, n_heads=32, n_kv_heads=4, intermediate=5632, vocab=32000,
             max_len=640, rms_eps=1e-5, rope_theta=1e4, weights_out_major=0)
    d.update(kw)
    return B.BnLlamaConfig(*d.values())


def test_llama_decode_validation():
    L = B.lib()
    c = llama_cfg()
    n = L.bn_llama_decode_workspace_size(C.byref(c))
    # residual + norm + qkv + o + attn + gate/up + act + mlp + logits rows, lens, and the
    # linear and decode partial sums: at least the activations of one step
    assert n >= 4 * (5 * 2048 + 2560 + 2 * 5632 + 5632 + 32000 + 640)
    assert L.bn_llama_decode_workspace_size(C.byref(llama_cfg(hidden=2048, n_heads=16))) == 0
    assert L.bn_llama_decode_workspace_size(None) == 0
    layers = (B.BnLlamaLayer * 22)()
    fake = 4096

    def dec(cfg, first, pos, n_tok, lay=layers, ptr=fake):
        return st("bn_llama_decode", C.byref(cfg), ptr, ptr, ptr, lay, first, pos, n_tok, ptr,
                  None, 0, None)

    s, m = dec(llama_cfg(n_heads=16), 0, 0, 1)
    assert s == B.BN_ERR_UNSUPPORTED and "head_dim" in m
    s, m = dec(llama_cfg(vocab=32002), 0, 0, 1)
    assert s == B.BN_ERR_UNSUPPORTED and "multiples of 4" in m
    s, m = dec(llama_cfg(n_layers=0), 0, 0, 1)
    assert s == B.BN_ERR_SHAPE
    # output-major weights stage each projection's input row (padded to 256
    # fp32) in 64 KB of LDS: wider rows are refused before any launch, and
    # the workspace query reports 0; row-major weights take them
    wide_i = llama_cfg(intermediate=16388, weights_out_major=1)
    assert L.bn_llama_decode_workspace_size(C.byref(wide_i)) == 0
    s, m = dec(wide_i, 0, 0, 1)
    assert s == B.BN_ERR_UNSUPPORTED and "output-major" in m
    wide_h = llama_cfg(hidden=16640, n_heads=260, weights_out_major=1)
    assert L.bn_llama_decode_workspace_size(C.byref(wide_h)) == 0
    assert L.bn_llama_decode_workspace_size(C.byref(llama_cfg(intermediate=16384, weights_out_major=1))) > 0
    assert L.bn_llama_decode_workspace_size(C.byref(llama_cfg(intermediate=16388))) > 0
    s, m = dec(c, 0, 600, 41)
    assert s == B.BN_ERR_SHAPE and "max_len" in m
    assert dec(c, 0, 600, 40)[0] != B.BN_ERR_SHAPE
    s, m = dec(c, 32000, 0, 1)
    assert s == B.BN_ERR_INVALID_ARG and "vocabulary" in m
    assert dec(c, 0, 0, 0) == (B.BN_OK, "")           # nothing to do: no device needed
    s, m = dec(c, 0, 0, 1, ptr=None)
    assert s == B.BN_ERR_INVALID_ARG and "NULL pointer" in m
    s, m = dec(c, 0, 0, 1)                            # layer pointers all NULL
    assert s == B.BN_ERR_INVALID_ARG and "layer 0" in m
    full = (B.BnLlamaLayer * 22)(*[B.BnLlamaLayer(*[fake] * 8) for _ in range(22)])
    s, m = st("bn_llama_decode", C.byref(c), fake, fake, fake, full, 0, 0, 1, fake,
              C.c_void_p(fake), 256, None)
    assert s == B.BN_ERR_INVALID_ARG and "need" in m
    s, m = st("bn_llama_decode", C.byref(c), fake, fake, fake, full, 0, 0, 1, fake,
              C.c_void_p(fake + 16), n, None)
    assert s == B.BN_ERR_UNSUPPORTED and "256-byte" in m


@pytest.mark.parametrize("kw,status,msg", [
    (dict(Hkv=3), B.BN_ERR_SHAPE, "multiple of n_kv_heads"),
    (dict(qw=1024), B.BN_ERR_SHAPE, "query and output"),
    (dict(kh=9), B.BN_ERR_SHAPE, "key and value"),
    (dict(H=32, Hkv=16, kw_=1024), B.BN_ERR_UNSUPPORTED, "<= 512"),
    (dict(D=6, qw=192, kw_=24, H=32, Hkv=4), B.BN_ERR_UNSUPPORTED, "head_dim % 4"),
    (dict(dt=B.BN_BF16), B.BN_ERR_UNSUPPORTED, "unsupported dtype"),
    (dict(), B.BN_ERR_NOT_DEVICE, "only GPU implementation available"),
])
def test_fused_head_attention_validation(kw, status, msg):
    """Shape, limit and dtype checks come before the device check (host
    views, never dereferenced: no GPU needed)."""
    a = dict(S=8, qw=2048, kh=8, kw_=256, H=32, Hkv=4, D=64, dt=B.BN_F32)
    a.update(kw)
    q = V(a["S"], a["qw"], dtype=a["dt"])
    k = V(a["kh"], a["kw_"])
    v = V(8, a["kw_"])
    o = V(a["S"], a["qw"])
    s, m = st("bn_fused_head_attention", q, k, v, o, a["H"], a["Hkv"], a["D"], 0.125, 1, 0, None)
    assert s == status, m
    assert m.startswith("Fused-head attention:") and msg in m, m


def test_decode_wrappers_refuse_layouts_they_cannot_pass():
    """bnhip.gqa_decode and gqa_decode_planned pass any cache whose key rows
    are contiguous (through the strided entry points) and refuse the rest on
    the host (CPU tensors: nothing reaches a device)."""
    import torch
    q = torch.zeros((2, 8, 64))
    kc = torch.zeros((2, 16, 2, 64))
    hm = torch.zeros((2, 2, 16, 64)).transpose(1, 2)
    lens = torch.zeros(2, dtype=torch.int32)
    with pytest.raises(ValueError, match="same shape and strides"):
        B.gqa_decode(q, kc, hm, lens)
    with pytest.raises(ValueError, match="stride 1 along head_dim"):
        cols = torch.zeros((2, 16, 2, 128))[..., ::2]
        B.gqa_decode(q, cols, cols, lens)
    with pytest.raises(ValueError, match="q and o must be contiguous"):
        B.gqa_decode(torch.zeros((8, 2, 64)).transpose(0, 1), kc, kc, lens)
    with pytest.raises(ValueError, match="same shape and strides"):
        B.gqa_decode_planned(q, kc, hm, lens, [16, 16])
    with pytest.raises(ValueError, match="stride 1 along head_dim"):
        cols = torch.zeros((2, 16, 2, 128))[..., ::2]
        B.gqa_decode_planned(q, cols, cols, lens, [16, 16])
