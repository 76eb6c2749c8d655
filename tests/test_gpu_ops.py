"""GPU parity of the op-surface kernels (RMSNorm, RoPE, fused RMSNorm+RoPE,
softmax, matmul, repeat_kv, elementwise, backward ops) against the CPU
oracle, called through the C ABI on torch-allocated device buffers."""
import ctypes as C

import numpy as np
import pytest
import torch

import bnhip as B
from oracle import oracle as O
from gpu_util import BF16_TOL, FP32_TOL, assert_close, bf16_round, dev, host, require_gpu

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def rng(s):
    return np.random.default_rng(s)


def V(t):
    """bn_view of t; the caller must keep t referenced until the launch is
    queued (a dropped temporary returns its block to torch's caching allocator
    and the next allocation may reuse it)."""
    return C.byref(B.view(t))


S0 = None  # legacy default stream


@pytest.mark.parametrize("rows,w,dtype", [(7, 2048, "f32"), (5, 300, "f32"), (64, 2048, "bf16"),
                                          (3, 4096, "f32"), (2, 6000, "f32"), (1, 2048, "bf16"),
                                          (8195, 256, "f32"), (8193, 2048, "bf16")])  # 4 rows/wave
def test_rmsnorm(rows, w, dtype):
    r = rng(1)
    x = r.standard_normal((rows, w)).astype(np.float32)
    wt = r.standard_normal((1, w)).astype(np.float32)
    td = torch.bfloat16 if dtype == "bf16" else torch.float32
    if dtype == "bf16":
        x, wt = bf16_round(x), bf16_round(wt)
    xd, wd = dev(x, td), dev(wt, td)
    yd = torch.empty_like(xd)
    B.call("bn_rmsnorm", V(xd), V(wd), V(yd), 1e-5, S0)
    assert_close(host(yd), O.rmsnorm(x, wt, 1e-5), BF16_TOL if dtype == "bf16" else FP32_TOL,
                 "rmsnorm")


def test_rmsnorm_strided_view():
    r = rng(2)
    big = r.standard_normal((10, 600)).astype(np.float32)
    wt = r.standard_normal((1, 256)).astype(np.float32)
    bd, wd = dev(big), dev(wt)
    xv = bd[2:9, 100:356]                       # column slice: strided rows
    yd = torch.empty((7, 256), device="cuda")
    B.call("bn_rmsnorm", V(xv), V(wd), V(yd), 1e-6, S0)
    assert_close(host(yd), O.rmsnorm(big[2:9, 100:356], wt, 1e-6), FP32_TOL)


@pytest.mark.parametrize("rows,w,dtype,inplace", [(7, 2048, "f32", False), (512, 2048, "f32", True),
                                                  (1, 2048, "f32", True), (5, 300, "f32", False),
                                                  (64, 2048, "bf16", False), (9, 300, "bf16", True),
                                                  (3, 6000, "f32", False)])
def test_add_rmsnorm(rows, w, dtype, inplace):
    """h = x + delta, y = RMSNorm(h): fast path (rows in registers), the
    composed fallback (bf16 width 300, width 6000), and h written over x."""
    r = rng(21)
    x = r.standard_normal((rows, w)).astype(np.float32)
    d = r.standard_normal((rows, w)).astype(np.float32)
    wt = r.standard_normal((1, w)).astype(np.float32)
    td = torch.bfloat16 if dtype == "bf16" else torch.float32
    if dtype == "bf16":
        x, d, wt = bf16_round(x), bf16_round(d), bf16_round(wt)
    xd, dd, wd = dev(x, td), dev(d, td), dev(wt, td)
    hd = xd if inplace else torch.empty_like(xd)
    yd = torch.empty_like(xd)
    B.call("bn_add_rmsnorm", V(xd), V(dd), V(wd), V(hd), V(yd), 1e-5, S0)
    h_ref, y_ref = O.add_rmsnorm(x, d, wt, 1e-5)
    if dtype == "bf16":  # h is stored in bf16 and the norm reads the stored h
        h_ref = bf16_round(h_ref)
        y_ref = O.rmsnorm(h_ref, wt, 1e-5)
    tol = BF16_TOL if dtype == "bf16" else FP32_TOL
    assert_close(host(hd), h_ref, tol, "h")
    assert_close(host(yd), y_ref, tol, "y")


def test_add_rmsnorm_strided_views():
    r = rng(22)
    big = r.standard_normal((10, 600)).astype(np.float32)
    dl = r.standard_normal((7, 256)).astype(np.float32)
    wt = r.standard_normal((1, 256)).astype(np.float32)
    bd, dd, wd = dev(big), dev(dl), dev(wt)
    xv = bd[2:9, 100:356]
    hd, yd = torch.empty((7, 256), device="cuda"), torch.empty((7, 256), device="cuda")
    B.call("bn_add_rmsnorm", V(xv), V(dd), V(wd), V(hd), V(yd), 1e-6, S0)
    h_ref, y_ref = O.add_rmsnorm(big[2:9, 100:356], dl, wt, 1e-6)
    assert_close(host(hd), h_ref, FP32_TOL, "h")
    assert_close(host(yd), y_ref, FP32_TOL, "y")


@pytest.mark.parametrize("rows,w,dtype", [(512, 5632, "f32"), (1, 5632, "f32"), (7, 300, "f32"),
                                          (64, 5632, "bf16"), (3, 36, "bf16")])
def test_silu_mul(rows, w, dtype):
    r = rng(23)
    g = (r.standard_normal((rows, w)) * 3).astype(np.float32)
    u = r.standard_normal((rows, w)).astype(np.float32)
    g[0, :4] = [0.0, -200.0, 200.0, -1e30]  # exp overflow must give -0, not NaN
    td = torch.bfloat16 if dtype == "bf16" else torch.float32
    if dtype == "bf16":
        g, u = bf16_round(g), bf16_round(u)
    gd, ud = dev(g, td), dev(u, td)
    od = torch.empty_like(gd)
    B.call("bn_silu_mul", V(gd), V(ud), V(od), S0)
    out = host(od)
    assert np.all(np.isfinite(out))
    assert_close(out, O.silu_mul(g, u), BF16_TOL if dtype == "bf16" else FP32_TOL, "silu_mul")
    # strided operands (transposed views) take the element kernel
    od2 = torch.empty((w, rows), device="cuda", dtype=td).t()
    B.call("bn_silu_mul", V(gd), V(ud), V(od2), S0)
    assert_close(host(od2), O.silu_mul(g, u), BF16_TOL if dtype == "bf16" else FP32_TOL, "silu_mul T")


@pytest.mark.parametrize("rows,w,D,off,dtype", [(16, 2048, 64, 0, "f32"), (3, 256, 64, 511, "f32"),
                                                (4, 64, 32, 7, "f32"), (8, 2048, 64, 16383, "f32"),
                                                (32, 2048, 64, 100, "bf16")])
def test_rope(rows, w, D, off, dtype):
    x = rng(3).standard_normal((rows, w)).astype(np.float32)
    td = torch.bfloat16 if dtype == "bf16" else torch.float32
    if dtype == "bf16":
        x = bf16_round(x)
    xd = dev(x, td)
    yd = torch.empty_like(xd)
    B.call("bn_rope", V(xd), V(yd), off, D, 1e4, S0)
    ref = O.rope(x, off, D, 1e4)
    assert_close(host(yd), ref, BF16_TOL if dtype == "bf16" else FP32_TOL, "rope")
    back = torch.empty_like(xd)
    B.call("bn_rope_backward", V(yd), V(back), off, D, 1e4, S0)
    assert_close(host(back), O.rope_backward(host(yd), off, D, 1e4),
                 BF16_TOL if dtype == "bf16" else FP32_TOL, "rope_back")


def test_rope_transposed_view():
    x = rng(4).standard_normal((128, 6)).astype(np.float32)   # stored transposed
    xd = dev(x)
    xt = xd.t()                                               # [6, 128] view, stride_w != 1
    yd = torch.empty((6, 128), device="cuda")
    B.call("bn_rope", V(xt), V(yd), 3, 64, 1e4, S0)
    assert_close(host(yd), O.rope(np.ascontiguousarray(x.T), 3, 64, 1e4), FP32_TOL)


@pytest.mark.parametrize("rows,w,off,dtype,hd", [(32, 2048, 0, "f32", 64), (9, 2048, 77, "f32", 64),
                                                 (64, 2048, 1000, "bf16", 64), (5, 512, 3, "bf16", 64),
                                                 (3, 320, 0, "f32", 64), (8194, 512, 5, "bf16", 64),
                                                 (8198, 2048, 0, "f32", 64),
                                                 # one angle per lane, shared (head_dim 32 / 128) and
                                                 # the per-chunk path (48: chunks start at varying
                                                 # offsets within their heads)
                                                 (7, 2048, 9, "bf16", 128), (7, 1024, 9, "f32", 32),
                                                 (5, 960, 3, "bf16", 48), (5, 960, 3, "f32", 48)])
def test_rmsnorm_rope(rows, w, off, dtype, hd):
    r = rng(5)
    x = r.standard_normal((rows, w)).astype(np.float32)
    wt = (1 + 0.1 * r.standard_normal((1, w))).astype(np.float32)
    td = torch.bfloat16 if dtype == "bf16" else torch.float32
    if dtype == "bf16":
        x, wt = bf16_round(x), bf16_round(wt)
    xd, wd = dev(x, td), dev(wt, td)
    yd = torch.empty_like(xd)
    B.call("bn_rmsnorm_rope", V(xd), V(wd), V(yd), 1e-5, off, hd, 1e4, S0)
    assert_close(host(yd), O.rmsnorm_rope(x, wt, 1e-5, off, hd, 1e4),
                 BF16_TOL if dtype == "bf16" else FP32_TOL, "rmsnorm_rope")


@pytest.mark.parametrize("rows,w,causal,off", [(33, 300, 1, 10), (8, 8, 1, 0), (16, 1000, 0, 0),
                                               (4, 128, 1, -2), (1, 4096, 1, 4095)])
def test_softmax(rows, w, causal, off):
    x = (3 * rng(6).standard_normal((rows, w))).astype(np.float32)
    xd = dev(x)
    yd = torch.empty_like(xd)
    B.call("bn_softmax", V(xd), V(yd), causal, off, S0)
    got, ref = host(yd), O.softmax(x, causal, off)
    assert_close(got, ref, FP32_TOL, "softmax")
    np.testing.assert_array_equal(got == 0, ref == 0)   # masked entries exactly 0
    dy = rng(7).standard_normal((rows, w)).astype(np.float32)
    dx, dyd = torch.empty_like(xd), dev(dy)
    B.call("bn_softmax_backward", V(yd), V(dyd), V(dx), S0)
    # the oracle gets the kernel's own y, so the comparison isolates the backward
    assert_close(host(dx), O.softmax_backward(got, dy), FP32_TOL, "softmax_back")


def test_softmax_known_answer():
    xd = dev(np.array([[1, 2, 3, 4]], np.float32))   # test_llama.py:96
    yd = torch.empty_like(xd)
    B.call("bn_softmax", V(xd), V(yd), 0, 0, S0)
    e = np.exp(np.arange(4) - 3.0)
    np.testing.assert_allclose(host(yd)[0], e / e.sum(), rtol=1e-6)


@pytest.mark.parametrize("m,k,n", [(70, 130, 50), (128, 2048, 256), (5, 7, 3), (256, 64, 256)])
def test_matmul(m, k, n):
    r = rng(8)
    a = r.standard_normal((m, k)).astype(np.float32)
    b = r.standard_normal((k, n)).astype(np.float32)
    cd, ad, bd = torch.empty((m, n), device="cuda"), dev(a), dev(b)
    B.call("bn_matmul", V(ad), V(bd), V(cd), S0)
    assert_close(host(cd), a.astype(np.float64) @ b, FP32_TOL, "matmul")
    # B given as the transpose view of a [n, k] buffer (the key.T of the layers)
    bt = dev(np.ascontiguousarray(b.T))
    B.call("bn_matmul", V(ad), V(bt.t()), V(cd), S0)
    assert_close(host(cd), O.matmul(a, b), FP32_TOL, "matmul(T view)")


@pytest.mark.parametrize("m,k,n", [(70, 130, 50), (128, 512, 256)])
def test_matmul_strided_views(m, k, n):
    """Operands with no unit stride (every other column) and a transposed
    output take the hand-written MFMA kernel instead of the library GEMM."""
    r = rng(18)
    a2 = r.standard_normal((m, 2 * k)).astype(np.float32)
    b2 = r.standard_normal((k, 2 * n)).astype(np.float32)
    ad, bd = dev(a2)[:, ::2], dev(b2)[:, ::2]
    ct = torch.zeros((n, m), device="cuda")
    c = ct.t()  # stride (1, m): a transposed output view
    B.call("bn_matmul", V(ad), V(bd), V(c), S0)
    ref = a2[:, ::2].astype(np.float64) @ b2[:, ::2]
    assert_close(host(c), ref, FP32_TOL, "matmul strided")


def test_repeat_kv_exact():
    kv = rng(9).standard_normal((33, 256)).astype(np.float32)
    out = torch.empty((33, 2048), device="cuda")
    kvd = dev(kv)
    B.call("bn_repeat_kv", V(kvd), V(out), 64, 8, S0)
    np.testing.assert_array_equal(host(out), O.repeat_kv(kv, 64, 8))


def test_elementwise_surface():
    r = rng(10)
    a = r.standard_normal((6, 9)).astype(np.float32)
    b = r.standard_normal((6, 9)).astype(np.float32)
    row = r.standard_normal((1, 9)).astype(np.float32)
    col = r.standard_normal((6, 1)).astype(np.float32)
    ad = dev(a)
    y = torch.empty_like(ad)
    for op, f in [(B.BN_ADD, np.add), (B.BN_SUB, np.subtract), (B.BN_MUL, np.multiply)]:
        for other in (b, row, col):
            od = dev(other)
            B.call("bn_binary", op, V(ad), V(od), V(y), S0)
            np.testing.assert_array_equal(host(y), f(a, other).astype(np.float32))
    eq = torch.empty((6, 9), dtype=torch.int32, device="cuda")
    pos = dev(np.where(a > 0, a, 0))
    B.call("bn_binary", B.BN_EQ, V(ad), V(pos), V(eq), S0)
    np.testing.assert_array_equal(host(eq), (a > 0).astype(np.float32))
    B.call("bn_unary", B.BN_RELU, V(ad), 0.0, V(y), S0)
    np.testing.assert_array_equal(host(y), np.maximum(a, 0))
    B.call("bn_unary", B.BN_MUL_SCALAR, V(ad), 0.125, V(y), S0)
    np.testing.assert_array_equal(host(y), a * np.float32(0.125))
    B.call("bn_unary", B.BN_SILU, V(ad), 0.0, V(y), S0)
    np.testing.assert_allclose(host(y), a / (1 + np.exp(-a.astype(np.float64))), rtol=1e-5, atol=1e-6)
    s0 = torch.empty((1, 9), device="cuda")
    B.call("bn_sum", V(ad), V(s0), 0, S0)
    np.testing.assert_allclose(host(s0), a.sum(0, keepdims=True), rtol=1e-5)
    am = torch.empty((6, 1), dtype=torch.int32, device="cuda")
    B.call("bn_argmax", V(ad), V(am), S0)
    np.testing.assert_array_equal(host(am)[:, 0], a.argmax(1))
    B.call("bn_fill", V(y), 2.5, S0)
    assert np.all(host(y) == 2.5)


def test_rmsnorm_backward():
    r = rng(11)
    x = r.standard_normal((6, 300)).astype(np.float32)
    wt = r.standard_normal((1, 300)).astype(np.float32)
    dy = r.standard_normal((6, 300)).astype(np.float32)
    dx = torch.empty((6, 300), device="cuda")
    dw = torch.full((1, 300), 5.0, device="cuda")   # overwritten, not accumulated into
    xd, wd, dyd = dev(x), dev(wt), dev(dy)   # kept alive across the launch
    B.call("bn_rmsnorm_backward", V(xd), V(wd), V(dyd), V(dx), V(dw), 1e-6, S0)
    rdx, rdw = O.rmsnorm_backward(x, wt, dy, 1e-6)
    assert_close(host(dx), rdx, FP32_TOL, "dx")
    assert_close(host(dw), rdw, FP32_TOL, "dw")


def test_pool_stream_ordered_alloc_free():
    s0 = B.BnPoolStats()
    B.call("bn_pool_get_stats", C.byref(s0))
    ptrs = []
    for n in (1 << 20, 3 << 20, 123):
        p = C.c_void_p()
        B.call("bn_alloc", C.byref(p), n, None)
        ptrs.append(p)
    s1 = B.BnPoolStats()
    B.call("bn_pool_get_stats", C.byref(s1))
    assert s1.bytes_in_use - s0.bytes_in_use == (1 << 20) + (3 << 20) + 123
    assert s1.n_live == s0.n_live + 3 and s1.bytes_reserved >= s1.bytes_in_use
    for p in ptrs:
        B.call("bn_free", p, None)
    B.call("bn_stream_synchronize", None)
    s2 = B.BnPoolStats()
    B.call("bn_pool_get_stats", C.byref(s2))
    assert s2.bytes_in_use == s0.bytes_in_use and s2.n_live == s0.n_live
    assert s2.n_frees == s0.n_frees + 3 and s2.peak_bytes_in_use >= s1.bytes_in_use
    # injected limit -> BN_ERR_OOM, and the pool keeps working afterwards
    B.call("bn_pool_set_limit", s2.bytes_in_use + 1000)
    p = C.c_void_p()
    code, msg = B.status_of("bn_alloc", C.byref(p), 4096, None)
    assert code == B.BN_ERR_OOM and "limit" in msg
    B.call("bn_pool_set_limit", 0)
    B.call("bn_alloc", C.byref(p), 4096, None)
    B.call("bn_free", p, None)


# ------------------------------------------------- projection + RoPE epilogue
LINEAR_CASES = [
    # M, K, N, rope_cols, position_offset
    (1, 2048, 2560, 2304, 37),      # config 4 decode step: fused QKV, split k
    (512, 2048, 2560, 2304, 0),     # config 4 prompt: fused QKV
    (512, 2048, 2048, 0, 0),        # output projection, no rotation
    (130, 72, 264, 128, 5),         # ragged rows, k not a multiple of the stage
    (3, 40, 200, 64, 1000),         # tiny, far position
    (64, 256, 512, 512, 3),         # every column rotated
    (2, 512, 512, 256, 3),          # few-rows path, 2 rows
    (5, 2048, 2560, 2304, 100),     # few-rows path, 8-row variant
    (8, 64, 128, 64, 0),            # few-rows path, one slab
    (9, 96, 264, 128, 1),           # first row count on the tiled path
]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("case", LINEAR_CASES)
def test_linear_rope(case, dtype):
    M, K, N, rc, off = case
    r = rng(60)
    x = r.standard_normal((M, K)).astype(np.float32)
    w = (r.standard_normal((K, N)) / np.sqrt(K)).astype(np.float32)
    if dtype == "bf16":
        x, w = bf16_round(x), bf16_round(w)
    td = torch.float32 if dtype == "f32" else torch.bfloat16
    y = B.linear_rope(dev(x, td), dev(w, td), rope_cols=rc, position_offset=off)
    ref = O.linear_rope(x, w, rc, off, 64, 1e4)
    assert_close(host(y), ref, FP32_TOL if dtype == "f32" else BF16_TOL, f"linear {case} {dtype}")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_linear_rope_strided_views_and_workspace(dtype):
    # x a column slice of a wider buffer, w the Q/K part of a fused weight,
    # y written into a column slice; a caller workspace gives the pool's bits
    td = torch.float32 if dtype == "f32" else torch.bfloat16
    r = rng(61)
    xb = r.standard_normal((9, 288)).astype(np.float32)
    wb = (r.standard_normal((256, 400)) / 16).astype(np.float32)
    if dtype == "bf16":
        xb, wb = bf16_round(xb), bf16_round(wb)
    xt, wt = dev(xb, td), dev(wb, td)
    x, w = xt[:, 16:272], wt[:, :320]
    yb = torch.full((9, 400), 7.0, dtype=td, device="cuda")
    y = yb[:, 40:360]
    B.linear_rope(x, w, y, rope_cols=256, position_offset=11)
    ref = O.linear_rope(xb[:, 16:272], wb[:, :320], 256, 11, 64, 1e4)
    got = host(yb)
    assert_close(got[:, 40:360], ref, FP32_TOL if dtype == "f32" else BF16_TOL, "strided")
    assert np.all(got[:, :40] == 7.0) and np.all(got[:, 360:] == 7.0)
    dt = B.BN_F32 if dtype == "f32" else B.BN_BF16
    n = B.lib().bn_linear_rope_workspace_size(dt, 9, 320, 256)
    assert n > 0  # 5 x 1 tiles: k is split
    ws = torch.empty(n // 4, dtype=torch.float32, device="cuda")
    y2 = B.linear_rope(x, w, rope_cols=256, position_offset=11, workspace=ws)
    assert torch.equal(y2, y)


@pytest.mark.parametrize("case", [(1, 2048, 2560, 2304, 511), (1, 5632, 2048, 0, 0), (2, 2048, 512, 256, 7),
                                  (3, 520, 320, 192, 40), (4, 1024, 256, 0, 0), (1, 68, 64, 64, 16383),
                                  (1, 8200, 128, 64, 3)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_linear_rope_output_major_weight(case, dtype):
    """w given as the transposed view of an [N, K] matrix (each output's
    weights contiguous): the few-rows kernel without a k split.  Config 4's
    decode shapes, k not a multiple of a wave-wide load, 1-4 rows, positions
    up to 16383; against the oracle and, bit for bit where the sums are the
    same, across the row-major path's rows."""
    M, K, N, rc, off = case
    if dtype == "bf16" and K % 8:
        pytest.skip("bf16 rows of 16 bytes need K % 8 == 0")
    r = rng(62)
    x = r.standard_normal((M, K)).astype(np.float32)
    wt = (r.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)  # [N, K] storage
    if dtype == "bf16":
        x, wt = bf16_round(x), bf16_round(wt)
    td = torch.float32 if dtype == "f32" else torch.bfloat16
    wd = dev(wt, td)
    y = B.linear_rope(dev(x, td), wd.t(), rope_cols=rc, position_offset=off)
    ref = O.linear_rope(x, np.ascontiguousarray(wt.T), rc, off, 64, 1e4)
    assert_close(host(y), ref, FP32_TOL if dtype == "f32" else BF16_TOL, f"out-major {case} {dtype}")
    # each output depends only on its own row of w and x: one row of x alone
    # gives the same bits as that row inside the batch
    if M > 1:
        y1 = B.linear_rope(dev(x[1:2], td), wd.t(), rope_cols=rc, position_offset=off + 1)
        assert torch.equal(y1[0], y[1])


def test_linear_rope_output_major_inf_in_last_span():
    """k = 5632 fp32 is 22 wave-wide loads: the last round of 8 has two slots
    past the row.  An Inf in the last span of x must give the reference's
    +/-Inf (Inf * w summed with finite terms), not the NaN of a zero weight
    met in a slot past the row."""
    M, K, N = 1, 5632, 256
    r = rng(64)
    x = r.standard_normal((M, K)).astype(np.float32)
    x[0, K - 1] = np.inf
    wt = (r.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)
    wt[:, K - 1] = np.where(wt[:, K - 1] >= 0, 0.5, -0.5)
    y = host(B.linear_rope(dev(x), dev(wt).t(), rope_cols=0))
    ref = O.linear_rope(x, np.ascontiguousarray(wt.T), 0, 0, 64, 1e4)
    assert not np.isnan(ref).any() and np.isinf(ref).all()
    np.testing.assert_array_equal(y, ref)


def test_linear_rope_output_major_strided_and_limits():
    # w the transposed view of the first 320 rows and 256 columns of a wider
    # [400, 264] buffer (stride between outputs 264), y a column slice
    r = rng(63)
    xb = r.standard_normal((2, 256)).astype(np.float32)
    wb = (r.standard_normal((400, 264)) / 16).astype(np.float32)
    w = dev(wb)[:320, :256].t()
    yb = torch.full((2, 400), 7.0, device="cuda")
    B.linear_rope(dev(xb), w, yb[:, 40:360], rope_cols=128, position_offset=9)
    got = host(yb)
    ref = O.linear_rope(xb, np.ascontiguousarray(wb[:320, :256].T), 128, 9, 64, 1e4)
    assert_close(got[:, 40:360], ref, FP32_TOL, "out-major strided")
    assert np.all(got[:, :40] == 7.0) and np.all(got[:, 360:] == 7.0)
    # more than 4 rows of bf16, or an odd output width, is refused for this layout
    with pytest.raises(B.BnError, match="at most 4 rows"):
        B.linear_rope(torch.randn((5, 256), device="cuda").bfloat16(), w.bfloat16())
    with pytest.raises(B.BnError, match="even output width"):
        B.linear_rope(dev(xb), dev(wb)[:319, :256].t())


@pytest.mark.parametrize("case", [(512, 2048, 2560, 2304, 0),    # config 4's prompt QKV + RoPE
                                  (512, 2048, 2048, 0, 0),       # its O projection
                                  (37, 5632, 2048, 0, 0),        # down, ragged row tile
                                  (5, 520, 330, 192, 40),        # ragged column tile, k not a multiple of 32
                                  (96, 64, 4032, 4032, 16000),   # every column rotated, late positions
                                  (40, 256, 512, 512, 5)])       # head_dim 256: angles per element
def test_linear_rope_output_major_many_rows(case):
    """fp32, w output-major (the transposed view of an [N, K] matrix), more
    than 4 rows: the matrix-core kernel of 32 x 160 output tiles; against the
    oracle's op_mm + op_rope, and the same bits for a row computed inside
    different row tiles (each output is one fixed-order sum)."""
    M, K, N, rc, off = case
    r = rng(65)
    x = r.standard_normal((M, K)).astype(np.float32)
    wt = (r.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)
    wd = dev(wt)
    hd = 256 if K == 256 else 64
    y = B.linear_rope(dev(x), wd.t(), rope_cols=rc, position_offset=off, head_dim=hd)
    ref = O.linear_rope(x, np.ascontiguousarray(wt.T), rc, off, hd, 1e4)
    assert_close(host(y), ref, FP32_TOL, f"out-major many rows {case}")
    if M > 40:   # rows 33.. as rows 0.. of a second call (another row tile position)
        y2 = B.linear_rope(dev(x[33:]), wd.t(), rope_cols=rc, position_offset=off + 33, head_dim=hd)
        assert torch.equal(y2, y[33:])


def test_linear_rope_empty_k_gives_zeros():
    x = torch.empty((5, 0), device="cuda")
    w = torch.empty((0, 64), device="cuda")
    y = B.linear_rope(x, w, rope_cols=64, position_offset=3)
    assert torch.count_nonzero(y).item() == 0


def test_linear_rope_empty_rows_is_noop():
    x = torch.empty((0, 64), device="cuda")
    w = torch.randn((64, 128), device="cuda")
    y = B.linear_rope(x, w, rope_cols=64)
    assert y.shape == (0, 128)


def _argmax_sequential(row):
    """The reference's rule (op_reduction.cuh:36-92 with MaxAccumFunc): the
    accumulator starts at column 0 and takes x when x > accumulator."""
    best, bi = row[0], 0
    for c in range(1, len(row)):
        if row[c] > best:
            best, bi = row[c], c
    return bi


def test_argmax_rows_ties_nan_strided():
    r = rng(12)
    a = r.standard_normal((7, 32000)).astype(np.float32)
    a[1, [5, 17000, 31999]] = 9.0                 # ties: the first one
    a[2, 0] = np.nan                              # NaN at column 0: index 0
    a[3, [3, 300]] = np.nan                       # NaN elsewhere never wins
    a[3, 20000] = 7.0
    a[4, :] = -np.inf                             # all equal: index 0
    a[5, :] = 1.0
    a[5, 0] = 0.5                                 # equal maxima after column 0: first one
    a[6, 31999] = 50.0                            # maximum in the last column
    ad = dev(a)
    am = torch.empty((7, 1), dtype=torch.int32, device="cuda")
    B.call("bn_argmax", V(ad), V(am), S0)
    want = [_argmax_sequential(row) for row in a]
    assert want[1] == 5 and want[2] == 0 and want[3] == 20000 and want[4] == 0 and want[5] == 1
    np.testing.assert_array_equal(host(am)[:, 0], want)
    # strided view (every other column of a wider buffer) and one short row
    wide = dev(np.repeat(a[:, :1000], 2, axis=1))
    B.call("bn_argmax", V(wide[:, ::2]), V(am), S0)
    np.testing.assert_array_equal(host(am)[:, 0], [_argmax_sequential(row) for row in a[:, :1000]])
    one = torch.empty((1, 1), dtype=torch.int32, device="cuda")
    B.call("bn_argmax", V(ad[6:7, :1]), V(one), S0)
    assert int(one.item()) == 0
    # contiguous widths around the fast path's rounds (1024 threads x 4 chunks
    # of 4 columns): one chunk, a partial round, several rounds; ties and NaN
    for wdt in (4, 100, 4100, 70000):
        b = np.round(r.standard_normal((4, wdt)) * 2).astype(np.float32)  # many ties
        b[1, 0] = np.nan
        b[2, 3::7] = np.nan
        b[3, -1] = 99.0
        bm = torch.empty((4, 1), dtype=torch.int32, device="cuda")
        B.call("bn_argmax", V(dev(b)), V(bm), S0)
        np.testing.assert_array_equal(host(bm)[:, 0], [_argmax_sequential(row) for row in b])
    # uint32 input
    u = r.integers(0, 1 << 31, (3, 5000)).astype(np.int32)
    u[0, [10, 4000]] = (1 << 31) - 1
    ud = torch.from_numpy(u).cuda()
    um = torch.empty((3, 1), dtype=torch.int32, device="cuda")
    B.call("bn_argmax", V(ud), V(um), S0)
    np.testing.assert_array_equal(host(um)[:, 0], [_argmax_sequential(row) for row in u])
