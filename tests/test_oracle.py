"""Pins the CPU oracle before it is trusted as the parity checker.

The reference ships no golden vectors or numeric assertions for this path
(test_llama.py only prints), so every oracle function is checked here against
an independent formulation (fp64 closed forms, torch fp64 SDPA, complex
multiplication for RoPE), against invariants the mathematics fixes, against
the one known-answer input the reference's tests hold (softmax of [1,2,3,4],
test_llama.py:96) and against brute force on tiny inputs.  Each check is
chosen so that a plausible slip (wrong pair index, rotate-half instead of
interleaved pairs, off-by-one mask, wrong KV head) fails it.
"""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O


def rng(seed=0):
    return np.random.default_rng(seed)


def relerr(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


# ---------------------------------------------------------------- RMSNorm
@pytest.mark.parametrize("rows,w", [(4, 64), (7, 2048), (3, 300), (2, 1)])
def test_rmsnorm_closed_form(rows, w):
    r = rng(1)
    x = r.standard_normal((rows, w)).astype(np.float32)
    wt = r.standard_normal((1, w)).astype(np.float32)
    eps = 1e-5
    y = O.rmsnorm(x, wt, eps)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + eps) * wt
    assert relerr(y, ref) < 2e-6


def test_rmsnorm_unit_rms_invariant():
    x = rng(2).standard_normal((5, 2048)).astype(np.float32) * 7.0
    y = O.rmsnorm(x, np.ones((1, 2048), np.float32), 1e-12)
    rms = np.sqrt((y.astype(np.float64) ** 2).mean(1))
    np.testing.assert_allclose(rms, 1.0, rtol=1e-6)
    # scale invariance y(a x) = y(x) when eps is negligible
    y2 = O.rmsnorm(x * 3.0, np.ones((1, 2048), np.float32), 1e-12)
    assert relerr(y2, y) < 1e-6


def test_rmsnorm_matches_torch():
    r = rng(3)
    x = r.standard_normal((8, 512)).astype(np.float32)
    wt = r.standard_normal((1, 512)).astype(np.float32)
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x).double(), (512,),
                                       torch.from_numpy(wt[0]).double(), eps=1e-6)
    assert relerr(O.rmsnorm(x, wt, 1e-6), ref.numpy()) < 2e-6


def test_add_rmsnorm_closed_form_and_reduction():
    r = rng(31)
    x = r.standard_normal((6, 2048)).astype(np.float32)
    d = r.standard_normal((6, 2048)).astype(np.float32)
    wt = r.standard_normal((1, 2048)).astype(np.float32)
    h, y = O.add_rmsnorm(x, d, wt, 1e-5)
    h64 = x.astype(np.float64) + d
    np.testing.assert_array_equal(h, (x + d).astype(np.float32))   # fp32 add, exact
    ref = h64 / np.sqrt((h64 ** 2).mean(1, keepdims=True) + 1e-5) * wt
    assert relerr(y, ref) < 2e-6
    # delta = 0 reduces to the plain RMSNorm
    h0, y0 = O.add_rmsnorm(x, np.zeros_like(x), wt, 1e-5)
    np.testing.assert_array_equal(h0, x)
    np.testing.assert_array_equal(y0, O.rmsnorm(x, wt, 1e-5))


def test_silu_mul_closed_form_and_limits():
    r = rng(32)
    g = (r.standard_normal((5, 300)) * 4).astype(np.float32)
    u = r.standard_normal((5, 300)).astype(np.float32)
    g64 = g.astype(np.float64)
    ref = g64 / (1.0 + np.exp(-g64)) * u
    assert relerr(O.silu_mul(g, u), ref) < 1e-6
    # silu(0) = 0, silu(g) -> g for large g, -> -0 for very negative g (no NaN)
    edge = np.array([[0.0, 30.0, -30.0, -1000.0, 1000.0]], np.float32)
    out = O.silu_mul(edge, np.ones_like(edge))
    assert out[0, 0] == 0.0 and abs(out[0, 1] - 30.0) < 1e-5 and abs(out[0, 2]) < 1e-10
    assert out[0, 3] == 0.0 and out[0, 4] == 1000.0 and np.all(np.isfinite(out))
    # torch's SiLU on the same values (an independent implementation)
    t = torch.nn.functional.silu(torch.from_numpy(g64)) * torch.from_numpy(u.astype(np.float64))
    assert relerr(O.silu_mul(g, u), t.numpy()) < 1e-6


# ---------------------------------------------------------------- RoPE
def rope_complex_fp64(x, pos_off, D, theta):
    """Independent restatement: interleaved pairs as complex numbers rotated by
    e^{i*angle}, angle formed in fp32 as pos*freq (op_rope.cuh:82-83)."""
    rows, w = x.shape
    z = x.astype(np.float64).reshape(rows, w // D, D // 2, 2)
    zc = z[..., 0] + 1j * z[..., 1]
    p = np.arange(D // 2)
    e = (2 * p).astype(np.float32) / np.float32(D)
    freq = np.float32(1.0 / np.float32(np.float64(theta) ** e.astype(np.float64)))
    pos = (np.arange(rows) + pos_off).astype(np.float32)
    ang = (pos[:, None] * freq[None, :]).astype(np.float32).astype(np.float64)
    out = zc * np.exp(1j * ang)[:, None, :]
    return np.stack([out.real, out.imag], -1).reshape(rows, w)


@pytest.mark.parametrize("rows,w,D,off", [(4, 64, 32, 0), (16, 2048, 64, 0),
                                          (3, 256, 64, 511), (2, 2048, 64, 16383),
                                          (5, 96, 16, 7)])
def test_rope_complex_restatement(rows, w, D, off):
    x = rng(4).standard_normal((rows, w)).astype(np.float32)
    y = O.rope(x, off, D, 10000.0)
    assert relerr(y, rope_complex_fp64(x, off, D, 10000.0)) < 1e-6


def test_rope_freq_formation():
    # freq = fp32(1 / fp32(theta^e)): two roundings, so within 1.5 ulp of the
    # exact theta^(-2p/D); a wrong exponent (p/D, 2p/(D-1)) is off by far more
    for D in (16, 32, 64, 128):
        for p in range(D // 2):
            f = O.rope_freq(p, D, 10000.0)
            exact = 10000.0 ** (-(2.0 * p) / D)
            assert abs(f - exact) <= 1.5 * np.spacing(np.float32(exact)), (D, p)


def test_rope_invariants():
    r = rng(5)
    x = r.standard_normal((12, 256)).astype(np.float32)
    y = O.rope(x, 3, 64, 10000.0)
    pn = lambda a: np.hypot(a[:, 0::2].astype(np.float64), a[:, 1::2])
    np.testing.assert_allclose(pn(y), pn(x), rtol=1e-6)          # pair norms kept
    np.testing.assert_array_equal(O.rope(x[:1], 0, 64, 1e4), x[:1])  # pos 0 = identity
    back = O.rope_backward(y, 3, 64, 10000.0)                     # inverse rotation
    assert relerr(back, x) < 1e-6
    # <rope_m(q), rope_n(k)> depends only on m - n
    q = r.standard_normal((1, 64)).astype(np.float32)
    k = r.standard_normal((1, 64)).astype(np.float32)
    d1 = float((O.rope(q, 10, 64, 1e4).astype(np.float64) @ O.rope(k, 4, 64, 1e4)[0])[0])
    d2 = float((O.rope(q, 106, 64, 1e4).astype(np.float64) @ O.rope(k, 100, 64, 1e4)[0])[0])
    assert abs(d1 - d2) < 1e-4 * max(1.0, abs(d1))


def test_rope_is_not_rotate_half():
    # the reference pairs (2p, 2p+1) (op_rope.cuh:76-77), unlike the torch model's
    # rotate-half (benchmark_latency.py:47-53): the two must differ
    x = rng(6).standard_normal((4, 64)).astype(np.float32)
    y = O.rope(x, 1, 64, 1e4)
    x1, x2 = x[:, :32].astype(np.float64), x[:, 32:]
    f = 10000.0 ** (-np.arange(0, 64, 2) / 64.0)
    ang = (np.arange(4) + 1)[:, None] * f[None]
    half = np.concatenate([x1 * np.cos(ang) - x2 * np.sin(ang),
                           x1 * np.sin(ang) + x2 * np.cos(ang)], 1)
    assert relerr(y, half) > 1e-2


def test_rmsnorm_rope_is_composition():
    r = rng(7)
    x = r.standard_normal((9, 2048)).astype(np.float32)
    wt = r.standard_normal((1, 2048)).astype(np.float32)
    y = O.rmsnorm_rope(x, wt, 1e-5, 5, 64, 1e4)
    np.testing.assert_array_equal(y, O.rope(O.rmsnorm(x, wt, 1e-5), 5, 64, 1e4))


# ---------------------------------------------------------------- softmax
def test_softmax_known_answer():
    # the reference's own test input (test_llama.py:96-100)
    y = O.softmax(np.array([[1, 2, 3, 4]], np.float32))
    e = np.exp(np.arange(4) - 3.0)
    np.testing.assert_allclose(y[0], e / e.sum(), rtol=1e-6)
    assert abs(float(y.sum()) - 1.0) < 1e-6


@pytest.mark.parametrize("rows,w,off", [(8, 8, 0), (5, 300, 0), (3, 700, 400), (4, 4, 2)])
def test_softmax_causal(rows, w, off):
    x = rng(8).standard_normal((rows, w)).astype(np.float32) * 3
    y = O.softmax(x, True, off)
    x64 = x.astype(np.float64)
    for r in range(rows):
        q = r + off
        vis = np.arange(w) <= q
        assert np.all(y[r, ~vis] == 0.0)          # masked entries exactly 0
        e = np.exp(x64[r, vis] - x64[r, vis].max())
        np.testing.assert_allclose(y[r, vis], e / e.sum(), rtol=2e-6, atol=1e-12)
        assert abs(float(y[r].astype(np.float64).sum()) - 1.0) < 1e-5


def test_softmax_fully_masked_row_is_zero():
    y = O.softmax(np.ones((2, 4), np.float32), True, -1)
    assert np.all(y[0] == 0.0) and y[1, 0] == 1.0


def test_softmax_backward_analytic():
    r = rng(9)
    x = r.standard_normal((3, 37)).astype(np.float32)
    dy = r.standard_normal((3, 37)).astype(np.float32)
    y = O.softmax(x)
    y64 = y.astype(np.float64)
    ref = y64 * (dy - (y64 * dy).sum(1, keepdims=True))
    assert relerr(O.softmax_backward(y, dy), ref) < 1e-5


@pytest.mark.parametrize("rows,w,causal,off", [(6, 50, False, 0), (9, 300, True, 0),
                                               (4, 700, True, 400), (5, 33, True, -2)])
def test_softmax_backward_vs_torch_autograd(rows, w, causal, off):
    """op_softmax_backward (op_softmax.cuh:182-246) pinned by torch fp64
    autograd through a masked softmax: dx = d/dx <softmax(x), dy>.  Masked
    positions get exactly zero gradient (y = 0 there)."""
    r = rng(31)
    x = (2 * r.standard_normal((rows, w))).astype(np.float32)
    dy = r.standard_normal((rows, w)).astype(np.float32)
    xt = torch.from_numpy(x.astype(np.float64)).requires_grad_(True)
    if causal:
        vis = torch.arange(w)[None, :] <= (torch.arange(rows)[:, None] + off)
        z = torch.where(vis, xt, torch.tensor(float("-inf"), dtype=torch.float64))
        yt = torch.softmax(z, dim=1)
        yt = torch.where(vis, yt, torch.zeros((), dtype=torch.float64))  # fully masked rows: 0
    else:
        yt = torch.softmax(xt, dim=1)
    (yt * torch.from_numpy(dy.astype(np.float64))).sum().backward()
    want = xt.grad.numpy()
    y = O.softmax(x, causal, off)
    got = O.softmax_backward(y, dy)
    assert relerr(got, want) < 1e-5
    if causal:
        assert np.all(got[~vis.numpy()] == 0.0)


def test_softmax_backward_planted_slip_fails_autograd_pin():
    # a softmax backward that drops the y * sum(y * dy) term must miss the pin
    r = rng(32)
    x = r.standard_normal((3, 40)).astype(np.float32)
    dy = r.standard_normal((3, 40)).astype(np.float32)
    xt = torch.from_numpy(x.astype(np.float64)).requires_grad_(True)
    (torch.softmax(xt, 1) * torch.from_numpy(dy.astype(np.float64))).sum().backward()
    y = O.softmax(x).astype(np.float64)
    assert relerr(y * dy, xt.grad.numpy()) > 1e-2


# ---------------------------------------------------------------- matmul / views
def test_matmul_and_views():
    r = rng(10)
    a = r.standard_normal((33, 70)).astype(np.float32)
    b = r.standard_normal((70, 17)).astype(np.float32)
    assert relerr(O.matmul(a, b), a.astype(np.float64) @ b) < 1e-5
    # transposed view (tensor.cuh:133-145) and a sliced view (:149-171)
    bt = np.ascontiguousarray(b.T)
    c = np.empty((33, 17), np.float32)
    O.matmul_views(O.view(a), O.OrView(O._ptr(bt), 0, 70, 17, 1, 70), O.view(c))
    assert relerr(c, a.astype(np.float64) @ b) < 1e-5
    c2 = np.empty((10, 5), np.float32)
    O.matmul_views(O.view(a, offset=3 * 70 + 4, h=10, w=20, stride_h=70),
                   O.view(b, offset=4 * 17 + 2, h=20, w=5, stride_h=17), O.view(c2))
    assert relerr(c2, a[3:13, 4:24].astype(np.float64) @ b[4:24, 2:7]) < 1e-5


def test_repeat_kv_mapping_exact():
    # KV head g holds the constant g+1: destination head h must hold h//n_rep + 1
    D, Hkv, n_rep = 64, 4, 8
    kv = np.repeat(np.arange(1, Hkv + 1, dtype=np.float32), D)[None].repeat(3, 0)
    out = O.repeat_kv(kv, D, n_rep)
    for h in range(Hkv * n_rep):
        assert np.all(out[:, h * D:(h + 1) * D] == h // n_rep + 1)


# ---------------------------------------------------------------- attention
def sdpa64(q, k, v, scale, causal, seq_offset):
    """torch fp64 SDPA with GQA; mask j <= i + seq_offset (op_softmax.cuh:89-99)."""
    qt = torch.from_numpy(q).double().permute(0, 2, 1, 3)
    kt = torch.from_numpy(k).double().permute(0, 2, 1, 3)
    vt = torch.from_numpy(v).double().permute(0, 2, 1, 3)
    Sq, Skv = q.shape[1], k.shape[1]
    mask = None
    if causal:
        mask = (torch.arange(Skv)[None, :] <= torch.arange(Sq)[:, None] + seq_offset)
    o = torch.nn.functional.scaled_dot_product_attention(
        qt, kt, vt, attn_mask=mask, scale=scale, enable_gqa=True)
    return o.permute(0, 2, 1, 3).numpy()


@pytest.mark.parametrize("B,Sq,Skv,H,Hkv,D,causal,off", [
    (2, 16, 16, 8, 2, 64, True, 0),
    (1, 64, 64, 32, 4, 64, True, 0),
    (2, 5, 40, 4, 1, 32, True, 35),
    (1, 33, 33, 4, 4, 16, False, 0),
    (1, 300, 300, 2, 1, 64, True, 0)])
def test_gqa_prefill_vs_sdpa(B, Sq, Skv, H, Hkv, D, causal, off):
    r = rng(11)
    q = r.standard_normal((B, Sq, H, D)).astype(np.float32)
    k = r.standard_normal((B, Skv, Hkv, D)).astype(np.float32)
    v = r.standard_normal((B, Skv, Hkv, D)).astype(np.float32)
    sc = 1.0 / math.sqrt(D)
    o = O.gqa_prefill(q, k, v, sc, causal, off)
    assert relerr(o, sdpa64(q, k, v, sc, causal, off)) < 1e-5


def test_gqa_prefill_mask_prefix_mean():
    # Q = 0 makes every visible key equally likely: row i is the mean of
    # V[0 .. i+off] of its KV head; an off-by-one moves it by >= 1/(2(i+1)).
    B, S, H, Hkv, D, off = 1, 24, 8, 2, 16, 3
    r = rng(12)
    q = np.zeros((B, S, H, D), np.float32)
    k = r.standard_normal((B, S + off, Hkv, D)).astype(np.float32)
    v = r.integers(0, 2, (B, S + off, Hkv, D)).astype(np.float32)
    o = O.gqa_prefill(q, k, v, 0.125, True, off)
    for i in range(S):
        for h in range(H):
            ref = v[0, :i + off + 1, h // (H // Hkv)].astype(np.float64).mean(0)
            np.testing.assert_allclose(o[0, i, h], ref, atol=1e-6)


def test_gqa_prefill_head_mapping_exact():
    # V of KV head g is the constant g+1: every output of query head h must be
    # exactly h // G + 1 (mapping of llama_layers.hpp:159-163)
    B, S, H, Hkv, D = 1, 9, 32, 4, 64
    r = rng(13)
    q = r.standard_normal((B, S, H, D)).astype(np.float32)
    k = r.standard_normal((B, S, Hkv, D)).astype(np.float32)
    v = np.broadcast_to(np.arange(1, Hkv + 1, dtype=np.float32)[None, None, :, None],
                        (B, S, Hkv, D)).copy()
    o = O.gqa_prefill(q, k, v, 0.125, True, 0)
    for h in range(H):
        np.testing.assert_allclose(o[0, :, h], h // 8 + 1, rtol=2e-7)


def test_gqa_prefill_brute_force():
    r = rng(14)
    B, S, H, Hkv, D = 1, 6, 4, 2, 8
    q = r.standard_normal((B, S, H, D)).astype(np.float32)
    k = r.standard_normal((B, S, Hkv, D)).astype(np.float32)
    v = r.standard_normal((B, S, Hkv, D)).astype(np.float32)
    o = O.gqa_prefill(q, k, v, 0.3, True, 0)
    ref = np.zeros((S, H, D))
    for h in range(H):
        g = h // 2
        for i in range(S):
            s = [0.3 * sum(float(q[0, i, h, d]) * float(k[0, j, g, d]) for d in range(D))
                 for j in range(i + 1)]
            m = max(s)
            e = [math.exp(x - m) for x in s]
            for d in range(D):
                ref[i, h, d] = sum(e[j] * float(v[0, j, g, d]) for j in range(i + 1)) / sum(e)
    assert relerr(o[0], ref) < 1e-5


def test_gqa_decode_equals_prefill_last_row():
    r = rng(15)
    B, Lmax, H, Hkv, D = 3, 50, 8, 2, 64
    lens = np.array([50, 1, 23], np.int32)
    kc = r.standard_normal((B, Lmax, Hkv, D)).astype(np.float32)
    vc = r.standard_normal((B, Lmax, Hkv, D)).astype(np.float32)
    q = r.standard_normal((B, H, D)).astype(np.float32)
    o = O.gqa_decode(q, kc, vc, lens, 0.125)
    for b in range(B):
        L = int(lens[b])
        qq = np.zeros((1, L, H, D), np.float32)
        qq[0, L - 1] = q[b]
        full = O.gqa_prefill(qq, kc[b:b + 1, :L], vc[b:b + 1, :L], 0.125, True, 0)
        np.testing.assert_array_equal(o[b], full[0, L - 1])
        ref = sdpa64(q[b:b + 1, None], kc[b:b + 1, :L], vc[b:b + 1, :L], 0.125, False, 0)
        assert relerr(o[b], ref[0, 0]) < 1e-5


# ---------------------------------------------------------------- layer chain
def layer_fp64(x, wq, wk, wv, wo, H, Hkv, theta, off, per_head):
    """numpy fp64 restatement of the layer op sequence (llama_layers.py:157-186)."""
    S, hid = x.shape
    D = hid // H
    G = H // Hkv
    x = x.astype(np.float64)
    q, k, v = x @ wq, x @ wk, x @ wv
    q = rope_complex_fp64(q, off, D, theta)
    k = rope_complex_fp64(k, off, D, theta)
    mask = np.arange(S)[None, :] <= np.arange(S)[:, None] + off
    if not per_head:
        krep = np.repeat(k.reshape(S, Hkv, D), G, axis=1).reshape(S, hid)
        vrep = np.repeat(v.reshape(S, Hkv, D), G, axis=1).reshape(S, hid)
        s = q @ krep.T / math.sqrt(D)
        s = np.where(mask, s, -np.inf)
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        o = p @ vrep
    else:
        o = np.zeros((S, hid))
        for h in range(H):
            g = h // G
            s = q[:, h * D:(h + 1) * D] @ k[:, g * D:(g + 1) * D].T / math.sqrt(D)
            s = np.where(mask, s, -np.inf)
            p = np.exp(s - s.max(1, keepdims=True))
            p /= p.sum(1, keepdims=True)
            o[:, h * D:(h + 1) * D] = p @ v[:, g * D:(g + 1) * D]
    return o @ wo


@pytest.mark.parametrize("per_head", [False, True])
def test_gqa_layer_chain(per_head):
    r = rng(16)
    S, hid, H, Hkv = 12, 128, 8, 2
    x = r.standard_normal((S, hid)).astype(np.float32)
    wq = (r.standard_normal((hid, hid)) * 0.05).astype(np.float32)
    wk = (r.standard_normal((hid, hid // 4)) * 0.05).astype(np.float32)
    wv = (r.standard_normal((hid, hid // 4)) * 0.05).astype(np.float32)
    wo = (r.standard_normal((hid, hid)) * 0.05).astype(np.float32)
    out = O.gqa_layer(x, wq, wk, wv, wo, H, Hkv, 1e4, 0, per_head)
    ref = layer_fp64(x, wq, wk, wv, wo, H, Hkv, 1e4, 0, per_head)
    assert relerr(out, ref) < 1e-5
    other = layer_fp64(x, wq, wk, wv, wo, H, Hkv, 1e4, 0, not per_head)
    assert relerr(out, other) > 1e-3   # fused-head and per-head really differ


def fused_head_torch64(q, k, v, D, n_rep, sc, causal, off):
    """The fused-head chain in torch fp64: heads expanded with
    repeat_interleave on a [S, Hkv, D] view, one masked softmax over the full
    width; rows with no visible key are zero (the chain's all-zero P row)."""
    q, k, v = (torch.from_numpy(np.asarray(a, np.float64)) for a in (q, k, v))
    Sq, Sk = q.shape[0], k.shape[0]
    kr = k.view(Sk, -1, D).repeat_interleave(n_rep, dim=1).reshape(Sk, -1)
    vr = v.view(Sk, -1, D).repeat_interleave(n_rep, dim=1).reshape(Sk, -1)
    s = (q @ kr.T) * sc
    if causal:
        i = torch.arange(Sq).unsqueeze(1)
        j = torch.arange(Sk).unsqueeze(0)
        s = s.masked_fill(j > i + off, float("-inf"))
    p = torch.nan_to_num(torch.softmax(s, dim=1), nan=0.0)
    return (p @ vr).numpy()


@pytest.mark.parametrize("Sq,Sk,H,Hkv,D,causal,off", [
    (12, 12, 8, 2, 16, True, 0), (9, 20, 4, 4, 8, True, 11), (7, 7, 6, 2, 4, False, 0),
    (5, 5, 4, 1, 8, True, -2)])
def test_fused_head_attention_vs_torch(Sq, Sk, H, Hkv, D, causal, off):
    r = rng(17)
    q = r.standard_normal((Sq, H * D)).astype(np.float32)
    k = r.standard_normal((Sk, Hkv * D)).astype(np.float32)
    v = r.standard_normal((Sk, Hkv * D)).astype(np.float32)
    sc = 1.0 / math.sqrt(D)
    out = O.fused_head_attention(q, k, v, D, H // Hkv, sc, causal, off)
    ref = fused_head_torch64(q, k, v, D, H // Hkv, sc, causal, off)
    assert relerr(out, ref) < 1e-5
    if off < 0:   # rows 0 and 1 see no key: exact zeros
        assert not out[:-off].any()


def test_fused_head_attention_uniform_keys_closed_form():
    # identical keys: every visible key gets the same weight, so row i of head
    # h is the mean of the visible rows of V's KV head h // n_rep
    r = rng(18)
    S, H, Hkv, D, off = 10, 8, 2, 4, 3
    q = r.standard_normal((S, H * D)).astype(np.float32)
    k = np.tile(r.standard_normal((1, Hkv * D)).astype(np.float32), (S, 1))
    v = r.standard_normal((S, Hkv * D)).astype(np.float32)
    out = O.fused_head_attention(q, k, v, D, H // Hkv, 0.5, True, off)
    for i in range(S):
        mean = v[:min(S, i + off + 1)].astype(np.float64).mean(0)
        for h in range(H):
            g = h // (H // Hkv)
            np.testing.assert_allclose(out[i, h * D:(h + 1) * D], mean[g * D:(g + 1) * D],
                                       rtol=1e-5, atol=1e-6)


def test_fused_head_check_catches_planted_group_slip():
    # head h reading KV head h % Hkv instead of h // n_rep fails the torch pin
    r = rng(19)
    S, H, Hkv, D = 8, 8, 2, 8
    q = r.standard_normal((S, H * D)).astype(np.float32)
    k = r.standard_normal((S, Hkv * D)).astype(np.float32)
    v = r.standard_normal((S, Hkv * D)).astype(np.float32)
    kt, vt = np.tile(k, (1, H // Hkv)), np.tile(v, (1, H // Hkv))   # the slip
    s = O.scale(O.matmul(q, np.ascontiguousarray(kt.T)), 0.25)
    slipped = O.matmul(O.softmax(s, True, 0), vt)
    ref = fused_head_torch64(q, k, v, D, H // Hkv, 0.25, True, 0)
    assert relerr(slipped, ref) > 1e-2


# ---------------------------------------------------------------- backward
def test_rmsnorm_backward_vs_torch():
    r = rng(17)
    x = r.standard_normal((6, 300)).astype(np.float32)
    wt = r.standard_normal((1, 300)).astype(np.float32)
    dy = r.standard_normal((6, 300)).astype(np.float32)
    xt = torch.from_numpy(x).double().requires_grad_()
    wtt = torch.from_numpy(wt).double().requires_grad_()
    y = xt / torch.sqrt((xt ** 2).mean(1, keepdim=True) + 1e-6) * wtt
    y.backward(torch.from_numpy(dy).double())
    dx, dw = O.rmsnorm_backward(x, wt, dy, 1e-6)
    assert relerr(dx, xt.grad.numpy()) < 1e-5
    assert relerr(dw, wtt.grad.numpy()) < 1e-5


# ---------------------------------------------------------------- sensitivity
def test_checks_catch_planted_mask_slip():
    # a mask shifted by one (seq_offset+1) must fail the SDPA comparison
    r = rng(18)
    q = r.standard_normal((1, 20, 4, 16)).astype(np.float32)
    k = r.standard_normal((1, 20, 2, 16)).astype(np.float32)
    v = r.standard_normal((1, 20, 2, 16)).astype(np.float32)
    wrong = O.gqa_prefill(q, k, v, 0.25, True, 1)
    assert relerr(wrong, sdpa64(q, k, v, 0.25, True, 0)) > 1e-2


def test_checks_catch_planted_pair_slip():
    # pairing (p, p + D/2) instead of (2p, 2p+1) must fail the restatement check
    x = rng(19).standard_normal((4, 64)).astype(np.float32)
    perm = np.arange(64).reshape(2, 32).T.reshape(-1)   # interleave halves
    wrong = O.rope(x[:, perm], 2, 64, 1e4)[:, np.argsort(perm)]
    assert relerr(wrong, rope_complex_fp64(x, 2, 64, 1e4)) > 1e-2


# ---------------------------------------------------- attention backward
@pytest.mark.parametrize("B,Sq,Skv,H,Hkv,causal,off", [(1, 40, 40, 8, 2, True, 0), (2, 17, 30, 4, 4, True, 13),
                                                       (1, 24, 24, 8, 1, False, 0), (1, 9, 12, 2, 1, True, -3)])
def test_gqa_prefill_backward_vs_torch_autograd(B, Sq, Skv, H, Hkv, causal, off):
    """The composed backward equals torch fp64 autograd through an explicit
    GQA attention (repeat_interleave of K/V, masked softmax)."""
    r = rng(41)
    q = r.standard_normal((B, Sq, H, 64))
    k = r.standard_normal((B, Skv, Hkv, 64))
    v = r.standard_normal((B, Skv, Hkv, 64))
    do = r.standard_normal((B, Sq, H, 64))
    dq, dk, dv = O.gqa_prefill_backward(q, k, v, do, 0.125, causal, off)
    tq, tk, tv = (torch.tensor(a, requires_grad=True) for a in (q, k, v))
    G = H // Hkv
    kr = tk.repeat_interleave(G, dim=2)
    vr = tv.repeat_interleave(G, dim=2)
    s = torch.einsum("bqhd,bkhd->bhqk", tq, kr) * 0.125
    i = torch.arange(Sq)[:, None]
    j = torch.arange(Skv)[None, :]
    vis = (j <= i + off) if causal else torch.ones(Sq, Skv, dtype=torch.bool)
    s = s.masked_fill(~vis, float("-inf"))
    p = torch.softmax(s, -1).nan_to_num(0.0)   # rows with no visible key -> 0
    o = torch.einsum("bhqk,bkhd->bqhd", p, vr)
    o.backward(torch.tensor(do))
    assert relerr(dq, tq.grad.numpy()) < 1e-6
    assert relerr(dk, tk.grad.numpy()) < 1e-6
    assert relerr(dv, tv.grad.numpy()) < 1e-6


def test_gqa_prefill_lse_closed_form():
    """lse is the log of the softmax denominator: exp(scale*s - lse) sums to 1
    over the visible keys, and matches a brute-force log-sum-exp."""
    r = rng(42)
    q = r.standard_normal((1, 20, 4, 64))
    k = r.standard_normal((1, 26, 2, 64))
    lse = O.gqa_prefill_lse(q, k, 0.125, True, 6)
    for h in range(4):
        for i in range(20):
            s = [0.125 * q[0, i, h] @ k[0, j, h // 2] for j in range(min(26, i + 7))]
            assert abs(lse[0, h, i] - math.log(sum(math.exp(x) for x in s))) < 1e-9


def test_backward_check_catches_planted_slip():
    """Dropping the rowsum term of the softmax backward (a plausible slip)
    moves dq far outside the tolerance the GPU is held to."""
    r = rng(43)
    q, k, v, do = (r.standard_normal(sh) for sh in ((1, 16, 2, 64), (1, 16, 1, 64), (1, 16, 1, 64), (1, 16, 2, 64)))
    dq, _, _ = O.gqa_prefill_backward(q, k, v, do, 0.125)
    vis = O._visible(16, 16, True, 0)
    wrong = np.zeros_like(dq)
    for h in range(2):
        s = np.where(vis, 0.125 * q[0, :, h] @ k[0, :, 0].T, -np.inf)
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        wrong[0, :, h] = 0.125 * (p * (do[0, :, h] @ v[0, :, 0].T)) @ k[0, :, 0]
    assert relerr(wrong, dq) > 0.05


@pytest.mark.parametrize("B,Sq,Skv,H,Hkv,causal,off", [(1, 40, 40, 8, 2, True, 0), (2, 17, 30, 4, 4, True, 13),
                                                       (1, 24, 24, 8, 1, False, 0), (1, 9, 12, 2, 1, True, -3)])
def test_backward_from_residuals_equals_chain_form(B, Sq, Skv, H, Hkv, causal, off):
    """Given the exact forward output and lse, the residual form (P from lse,
    D = rowsum(dO*O)) reproduces the chain form; a natural-vs-base-2 lse slip
    does not."""
    r = rng(44)
    q, k, v, do = (r.standard_normal(sh) for sh in ((B, Sq, H, 64), (B, Skv, Hkv, 64),
                                                     (B, Skv, Hkv, 64), (B, Sq, H, 64)))
    G = H // Hkv
    vis = O._visible(Sq, Skv, causal, off)
    o = np.zeros_like(q)
    for b in range(B):
        for h in range(H):
            s = np.where(vis, 0.125 * q[b, :, h] @ k[b, :, h // G].T, -np.inf)
            m = s.max(1, keepdims=True)
            e = np.where(vis, np.exp(s - np.where(np.isfinite(m), m, 0.0)), 0.0)
            t = e.sum(1, keepdims=True)
            o[b, :, h] = np.divide(e, t, out=np.zeros_like(e), where=t > 0) @ v[b, :, h // G]
    lse = O.gqa_prefill_lse(q, k, 0.125, causal, off)
    chain = O.gqa_prefill_backward(q, k, v, do, 0.125, causal, off)
    res = O.gqa_prefill_backward_from_residuals(q, k, v, o, lse, do, 0.125, causal, off)
    for a, b_ in zip(res, chain):
        assert relerr(a, b_) < 1e-6
    wrong = O.gqa_prefill_backward_from_residuals(q, k, v, o, lse / math.log(2), do, 0.125, causal, off)
    assert relerr(wrong[0], chain[0]) > 0.05


# ---------------------------------------------------- projection + RoPE
def test_linear_rope_pins():
    """Without rotation it is op_mm's product; the rotation is the identity at
    position 0, keeps every pair's norm, is undone by the pinned RoPE backward
    (the transpose rotation), and leaves columns past rope_cols alone."""
    r = rng(45)
    x = r.standard_normal((6, 40)).astype(np.float32)
    w = r.standard_normal((40, 192)).astype(np.float32)
    plain = O.linear_rope(x, w)
    assert relerr(plain, O.matmul(x, w)) < 1e-5
    y = O.linear_rope(x, w, 128, 0, 64, 1e4)
    assert np.allclose(y[0], plain[0], rtol=1e-6, atol=1e-6)          # row 0: angle 0
    assert np.array_equal(y[:, 128:], plain[:, 128:])
    n_y = np.hypot(y[:, :128:2], y[:, 1:128:2])
    n_p = np.hypot(plain[:, :128:2], plain[:, 1:128:2])
    assert np.allclose(n_y, n_p, rtol=1e-5)
    y7 = O.linear_rope(x, w, 128, 7, 64, 1e4)
    back = O.rope_backward(y7[:, :128], 7, 64, 1e4)
    assert relerr(back, plain[:, :128]) < 1e-5
    # a planted slip: rotating the V columns too moves them
    wrong = plain.copy()
    wrong[:, :] = O.rope(plain, 7, 64, 1e4)
    assert relerr(wrong[:, 128:], y7[:, 128:]) > 1e-2
