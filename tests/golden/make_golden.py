"""Writes the golden fixtures `tests/golden/*.npz`: small seeded inputs and the
CPU oracle's outputs for every function on the path, at tiny shapes.

Test infrastructure: it imports the oracle as the checker and torch (CPU) as
the independent check.  Before a fixture is written, each expected output is
compared with an independent fp64 computation (torch autograd, SDPA with the
GQA head expansion, closed forms), so a fixture never records an oracle slip.
Each file holds the inputs, the expected outputs, the seed and the scalar
parameters (`p_*` entries); `tests/test_golden.py` checks that the oracle still
reproduces them bit for bit, `tests/test_gpu_golden.py` runs the HIP kernels on
the same inputs.

Run from the repository root:  python tests/golden/make_golden.py
"""
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import oracle as O  # noqa: E402


def t64(a):
    return torch.from_numpy(np.asarray(a, np.float64))


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(float(np.max(np.abs(b))), 1e-30))


def bf16(a):
    return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16).float().numpy()


def check(name, got, ref, tol):
    r = rel(got, ref)
    assert r <= tol, f"{name}: oracle vs independent fp64 check {r:.3e} > {tol:.0e}"


def rope_ref(x, off, D, theta):
    """op_rope in fp64 on the reference's fp32 angle formation (op_rope.cuh:79-98)."""
    x = np.asarray(x, np.float64)
    y = x.copy()
    for c in range(0, x.shape[1], 2):
        p = (c % D) // 2
        e = np.float32(2 * p) / np.float32(D)
        freq = np.float32(1.0 / float(np.float32(np.power(np.float32(theta), e))))
        for r in range(x.shape[0]):
            ang = float(np.float32(np.float32(r + off) * freq))
            cs, sn = math.cos(ang), math.sin(ang)
            y[r, c] = x[r, c] * cs - x[r, c + 1] * sn
            y[r, c + 1] = x[r, c] * sn + x[r, c + 1] * cs
    return y


def sdpa_ref(q, k, v, scale, causal, off):
    """Per-head GQA attention in torch fp64: q [B,Sq,H,D], k/v [B,Skv,Hkv,D]."""
    q, k, v = t64(q), t64(k), t64(v)
    G = q.shape[2] // k.shape[2]
    k = k.repeat_interleave(G, dim=2)
    v = v.repeat_interleave(G, dim=2)
    s = torch.einsum("bqhd,bkhd->bhqk", q, k) * scale
    if causal:
        i = torch.arange(q.shape[1])[:, None]
        j = torch.arange(k.shape[1])[None, :]
        s = s.masked_fill(j > i + off, float("-inf"))
    p = torch.nan_to_num(torch.softmax(s, -1), nan=0.0)
    return torch.einsum("bhqk,bkhd->bqhd", p, v).numpy()


def write(name, seed, params, **arrays):
    kw = {k: np.asarray(v) for k, v in arrays.items()}
    for k, v in params.items():
        kw["p_" + k] = np.asarray(v)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), seed=np.int64(seed), **kw)
    print(f"{name}: {', '.join(f'{k}{list(np.shape(v))}' for k, v in arrays.items())}")


def main():
    O.build()
    # ------------------------------------------------ RMSNorm / RoPE / fused
    r = np.random.default_rng(11)
    x = r.standard_normal((5, 300)).astype(np.float32)
    w = r.uniform(0.5, 1.5, (1, 300)).astype(np.float32)
    y = O.rmsnorm(x, w, 1e-5)
    xt = t64(x)
    check("rmsnorm", y, (xt / torch.sqrt((xt * xt).mean(1, keepdim=True) + 1e-5) * t64(w)).numpy(), 1e-6)
    write("rmsnorm", 11, {"eps": 1e-5}, x=x, weight=w, y=y)

    r = np.random.default_rng(12)
    x = r.standard_normal((6, 256)).astype(np.float32)
    y = O.rope(x, 3, 64, 1e4)
    check("rope", y, rope_ref(x, 3, 64, 1e4), 1e-5)
    dy = r.standard_normal((6, 256)).astype(np.float32)
    dx = O.rope_backward(dy, 3, 64, 1e4)
    check("rope_backward", O.rope(dx, 3, 64, 1e4), dy, 1e-5)   # the inverse rotation
    write("rope", 12, {"offset": 3, "head_dim": 64, "theta": 1e4}, x=x, y=y, dy=dy, dx=dx)

    r = np.random.default_rng(13)
    x = bf16(r.standard_normal((4, 256)))
    w = bf16(r.uniform(0.5, 1.5, (1, 256)))
    y = O.rmsnorm_rope(x, w, 1e-5, 5, 64, 1e4)
    check("rmsnorm_rope", y, rope_ref(O.rmsnorm(x, w, 1e-5), 5, 64, 1e4), 1e-5)
    write("rmsnorm_rope", 13, {"eps": 1e-5, "offset": 5, "head_dim": 64, "theta": 1e4},
          x=x, weight=w, y=y)

    r = np.random.default_rng(14)
    x = r.standard_normal((5, 300)).astype(np.float32)
    w = r.uniform(0.5, 1.5, (1, 300)).astype(np.float32)
    dy = r.standard_normal((5, 300)).astype(np.float32)
    dx, dw = O.rmsnorm_backward(x, w, dy, 1e-5)
    xt, wt = t64(x).requires_grad_(), t64(w).requires_grad_()
    (xt / torch.sqrt((xt * xt).mean(1, keepdim=True) + 1e-5) * wt).backward(t64(dy))
    check("rmsnorm_backward dx", dx, xt.grad.numpy(), 1e-5)
    check("rmsnorm_backward dw", dw, wt.grad.numpy(), 1e-5)
    write("rmsnorm_backward", 14, {"eps": 1e-5}, x=x, weight=w, dy=dy, dx=dx, dw=dw)

    r = np.random.default_rng(15)
    x = r.standard_normal((3, 256)).astype(np.float32)
    d = r.standard_normal((3, 256)).astype(np.float32)
    w = r.uniform(0.5, 1.5, (1, 256)).astype(np.float32)
    h, y = O.add_rmsnorm(x, d, w, 1e-5)
    ht = t64(x) + t64(d)
    check("add_rmsnorm", y, (ht / torch.sqrt((ht * ht).mean(1, keepdim=True) + 1e-5) * t64(w)).numpy(), 1e-6)
    write("add_rmsnorm", 15, {"eps": 1e-5}, x=x, delta=d, weight=w, h=h, y=y)

    r = np.random.default_rng(16)
    g = (3 * r.standard_normal((4, 128))).astype(np.float32)
    u = r.standard_normal((4, 128)).astype(np.float32)
    o = O.silu_mul(g, u)
    check("silu_mul", o, (torch.nn.functional.silu(t64(g)) * t64(u)).numpy(), 1e-6)
    write("silu_mul", 16, {}, gate=g, up=u, out=o)

    # ------------------------------------------------ softmax and its backward
    r = np.random.default_rng(17)
    cases = {}
    for tag, (rows, cols, causal, off) in {"c0": (8, 8, 1, 0), "c2": (5, 9, 1, 2),
                                           "full": (4, 7, 0, 0)}.items():
        x = (3 * r.standard_normal((rows, cols))).astype(np.float32)
        y = O.softmax(x, bool(causal), off)
        s = t64(x)
        if causal:
            s = s.masked_fill(torch.arange(cols)[None, :] > torch.arange(rows)[:, None] + off, float("-inf"))
        check("softmax " + tag, y, torch.softmax(s, 1).numpy(), 1e-6)
        dy = r.standard_normal((rows, cols)).astype(np.float32)
        dx = O.softmax_backward(y, dy)
        yt = t64(y)
        check("softmax_backward " + tag, dx, (yt * (t64(dy) - (yt * t64(dy)).sum(1, keepdim=True))).numpy(), 1e-5)
        cases.update({f"x_{tag}": x, f"y_{tag}": y, f"dy_{tag}": dy, f"dx_{tag}": dx,
                      f"cfg_{tag}": np.array([rows, cols, causal, off])})
    ka = O.softmax(np.array([[1, 2, 3, 4]], np.float32))  # test_llama.py:96
    e = np.exp(np.arange(4) - 3.0)
    check("softmax known answer", ka, (e / e.sum())[None], 1e-6)
    write("softmax", 17, {}, x_known=np.array([[1, 2, 3, 4]], np.float32), y_known=ka, **cases)

    # ------------------------------------------------ layer surface
    r = np.random.default_rng(18)
    kv = r.standard_normal((5, 128)).astype(np.float32)
    rep = O.repeat_kv(kv, 64, 4)
    assert np.array_equal(rep, np.repeat(kv.reshape(5, 2, 64), 4, axis=1).reshape(5, 512))
    a = r.standard_normal((7, 33)).astype(np.float32)
    b = r.standard_normal((33, 5)).astype(np.float32)
    c = O.matmul(a, b)
    check("matmul", c, a.astype(np.float64) @ b, 1e-6)
    xl = r.standard_normal((3, 96)).astype(np.float32)
    wl = (r.standard_normal((96, 192)) / 10).astype(np.float32)
    yl = O.linear_rope(xl, wl, 128, 7, 64, 1e4)
    ref = xl.astype(np.float64) @ wl
    ref[:, :128] = rope_ref(ref[:, :128], 7, 64, 1e4)
    check("linear_rope", yl, ref, 1e-5)
    write("surface", 18, {"head_dim": 64, "n_rep": 4, "rope_cols": 128, "offset": 7, "theta": 1e4},
          kv=kv, repeat_kv=rep, a=a, b=b, c=c, x=xl, w=wl, y_linear_rope=yl)

    # ------------------------------------------------ attention
    # inputs exactly representable in bf16: one set serves the fp32 and bf16 kernels
    r = np.random.default_rng(19)
    q = bf16(r.standard_normal((1, 48, 8, 64)))
    k = bf16(r.standard_normal((1, 48, 2, 64)))
    v = bf16(r.standard_normal((1, 48, 2, 64)))
    o = O.gqa_prefill(q, k, v, 0.125, True, 0)
    check("gqa_prefill", o, sdpa_ref(q, k, v, 0.125, True, 0), 1e-5)
    lse = O.gqa_prefill_lse(q, k, 0.125, True, 0).astype(np.float32)
    q2 = r.standard_normal((1, 16, 8, 64)).astype(np.float32)
    k2 = r.standard_normal((1, 40, 2, 64)).astype(np.float32)
    v2 = r.standard_normal((1, 40, 2, 64)).astype(np.float32)
    o2 = O.gqa_prefill(q2, k2, v2, 0.125, True, 24)
    check("gqa_prefill offset", o2, sdpa_ref(q2, k2, v2, 0.125, True, 24), 1e-5)
    write("gqa_prefill", 19, {"scale": 0.125, "offset2": 24}, q=q, k=k, v=v, o=o, lse=lse,
          q2=q2, k2=k2, v2=v2, o2=o2)

    r = np.random.default_rng(20)
    qd = r.standard_normal((3, 8, 64)).astype(np.float32)
    kc = r.standard_normal((3, 40, 2, 64)).astype(np.float32)
    vc = r.standard_normal((3, 40, 2, 64)).astype(np.float32)
    lens = np.array([40, 17, 1], np.int32)
    od = O.gqa_decode(qd, kc, vc, lens, 0.125)
    for bb, L in enumerate(lens):
        check(f"gqa_decode b={bb}", od[bb], sdpa_ref(qd[bb][None, None], kc[bb:bb + 1, :L],
                                                     vc[bb:bb + 1, :L], 0.125, False, 0)[0, 0], 1e-5)
    write("gqa_decode", 20, {"scale": 0.125}, q=qd, k_cache=kc, v_cache=vc, seq_lens=lens, o=od)

    r = np.random.default_rng(21)
    qf = r.standard_normal((16, 512)).astype(np.float32)
    kf = r.standard_normal((16, 128)).astype(np.float32)
    vf = r.standard_normal((16, 128)).astype(np.float32)
    of = O.fused_head_attention(qf, kf, vf, 64, 4, 0.125, True, 0)
    kr = t64(kf).view(16, 2, 64).repeat_interleave(4, dim=1).reshape(16, 512)
    vr = t64(vf).view(16, 2, 64).repeat_interleave(4, dim=1).reshape(16, 512)
    s = (t64(qf) @ kr.T) * 0.125
    s = s.masked_fill(torch.arange(16)[None, :] > torch.arange(16)[:, None], float("-inf"))
    check("fused_head_attention", of, (torch.softmax(s, 1) @ vr).numpy(), 1e-5)
    write("fused_head_attention", 21, {"n_heads": 8, "n_kv_heads": 2, "head_dim": 64, "scale": 0.125},
          q=qf, k=kf, v=vf, o=of)

    r = np.random.default_rng(22)
    qg = bf16(r.standard_normal((1, 32, 4, 64)))
    kg = bf16(r.standard_normal((1, 32, 2, 64)))
    vg = bf16(r.standard_normal((1, 32, 2, 64)))
    dog = bf16(r.standard_normal((1, 32, 4, 64)))
    dq, dk, dv = O.gqa_prefill_backward(qg, kg, vg, dog, 0.125, True, 0)
    qt, kt, vt = (t64(a).requires_grad_() for a in (qg, kg, vg))
    G = 2
    s = torch.einsum("bqhd,bkhd->bhqk", qt, kt.repeat_interleave(G, dim=2)) * 0.125
    s = s.masked_fill(torch.arange(32)[None, :] > torch.arange(32)[:, None], float("-inf"))
    ot = torch.einsum("bhqk,bkhd->bqhd", torch.softmax(s, -1), vt.repeat_interleave(G, dim=2))
    ot.backward(t64(dog))
    for nm, got, ref in (("dq", dq, qt.grad), ("dk", dk, kt.grad), ("dv", dv, vt.grad)):
        check("gqa_prefill_backward " + nm, got, ref.numpy(), 1e-5)
    write("gqa_prefill_backward", 22, {"scale": 0.125}, q=qg, k=kg, v=vg, do=dog,
          dq=np.asarray(dq, np.float32), dk=np.asarray(dk, np.float32), dv=np.asarray(dv, np.float32))


if __name__ == "__main__":
    main()
