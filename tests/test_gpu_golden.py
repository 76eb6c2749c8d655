"""GPU kernels against the committed golden fixtures (`tests/golden/*.npz`):
the same seeded inputs the CPU oracle's expected outputs were computed from
(and checked against torch fp64 when written), run through the C ABI.  Bounds:
fp32 max relative error 1e-4, bf16 2e-2; the repeat_kv mapping exact."""
import ctypes as C
import os

import numpy as np
import pytest
import torch

import bnhip as B
from gpu_util import BF16_TOL, FP32_TOL, assert_close, dev, host, require_gpu

pytestmark = pytest.mark.gpu
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def load(name):
    print(f"golden fixture {name}", flush=True)
    return np.load(os.path.join(HERE, name + ".npz"))


def V(t):
    return C.byref(B.view(t))


def test_golden_norm_rope():
    f = load("rmsnorm")
    x, w = dev(f["x"]), dev(f["weight"])
    y = torch.empty_like(x)
    B.call("bn_rmsnorm", V(x), V(w), V(y), float(f["p_eps"]), None)
    assert_close(host(y), f["y"], FP32_TOL, "rmsnorm")
    f = load("rope")
    a = (int(f["p_offset"]), int(f["p_head_dim"]), float(f["p_theta"]))
    x, dy = dev(f["x"]), dev(f["dy"])
    y, dx = torch.empty_like(x), torch.empty_like(dy)
    B.call("bn_rope", V(x), V(y), *a, None)
    B.call("bn_rope_backward", V(dy), V(dx), *a, None)
    assert_close(host(y), f["y"], FP32_TOL, "rope")
    assert_close(host(dx), f["dx"], FP32_TOL, "rope_backward")
    f = load("rmsnorm_rope")
    args = (float(f["p_eps"]), int(f["p_offset"]), int(f["p_head_dim"]), float(f["p_theta"]))
    for dt, tol in ((torch.float32, FP32_TOL), (torch.bfloat16, BF16_TOL)):  # x is bf16-exact
        x, w = dev(f["x"], dt), dev(f["weight"], dt)
        y = torch.empty_like(x)
        B.call("bn_rmsnorm_rope", V(x), V(w), V(y), *args, None)
        assert_close(host(y), f["y"], tol, f"rmsnorm_rope {dt}")
    f = load("rmsnorm_backward")
    x, w, dy = dev(f["x"]), dev(f["weight"]), dev(f["dy"])
    dx, dw = torch.empty_like(x), torch.empty_like(w)
    B.call("bn_rmsnorm_backward", V(x), V(w), V(dy), V(dx), V(dw), float(f["p_eps"]), None)
    assert_close(host(dx), f["dx"], FP32_TOL, "rmsnorm_backward dx")
    assert_close(host(dw), f["dw"], FP32_TOL, "rmsnorm_backward dw")
    f = load("add_rmsnorm")
    h, y = B.add_rmsnorm(dev(f["x"]), dev(f["delta"]), dev(f["weight"]), float(f["p_eps"]))
    assert_close(host(h), f["h"], FP32_TOL, "add_rmsnorm h")
    assert_close(host(y), f["y"], FP32_TOL, "add_rmsnorm y")
    f = load("silu_mul")
    assert_close(host(B.silu_mul(dev(f["gate"]), dev(f["up"]))), f["out"], FP32_TOL, "silu_mul")


def test_golden_softmax():
    f = load("softmax")
    for tag in ("known", "c0", "c2", "full"):
        x = dev(f[f"x_{tag}"])
        rows, cols, causal, off = (x.shape[0], x.shape[1], 0, 0) if tag == "known" else \
            (int(v) for v in f[f"cfg_{tag}"])
        y = torch.empty_like(x)
        B.call("bn_softmax", V(x), V(y), causal, off, None)
        assert_close(host(y), f[f"y_{tag}"], FP32_TOL, f"softmax {tag}")
        if tag != "known":
            yd, dyd = dev(f[f"y_{tag}"]), dev(f[f"dy_{tag}"])
            dx = torch.empty_like(yd)
            B.call("bn_softmax_backward", V(yd), V(dyd), V(dx), None)
            assert_close(host(dx), f[f"dx_{tag}"], FP32_TOL, f"softmax_backward {tag}")


def test_golden_surface():
    f = load("surface")
    kv = dev(f["kv"])
    rep = torch.empty((kv.shape[0], kv.shape[1] * int(f["p_n_rep"])), device="cuda")
    B.call("bn_repeat_kv", V(kv), V(rep), int(f["p_head_dim"]), int(f["p_n_rep"]), None)
    np.testing.assert_array_equal(host(rep), f["repeat_kv"])
    a, b = dev(f["a"]), dev(f["b"])
    c = torch.empty((a.shape[0], b.shape[1]), device="cuda")
    B.call("bn_matmul", V(a), V(b), V(c), None)
    assert_close(host(c), f["c"], FP32_TOL, "matmul")
    y = B.linear_rope(dev(f["x"]), dev(f["w"]), rope_cols=int(f["p_rope_cols"]),
                      position_offset=int(f["p_offset"]), head_dim=int(f["p_head_dim"]),
                      theta=float(f["p_theta"]))
    assert_close(host(y), f["y_linear_rope"], FP32_TOL, "linear_rope")


def test_golden_attention():
    f = load("gqa_prefill")
    sc = float(f["p_scale"])
    for dt, tol in ((torch.float32, FP32_TOL), (torch.bfloat16, BF16_TOL)):  # bf16-exact inputs
        q, k, v = dev(f["q"], dt), dev(f["k"], dt), dev(f["v"], dt)
        o, lse = B.gqa_prefill_lse(q, k, v, scale=sc)
        assert_close(host(o), f["o"], tol, f"gqa_prefill {dt}")
        assert_close(host(lse), f["lse"], FP32_TOL if dt == torch.float32 else 1e-3, f"lse {dt}")
    # Sk != Sq with a position offset (fp32 inputs: the fp32 kernel)
    o2 = B.gqa_prefill(dev(f["q2"]), dev(f["k2"]), dev(f["v2"]), scale=sc, causal=True,
                       seq_offset=int(f["p_offset2"]))
    assert_close(host(o2), f["o2"], FP32_TOL, "gqa_prefill offset")
    f = load("gqa_decode")
    o = B.gqa_decode(dev(f["q"]), dev(f["k_cache"]), dev(f["v_cache"]),
                     torch.from_numpy(f["seq_lens"]).cuda(), scale=float(f["p_scale"]))
    assert_close(host(o), f["o"], FP32_TOL, "gqa_decode")
    f = load("fused_head_attention")
    o = B.fused_head_attention(dev(f["q"]), dev(f["k"]), dev(f["v"]), int(f["p_n_heads"]),
                               int(f["p_n_kv_heads"]), int(f["p_head_dim"]), scale=float(f["p_scale"]))
    assert_close(host(o), f["o"], FP32_TOL, "fused_head_attention")


def test_golden_backward():
    f = load("gqa_prefill_backward")
    sc = float(f["p_scale"])
    q, k, v, do = (dev(f[n], torch.bfloat16) for n in ("q", "k", "v", "do"))  # bf16-exact
    o, lse = B.gqa_prefill_lse(q, k, v, scale=sc)
    dq, dk, dv = B.gqa_prefill_backward(q, k, v, o, do, lse, scale=sc)
    for nm, got in (("dq", dq), ("dk", dk), ("dv", dv)):
        assert_close(host(got), f[nm], BF16_TOL, f"gqa_prefill_backward {nm}")
