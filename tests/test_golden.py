"""The committed golden fixtures (`tests/golden/*.npz`, written by
`tests/golden/make_golden.py` after checking every expected output against an
independent torch fp64 computation) stay reproduced by the CPU oracle: the C
restatements bit for bit, the fp64-numpy compositions (the projection, lse,
backward) to the last fp32 ulp.  A change to the oracle that moves any of
these values fails here before it can move a GPU parity verdict."""
import os

import numpy as np
import pytest

from oracle import oracle as O

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(HERE, name + ".npz"))


NAMES = ["rmsnorm", "rope", "rmsnorm_rope", "rmsnorm_backward", "add_rmsnorm", "silu_mul",
         "softmax", "surface", "gqa_prefill", "gqa_decode", "fused_head_attention",
         "gqa_prefill_backward"]


def test_every_fixture_present_with_seed():
    for n in NAMES:
        f = load(n)
        assert "seed" in f.files and int(f["seed"]) > 0, n


def eq(got, ref):
    np.testing.assert_array_equal(np.asarray(got, np.float32), ref)


def close(got, ref):
    np.testing.assert_allclose(np.asarray(got, np.float32), ref, rtol=1e-6, atol=1e-7)


def test_norm_rope_fixtures():
    f = load("rmsnorm")
    eq(O.rmsnorm(f["x"], f["weight"], float(f["p_eps"])), f["y"])
    f = load("rope")
    a = (int(f["p_offset"]), int(f["p_head_dim"]), float(f["p_theta"]))
    eq(O.rope(f["x"], *a), f["y"])
    eq(O.rope_backward(f["dy"], *a), f["dx"])
    f = load("rmsnorm_rope")
    eq(O.rmsnorm_rope(f["x"], f["weight"], float(f["p_eps"]), int(f["p_offset"]),
                      int(f["p_head_dim"]), float(f["p_theta"])), f["y"])
    f = load("rmsnorm_backward")
    dx, dw = O.rmsnorm_backward(f["x"], f["weight"], f["dy"], float(f["p_eps"]))
    eq(dx, f["dx"])
    eq(dw, f["dw"])
    f = load("add_rmsnorm")
    h, y = O.add_rmsnorm(f["x"], f["delta"], f["weight"], float(f["p_eps"]))
    eq(h, f["h"])
    eq(y, f["y"])
    f = load("silu_mul")
    eq(O.silu_mul(f["gate"], f["up"]), f["out"])


def test_softmax_fixtures():
    f = load("softmax")
    eq(O.softmax(f["x_known"]), f["y_known"])
    for tag in ("c0", "c2", "full"):
        rows, cols, causal, off = (int(v) for v in f[f"cfg_{tag}"])
        eq(O.softmax(f[f"x_{tag}"], bool(causal), off), f[f"y_{tag}"])
        eq(O.softmax_backward(f[f"y_{tag}"], f[f"dy_{tag}"]), f[f"dx_{tag}"])


def test_surface_fixtures():
    f = load("surface")
    eq(O.repeat_kv(f["kv"], int(f["p_head_dim"]), int(f["p_n_rep"])), f["repeat_kv"])
    eq(O.matmul(f["a"], f["b"]), f["c"])
    close(O.linear_rope(f["x"], f["w"], int(f["p_rope_cols"]), int(f["p_offset"]),
                        int(f["p_head_dim"]), float(f["p_theta"])), f["y_linear_rope"])


def test_attention_fixtures():
    f = load("gqa_prefill")
    sc = float(f["p_scale"])
    eq(O.gqa_prefill(f["q"], f["k"], f["v"], sc, True, 0), f["o"])
    eq(O.gqa_prefill(f["q2"], f["k2"], f["v2"], sc, True, int(f["p_offset2"])), f["o2"])
    close(O.gqa_prefill_lse(f["q"], f["k"], sc, True, 0), f["lse"])
    f = load("gqa_decode")
    eq(O.gqa_decode(f["q"], f["k_cache"], f["v_cache"], f["seq_lens"], float(f["p_scale"])), f["o"])
    f = load("fused_head_attention")
    eq(O.fused_head_attention(f["q"], f["k"], f["v"], int(f["p_head_dim"]),
                              int(f["p_n_heads"]) // int(f["p_n_kv_heads"]), float(f["p_scale"]),
                              True, 0), f["o"])
    f = load("gqa_prefill_backward")
    dq, dk, dv = O.gqa_prefill_backward(f["q"], f["k"], f["v"], f["do"], float(f["p_scale"]), True, 0)
    close(dq, f["dq"])
    close(dk, f["dk"])
    close(dv, f["dv"])
