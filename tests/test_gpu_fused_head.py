"""GPU parity of bn_fused_head_attention (the reference's fused-head chain
repeat_kv -> q @ k_rep^T -> * scale -> causal softmax -> @ v_rep in one
launch) against the oracle's op-by-op chain, called through the C ABI on
torch-allocated device buffers.  Bound: fp32, max relative error 1e-4."""
import ctypes as C

import numpy as np
import pytest
import torch

import bnhip as B
from gpu_util import FP32_TOL, assert_close, dev, host, require_gpu
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def V(t):
    return C.byref(B.view(t))


def run(q, k, v, H, Hkv, D, sc, causal, off, out=None):
    out = torch.full((q.shape[0], H * D), float("nan"), device="cuda") if out is None else out
    print(f"fused-head attention Sq={q.shape[0]} Sk={k.shape[0]} H={H} Hkv={Hkv} D={D} "
          f"causal={causal} off={off}", flush=True)
    B.call("bn_fused_head_attention", V(q), V(k), V(v), V(out), H, Hkv, D, sc, int(causal), off,
           None)
    return out


@pytest.mark.parametrize("Sq,Sk,H,Hkv,D,causal,off", [
    (128, 128, 32, 4, 64, True, 0),      # config 1
    (1, 1, 32, 4, 64, True, 0),
    (3, 3, 32, 4, 64, True, 0),
    (65, 65, 32, 4, 64, True, 0),        # one row past a 4-row block, keys past a 64-key tile
    (130, 130, 32, 4, 64, False, 0),
    (16, 40, 32, 4, 64, True, 24),       # rows at positions 24..39 of a 40-key context
    (7, 7, 32, 4, 64, True, -3),         # rows 0..2 see no key: zeros
    (33, 33, 8, 8, 64, True, 0),         # n_rep 1, KV*D = 512 (the limit)
    (20, 20, 4, 1, 64, True, 2),         # one KV head: KV*D = 64
    (512, 512, 32, 4, 64, True, 0),      # the 512-token prompt of config 4 (matrix-core path)
    (511, 511, 32, 4, 64, True, 0),      # the longest prompt of the VALU kernel
    (50, 50, 12, 4, 4, True, 0),         # head_dim 4
])
def test_fused_head_attention(Sq, Sk, H, Hkv, D, causal, off):
    r = np.random.default_rng(Sq * 131 + Sk)
    q = r.standard_normal((Sq, H * D)).astype(np.float32)
    k = r.standard_normal((Sk, Hkv * D)).astype(np.float32)
    v = r.standard_normal((Sk, Hkv * D)).astype(np.float32)
    sc = 1.0 / np.sqrt(D)
    qd, kd, vd = dev(q), dev(k), dev(v)
    got = host(run(qd, kd, vd, H, Hkv, D, sc, causal, off))
    ref = O.fused_head_attention(q, k, v, D, H // Hkv, sc, causal, off)
    assert_close(got, ref, FP32_TOL, "fused-head attention")
    if off < 0:
        assert not got[:-off].any()


def test_fused_head_attention_packed_views_and_strided_output():
    """q, k, v as column slices of one [S, (H+2Hkv)D] projection (the QKV
    layout of the model), output into a column slice of a wider buffer."""
    S, H, Hkv, D = 77, 32, 4, 64
    r = np.random.default_rng(5)
    qkv = r.standard_normal((S, (H + 2 * Hkv) * D)).astype(np.float32)
    q, k, v = qkv[:, :H * D], qkv[:, H * D:(H + Hkv) * D], qkv[:, (H + Hkv) * D:]
    d = dev(qkv)
    big = torch.full((S, H * D + 64), float("nan"), device="cuda")
    out = big[:, 32:32 + H * D]
    run(d[:, :H * D], d[:, H * D:(H + Hkv) * D], d[:, (H + Hkv) * D:], H, Hkv, D, 0.125, True, 0,
        out=out)
    got = host(big)
    ref = O.fused_head_attention(q, k, v, D, H // Hkv, 0.125, True, 0)
    assert_close(got[:, 32:32 + H * D], ref, FP32_TOL, "packed views")
    assert np.isnan(got[:, :32]).all() and np.isnan(got[:, 32 + H * D:]).all()  # untouched


def test_fused_head_attention_large_scores_and_no_keys():
    """Scores with a standard deviation of ~45 (the running max moves as tiles
    arrive; beyond that, fp32 reassociation of the dots alone moves the
    near-tied weights past 1e-4) and an empty key set (seq_kv = 0: the
    chain's P @ V over nothing is 0)."""
    S, H, Hkv, D = 200, 8, 2, 64
    r = np.random.default_rng(6)
    q = (r.standard_normal((S, H * D)) * 2).astype(np.float32)
    k = (r.standard_normal((S, Hkv * D)) * 2).astype(np.float32)
    v = r.standard_normal((S, Hkv * D)).astype(np.float32)
    got = host(run(dev(q), dev(k), dev(v), H, Hkv, D, 0.5, True, 0))
    ref = O.fused_head_attention(q, k, v, D, H // Hkv, 0.5, True, 0)
    assert_close(got, ref, FP32_TOL, "large scores")
    k0 = torch.empty((0, Hkv * D), device="cuda")
    got0 = host(run(dev(q), k0, k0, H, Hkv, D, 1.0, True, 0))
    assert not got0.any()


def test_fused_head_attention_rejects_misaligned_rows():
    """Rows off a 16-byte boundary are refused before any launch (the kernel
    reads float4s); the op-by-op chain serves such views."""
    q2 = torch.zeros((4, 2049), device="cuda")
    k = torch.zeros((4, 256), device="cuda")
    out = torch.zeros((4, 2048), device="cuda")
    with pytest.raises(RuntimeError, match="16-byte"):
        B.call("bn_fused_head_attention", V(q2[:, 1:]), V(k), V(k), V(out), 32, 4, 64, 0.125, 1,
               0, None)


@pytest.mark.parametrize("Sq,Sk,H,Hkv,causal,off,D", [
    (600, 1100, 32, 4, False, 0, 64),   # non-causal, ragged row tile and key block
    (700, 700, 16, 4, True, 0, 64),     # n_rep 4
    (530, 800, 32, 4, True, 270, 64),   # rows at positions 270..799 of an 800-key context
    (560, 560, 32, 4, True, -40, 64),   # rows 0..39 see no key: zeros
    (520, 520, 16, 2, True, 0, 128),    # head_dim 128, two KV heads (KV*D = 256)
    (515, 515, 8, 8, True, 3, 32),      # head_dim 32, n_rep 1
])
def test_fused_head_attention_matrix_core_rows(Sq, Sk, H, Hkv, causal, off, D):
    """The matrix-core path (seq_q >= 512, KV*D = 256): the whole output
    computed, 64-row blocks at both ends checked against the oracle chain on
    the same rows (a block starting at row i0 sits at position i0 + off)."""
    r = np.random.default_rng(Sq * 7 + Sk)
    q = r.standard_normal((Sq, H * D)).astype(np.float32)
    k = r.standard_normal((Sk, Hkv * D)).astype(np.float32)
    v = r.standard_normal((Sk, Hkv * D)).astype(np.float32)
    sc = 1.0 / np.sqrt(D)
    got = host(run(dev(q), dev(k), dev(v), H, Hkv, D, sc, causal, off))
    assert np.isfinite(got).all()
    if off < 0:
        assert not got[:-off].any()
    for i0 in (max(0, -off), Sq - 64):
        ref = O.fused_head_attention(q[i0:i0 + 64], k, v, D, H // Hkv, sc, causal, i0 + off)
        assert_close(got[i0:i0 + 64], ref, FP32_TOL, f"rows {i0}..{i0 + 63}")


@pytest.mark.parametrize("S", [2048])
def test_fused_head_attention_long_prompt_blocks(S):
    """The matrix-core path at S = 2048 (TinyLLaMA's heads): 64-row blocks at
    the start, middle and end of the causal output against the oracle chain
    on the same rows (rows i0.. at positions i0.. see keys 0..i0+r), and
    every row of the output finite."""
    H, Hkv, D = 32, 4, 64
    r = np.random.default_rng(2048)
    q = r.standard_normal((S, H * D)).astype(np.float32)
    k = r.standard_normal((S, Hkv * D)).astype(np.float32)
    v = r.standard_normal((S, Hkv * D)).astype(np.float32)
    got = host(run(dev(q), dev(k), dev(v), H, Hkv, D, 0.125, True, 0))
    assert np.isfinite(got).all()
    for i0 in (0, 1000, S - 64):
        ref = O.fused_head_attention(q[i0:i0 + 64], k[:i0 + 64], v[:i0 + 64], D, H // Hkv, 0.125,
                                     True, i0)
        assert_close(got[i0:i0 + 64], ref, FP32_TOL, f"S={S} rows {i0}..{i0 + 63}")


def test_fused_head_attention_matrix_core_views_and_repeats():
    """The matrix-core path on packed column views of one QKV buffer, into a
    column slice of a wider output (columns outside untouched), and the same
    bits on a repeated call."""
    S, H, Hkv, D = 540, 32, 4, 64
    r = np.random.default_rng(7)
    qkv = r.standard_normal((S, (H + 2 * Hkv) * D)).astype(np.float32)
    q, k, v = qkv[:, :H * D], qkv[:, H * D:(H + Hkv) * D], qkv[:, (H + Hkv) * D:]
    d = dev(qkv)
    big = torch.full((S, H * D + 64), float("nan"), device="cuda")
    out = big[:, 32:32 + H * D]
    args = (d[:, :H * D], d[:, H * D:(H + Hkv) * D], d[:, (H + Hkv) * D:], H, Hkv, D, 0.125, True, 0)
    run(*args, out=out)
    got = host(big)
    ref = O.fused_head_attention(q, k, v, D, H // Hkv, 0.125, True, 0)
    assert_close(got[:, 32:32 + H * D], ref, FP32_TOL, "matrix-core packed views")
    assert np.isnan(got[:, :32]).all() and np.isnan(got[:, 32 + H * D:]).all()
    run(*args, out=out)
    assert np.array_equal(host(big), got, equal_nan=True)
