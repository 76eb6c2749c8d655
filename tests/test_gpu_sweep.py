"""Seeded random-shape parity sweep of the attention kernels against the CPU oracle.

The fixed cases in test_gpu_attention.py pin known edges one by one; this
sweep draws shapes from the regions the launch code treats differently and
compares every element with the oracle:

* prefill: query heads per KV head 1-16 (powers of two and not), so both the
  head-packed bf16 kernel (4 or 8 heads per KV head) and the per-head kernel
  with one and two row tiles per wave run; ragged row and key tails; causal
  offsets below zero, at Skv - Sq and past it; non-causal; the row
  log-sum-exp beside the output;
* decode: every kernel the host can pick (fp32 short-cache split, fp32 split-K,
  bf16 one workgroup per (sequence, KV head), bf16 split rows, bf16 split
  MFMA), with lengths 0, 1, max_len and past max_len among the random ones;
* backward (bf16): random groups, offsets and both mask modes;
* projection + RoPE (fp32, bf16): row-major weights over 1-300 rows (the
  tiled kernel, with and without a k split, and the few-rows streaming
  kernel) and output-major weights over 1-4 rows, random widths, rotated
  column counts and positions.

Each case prints its shape in the assertion message, and the seeds are fixed,
so a failure names a reproducible input.
"""
import numpy as np
import pytest
import torch

import bnhip as B
from oracle import oracle as O
from gpu_util import BF16_TOL, FP32_TOL, assert_close, bf16_round, dev, host, require_gpu
from test_gpu_attention import check_backward, nan_like

pytestmark = pytest.mark.gpu
TD = {"f32": torch.float32, "bf16": torch.bfloat16}
TOL = {"f32": FP32_TOL, "bf16": BF16_TOL}
SCALE = 0.125


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def draw(rng, shape, dtype):
    a = rng.standard_normal(shape).astype(np.float32)
    return bf16_round(a) if dtype == "bf16" else a


# ------------------------------------------------------------------- prefill
def prefill_case(i):
    """(B, Sq, Skv, H, Hkv, causal, off, dtype) of sweep case i."""
    rng = np.random.default_rng(7000 + i)
    dtype = ("f32", "bf16")[i % 2]
    group = int(rng.choice([1, 2, 3, 4, 5, 8, 16]))
    n_kv = int(rng.integers(1, 5))
    if group * n_kv > 48:
        n_kv = 48 // group
    Bn = int(rng.integers(1, 4))
    Sq, Skv = int(rng.integers(1, 330)), int(rng.integers(1, 330))
    causal = bool(rng.random() < 0.75)
    off = Skv - Sq + int(rng.integers(-40, 41)) if causal else 0
    return Bn, Sq, Skv, group * n_kv, n_kv, causal, off, dtype


@pytest.mark.parametrize("i", range(32))
def test_prefill_sweep(i):
    Bn, Sq, Skv, H, Hkv, causal, off, dtype = case = prefill_case(i)
    rng = np.random.default_rng(9000 + i)
    q = draw(rng, (Bn, Sq, H, 64), dtype)
    k = draw(rng, (Bn, Skv, Hkv, 64), dtype)
    v = draw(rng, (Bn, Skv, Hkv, 64), dtype)
    o, lse = B.gqa_prefill_lse(dev(q, TD[dtype]), dev(k, TD[dtype]), dev(v, TD[dtype]),
                               scale=SCALE, causal=causal, seq_offset=off)
    got = host(o)
    assert_close(got, O.gqa_prefill(q, k, v, SCALE, causal, off), TOL[dtype], f"prefill {case}")
    ref_lse = O.gqa_prefill_lse(q, k, SCALE, causal, off)
    got_lse = host(lse)
    fin = np.isfinite(ref_lse)
    assert np.array_equal(np.isfinite(got_lse), fin), f"lse {case}: visible-key rows differ"
    assert np.all(got_lse[~fin] == -np.inf)
    if fin.any():
        err = float(np.max(np.abs(got_lse[fin] - ref_lse[fin])))
        assert err <= TOL[dtype], f"lse {case}: max abs error {err:.3e}"
    if causal:  # rows that see no key are exactly zero
        blind = np.arange(Sq) + off < 0
        assert np.all(got[:, blind] == 0.0), f"prefill {case}: rows with no visible key"


@pytest.mark.parametrize("group,Hkv", [(16, 4), (1, 64), (2, 32)])
def test_prefill_sweep_two_row_tiles(group, Hkv):
    """bf16 groups that are not head-packed, at the size where each wave takes
    two 32-row tiles (B*H*ceil(Sq/256) >= 1024 workgroups' worth), checked on
    sampled (batch, head) pairs over the full causal range."""
    Bn, Sq, H = 2, 2048, group * Hkv
    assert Bn * H * ((Sq + 255) // 256) >= 1024
    rng = np.random.default_rng(9100 + group)
    q = draw(rng, (Bn, Sq, H, 64), "bf16")
    k = draw(rng, (Bn, Sq, Hkv, 64), "bf16")
    v = draw(rng, (Bn, Sq, Hkv, 64), "bf16")
    got = host(B.gqa_prefill(dev(q, torch.bfloat16), dev(k, torch.bfloat16), dev(v, torch.bfloat16),
                             scale=SCALE, causal=True))
    for b, h in [(0, 0), (1, H - 1), (int(rng.integers(Bn)), int(rng.integers(H)))]:
        g = h // group
        ref = O.gqa_prefill(q[b:b + 1, :, h:h + 1], k[b:b + 1, :, g:g + 1], v[b:b + 1, :, g:g + 1],
                            SCALE, True, 0)
        assert_close(got[b:b + 1, :, h:h + 1], ref, BF16_TOL, f"prefill G={group} b={b} h={h}")


# ------------------------------------------------------------------- decode
CUS = 256   # MI355X compute units: B * Hkv at or above this takes the whole-cache bf16 kernel


def decode_path(dtype, Bn, L, H, Hkv):
    """The kernel the host picks (mirrors the launch rules of bn_gqa_decode)."""
    if dtype == "f32":
        return "f32_short" if L <= 1024 and Bn * H <= 256 else "f32_split"
    if Bn * Hkv >= CUS:
        return "bf16_whole"
    return "bf16_rows" if Hkv % 4 == 0 else "bf16_mfma"


DECODE_TARGETS = ["f32_short", "f32_split", "bf16_whole", "bf16_rows", "bf16_mfma"]


def decode_case(target, i):
    rng = np.random.default_rng(8000 + 97 * DECODE_TARGETS.index(target) + i)
    G = int(rng.choice([1, 2, 4, 8]))
    if target == "f32_short":
        dtype, Hkv, L = "f32", int(rng.choice([1, 2, 4])), int(rng.integers(1, 1025))
        Bn = int(rng.integers(1, max(2, 256 // (G * Hkv)) + 1))
    elif target == "f32_split":
        dtype, Hkv, L = "f32", int(rng.choice([1, 2, 4])), int(rng.integers(1025, 3000))
        Bn = int(rng.integers(1, 6))
    elif target == "bf16_whole":
        dtype, Hkv, L = "bf16", int(rng.choice([4, 8])), int(rng.integers(64, 700))
        Bn = -(-CUS // Hkv) + int(rng.integers(0, 8))
    elif target == "bf16_rows":
        dtype, Hkv, L = "bf16", int(rng.choice([4, 8])), int(rng.integers(1, 3000))
        Bn = int(rng.integers(1, 9))
    else:
        dtype, Hkv, L = "bf16", int(rng.choice([1, 2, 3, 6])), int(rng.integers(1, 3000))
        Bn = int(rng.integers(1, 9))
    H = G * Hkv
    lens = rng.integers(1, L + 1, size=Bn)
    # the edges among the random lengths: empty, one key, the whole cache, past it
    for j, e in enumerate([0, 1, L, L + 3]):
        if Bn > j and rng.random() < 0.5:
            lens[rng.integers(Bn)] = e
    return dtype, Bn, L, H, Hkv, lens.astype(np.int32)


DECODE_SWEEP = [(t, i) for t in DECODE_TARGETS for i in range(4)] + \
    [("f32_short", i) for i in range(4, 12)]   # the in-launch merge of the short-cache split


@pytest.mark.parametrize("target,i", DECODE_SWEEP)
def test_decode_sweep(target, i):
    dtype, Bn, L, H, Hkv, lens = decode_case(target, i)
    assert decode_path(dtype, Bn, L, H, Hkv) == target
    what = f"decode {target} B={Bn} L={L} H={H} Hkv={Hkv}"
    rng = np.random.default_rng(8500 + 97 * DECODE_TARGETS.index(target) + i)
    q = draw(rng, (Bn, H, 64), dtype)
    kc = draw(rng, (Bn, L, Hkv, 64), dtype)
    vc = draw(rng, (Bn, L, Hkv, 64), dtype)
    qd, kd, vd = dev(q, TD[dtype]), dev(kc, TD[dtype]), dev(vc, TD[dtype])
    ld = torch.from_numpy(lens).cuda()
    out = B.gqa_decode(qd, kd, vd, ld, scale=SCALE)
    got = host(out)
    for b in range(Bn):
        Lb = int(min(max(lens[b], 0), L))
        if Lb == 0:
            assert np.all(got[b] == 0.0), f"{what}: empty cache b={b}"
            continue
        ref = O.gqa_decode(q[b:b + 1], kc[b:b + 1, :Lb], vc[b:b + 1, :Lb],
                           np.array([Lb], np.int32), SCALE)
        assert_close(got[b:b + 1], ref, TOL[dtype], f"{what} b={b} len={Lb}")
    # the same caches in a random other layout (bn_gqa_decode_strided): the same bits
    head_major, gap, pad = bool(rng.integers(2)), int(rng.choice([0, 1, 5])), int(rng.choice([0, 8, 32]))
    ks, vs = (strided_cache(c, head_major, gap, pad) for c in (kd, vd))
    got_s = B.gqa_decode(qd, ks, vs, ld, scale=SCALE)
    what_s = f"{what}: strided (head_major={head_major}, gap={gap}, pad={pad})"
    if target == "bf16_whole" and head_major and pad == 0:
        # a head's rows contiguous: long caches may stream with six waves
        assert_close(host(got_s), got, TOL[dtype], what_s)
    else:
        assert torch.equal(got_s, out), f"{what_s} differs"


def strided_cache(c, head_major, gap, pad):
    """c [B, L, Hkv, 64] copied into a wider storage -- head-major [B, Hkv, L + gap, 64 + pad]
    or token-major [B, L + gap, Hkv, 64 + pad], the unused elements NaN -- returned as a
    [B, L, Hkv, 64] view of it."""
    Bn, L, Hkv, D = c.shape
    if head_major:
        s = torch.full((Bn, Hkv, L + gap, D + pad), float("nan"), dtype=c.dtype, device=c.device)
        v = s[:, :, :L, :D].transpose(1, 2)
    else:
        s = torch.full((Bn, L + gap, Hkv, D + pad), float("nan"), dtype=c.dtype, device=c.device)
        v = s[:, :L, :, :D]
    v.copy_(c)
    return v


# ------------------------------------------------------------------- backward
@pytest.mark.parametrize("i", range(10))
def test_prefill_backward_sweep(i):
    rng = np.random.default_rng(7500 + i)
    group = int(rng.choice([1, 2, 3, 4, 8]))
    Hkv = int(rng.integers(1, 4))
    Bn, Sq, Skv = int(rng.integers(1, 3)), int(rng.integers(1, 260)), int(rng.integers(1, 260))
    causal = bool(rng.random() < 0.7)
    off = Skv - Sq + int(rng.integers(-30, 31)) if causal else 0
    H = group * Hkv
    case = (Bn, Sq, Skv, H, Hkv, causal, off)
    q = draw(rng, (Bn, Sq, H, 64), "bf16")
    k = draw(rng, (Bn, Skv, Hkv, 64), "bf16")
    v = draw(rng, (Bn, Skv, Hkv, 64), "bf16")
    do = draw(rng, (Bn, Sq, H, 64), "bf16")
    qd, kd, vd, dod = (dev(a, torch.bfloat16) for a in (q, k, v, do))
    o, lse = B.gqa_prefill_lse(qd, kd, vd, scale=SCALE, causal=causal, seq_offset=off)
    dq, dk, dv = B.gqa_prefill_backward(qd, kd, vd, o, dod, lse, scale=SCALE, causal=causal,
                                        seq_offset=off, dq=nan_like(qd), dk=nan_like(kd),
                                        dv=nan_like(vd))
    got = (host(dq), host(dk), host(dv))
    check_backward(got, q, k, v, do, host(o), host(lse), causal, off, f"backward sweep {case}")
    if causal:
        vis = np.arange(Skv)[None, :] <= np.arange(Sq)[:, None] + off
        assert np.all(got[0][:, ~vis.any(1)] == 0.0)
        assert np.all(got[1][:, ~vis.any(0)] == 0.0) and np.all(got[2][:, ~vis.any(0)] == 0.0)


# -------------------------------------------------- projection + RoPE
def linear_case(layout, i):
    """(M, K, N, rope_cols, offset, dtype): row-major w takes the tiled MFMA
    kernel (k split when the grid is small) or, for a few rows, the
    streaming kernel and its slab reduction; output-major w (the transposed
    view of [N, K] storage) the one-launch streaming kernel (1-4 rows)."""
    rng = np.random.default_rng(6000 + 31 * (layout == "out") + i)
    dtype = ("f32", "bf16")[i % 2]
    if layout == "row":
        M = int(rng.choice([1, 2, 3, 8, 9, 64, 65, 300]))
        K, N = 8 * int(rng.integers(1, 190)), 8 * int(rng.integers(1, 150))
    else:
        M = int(rng.integers(1, 5))
        K, N = 8 * int(rng.integers(1, 1100)), 2 * int(rng.integers(1, 1500))
        K = min(K, (16384 // M - 512) // 8 * 8)  # the staged x rows fit the kernel's LDS
    rc = 64 * int(rng.integers(0, N // 64 + 1))
    return M, K, N, rc, int(rng.integers(0, 5000)), dtype


@pytest.mark.parametrize("i", range(10))
@pytest.mark.parametrize("layout", ["row", "out"])
def test_linear_rope_sweep(layout, i):
    M, K, N, rc, off, dtype = case = linear_case(layout, i)
    rng = np.random.default_rng(6500 + 31 * (layout == "out") + i)
    x = draw(rng, (M, K), dtype)
    w = (draw(rng, (K, N), dtype) / np.sqrt(K)).astype(np.float32)
    if dtype == "bf16":
        w = bf16_round(w)
    if layout == "row":
        wd = dev(w, TD[dtype])
    else:  # [N, K] storage passed as its [K, N] view
        wd = dev(np.ascontiguousarray(w.T), TD[dtype]).t()
    y = B.linear_rope(dev(x, TD[dtype]), wd, rope_cols=rc, position_offset=off)
    ref = O.linear_rope(x, w, rc, off, 64, 1e4)
    assert_close(host(y), ref, TOL[dtype], f"linear_rope {layout} {case}")
