"""GPU parity of the planned ragged decode (bn_gqa_decode_planned).

The host lengths choose equal shares of the batch's tiles per compute unit;
a cut cache is merged in the same launch by its head part (its first tiles),
from the records its later parts' waves wrote with this launch's epoch.  Every sequence
of every case is compared with the CPU oracle at the bf16 bound (2e-2), and
the planned call with bn_gqa_decode (which it must agree with to the same
bound: both are the same softmax row).  Length sets: config 3's ragged draw
(the bench's), two length classes, a few long caches among short ones,
sequences of length 0 and 1, other query-group sizes, and batches the plan
does not take (balanced, or more than 256 units) which run bn_gqa_decode.
"""
import os

import numpy as np
import pytest
import torch

import bnhip as B
from oracle import oracle as O
from gpu_util import BF16_TOL, assert_close, bf16_round, dev, host, require_gpu

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def lengths(kind, Bn, L, seed=2):
    r = np.random.default_rng(seed)
    if kind == "ragged":            # config 3's ragged variant, as bench.py draws it
        return r.integers(512, L + 1, Bn).astype(np.int32)
    if kind == "two_class":
        return np.where(np.arange(Bn) % 2 == 0, 512, L).astype(np.int32)
    if kind == "skewed":            # four long caches among short ones
        out = np.full(Bn, 600, np.int32)
        out[[3, 20, 41, 62]] = L
        return out
    if kind == "zeros":             # empty and one-key sequences among ragged ones
        out = r.integers(512, L + 1, Bn).astype(np.int32)
        out[[0, 5, 6, 33]] = 0
        out[[1, 34]] = 1
        out[-1] = L
        return out
    if kind == "uniform":
        return np.full(Bn, L, np.int32)
    raise ValueError(kind)


def head_major(c):
    """The same values as the contiguous cache c [B, L, Hkv, 64], stored
    [B, Hkv, L, 64], as a [B, L, Hkv, 64] view."""
    return c.transpose(1, 2).contiguous().transpose(1, 2)


def run_case(Bn, L, H, Hkv, lens, seed=9, workspace=True):
    r = np.random.default_rng(seed)
    q = bf16_round(r.standard_normal((Bn, H, 64)).astype(np.float32))
    kc = bf16_round(r.standard_normal((Bn, L, Hkv, 64)).astype(np.float32))
    vc = bf16_round(r.standard_normal((Bn, L, Hkv, 64)).astype(np.float32))
    qd, kd, vd = dev(q, torch.bfloat16), dev(kc, torch.bfloat16), dev(vc, torch.bfloat16)
    ld = torch.from_numpy(lens).cuda()
    ws = None
    if workspace:
        n = B.lib().bn_gqa_decode_planned_workspace_size(Bn, L, H, Hkv, 64)
        ws = torch.empty(n, dtype=torch.uint8, device="cuda")
    o1 = torch.full((Bn, H, 64), float("nan"), dtype=torch.bfloat16, device="cuda")
    B.gqa_decode_planned(qd, kd, vd, ld, lens, o1, scale=0.125, workspace=ws)
    o2 = B.gqa_decode_planned(qd, kd, vd, ld, lens, scale=0.125, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2), "a second call on the same workspace gives other bits"
    got = host(o1)
    for b in range(Bn):
        Lb = int(lens[b])
        if Lb == 0:
            assert np.all(got[b] == 0.0), f"b={b}: no key gives zeros"
            continue
        ref = O.gqa_decode(q[b:b + 1], kc[b:b + 1, :Lb], vc[b:b + 1, :Lb],
                           np.array([Lb], np.int32), 0.125)
        assert_close(got[b:b + 1], ref, BF16_TOL, f"b={b} L={Lb}")
    plain = host(B.gqa_decode(qd, kd, vd, ld, scale=0.125, workspace=B.decode_workspace(Bn, L, H)))
    assert_close(got, plain, BF16_TOL, "planned vs bn_gqa_decode")
    return got


@pytest.mark.parametrize("kind", ["ragged", "two_class", "skewed", "zeros"])
def test_planned_decode_config3(kind):
    Bn, L, H, Hkv = 64, 4096, 32, 4
    run_case(Bn, L, H, Hkv, lengths(kind, Bn, L))


@pytest.mark.parametrize("H,Hkv,Bn", [(16, 4, 64), (32, 8, 32), (8, 4, 64)])
def test_planned_decode_group_sizes(H, Hkv, Bn):
    # 4, 4 and 2 query heads per KV head; 256 units each
    L = 2048
    run_case(Bn, L, H, Hkv, lengths("ragged", Bn, L, seed=5), seed=11)


def test_planned_decode_pool_workspace():
    Bn, L, H, Hkv = 64, 1024, 32, 4
    run_case(Bn, L, H, Hkv, lengths("skewed", Bn, L), seed=12, workspace=False)


@pytest.mark.parametrize("kind,Bn", [("uniform", 64), ("ragged", 96)])
def test_planned_decode_unplanned_batches(kind, Bn):
    # balanced lengths, or 384 units: bn_gqa_decode runs, same results
    L = 1024
    run_case(Bn, L, 32, 4, lengths(kind, Bn, L), seed=13)


def test_planned_decode_head_major_caches():
    """bn_gqa_decode_planned_strided on head-major caches: the same kernel and
    plan, only the row addresses change -- bit for bit the contiguous call."""
    Bn, L, H, Hkv = 64, 4096, 32, 4
    lens = lengths("ragged", Bn, L)
    g = torch.Generator(device="cuda").manual_seed(21)
    q = torch.randn((Bn, H, 64), generator=g, device="cuda").bfloat16()
    kc = torch.randn((Bn, L, Hkv, 64), generator=g, device="cuda").bfloat16()
    vc = torch.randn((Bn, L, Hkv, 64), generator=g, device="cuda").bfloat16()
    ld = torch.from_numpy(lens).cuda()
    ws = torch.empty(B.lib().bn_gqa_decode_planned_workspace_size(Bn, L, H, Hkv, 64),
                     dtype=torch.uint8, device="cuda")
    want = B.gqa_decode_planned(q, kc, vc, ld, lens, scale=0.125, workspace=ws)
    ks, vs = head_major(kc), head_major(vc)
    assert not ks.is_contiguous()
    for _ in range(2):
        got = B.gqa_decode_planned(q, ks, vs, ld, lens, scale=0.125, workspace=ws)
        assert torch.equal(got, want)
    ref = host(B.gqa_decode(q, ks, vs, ld, scale=0.125))  # the whole-cache kernel, same layout
    assert_close(host(want), ref, BF16_TOL, "planned vs bn_gqa_decode_strided")


@pytest.mark.parametrize("kind", ["ragged", "skewed", "zeros"])
def test_planned_decode_fallback_path(kind):
    """BN_PLAN_FALLBACK=1 makes every head ignore the records and stream its
    cut cache's later keys itself -- what a head does if a record never
    arrives.  Forced from the host, so no kernel waits on anything; the results
    must hold the same bounds, and repeat bit for bit."""
    Bn, L, H, Hkv = 64, 4096, 32, 4
    os.environ["BN_PLAN_FALLBACK"] = "1"
    try:
        run_case(Bn, L, H, Hkv, lengths(kind, Bn, L), seed=17)
    finally:
        del os.environ["BN_PLAN_FALLBACK"]
