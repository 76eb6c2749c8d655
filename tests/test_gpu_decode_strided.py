"""GPU parity of bn_gqa_decode_strided: KV caches in other layouts than the
contiguous [batch, max_len, n_kv_heads, 64].

The kernels run the same arithmetic in the same order whatever the strides,
so each strided call must equal the contiguous call on the same values bit
for bit -- except on the one-workgroup-per-(sequence, KV head) bf16 path when
a KV head's rows are contiguous (head-major) and the batch holds at most 512
sequences: there a cache longer than 1.25x
the batch's mean streams with six waves instead of four, the same row in
another summation order, held to the bf16 bound against the contiguous call.
A few sequences per case are also checked against the CPU oracle
Cases cover every decode path: the one-workgroup-
per-(sequence, KV head) bf16 kernel (config 3's shape, uniform and ragged),
the split-K bf16 kernels (whole-row and per-head), the fp32 split kernel and
the fp32 short-cache split with its in-launch merge.
"""
import numpy as np
import pytest
import torch

import bnhip as B
from oracle import oracle as O
from gpu_util import BF16_TOL, FP32_TOL, assert_close, host, require_gpu

pytestmark = pytest.mark.gpu
TD = {"f32": torch.float32, "bf16": torch.bfloat16}
TOL = {"f32": FP32_TOL, "bf16": BF16_TOL}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def relayout(c, layout):
    """The same values as the contiguous cache c [B, L, Hkv, 64] in another
    storage, returned as a [B, L, Hkv, 64] view of it."""
    Bn, L, Hkv, D = c.shape
    if layout == "head_major":        # [B, Hkv, L, 64]
        s = torch.empty((Bn, Hkv, L, D), dtype=c.dtype, device=c.device)
        s.copy_(c.transpose(1, 2))
        return s.transpose(1, 2)
    if layout == "padded_rows":       # [B, L, Hkv, 96]: 32 unused elements per key row
        s = torch.full((Bn, L, Hkv, 96), float("nan"), dtype=c.dtype, device=c.device)
        s[..., :D].copy_(c)
        return s[..., :D]
    if layout == "head_major_gap":    # [B, Hkv, L + 3, 64]: 3 unused rows per head
        s = torch.full((Bn, Hkv, L + 3, D), float("nan"), dtype=c.dtype, device=c.device)
        s[:, :, :L].copy_(c.transpose(1, 2))
        return s[:, :, :L].transpose(1, 2)
    raise ValueError(layout)


def lengths(Bn, L, kind, seed):
    r = np.random.default_rng(seed)
    if kind == "uniform":
        return np.full(Bn, L, np.int32)
    lens = r.integers(1, L + 1, Bn).astype(np.int32)
    lens[: min(Bn, 4)] = [L, 1, 33, L + 7][: min(Bn, 4)]  # full, one key, tile edge, clamped
    return lens


CASES = [
    # dtype, B, Lmax, H, Hkv, lengths   (the path each one takes)
    ("bf16", 64, 4096, 32, 4, "uniform"),  # config 3: one workgroup per (sequence, KV head)
    ("bf16", 64, 4096, 32, 4, "ragged"),
    ("bf16", 80, 300, 16, 4, "ragged"),    # the same kernel, G = 4, short caches
    ("bf16", 512, 96, 16, 2, "ragged"),    # the same kernel, the largest batch that sums its lengths
    ("bf16", 520, 96, 16, 2, "ragged"),    # past it: four waves for every cache, any layout
    ("bf16", 2, 4096, 32, 4, "ragged"),    # split-K, whole-row kernel (4 KV heads per workgroup)
    ("bf16", 3, 1000, 16, 2, "ragged"),    # split-K, per-head kernel (n_kv_heads not a multiple of 4)
    ("f32", 2, 2048, 32, 4, "ragged"),     # fp32 split-K
    ("f32", 1, 640, 32, 4, "uniform"),     # fp32 short-cache split, merged in the launch
    ("f32", 3, 300, 8, 2, "ragged"),
]


@pytest.mark.parametrize("layout", ["head_major", "padded_rows", "head_major_gap"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(map(str, c)))
def test_strided_equals_contiguous_and_oracle(case, layout):
    dtype, Bn, L, H, Hkv, kind = case
    print(f"strided decode {layout} {case}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(Bn * 7 + L)
    q = torch.randn((Bn, H, 64), generator=g, device="cuda").to(TD[dtype])
    kc = torch.randn((Bn, L, Hkv, 64), generator=g, device="cuda").to(TD[dtype])
    vc = torch.randn((Bn, L, Hkv, 64), generator=g, device="cuda").to(TD[dtype])
    lens = lengths(Bn, L, kind, Bn + L)
    ld = torch.from_numpy(lens).cuda()
    ks, vs = relayout(kc, layout), relayout(vc, layout)
    assert not ks.is_contiguous() and torch.equal(ks, kc) and torch.equal(vs, vc)
    ws = B.decode_workspace(Bn, L, H)
    want = B.gqa_decode(q, kc, vc, ld, scale=0.125, workspace=ws)
    got = B.gqa_decode(q, ks, vs, ld, scale=0.125, workspace=ws)
    torch.cuda.synchronize()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    # rows of a head contiguous, batch of at most 512 sequences: the adaptive kernel
    wide = dtype == "bf16" and Bn * Hkv >= cus and ks.stride(1) == 64 and Bn <= 512
    if wide and kind == "ragged":
        assert_close(host(got), host(want), TOL[dtype], f"{layout}: against the contiguous call")
    else:
        assert torch.equal(got, want), f"{layout}: differs from the contiguous call"
    gh = host(got)
    assert np.all(np.isfinite(gh))
    for b in sorted({0, 1, 2, 3, Bn - 1} & set(range(Bn))):
        Lb = int(min(lens[b], L))
        ref = O.gqa_decode(host(q[b:b + 1]), host(kc[b:b + 1, :Lb]), host(vc[b:b + 1, :Lb]),
                           np.array([Lb], np.int32), 0.125)
        assert_close(gh[b:b + 1], ref, TOL[dtype], f"{layout} b={b} len={Lb}")


def test_strided_pool_workspace_and_repeats():
    """No workspace (the pool supplies the split path's partials) and three
    calls in a row on a head-major cache: identical results each time."""
    Bn, L, H, Hkv = 2, 4096, 32, 4
    g = torch.Generator(device="cuda").manual_seed(5)
    q = torch.randn((Bn, H, 64), generator=g, device="cuda").bfloat16()
    kc = torch.randn((Bn, L, Hkv, 64), generator=g, device="cuda").bfloat16()
    vc = torch.randn((Bn, L, Hkv, 64), generator=g, device="cuda").bfloat16()
    ld = torch.tensor([4000, 77], dtype=torch.int32, device="cuda")
    ks, vs = relayout(kc, "head_major"), relayout(vc, "head_major")
    want = B.gqa_decode(q, kc, vc, ld, scale=0.125)
    for _ in range(3):
        assert torch.equal(B.gqa_decode(q, ks, vs, ld, scale=0.125), want)
