"""bn_gqa_decode_noalloc: the decode entry point that allocates nothing.

It runs bn_gqa_decode's kernels with the split-K partials in a file-scope
device array instead of a workspace, so its output must equal
bn_gqa_decode's bit for bit on every path (bf16 whole-cache, bf16 whole-row
split, bf16 per-KV-head split, fp32 split, fp32 short-cache split), over two calls
in a row where the second is smaller and finds the first call's partials
still in the array.  The pool's allocation count must not move.  (The
refusal of partials larger than the array is a host-side check, tested
without a GPU in test_abi.py.)
"""
import ctypes as C

import numpy as np
import pytest
import torch

import bnhip as B
from oracle import oracle as O
from gpu_util import BF16_TOL, FP32_TOL, assert_close, bf16_round, host, require_gpu

pytestmark = pytest.mark.gpu
TD = {"f32": torch.float32, "bf16": torch.bfloat16}
TOL = {"f32": FP32_TOL, "bf16": BF16_TOL}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def pool_allocs():
    s = B.BnPoolStats()
    B.check(B.lib().bn_pool_get_stats(C.byref(s)))
    return int(s.n_allocs)


def make_case(dtype, Bn, L, H, Hkv, lens, seed):
    r = np.random.default_rng(seed)
    q, kc, vc = (r.standard_normal(s).astype(np.float32)
                 for s in ((Bn, H, 64), (Bn, L, Hkv, 64), (Bn, L, Hkv, 64)))
    if dtype == "bf16":
        q, kc, vc = bf16_round(q), bf16_round(kc), bf16_round(vc)
    t = TD[dtype]
    dev = [torch.from_numpy(a).to(t).cuda() for a in (q, kc, vc)]
    ld = torch.tensor(lens, dtype=torch.int32, device="cuda")
    return (q, kc, vc), dev, ld


def run_noalloc(dtype, qd, kd, vd, ld, o):
    Bn, H, D = qd.shape
    _, L, Hkv, _ = kd.shape
    code = B.BN_BF16 if dtype == "bf16" else B.BN_F32
    return B.lib().bn_gqa_decode_noalloc(code, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                                         ld.data_ptr(), o.data_ptr(), Bn, L, H, Hkv, D, 0.125,
                                         None)


# (dtype, H, Hkv, first call (B, L, lens), second call (B, L, lens)); the
# second call is smaller in batch and cache length
PATHS = {
    "bf16_rows_split": ("bf16", 32, 4, (6, 3000, [3000, 1, 2047, 129, 3000, 700]),
                        (3, 1000, [1000, 300, 5])),
    "bf16_head_split": ("bf16", 16, 2, (5, 2500, [2500, 17, 1024, 2000, 64]),
                        (2, 700, [699, 700])),
    "f32_split": ("f32", 32, 4, (4, 2100, [2100, 1, 1500, 64]), (2, 1500, [1500, 900])),
    "f32_short": ("f32", 32, 4, (2, 640, [640, 313]), (1, 300, [257])),
    "bf16_whole": ("bf16", 32, 4, (None, 700, None), (None, 300, None)),
}


def lens_for(Bn, L, lens, seed):
    if lens is not None:
        return lens
    r = np.random.default_rng(seed)
    return [int(x) for x in r.integers(1, L + 1, Bn)]


@pytest.mark.parametrize("path", sorted(PATHS))
def test_noalloc_matches_decode_two_calls(path):
    dtype, H, Hkv, first, second = PATHS[path]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    for call, (Bn, L, lens) in enumerate((first, second)):
        if Bn is None:  # enough (sequence, KV head) pairs to fill the CUs
            Bn = -(-cus // Hkv) + (8 if call == 0 else 0)
        lens = lens_for(Bn, L, lens, 100 + call)
        print(f"noalloc {path} call {call}: B={Bn} L={L} H={H} Hkv={Hkv}", flush=True)
        (q, kc, vc), (qd, kd, vd), ld = make_case(dtype, Bn, L, H, Hkv, lens, 7 * call + len(path))
        ref_o = B.gqa_decode(qd, kd, vd, ld, scale=0.125)  # pool workspace
        o = torch.full_like(qd, float("nan"))
        torch.cuda.synchronize()
        n0 = pool_allocs()
        st = run_noalloc(dtype, qd, kd, vd, ld, o)
        assert st == B.BN_OK, B.lib().bn_last_error().decode()
        torch.cuda.synchronize()
        assert pool_allocs() == n0, "the no-allocation entry point allocated from the pool"
        got, want = o.cpu(), ref_o.cpu()
        assert torch.equal(got.view(torch.int16) if dtype == "bf16" else got.view(torch.int32),
                           want.view(torch.int16) if dtype == "bf16" else want.view(torch.int32)), \
            f"{path} call {call}: differs from bn_gqa_decode"
        gotf = host(o)
        for b in (0, Bn - 1):
            Lb = int(lens[b])
            ref = O.gqa_decode(q[b:b + 1], kc[b:b + 1, :Lb], vc[b:b + 1, :Lb],
                               np.array([Lb], np.int32), 0.125)
            assert_close(gotf[b:b + 1], ref, TOL[dtype], f"{path} call {call} b={b}")


def test_noalloc_after_nan_partials():
    """A call whose partials are all NaN (NaN cache data, in range) leaves them
    in the array; a ragged call after it reads only records it wrote itself."""
    H, Hkv, L = 32, 4, 3000
    _, (qd, kd, vd), ld = make_case("bf16", 6, L, H, Hkv, [L] * 6, 1)
    kd.fill_(float("nan"))
    o = torch.empty_like(qd)
    assert run_noalloc("bf16", qd, kd, vd, ld, o) == B.BN_OK
    torch.cuda.synchronize()
    assert torch.isnan(o.float()).all()
    lens = [1, 200, 3000, 64, 129, 1000]
    (q, kc, vc), (qd, kd, vd), ld = make_case("bf16", 6, L, H, Hkv, lens, 2)
    o = torch.empty_like(qd)
    assert run_noalloc("bf16", qd, kd, vd, ld, o) == B.BN_OK
    got = host(o)
    assert np.all(np.isfinite(got))
    assert torch.equal(o.cpu().view(torch.int16),
                       B.gqa_decode(qd, kd, vd, ld, scale=0.125).cpu().view(torch.int16))
    for b in range(6):
        ref = O.gqa_decode(q[b:b + 1], kc[b:b + 1, :lens[b]], vc[b:b + 1, :lens[b]],
                           np.array([lens[b]], np.int32), 0.125)
        assert_close(got[b:b + 1], ref, BF16_TOL, f"b={b}")

