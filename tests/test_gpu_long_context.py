"""Long-context causal GQA prefill at its full size: B=1, S=16384, 32/4
heads, head_dim 64, bf16, with the fused RMSNorm+RoPE on the [16384, 2048]
input feeding the queries.

The kernels run at the full size; the oracle checks them where it finishes in
seconds:
  * the fused RMSNorm+RoPE over the whole [16384, 2048] tensor (RoPE angles
    pos*freq formed in fp32 up to position 16383, op_rope.cuh:79-83);
  * the prefill on contiguous blocks of 64 query rows at the start, middle
    and end of the sequence, every head, against the oracle run with
    seq_offset = the block's first row (op_softmax.cuh:89-99) over the keys
    the block can see -- the masked keys past them contribute exact zeros in
    the reference's softmax, so leaving them out changes no bit of the oracle;
  * Q = 0 over the whole output: every row is the mean of V over its prefix
    (exact in the kernel: every probability is 1), which an off-by-one in the
    causal range of any of the 256 key blocks would shift.
"""
import ctypes as C

import numpy as np
import pytest
import torch

import bnhip as B
from oracle import oracle as O
from gpu_util import BF16_TOL, assert_close, bf16_round, host, require_gpu

pytestmark = pytest.mark.gpu
S, H, HKV, D, HID = 16384, 32, 4, 64, 2048


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


@pytest.fixture(scope="module")
def config5():
    """x ~ N(0,1) [S, 2048] -> RMSNorm(eps 1e-5, w = ones) + RoPE(theta 1e4) =
    Q; K, V ~ N(0,1) [S, 4, 64]; all bf16 (round-to-nearest-even casts)."""
    r = np.random.default_rng(0)
    x = bf16_round(r.standard_normal((S, HID)).astype(np.float32))
    k = bf16_round(r.standard_normal((1, S, HKV, D)).astype(np.float32))
    v = bf16_round(r.standard_normal((1, S, HKV, D)).astype(np.float32))
    xd = torch.from_numpy(x).to(torch.bfloat16).cuda()
    wd = torch.ones((1, HID), dtype=torch.bfloat16, device="cuda")
    qd = torch.empty_like(xd)
    print("config 5: fused RMSNorm+RoPE [16384, 2048] bf16", flush=True)
    B.call("bn_rmsnorm_rope", C.byref(B.view(xd)), C.byref(B.view(wd)), C.byref(B.view(qd)),
           1e-5, 0, D, 1e4, B.stream_of())
    kd = torch.from_numpy(k).to(torch.bfloat16).cuda()
    vd = torch.from_numpy(v).to(torch.bfloat16).cuda()
    print("config 5: prefill S=16384 bf16", flush=True)
    od = B.gqa_prefill(qd.view(1, S, H, D), kd, vd, scale=0.125)
    torch.cuda.synchronize()
    return dict(x=x, k=k, v=v, kd=kd, vd=vd, q=host(qd), o=host(od))


def test_rmsnorm_rope_full_config5_input(config5):
    ref = O.rmsnorm_rope(config5["x"], np.ones((1, HID), np.float32), 1e-5, 0, D, 1e4)
    got = config5["q"]
    assert_close(got, ref, BF16_TOL, "rmsnorm_rope [16384, 2048] bf16")
    # the kernel rounds its fp32 result once: within one bf16 rounding of the
    # oracle, plus fp32-level noise (sin/cos ulps) that only shows on outputs
    # near zero, where the pair rotation cancels
    noise = 2.0 ** -16 * np.max(np.abs(ref))
    excess = np.abs(got - ref) - np.abs(ref) * 2.0 ** -8
    assert np.all(excess <= noise), f"more than one bf16 rounding: {excess.max():.3e} > {noise:.3e}"
    # high positions: the last rows carry angles up to 16383 * freq
    assert_close(got[-64:], ref[-64:], BF16_TOL, "last 64 rows")


@pytest.mark.parametrize("r0", [0, 8192, S - 64])
def test_prefill_config5_row_blocks(config5, r0):
    q = config5["q"].reshape(1, S, H, D)[:, r0:r0 + 64]
    kv_end = r0 + 64  # keys past the block's last row are masked for every row of it
    ref = O.gqa_prefill(q, config5["k"][:, :kv_end], config5["v"][:, :kv_end], 0.125, True, r0)
    got = config5["o"][:, r0:r0 + 64]
    assert np.all(np.isfinite(got))
    assert_close(got, ref, BF16_TOL, f"rows {r0}..{r0 + 63}, all heads")


def test_prefill_config5_zero_query_prefix_means(config5):
    q = torch.zeros((1, S, H, D), dtype=torch.bfloat16, device="cuda")
    got = host(B.gqa_prefill(q, config5["kd"], config5["vd"], scale=0.125))
    v = config5["v"].astype(np.float64)
    means = np.cumsum(v, axis=1) / np.arange(1, S + 1)[None, :, None, None]
    ref = np.repeat(means, H // HKV, axis=2)
    assert_close(got, ref, BF16_TOL, "prefix means, S=16384")
    # the output is the bf16 rounding of an fp32 mean: within one rounding,
    # plus the fp32 accumulation error of up to 16384 terms
    noise = 2.0 ** -16 * np.max(np.abs(ref))
    excess = np.abs(got - ref) - np.abs(ref) * 2.0 ** -8
    assert np.all(excess <= noise), f"more than one bf16 rounding: {excess.max():.3e} > {noise:.3e}"
