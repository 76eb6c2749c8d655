"""GPU parity of the fused GQA prefill and KV-cache decode kernels.

Small shapes are compared with the CPU oracle element for element (every
head, every row); the full benchmark shapes (B=4, S=2048 prefill; B=64, L=4096
decode) are checked on sampled (batch, head) pairs against the oracle and on
size-independent properties (Q=0 gives prefix means of V; constant-per-head
V exposes the GQA head mapping; decode equals the prefill's last row).
Tolerances are the north star's: max relative error 1e-4 (fp32), 2e-2 (bf16).
"""
import math

import numpy as np
import pytest
import torch

import bnhip as B
from oracle import oracle as O
from gpu_util import BF16_TOL, FP32_TOL, assert_close, bf16_round, dev, host, relerr, require_gpu

pytestmark = pytest.mark.gpu
TD = {"f32": torch.float32, "bf16": torch.bfloat16}
TOL = {"f32": FP32_TOL, "bf16": BF16_TOL}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def draw(shape, seed, dtype):
    a = np.random.default_rng(seed).standard_normal(shape).astype(np.float32)
    return bf16_round(a) if dtype == "bf16" else a


PREFILL_CASES = [
    # B, Sq, Skv, H, Hkv, causal, off
    (2, 128, 128, 8, 2, 1, 0),
    (1, 200, 200, 32, 4, 1, 0),     # ragged last row tile, TinyLLaMA heads
    (1, 64, 64, 4, 4, 0, 0),        # non-causal, no grouping
    (1, 50, 250, 8, 1, 1, 200),     # query rows at the end of a longer key range
    (2, 70, 70, 2, 1, 1, -5),       # negative offset: first rows see no key -> 0
    (1, 1, 300, 8, 2, 1, 299),      # one query row (decode as prefill)
    (3, 257, 257, 16, 4, 1, 0),
    (1, 130, 90, 4, 2, 0, 0),       # non-causal, Skv not a multiple of 64
]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("case", PREFILL_CASES)
def test_prefill_vs_oracle(case, dtype):
    Bn, Sq, Skv, H, Hkv, causal, off = case
    q = draw((Bn, Sq, H, 64), 1, dtype)
    k = draw((Bn, Skv, Hkv, 64), 2, dtype)
    v = draw((Bn, Skv, Hkv, 64), 3, dtype)
    o = B.gqa_prefill(dev(q, TD[dtype]), dev(k, TD[dtype]), dev(v, TD[dtype]), scale=0.125,
                      causal=bool(causal), seq_offset=off)
    ref = O.gqa_prefill(q, k, v, 0.125, bool(causal), off)
    got = host(o)
    assert_close(got, ref, TOL[dtype], f"prefill {case} {dtype}")
    if off < 0:  # rows with no visible key are exactly zero, as the reference's P @ V
        assert np.all(got[:, :-off] == 0.0)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_prefill_strided_rows(dtype):
    # q/k/v as column slices of wider rows (e.g. a fused QKV projection output)
    Bn, S, H, Hkv = 2, 96, 8, 2
    qkv = draw((Bn, S, (H + 2 * Hkv) * 64), 4, dtype)
    t = dev(qkv, TD[dtype])
    q = t[:, :, :H * 64].unflatten(2, (H, 64))
    k = t[:, :, H * 64:(H + Hkv) * 64].unflatten(2, (Hkv, 64))
    v = t[:, :, (H + Hkv) * 64:].unflatten(2, (Hkv, 64))
    o = B.gqa_prefill(q, k, v, scale=0.125)
    qn = qkv[:, :, :H * 64].reshape(Bn, S, H, 64)
    kn = qkv[:, :, H * 64:(H + Hkv) * 64].reshape(Bn, S, Hkv, 64)
    vn = qkv[:, :, (H + Hkv) * 64:].reshape(Bn, S, Hkv, 64)
    assert_close(host(o), O.gqa_prefill(qn, kn, vn, 0.125, True, 0), TOL[dtype])


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_prefill_head_mapping(dtype):
    # V of KV head g is the constant g+1: query head h must return h//G + 1
    Bn, S, H, Hkv = 1, 192, 32, 4
    q = draw((Bn, S, H, 64), 5, dtype)
    k = draw((Bn, S, Hkv, 64), 6, dtype)
    v = np.broadcast_to(np.arange(1, Hkv + 1, dtype=np.float32)[None, None, :, None],
                        (Bn, S, Hkv, 64)).copy()
    got = host(B.gqa_prefill(dev(q, TD[dtype]), dev(k, TD[dtype]), dev(v, TD[dtype])))
    for h in range(H):
        want = h // (H // Hkv) + 1
        np.testing.assert_array_equal(np.rint(got[0, :, h]), want)
        assert np.max(np.abs(got[0, :, h] - want)) < (1e-5 if dtype == "f32" else 2e-2 * want)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_prefill_baseline_shape(dtype):
    """config 2: B=4, S=2048, 32/4 heads, D=64, causal, scale 1/8."""
    Bn, S, H, Hkv = 4, 2048, 32, 4
    rngs = np.random.default_rng(0)
    q = rngs.standard_normal((Bn, S, H, 64)).astype(np.float32)
    k = rngs.standard_normal((Bn, S, Hkv, 64)).astype(np.float32)
    v = rngs.standard_normal((Bn, S, Hkv, 64)).astype(np.float32)
    if dtype == "bf16":
        q, k, v = bf16_round(q), bf16_round(k), bf16_round(v)
    got = host(B.gqa_prefill(dev(q, TD[dtype]), dev(k, TD[dtype]), dev(v, TD[dtype]),
                             scale=0.125))
    assert np.all(np.isfinite(got))
    for b, h in [(0, 0), (3, 31), (1, 13)]:   # sampled heads, full length, every row
        g = h // 8
        ref = O.gqa_prefill(q[b:b + 1, :, h:h + 1], k[b:b + 1, :, g:g + 1],
                            v[b:b + 1, :, g:g + 1], 0.125, True, 0)
        assert_close(got[b:b + 1, :, h:h + 1], ref, TOL[dtype], f"b={b} h={h}")


@pytest.mark.parametrize("growth", [1 / 8, -1 / 600])
def test_prefill_score_jumps(growth):
    """Scores that grow along the sequence (K row j scaled by 1 + growth*j) take
    the kernel's exact rescale path many times (later keys exceed the first
    tile's max by far more than 2^16 in probability); shrinking scores make the
    first keys dominate and later ones underflow.  Both must match the oracle."""
    Bn, S, H, Hkv = 1, 600, 8, 2
    q = draw((Bn, S, H, 64), 11, "bf16")
    k = draw((Bn, S, Hkv, 64), 12, "f32") * (1 + growth * np.arange(S))[None, :, None, None]
    k = bf16_round(k.astype(np.float32))
    v = draw((Bn, S, Hkv, 64), 13, "bf16")
    o = B.gqa_prefill(dev(q, torch.bfloat16), dev(k, torch.bfloat16), dev(v, torch.bfloat16),
                      scale=0.125)
    assert_close(host(o), O.gqa_prefill(q, k, v, 0.125, True, 0), BF16_TOL, f"growth {growth}")


def test_prefill_zero_query_prefix_means():
    # size-independent property at the full shape: Q = 0 -> row i is mean(V[0..i])
    Bn, S, H, Hkv = 4, 2048, 32, 4
    v = np.random.default_rng(7).standard_normal((Bn, S, Hkv, 64)).astype(np.float32)
    k = np.random.default_rng(8).standard_normal((Bn, S, Hkv, 64)).astype(np.float32)
    q = torch.zeros((Bn, S, H, 64), device="cuda")
    got = host(B.gqa_prefill(q, dev(k), dev(v), scale=0.125))
    means = np.cumsum(v.astype(np.float64), axis=1) / np.arange(1, S + 1)[None, :, None, None]
    ref = np.repeat(means, H // Hkv, axis=2)
    assert_close(got, ref, FP32_TOL, "prefix means")


@pytest.mark.parametrize("shape", [(4, 2048, 2048, 32, 4, 0), (2, 4100, 4160, 32, 4, 60),
                                   (1, 16384, 16384, 16, 2, 0)])
def test_prefill_bf16_every_row_prefix_means(shape):
    """Q = 0 in bf16 at config 2's shape, a ragged one with an offset and a
    long one with two KV heads: every output row of every head is the mean of
    the V rows it sees (query i sees keys 0 .. i + offset), so a row tile
    computed twice, skipped or given the wrong keys shows (the output starts
    as NaN)."""
    Bn, Sq, Skv, H, Hkv, off = shape
    v = bf16_round(np.random.default_rng(21).standard_normal((Bn, Skv, Hkv, 64)).astype(np.float32))
    k = bf16_round(np.random.default_rng(22).standard_normal((Bn, Skv, Hkv, 64)).astype(np.float32))
    q = torch.zeros((Bn, Sq, H, 64), device="cuda", dtype=torch.bfloat16)
    o = torch.full((Bn, Sq, H, 64), float("nan"), device="cuda", dtype=torch.bfloat16)
    B.gqa_prefill(q, dev(k, torch.bfloat16), dev(v, torch.bfloat16), o, scale=0.125, seq_offset=off)
    got = host(o)
    csum = np.cumsum(v.astype(np.float64), axis=1)
    last = np.minimum(np.arange(Sq) + off, Skv - 1)
    means = csum[:, last] / (last + 1)[None, :, None, None]
    ref = np.repeat(means, H // Hkv, axis=2)
    assert np.all(np.isfinite(got))
    assert_close(got, ref, BF16_TOL, f"bf16 prefix means {shape}")


def test_prefill_bf16_long_offset_shape_vs_oracle():
    """B=2, Sq=4100 (a ragged last row tile), Skv=4160, offset 60, 32/4 heads
    (1032 head-packed row tiles): whole heads against the oracle, and a second
    call on the same buffers gives the same bits."""
    Bn, Sq, Skv, H, Hkv, off = 2, 4100, 4160, 32, 4, 60
    q = draw((Bn, Sq, H, 64), 31, "bf16")
    k = draw((Bn, Skv, Hkv, 64), 32, "bf16")
    v = draw((Bn, Skv, Hkv, 64), 33, "bf16")
    qd, kd, vd = dev(q, torch.bfloat16), dev(k, torch.bfloat16), dev(v, torch.bfloat16)
    o1 = B.gqa_prefill(qd, kd, vd, scale=0.125, seq_offset=off)
    o2 = B.gqa_prefill(qd, kd, vd, scale=0.125, seq_offset=off)
    assert torch.equal(o1, o2)
    got = host(o1)
    for b, h in [(0, 5), (1, 30)]:
        g = h // 8
        ref = O.gqa_prefill(q[b:b + 1, :, h:h + 1], k[b:b + 1, :, g:g + 1], v[b:b + 1, :, g:g + 1],
                            0.125, True, off)
        assert_close(got[b:b + 1, :, h:h + 1], ref, BF16_TOL, f"b={b} h={h}")


# ------------------------------------------------------------------- decode
DECODE_CASES = [
    # B, Lmax, H, Hkv, lens
    (8, 1000, 32, 4, [1000, 1, 513, 64, 999, 2, 700, 128]),
    (3, 300, 8, 8, [300, 17, 150]),
    (5, 4096, 32, 4, [4096, 512, 3000, 1, 4095]),
    (2, 77, 4, 2, [77, 40]),
    (4, 256, 16, 4, [0, 256, 300, 5]),   # 0 -> zeros; above max_len -> clamped
]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("case", DECODE_CASES)
def test_decode_vs_oracle(case, dtype):
    Bn, L, H, Hkv, lens = case
    q = draw((Bn, H, 64), 11, dtype)
    kc = draw((Bn, L, Hkv, 64), 12, dtype)
    vc = draw((Bn, L, Hkv, 64), 13, dtype)
    lens = np.array(lens, np.int32)
    got = host(B.gqa_decode(dev(q, TD[dtype]), dev(kc, TD[dtype]), dev(vc, TD[dtype]),
                            torch.from_numpy(lens).cuda(), scale=0.125))
    for b in range(Bn):
        Lb = int(min(max(lens[b], 0), L))
        if Lb == 0:
            assert np.all(got[b] == 0.0)
            continue
        ref = O.gqa_decode(q[b:b + 1], kc[b:b + 1, :Lb], vc[b:b + 1, :Lb],
                           np.array([Lb], np.int32), 0.125)
        assert_close(got[b:b + 1], ref, TOL[dtype], f"decode b={b} len={Lb}")


@pytest.mark.parametrize("L,H,Hkv", [(300, 32, 4), (130, 16, 4), (200, 8, 4), (96, 16, 2),
                                     (70, 4, 4)])
def test_decode_bf16_one_workgroup_per_kv_head(L, H, Hkv):
    """bf16 with at least as many (sequence, KV head) pairs as CUs takes the
    single-pass kernel (one workgroup per pair, per-wave key ranges merged in
    LDS): G = 8, 4, 2, 1; empty, one-key, tile-edge, clamped and short
    lengths that leave some waves without keys."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    Bn = -(-cus // Hkv)
    r = np.random.default_rng(L + H)
    lens = r.integers(1, L + 1, Bn).astype(np.int32)
    lens[:8] = [0, 1, 31, 32, 33, L, L + 5, min(255, L)]
    q = bf16_round(r.standard_normal((Bn, H, 64)).astype(np.float32))
    kc = bf16_round(r.standard_normal((Bn, L, Hkv, 64)).astype(np.float32))
    vc = bf16_round(r.standard_normal((Bn, L, Hkv, 64)).astype(np.float32))
    got = host(B.gqa_decode(dev(q, torch.bfloat16), dev(kc, torch.bfloat16),
                            dev(vc, torch.bfloat16), torch.from_numpy(lens).cuda(), scale=0.125))
    for b in list(range(8)) + list(range(8, Bn, 7)):
        Lb = int(min(max(lens[b], 0), L))
        if Lb == 0:
            assert np.all(got[b] == 0.0)
            continue
        ref = O.gqa_decode(q[b:b + 1], kc[b:b + 1, :Lb], vc[b:b + 1, :Lb],
                           np.array([Lb], np.int32), 0.125)
        assert_close(got[b:b + 1], ref, BF16_TOL, f"b={b} len={Lb}")


@pytest.mark.parametrize("lens_kind", ["skewed", "two_groups"])
def test_decode_bf16_whole_cache_skewed_lengths(lens_kind):
    """The one-workgroup-per-(sequence, KV head) kernel on batches whose
    lengths differ by far: a few long caches among short ones (skewed) or
    two length classes (two_groups); every sequence matches the oracle."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    H, Hkv, L = 32, 4, 4096
    Bn = -(-cus // Hkv)
    r = np.random.default_rng(71)
    if lens_kind == "skewed":
        lens = np.full(Bn, 64, np.int32)
        lens[:4] = [4096, 4095, 3000, 2049]
    else:
        lens = np.where(np.arange(Bn) % 2 == 0, 1000, 3000).astype(np.int32)
    q = bf16_round(r.standard_normal((Bn, H, 64)).astype(np.float32))
    kc = bf16_round(r.standard_normal((Bn, L, Hkv, 64)).astype(np.float32))
    vc = bf16_round(r.standard_normal((Bn, L, Hkv, 64)).astype(np.float32))
    got = host(B.gqa_decode(dev(q, torch.bfloat16), dev(kc, torch.bfloat16),
                            dev(vc, torch.bfloat16), torch.from_numpy(lens).cuda(), scale=0.125))
    assert np.all(np.isfinite(got))
    for b in [0, 1, 2, 3, 4, 5, Bn - 1]:
        Lb = int(lens[b])
        ref = O.gqa_decode(q[b:b + 1], kc[b:b + 1, :Lb], vc[b:b + 1, :Lb],
                           np.array([Lb], np.int32), 0.125)
        assert_close(got[b:b + 1], ref, BF16_TOL, f"{lens_kind} b={b} len={Lb}")


@pytest.mark.parametrize("dtype,Bn,L,H,Hkv", [("f32", 1, 640, 32, 4), ("f32", 3, 300, 8, 2),
                                              ("bf16", 2, 300, 32, 4), ("bf16", 80, 200, 16, 4)])
def test_decode_ignores_cache_rows_past_len(dtype, Bn, L, H, Hkv):
    """Cache rows at or past a sequence's length hold NaN (memory the caller
    never wrote): no kernel may let them reach the output (short-cache split fp32,
    split and per-KV-head bf16 paths)."""
    r = np.random.default_rng(Bn + L)
    lens = r.integers(1, L + 1, Bn).astype(np.int32)
    lens[0] = L // 2
    q = draw((Bn, H, 64), 50, dtype)
    kc = draw((Bn, L, Hkv, 64), 51, dtype)
    vc = draw((Bn, L, Hkv, 64), 52, dtype)
    kn, vn = kc.copy(), vc.copy()
    for b in range(Bn):
        kn[b, lens[b]:] = np.nan
        vn[b, lens[b]:] = np.nan
    got = host(B.gqa_decode(dev(q, TD[dtype]), dev(kn, TD[dtype]), dev(vn, TD[dtype]),
                            torch.from_numpy(lens).cuda(), scale=0.125))
    assert np.all(np.isfinite(got))
    for b in range(Bn):
        Lb = int(lens[b])
        ref = O.gqa_decode(q[b:b + 1], kc[b:b + 1, :Lb], vc[b:b + 1, :Lb],
                           np.array([Lb], np.int32), 0.125)
        assert_close(got[b:b + 1], ref, TOL[dtype], f"b={b} len={Lb}")


@pytest.mark.parametrize("dtype,Hkv", [("bf16", 4), ("bf16", 2), ("f32", 4)])
def test_decode_workspace_reuse(dtype, Hkv):
    """One workspace across calls of different batches and lengths (the
    whole-row, per-head and fp32 kernels): every result matches the oracle."""
    H, L = 8 * Hkv, 1500
    ws = B.decode_workspace(6, L, H)
    for call, lens in enumerate([[1500, 700, 1, 129, 1024, 0], [33, 1500], [1499, 2, 900, 640]]):
        Bn = len(lens)
        q = draw((Bn, H, 64), 20 + call, dtype)
        kc = draw((Bn, L, Hkv, 64), 30 + call, dtype)
        vc = draw((Bn, L, Hkv, 64), 40 + call, dtype)
        ld = torch.tensor(lens, dtype=torch.int32, device="cuda")
        got = host(B.gqa_decode(dev(q, TD[dtype]), dev(kc, TD[dtype]), dev(vc, TD[dtype]), ld,
                                scale=0.125, workspace=ws))
        for b, Lb in enumerate(lens):
            if Lb == 0:
                assert np.all(got[b] == 0.0)
                continue
            ref = O.gqa_decode(q[b:b + 1], kc[b:b + 1, :Lb], vc[b:b + 1, :Lb],
                               np.array([Lb], np.int32), 0.125)
            assert_close(got[b:b + 1], ref, TOL[dtype], f"call {call} b={b} len={Lb}")


def test_decode_short_split_many_calls():
    """fp32 short caches (config 4's decode): each (sequence, query head)'s
    keys are cut into 4 splits and the unit's last split to arrive merges the
    records in the same launch, counting on a slot of a 16-slot counter ring.
    40 calls in a row (the ring wraps twice) with lengths that leave splits
    empty (0..5 keys), cut lanes groups (63, 65) and the whole cache: every
    call matches the oracle, and a call repeated later gives the same bits."""
    H, Hkv, L = 32, 4, 640
    Bn = 3
    q = draw((Bn, H, 64), 90, "f32")
    kc = draw((Bn, L, Hkv, 64), 91, "f32")
    vc = draw((Bn, L, Hkv, 64), 92, "f32")
    qd, kd, vd = dev(q, torch.float32), dev(kc, torch.float32), dev(vc, torch.float32)
    pattern = [[0, 1, 2], [3, 4, 5], [63, 64, 65], [520, 576, 640], [1, 639, 17]]
    first = {}
    for call in range(40):
        lens = pattern[call % len(pattern)]
        got = host(B.gqa_decode(qd, kd, vd, torch.tensor(lens, dtype=torch.int32, device="cuda"),
                                scale=0.125))
        key = call % len(pattern)
        if key in first:
            assert np.array_equal(got, first[key]), f"call {call}: not the bits of call {key}"
            continue
        first[key] = got
        for b, Lb in enumerate(lens):
            if Lb == 0:
                assert np.all(got[b] == 0.0)
                continue
            ref = O.gqa_decode(q[b:b + 1], kc[b:b + 1, :Lb], vc[b:b + 1, :Lb],
                               np.array([Lb], np.int32), 0.125)
            assert_close(got[b:b + 1], ref, FP32_TOL, f"call {call} b={b} len={Lb}")


def test_decode_short_split_graph_replays():
    """The short-cache decode captured in a HIP graph (as bench.py replays a
    generate's decode launches): three calls on three caches per replay, five
    replays with eager work and synchronisations between them; every replay
    equals the eager result bit for bit (the split counters return to zero
    at the end of each launch, so replays reuse their slots)."""
    H, Hkv, L = 32, 4, 640
    lens_list = [[577], [640], [1]]
    cases = []
    for i, lens in enumerate(lens_list):
        q = dev(draw((1, H, 64), 100 + i, "f32"), torch.float32)
        kc = dev(draw((1, L, Hkv, 64), 110 + i, "f32"), torch.float32)
        vc = dev(draw((1, L, Hkv, 64), 120 + i, "f32"), torch.float32)
        ld = torch.tensor(lens, dtype=torch.int32, device="cuda")
        o = torch.empty((1, H, 64), device="cuda")
        ws = B.decode_workspace(1, L, H)
        cases.append((q, kc, vc, ld, o, ws))

    def calls():
        for q, kc, vc, ld, o, ws in cases:
            B.gqa_decode(q, kc, vc, ld, o=o, scale=0.125, workspace=ws)

    calls()
    torch.cuda.synchronize()
    eager = [c[4].clone() for c in cases]
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            calls()
    torch.cuda.synchronize()
    for rep in range(5):
        for c in cases:
            c[4].fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for i, c in enumerate(cases):
            assert torch.equal(c[4], eager[i]), f"replay {rep} call {i}"
        calls()  # eager work between the replays
        torch.cuda.synchronize()
        for i, c in enumerate(cases):
            assert torch.equal(c[4], eager[i]), f"eager after replay {rep} call {i}"


@pytest.mark.parametrize("dtype,H,Hkv,L", [("bf16", 32, 4, 3000),   # whole-row split kernel
                                           ("bf16", 16, 2, 3000),   # per-KV-head split kernel
                                           ("f32", 32, 4, 3000)])   # fp32 split kernel
def test_decode_workspace_holding_nan(dtype, H, Hkv, L):
    """A reused workspace may hold anything (NaN, Inf) in the partial slots of
    chunks past a sequence's length: the combine never lets them reach the
    output.  Short ragged lengths leave most chunk slots unwritten."""
    Bn = 5
    lens = np.array([1, 129, 3000, 40, 700], np.int32)
    ws = B.decode_workspace(Bn, L, H)
    ws.view(torch.float32).fill_(float("nan"))
    ws.view(torch.float32)[1::7] = float("inf")
    q = draw((Bn, H, 64), 60, dtype)
    kc = draw((Bn, L, Hkv, 64), 61, dtype)
    vc = draw((Bn, L, Hkv, 64), 62, dtype)
    got = host(B.gqa_decode(dev(q, TD[dtype]), dev(kc, TD[dtype]), dev(vc, TD[dtype]),
                            torch.from_numpy(lens).cuda(), scale=0.125, workspace=ws))
    assert np.all(np.isfinite(got))
    for b in range(Bn):
        Lb = int(lens[b])
        ref = O.gqa_decode(q[b:b + 1], kc[b:b + 1, :Lb], vc[b:b + 1, :Lb],
                           np.array([Lb], np.int32), 0.125)
        assert_close(got[b:b + 1], ref, TOL[dtype], f"b={b} len={Lb}")


@pytest.mark.parametrize("ragged", [False, True])
def test_decode_baseline_shape(ragged):
    """config 3: B=64, bf16 cache of 4096, 32/4 heads; ragged lengths in [512, 4096]."""
    Bn, L, H, Hkv = 64, 4096, 32, 4
    r = np.random.default_rng(2)
    lens = r.integers(512, 4097, Bn).astype(np.int32) if ragged else np.full(Bn, L, np.int32)
    q = bf16_round(r.standard_normal((Bn, H, 64)).astype(np.float32))
    kc = bf16_round(r.standard_normal((Bn, L, Hkv, 64)).astype(np.float32))
    vc = bf16_round(r.standard_normal((Bn, L, Hkv, 64)).astype(np.float32))
    qd, kd, vd = dev(q, torch.bfloat16), dev(kc, torch.bfloat16), dev(vc, torch.bfloat16)
    ld = torch.from_numpy(lens).cuda()
    ws = B.decode_workspace(Bn, L, H)
    got = host(B.gqa_decode(qd, kd, vd, ld, scale=0.125, workspace=ws))
    for b in (0, 17, 63):
        Lb = int(lens[b])
        ref = O.gqa_decode(q[b:b + 1], kc[b:b + 1, :Lb], vc[b:b + 1, :Lb],
                           np.array([Lb], np.int32), 0.125)
        assert_close(got[b:b + 1], ref, BF16_TOL, f"b={b}")
    # decode == the last row of the (independent) prefill kernel, every sequence
    for b in range(0, Bn, 9):
        Lb = int(lens[b])
        last = B.gqa_prefill(qd[b:b + 1, None], kd[b:b + 1, :Lb], vd[b:b + 1, :Lb],
                             scale=0.125, causal=True, seq_offset=Lb - 1)
        assert_close(got[b], host(last)[0, 0], BF16_TOL, f"decode vs prefill b={b}")


# ---------------------------------------------------------------- forward lse
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("case", PREFILL_CASES)
def test_prefill_lse_vs_oracle(case, dtype):
    # lse is compared in absolute terms: an absolute lse error is the relative
    # error of the row's softmax denominator, bounded by the dtype tolerance
    Bn, Sq, Skv, H, Hkv, causal, off = case
    q = draw((Bn, Sq, H, 64), 1, dtype)
    k = draw((Bn, Skv, Hkv, 64), 2, dtype)
    v = draw((Bn, Skv, Hkv, 64), 3, dtype)
    o, lse = B.gqa_prefill_lse(dev(q, TD[dtype]), dev(k, TD[dtype]), dev(v, TD[dtype]),
                               scale=0.125, causal=bool(causal), seq_offset=off)
    assert_close(host(o), O.gqa_prefill(q, k, v, 0.125, bool(causal), off), TOL[dtype],
                 f"prefill_lse o {case} {dtype}")
    ref = O.gqa_prefill_lse(q, k, 0.125, bool(causal), off)
    got = host(lse)
    fin = np.isfinite(ref)
    assert np.array_equal(np.isfinite(got), fin), "rows with / without visible keys differ"
    assert np.all(got[~fin] == -np.inf)
    if fin.any():
        err = float(np.max(np.abs(got[fin] - ref[fin])))
        assert err <= TOL[dtype], f"lse {case} {dtype}: max abs error {err:.3e}"


# ------------------------------------------------------------------- backward
BWD_CASES = PREFILL_CASES + [
    (1, 300, 40, 4, 2, 1, 0),       # causal, fewer keys than query rows
    (1, 96, 500, 8, 4, 0, 0),       # non-causal, many key blocks per query block
]


def bwd_inputs(case, seed=10):
    Bn, Sq, Skv, H, Hkv, _, _ = case
    return (draw((Bn, Sq, H, 64), seed, "bf16"), draw((Bn, Skv, Hkv, 64), seed + 1, "bf16"),
            draw((Bn, Skv, Hkv, 64), seed + 2, "bf16"), draw((Bn, Sq, H, 64), seed + 3, "bf16"))


def nan_like(t):
    return torch.full_like(t, float("nan"))


BF16_U = 2.0 ** -8   # bf16 unit roundoff


def check_backward(got, q, k, v, do, o, lse, causal, off, what):
    """got = (dq, dk, dv) on the host.  Against the exact chain form: the
    north-star bound, max relative error <= 2e-2.  Element-wise (assert_close)
    against the residual form evaluated in fp64 on the forward's own bf16 o
    and fp32 lse, since the backward inherits the rounding of those residuals
    (D = rowsum(dO*O) from a bf16 O moves a row's dq coherently), which the
    exact chain form does not carry.  The element-wise bound is the larger of
    2e-2 * max(|ref|, rms(ref)) and the bf16 error model of the products
    dq = dS K, dk = dS^T Q, dv = P^T dO: dS and P enter the MFMA rounded to
    bf16 (u = 2^-8) and the result is rounded to bf16 (u), so |error| <=
    2u * sum|a||b|; 2.5u leaves room for the fp32 accumulation and the
    recomputed exponential.  Without it, rows with one or two visible keys
    (large dS of opposite signs whose products with K cancel) exceed 2% of
    the rms in a few elements."""
    chain = O.gqa_prefill_backward(q, k, v, do, 0.125, bool(causal), off)
    res, cond = O.gqa_prefill_backward_from_residuals(q, k, v, o, lse, do, 0.125, bool(causal),
                                                      off, with_condition=True)
    for name, g, c, r, m in zip(("dq", "dk", "dv"), got, chain, res, cond):
        e = relerr(g, c)
        assert e <= BF16_TOL, f"{name} {what}: max relative error {e:.3e} vs the chain form"
        assert_close(g, r, BF16_TOL, f"{name} {what} vs the residual form", floor=2.5 * BF16_U * m)


@pytest.mark.parametrize("case", BWD_CASES)
def test_prefill_backward_vs_oracle(case):
    Bn, Sq, Skv, H, Hkv, causal, off = case
    q, k, v, do = bwd_inputs(case)
    qd, kd, vd, dod = (dev(a, torch.bfloat16) for a in (q, k, v, do))
    o, lse = B.gqa_prefill_lse(qd, kd, vd, scale=0.125, causal=bool(causal), seq_offset=off)
    # outputs start as NaN: every element is written, nothing accumulates
    dq, dk, dv = B.gqa_prefill_backward(qd, kd, vd, o, dod, lse, scale=0.125,
                                        causal=bool(causal), seq_offset=off, dq=nan_like(qd),
                                        dk=nan_like(kd), dv=nan_like(vd))
    gq, gk, gv = host(dq), host(dk), host(dv)
    check_backward((gq, gk, gv), q, k, v, do, host(o), host(lse), causal, off, str(case))
    if causal:
        # query rows that see no key and keys that no query row sees: exactly 0
        vis = np.arange(Skv)[None, :] <= np.arange(Sq)[:, None] + off
        assert np.all(gq[:, ~vis.any(1)] == 0.0)
        assert np.all(gk[:, ~vis.any(0)] == 0.0) and np.all(gv[:, ~vis.any(0)] == 0.0)


def test_prefill_backward_strided_rows():
    # q/k/v as column slices of a fused QKV row, the gradients as slices of a
    # fused dQKV row with the same strides
    Bn, S, H, Hkv = 2, 160, 8, 2
    W = (H + 2 * Hkv) * 64
    qkv = draw((Bn, S, W), 21, "bf16")
    do = draw((Bn, S, H, 64), 22, "bf16")
    t = dev(qkv, torch.bfloat16)
    g = torch.full_like(t, float("nan"))

    def split(x):
        return (x[:, :, :H * 64].unflatten(2, (H, 64)),
                x[:, :, H * 64:(H + Hkv) * 64].unflatten(2, (Hkv, 64)),
                x[:, :, (H + Hkv) * 64:].unflatten(2, (Hkv, 64)))

    q, k, v = split(t)
    dq, dk, dv = split(g)
    o, lse = B.gqa_prefill_lse(q, k, v, scale=0.125)
    B.gqa_prefill_backward(q, k, v, o, dev(do, torch.bfloat16), lse, scale=0.125, dq=dq, dk=dk,
                           dv=dv)
    qn = qkv[:, :, :H * 64].reshape(Bn, S, H, 64)
    kn = qkv[:, :, H * 64:(H + Hkv) * 64].reshape(Bn, S, Hkv, 64)
    vn = qkv[:, :, (H + Hkv) * 64:].reshape(Bn, S, Hkv, 64)
    check_backward((host(dq), host(dk), host(dv)), qn, kn, vn, do, host(o), host(lse), 1, 0,
                   "strided")


def test_prefill_backward_workspace_and_repeat():
    # a caller workspace gives the same bits as the pool, and a second call
    # over the same buffers reproduces the first
    case = (2, 200, 200, 8, 2, 1, 0)
    q, k, v, do = (dev(a, torch.bfloat16) for a in bwd_inputs(case, 30))
    o, lse = B.gqa_prefill_lse(q, k, v, scale=0.125)
    a = B.gqa_prefill_backward(q, k, v, o, do, lse, scale=0.125)
    ws = torch.empty(B.lib().bn_gqa_prefill_backward_workspace_size(2, 200, 200, 8, 2, 64, 1) // 4,
                     dtype=torch.float32, device="cuda")
    b = B.gqa_prefill_backward(q, k, v, o, do, lse, scale=0.125, workspace=ws)
    c = B.gqa_prefill_backward(q, k, v, o, do, lse, scale=0.125, workspace=ws)
    for x, y, z in zip(a, b, c):
        assert torch.equal(x, y) and torch.equal(y, z)


def test_prefill_backward_baseline_shape():
    # config-2 shape (B=4, S=2048, 32 heads over 4 KV heads): two (batch, KV
    # head) groups against the oracle, and every group on two properties that
    # hold at any size: each probability row sums to 1, so sum_key dv equals
    # sum over the group's heads and rows of dout; each dS row sums to 0, so
    # sum_key dk vanishes
    Bn, S, H, Hkv = 4, 2048, 32, 4
    G = H // Hkv
    rng = np.random.default_rng(40)
    q, k, v, do = (bf16_round(rng.standard_normal(s).astype(np.float32))
                   for s in ((Bn, S, H, 64), (Bn, S, Hkv, 64), (Bn, S, Hkv, 64), (Bn, S, H, 64)))
    qd, kd, vd, dod = (dev(a, torch.bfloat16) for a in (q, k, v, do))
    o, lse = B.gqa_prefill_lse(qd, kd, vd, scale=0.125)
    dq, dk, dv = B.gqa_prefill_backward(qd, kd, vd, o, dod, lse, scale=0.125)
    gq, gk, gv = host(dq), host(dk), host(dv)
    on, ln = host(o), host(lse)
    assert np.all(np.isfinite(gq)) and np.all(np.isfinite(gk)) and np.all(np.isfinite(gv))
    for b, g in ((3, 1), (0, 3)):
        hs, gs, bs = slice(g * G, (g + 1) * G), slice(g, g + 1), slice(b, b + 1)
        check_backward((gq[bs, :, hs], gk[bs, :, gs], gv[bs, :, gs]), q[bs, :, hs], k[bs, :, gs],
                       v[bs, :, gs], do[bs, :, hs], on[bs, :, hs], ln[bs, hs], 1, 0, f"b{b} g{g}")
    for b in range(Bn):
        for g in range(Hkv):
            want = do[b, :, g * G:(g + 1) * G].astype(np.float64).sum((0, 1))
            got = gv[b, :, g].astype(np.float64).sum(0)
            assert np.max(np.abs(got - want)) <= BF16_TOL * np.max(np.abs(want)), (b, g)
            zs = np.abs(gk[b, :, g].astype(np.float64).sum(0))
            assert np.all(zs <= BF16_TOL * np.abs(gk[b, :, g]).sum(0)), (b, g)


def test_bten_surface_backward_matches_c_abi():
    # the pybind11 surface (rows = tokens, [batch*seq, heads*64]) runs the same
    # kernels: identical bits to the ctypes path, and the oracle's gradients
    import bten
    case = (2, 150, 150, 8, 2, 1, 0)
    Bn, S, _, H, Hkv, _, _ = case
    q, k, v, do = bwd_inputs(case, 50)

    def t(a):
        rows, cols = a.shape[0] * a.shape[1], a.shape[2] * a.shape[3]
        x = bten.TensorBF16(rows, cols, True)
        x.copy_from_numpy(np.ascontiguousarray(a.reshape(rows, cols)))
        return x

    tq, tk, tv, tdo = t(q), t(k), t(v), t(do)
    o, lse = bten.gqa_prefill_lse(tq, tk, tv, Bn, H, Hkv, 64, 0.125)
    dq, dk, dv = bten.gqa_prefill_backward(tq, tk, tv, o, tdo, lse, Bn, H, Hkv, 64, 0.125)
    bten.synchronize()
    got = [x.to_numpy().reshape(sh) for x, sh in ((dq, q.shape), (dk, k.shape), (dv, v.shape))]
    qd, kd, vd, dod = (dev(a, torch.bfloat16) for a in (q, k, v, do))
    o2, lse2 = B.gqa_prefill_lse(qd, kd, vd, scale=0.125)
    ref = B.gqa_prefill_backward(qd, kd, vd, o2, dod, lse2, scale=0.125)
    assert np.array_equal(lse.to_numpy().reshape(Bn, H, S), host(lse2))
    for g, r in zip(got, ref):
        assert np.array_equal(g, host(r))
    check_backward(got, q, k, v, do, host(o2), host(lse2), 1, 0, "bten")


@pytest.mark.parametrize("Sq,Skv", [(0, 96), (70, 0)])
def test_prefill_backward_empty_sides(Sq, Skv):
    # no query rows: every key gets dK = dV = 0 (written, not left as they
    # were); no keys: every row gets dQ = 0
    H, Hkv = 8, 2
    q = torch.zeros((1, Sq, H, 64), dtype=torch.bfloat16, device="cuda")
    k = torch.randn((1, Skv, Hkv, 64), device="cuda").to(torch.bfloat16)
    v = torch.randn((1, Skv, Hkv, 64), device="cuda").to(torch.bfloat16)
    o = torch.zeros_like(q)
    do = torch.randn((1, Sq, H, 64), device="cuda").to(torch.bfloat16)
    lse = torch.full((1, H, Sq), float("-inf"), device="cuda")
    dq, dk, dv = B.gqa_prefill_backward(q, k, v, o, do, lse, scale=0.125, dq=nan_like(q),
                                        dk=nan_like(k), dv=nan_like(v))
    torch.cuda.synchronize()
    assert torch.count_nonzero(dq.float()).item() == 0 and not torch.isnan(dq.float()).any()
    assert torch.count_nonzero(dk.float()).item() == 0 and not torch.isnan(dk.float()).any()
    assert torch.count_nonzero(dv.float()).item() == 0 and not torch.isnan(dv.float()).any()
