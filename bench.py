#!/usr/bin/env python3
"""Benchmark of the MI355X GQA attention path (one JSON line on stdout).

Headline (``value``): causal GQA prefill, config 2 in bf16
(B=4, S=2048, 32 query / 4 KV heads, head_dim 64, scale 1/8), in TFLOP/s of
algorithmic work 4*B*H*D*S(S+1)/2 (unmasked QK^T and PV MACs x 2).
One step = one prefill launch over the whole batch, inputs resident in HBM.

Also measured in the same run and reported as sub-objects:
  decode        config 3: B=64 one-token decode over a bf16 cache of 4096
                (uniform), in GB/s of K/V + q + o bytes; two cache sets are
                rotated so the 268 MB cache cannot sit in the 256 MB MALL;
                caches stored head-major [B, Hkv, L, 64] (bn_gqa_decode_strided),
                the token-major [B, L, Hkv, 64] figure (bn_gqa_decode) beside it
  decode_ragged config 3 with lengths uniform in [512, 4096], the same two layouts
  prefill_fp32  config 2 in fp32
  rmsnorm_rope  config 5's fused RMSNorm+RoPE on [16384, 2048] bf16, GB/s
  prefill_long  config 5's prefill, B=1, S=16384, bf16
  add_rmsnorm   fused residual add + RMSNorm, bf16 [16384, 2048], GB/s
  silu_mul      SwiGLU activation, bf16 [16384, 5632], GB/s
  linear_rope   config 4's fused QKV projection with RoPE in the epilogue, fp32:
                prompt (M=512, TFLOP/s) and decode step (M=1, GB/s of weights)
  prefill_backward  config 2's flash-style backward (dQ, dK, dV), bf16,
                TFLOP/s of 2.5x the forward's algorithmic flops
Each carries a ``roofline`` object priced against MI355X peaks (bf16 MFMA
2.5 PFLOP/s dense, fp32 MFMA 157.3 TFLOP/s, HBM 8 TB/s).  ``cpu_baseline``
times the CPU oracle (a single-threaded C restatement of the reference
kernels, test infrastructure) on a bounded sample of the same workload.

Timing: hip events recorded on the stream the kernels are launched on (the
current torch stream, passed to the C ABI), around K back-to-back launches
after W warm-up launches followed by at least --warm-seconds (default 1 s)
of untimed back-to-back launches of the same workload (GPU clock settled),
with torch.cuda.synchronize() on both sides.
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "baranet-bdml_amd"))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
METRIC = "GQA prefill attention TFLOP/s + % MFMA peak; decode KV GB/s + % HBM peak"


def prefill_flops(B, S, H, D):
    return 4 * B * H * D * S * (S + 1) // 2


def decode_bytes(lens, Hkv, D, B, H, elem):
    return int(sum(2 * int(L) * Hkv * D * elem for L in lens) + 2 * B * H * D * elem)


WARM_SECONDS = 1.0  # --warm-seconds


def time_launches(fn, steps, warmup):
    """Average launch duration (ms) of fn() over `steps` back-to-back calls.

    Untimed warm-up: `warmup` calls, then more calls until WARM_SECONDS of
    back-to-back work have run, so the GPU clock has left its idle state
    (a cold GPU runs the first ~100 ms of MFMA work ~20% slower)."""
    import torch
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    t0, i, burst = time.perf_counter(), warmup, 4
    while time.perf_counter() - t0 < WARM_SECONDS:
        tb = time.perf_counter()
        for _ in range(burst):
            fn(i)
            i += 1
        torch.cuda.synchronize()
        if time.perf_counter() - tb < 0.05:
            burst *= 2
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for i in range(steps):
        fn(i)
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps


def time_graph(fn, n, steps, warmup, check=None):
    """Average duration (ms) of one fn(i) call, from a graph of fn(0..n-1)
    captured once and replayed: no host launch cost in the timed region.  The
    output tensor `check` after a replay must equal its eager value."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(n):
            fn(i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    eager = check.clone() if check is not None else None
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n):
            fn(i)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        if eager is not None and not torch.equal(check, eager):
            raise RuntimeError("graph replay differs from the eager result")
    return time_launches(lambda i: g.replay(), steps, warmup) / n


def measured_traffic(key):
    """HBM bytes per launch of the workload's dominant kernel, from the
    calibrated FETCH_SIZE + WRITE_SIZE counter passes kept in
    profiles/traffic.json (rocprofv3 cannot run inside this process)."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            return json.load(f)[key]["total"]
    except (OSError, KeyError, ValueError):
        return None


def roofline(bound, achieved, peak, unit, traffic=None):
    return {"bound": bound, "achieved": round(achieved, 3), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic}


def cpu_meta():
    """Host the CPU baselines ran on: logical CPUs of the machine, CPUs this
    process may run on, and the CPU model from /proc/cpuinfo."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        allowed = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        allowed = os.cpu_count()
    return {"nproc": os.cpu_count(), "cpus_allowed": allowed, "cpu_model": model}


def cpu_result(value, unit, sample, cores=1):
    """A cpu_baseline object: the single-threaded C oracle (kind "port": a
    restatement of the reference kernels' loops) on a bounded sample."""
    return dict({"value": value, "unit": unit, "cores": cores, "kind": "port", "sample": sample},
                **cpu_meta())


def bench_prefill(B_, S, H, Hkv, dtype, steps, warmup, seed=0):
    import torch
    import bnhip
    g = torch.Generator(device="cuda").manual_seed(seed)
    td = torch.bfloat16 if dtype == "bf16" else torch.float32
    q = torch.randn((B_, S, H, 64), generator=g, device="cuda").to(td)
    k = torch.randn((B_, S, Hkv, 64), generator=g, device="cuda").to(td)
    v = torch.randn((B_, S, Hkv, 64), generator=g, device="cuda").to(td)
    o = torch.empty_like(q)
    ms = time_launches(lambda i: bnhip.gqa_prefill(q, k, v, o, scale=0.125), steps, warmup)
    fl = prefill_flops(B_, S, H, 64)
    tflops = fl / (ms * 1e-3) / 1e12
    peak = PEAK_BF16_TFLOPS if dtype == "bf16" else PEAK_FP32_TFLOPS
    return {"value": round(tflops, 3), "unit": "TFLOP/s", "ms_per_launch": round(ms, 5),
            "flops_per_launch": fl,
            "roofline": roofline("mfma", tflops, peak, "TFLOP/s",
                                 measured_traffic({("bf16", 2048): "prefill_bf16",
                                                   ("fp32", 2048): "prefill_fp32",
                                                   ("bf16", 16384): "prefill_long"}.get((dtype, S),
                                                                                        "")))}


def bench_backward(steps, warmup, seed=5):
    """Config 2's backward: one step = bn_gqa_prefill_backward (the dQ kernel,
    then the dK/dV kernel) from the forward's o and lse.  Algorithmic work:
    five products over the causal half, 2.5x the forward's flops (S = QK^T
    recomputed, dP = dO V^T, dQ = dS K, dK = dS^T Q, dV = P^T dO)."""
    import torch
    import bnhip
    g = torch.Generator(device="cuda").manual_seed(seed)
    B_, S, H, Hkv = 4, 2048, 32, 4
    q = torch.randn((B_, S, H, 64), generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn((B_, S, Hkv, 64), generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn((B_, S, Hkv, 64), generator=g, device="cuda").to(torch.bfloat16)
    do = torch.randn((B_, S, H, 64), generator=g, device="cuda").to(torch.bfloat16)
    o, lse = bnhip.gqa_prefill_lse(q, k, v, scale=0.125)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws = torch.empty(bnhip.lib().bn_gqa_prefill_backward_workspace_size(B_, S, S, H, Hkv, 64, 1) // 4,
                     dtype=torch.float32, device="cuda")
    ms = time_launches(lambda i: bnhip.gqa_prefill_backward(q, k, v, o, do, lse, scale=0.125,
                                                            dq=dq, dk=dk, dv=dv, workspace=ws),
                       steps, warmup)
    fl = 5 * prefill_flops(B_, S, H, 64) // 2
    tflops = fl / (ms * 1e-3) / 1e12
    return {"value": round(tflops, 3), "unit": "TFLOP/s", "ms_per_launch": round(ms, 5),
            "flops_per_launch": fl, "config": "config 2 backward, bf16",
            "roofline": roofline("mfma", tflops, PEAK_BF16_TFLOPS, "TFLOP/s",
                                 measured_traffic("prefill_backward")),
            "traffic_kernel": "dK/dV kernel (the longest of the three launches)"}


def bench_linear(steps, warmup, seed=6):
    """Config 4's fused QKV projection with RoPE on its Q/K columns, fp32:
    x [M, 2048] @ w [2048, 2560], rope_cols 2304, for the prompt (M = 512,
    MFMA-bound, flops 2*M*K*N, row-major w) and a decode step (M = 1,
    HBM-bound on w, bytes K*N*4 + x + y; timed from a replayed graph of 16
    launches; w output-major, as the TinyLLaMA driver stores it, with the
    row-major split-k path beside it).  Beside each, the unfused path it
    replaces: torch's library GEMM (x @ w) followed by bn_rope on the Q/K
    columns."""
    import torch
    import bnhip
    g = torch.Generator(device="cuda").manual_seed(seed)
    K, N, RC = 2048, 2560, 2304
    # 16 weight copies (336 MB) rotated per launch, so that the decode step's
    # 21 MB weight cannot sit in the 256 MB MALL between launches, as in the
    # model, where each layer has its own
    ws_all = [torch.randn((K, N), generator=g, device="cuda") / 45.0 for _ in range(16)]
    out = {}
    for M in (512, 1):
        x = torch.randn((M, K), generator=g, device="cuda")
        y = torch.empty((M, N), device="cuda")
        ws = torch.empty(max(bnhip.lib().bn_linear_rope_workspace_size(0, M, N, K) // 4, 1),
                         device="cuda")
        # the decode step reads the weights output-major ([N, K] storage, the
        # [K, N] view transposed): the few-rows kernel without a k split
        wts = ws_all if M > 1 else [w.t().contiguous().t() for w in ws_all]
        fused = lambda i: bnhip.linear_rope(x, wts[i % 16], y, rope_cols=RC, position_offset=7,
                                             workspace=ws)
        yt = torch.empty((M, N), device="cuda")

        def unfused(i):
            torch.matmul(x, wts[i % 16], out=yt)
            q = yt[:, :RC]
            bnhip.call("bn_rope", bnhip.C.byref(bnhip.view(q)), bnhip.C.byref(bnhip.view(q)), 7, 64,
                       1e4, bnhip.stream_of())
        if M > 1:
            ms = time_launches(fused, steps, warmup)
            ms_ref = time_launches(unfused, steps, warmup)
        else:
            # a decode step's kernels are shorter than a Python launch: time 16
            # launches (one per weight copy) replayed from a captured graph
            ms = time_graph(fused, 16, steps, warmup, check=y)
            ms_ref = time_graph(unfused, 16, steps, warmup, check=yt)
            ms_rm = time_graph(lambda i: bnhip.linear_rope(x, ws_all[i % 16], y, rope_cols=RC,
                                                           position_offset=7, workspace=ws),
                               16, steps, warmup, check=y)
            del wts
        fl = 2 * M * K * N
        byt = 4 * (K * N + M * K + M * N)
        if M > 1:
            v = fl / (ms * 1e-3) / 1e12
            out["prompt"] = {"value": round(v, 3), "unit": "TFLOP/s", "ms_per_launch": round(ms, 5),
                             "m": M, "unfused_ms": round(ms_ref, 5),
                             "roofline": roofline("mfma", v, PEAK_FP32_TFLOPS, "TFLOP/s",
                                                  measured_traffic("linear_rope_prompt"))}
        else:
            v = byt / (ms * 1e-3) / 1e9
            out["decode_step"] = {"value": round(v, 1), "unit": "GB/s", "ms_per_launch": round(ms, 5),
                                  "m": M, "unfused_ms": round(ms_ref, 5),
                                  "weights": "output-major ([N, K] storage)",
                                  "row_major_split_k_ms": round(ms_rm, 5),
                                  "roofline": roofline("hbm", v, PEAK_HBM_GBS, "GB/s",
                                                       measured_traffic("linear_rope_decode"))}
    out["config"] = "config 4 QKV projection + RoPE, fp32, K=2048, N=2560, rope_cols=2304"
    # the product runs this kernel on the decode steps (prompts: library GEMM + RoPE)
    out["roofline"] = dict(out["decode_step"]["roofline"], kind="decode_step")
    return out


def decode_lengths(kind, B_=64, L=4096, seed=2):
    """Config 3's lengths: uniform 4096, the ragged U[512, 4096] draw, and two
    more ragged patterns for the planned path: two length classes (512 and
    4096 alternating) and four 4096-key caches among 600-key ones."""
    import numpy as np
    r = np.random.default_rng(seed)
    if kind == "ragged":
        return r.integers(512, L + 1, B_).astype(np.int32)
    if kind == "two_class":
        return np.where(np.arange(B_) % 2 == 0, 512, L).astype(np.int32)
    if kind == "skewed":
        out = np.full(B_, 600, np.int32)
        out[[3, 20, 41, 62]] = L
        return out
    return np.full(B_, L, np.int32)


def bench_decode(kind, steps, warmup, seed=2, planned=False, layout="token_major"):
    """Config 3 decode; planned=True times bn_gqa_decode_planned (the host
    lengths plan equal tile shares per compute unit) instead of
    bn_gqa_decode.  layout: the caches' storage -- "token_major"
    [B, L, Hkv, 64] contiguous (bn_gqa_decode) or "head_major" [B, Hkv, L, 64]
    (each (sequence, KV head)'s rows contiguous; bn_gqa_decode_strided)."""
    import torch
    import bnhip
    B_, L, H, Hkv = 64, 4096, 32, 4
    lens = decode_lengths(kind, B_, L, seed)
    g = torch.Generator(device="cuda").manual_seed(seed)
    cache = ((lambda: torch.randn((B_, L, Hkv, 64), generator=g, device="cuda").bfloat16())
             if layout == "token_major" else
             (lambda: torch.randn((B_, Hkv, L, 64), generator=g, device="cuda").bfloat16()
              .transpose(1, 2)))
    sets = []
    for _ in range(2):  # 2 x 268 MB > 256 MB MALL: every launch streams from HBM
        sets.append((torch.randn((B_, H, 64), generator=g, device="cuda").bfloat16(), cache(),
                     cache()))
    ld = torch.from_numpy(lens).cuda()
    nws = bnhip.lib().bn_gqa_decode_planned_workspace_size(B_, L, H, Hkv, 64)
    ws = torch.empty(nws, dtype=torch.uint8, device="cuda")
    o = torch.empty((B_, H, 64), device="cuda", dtype=torch.bfloat16)

    def run(i):
        q, kc, vc = sets[i % 2]
        if planned:
            bnhip.gqa_decode_planned(q, kc, vc, ld, lens, o, scale=0.125, workspace=ws)
        else:
            bnhip.gqa_decode(q, kc, vc, ld, o, scale=0.125, workspace=ws)

    ms = time_launches(run, steps, warmup)
    nb = decode_bytes(lens, Hkv, 64, B_, H, 2)
    gbs = nb / (ms * 1e-3) / 1e9
    desc = {"uniform": "uniform 4096", "ragged": f"ragged U[512,4096] seed {seed}",
            "two_class": "512 and 4096 alternating", "skewed": "four 4096 among 600"}[kind]
    key = {"uniform": "decode", "ragged": "decode_ragged"}.get(kind, "")
    if layout == "head_major":
        key += "_head_major"
    return {"value": round(gbs, 2), "unit": "GB/s", "ms_per_launch": round(ms, 5),
            "bytes_per_launch": nb, "lengths": f"{desc}, sum {int(lens.sum())}",
            "cache_layout": "[B, L, Hkv, 64]" if layout == "token_major" else "[B, Hkv, L, 64]",
            "entry_point": (("bn_gqa_decode_planned" if layout == "token_major"
                             else "bn_gqa_decode_planned_strided") if planned else
                            "bn_gqa_decode" if layout == "token_major" else "bn_gqa_decode_strided"),
            "roofline": roofline("hbm", gbs, PEAK_HBM_GBS, "GB/s",
                                 measured_traffic("decode_planned_" + kind +
                                                  ("_head_major" if layout == "head_major" else ""))
                                 if planned else measured_traffic(key))}


def bench_decode_planned(steps, warmup):
    """The planned decode beside the whole-cache kernel on three ragged
    patterns, both on head-major caches (the config-3 lines' layout)."""
    out = {}
    for kind in ("ragged", "two_class", "skewed"):
        pl = bench_decode(kind, steps, warmup, planned=True, layout="head_major")
        plain = bench_decode(kind, steps, warmup, layout="head_major") if kind != "ragged" else None
        out[kind] = {"planned": pl}
        if plain is not None:
            out[kind]["bn_gqa_decode"] = plain
    out["roofline"] = dict(out["two_class"]["planned"]["roofline"], kind="two_class planned")
    return out


def bench_rmsnorm_rope(steps, warmup):
    import ctypes as C
    import torch
    import bnhip
    rows, w = 16384, 2048
    g = torch.Generator(device="cuda").manual_seed(5)
    # 4 input/output sets of 67 MB each (537 MB) rotated per launch: the input
    # of a launch was last touched 3 launches ago, past the 256 MB MALL
    NS = 4
    xs = [torch.randn((rows, w), generator=g, device="cuda").bfloat16() for _ in range(NS)]
    ys = [torch.empty_like(xs[0]) for _ in range(NS)]
    wt = torch.ones((1, w), device="cuda", dtype=torch.bfloat16)
    wv = bnhip.view(wt)
    views = [(bnhip.view(x), bnhip.view(y)) for x, y in zip(xs, ys)]
    st = bnhip.stream_of()

    def run(i):
        xv, yv = views[i % NS]
        bnhip.call("bn_rmsnorm_rope", C.byref(xv), C.byref(wv), C.byref(yv), 1e-5, 0, 64,
                   1e4, st)

    ms = time_launches(run, steps, warmup)
    nb = 2 * rows * w * 2 + w * 2
    gbs = nb / (ms * 1e-3) / 1e9
    return {"value": round(gbs, 2), "unit": "GB/s", "ms_per_launch": round(ms, 5),
            "bytes_per_launch": nb,
            "roofline": roofline("hbm", gbs, PEAK_HBM_GBS, "GB/s", measured_traffic("rmsnorm_rope"))}


def bench_add_rmsnorm(steps, warmup):
    """Fused residual add + RMSNorm on a config-5-sized bf16 row block
    [16384, 2048]: read x, delta (and the weight), write h and y."""
    import ctypes as C
    import torch
    import bnhip
    rows, w = 16384, 2048
    g = torch.Generator(device="cuda").manual_seed(6)
    sets = [[torch.randn((rows, w), generator=g, device="cuda").bfloat16() for _ in range(4)]
            for _ in range(2)]  # 2 x 268 MB > 256 MB MALL
    wt = torch.ones((1, w), device="cuda", dtype=torch.bfloat16)
    wv = bnhip.view(wt)
    views = [[bnhip.view(t) for t in st] for st in sets]
    st_ = bnhip.stream_of()

    def run(i):
        xv, dv, hv, yv = views[i % 2]
        bnhip.call("bn_add_rmsnorm", C.byref(xv), C.byref(dv), C.byref(wv), C.byref(hv), C.byref(yv),
                   1e-5, st_)

    ms = time_launches(run, steps, warmup)
    nb = 4 * rows * w * 2 + w * 2
    gbs = nb / (ms * 1e-3) / 1e9
    return {"value": round(gbs, 2), "unit": "GB/s", "ms_per_launch": round(ms, 5),
            "bytes_per_launch": nb, "shape": [rows, w], "dtype": "bf16",
            "roofline": roofline("hbm", gbs, PEAK_HBM_GBS, "GB/s", measured_traffic("add_rmsnorm"))}


def bench_silu_mul(steps, warmup):
    """SwiGLU activation silu(gate) * up on a [16384, 5632] bf16 block (the
    TinyLLaMA MLP width at config 5's row count): read gate and up, write out."""
    import ctypes as C
    import torch
    import bnhip
    rows, w = 16384, 5632
    g = torch.Generator(device="cuda").manual_seed(7)
    gt, ut = (torch.randn((rows, w), generator=g, device="cuda").bfloat16() for _ in range(2))
    ot = torch.empty_like(gt)
    gv, uv, ov = bnhip.view(gt), bnhip.view(ut), bnhip.view(ot)
    st_ = bnhip.stream_of()

    def run(i):
        bnhip.call("bn_silu_mul", C.byref(gv), C.byref(uv), C.byref(ov), st_)

    ms = time_launches(run, steps, warmup)
    nb = 3 * rows * w * 2  # 554 MB per launch: larger than the MALL
    gbs = nb / (ms * 1e-3) / 1e9
    return {"value": round(gbs, 2), "unit": "GB/s", "ms_per_launch": round(ms, 5),
            "bytes_per_launch": nb, "shape": [rows, w], "dtype": "bf16",
            "roofline": roofline("hbm", gbs, PEAK_HBM_GBS, "GB/s", measured_traffic("silu_mul"))}


def bench_copy(steps, warmup):
    """Plain device copy of a known size: the calibration point that turns the
    FETCH_SIZE / WRITE_SIZE counters into HBM bytes (bytes per launch known)."""
    import torch
    n = 64 << 20  # 64 Mi fp32 = 256 MiB read + 256 MiB written per launch
    xs = [torch.ones(n, device="cuda") for _ in range(2)]
    y = torch.empty(n, device="cuda")
    ms = time_launches(lambda i: y.copy_(xs[i % 2]), steps, warmup)
    nb = 2 * 4 * n
    return {"value": round(nb / (ms * 1e-3) / 1e9, 2), "unit": "GB/s",
            "ms_per_launch": round(ms, 5), "bytes_read": 4 * n, "bytes_written": 4 * n}


def bench_block(steps, warmup):
    """Config 1: one TinyLLaMA attention block through the `bten` surface, fp32,
    B=1 S=128: RMSNorm(1e-5) -> Q/K/V -> RoPE -> causal softmax(QK^T/8)V -> O.
    fused_head = the reference's chain (one S x S probability matrix over the
    2048-wide rows); per_head = GQA with the fused prefill kernel."""
    import numpy as np
    import torch
    import bten
    from llama_layers import GroupedQueryAttention, RMSNorm
    S, hid = 128, 2048
    x = np.random.default_rng(0).standard_normal((S, hid)).astype(np.float32)
    rw = np.random.default_rng(1)
    ws = [(rw.standard_normal(sh) * 0.02).astype(np.float32)
          for sh in ((hid, hid), (hid, 256), (hid, 256), (hid, hid))]
    xt = bten.TensorF(S, hid)
    xt.copy_from_numpy(x)
    out = {}
    for mode in ("fused_head", "fused_head_ops", "per_head"):
        norm = RMSNorm(hid, eps=1e-5)
        attn = GroupedQueryAttention(bten.LLaMAConfig(), mode=mode)
        attn.load_weights(*ws)
        ms = time_launches(lambda i: attn(norm(xt)), steps, warmup)
        out[mode] = {"ms_per_block": round(ms, 4)}
    out["note"] = ("bten launches on the legacy default stream, timed with events on the same "
                   "stream; includes the per-op pool allocations of the op surface. fused_head = "
                   "the chain's attention in one launch (bn_fused_head_attention); "
                   "fused_head_ops = the same chain op by op (repeat_kv x2, QK^T GEMM, scale, "
                   "softmax, PV GEMM)")
    out["fused_head_kernel"] = bench_fused_head_kernel(steps, warmup)
    out["fused_head_long"] = bench_fused_head_long(steps, warmup)
    # the block's dominant device kernel is the attention launch
    out["roofline"] = dict(out["fused_head_kernel"]["roofline"], kind="fused_head_kernel")
    return out, (x, ws)


def bench_fused_head_kernel(steps, warmup, S=128):
    """The attention of config 1 alone through the C ABI: bn_fused_head_attention
    against the op-by-op chain it replaces, on the same torch buffers (q
    [128, 2048], k/v [128, 256], fp32).  Device time from graph replays of 20
    back-to-back launches (no host gaps); the chain eagerly (its GEMMs are
    library calls)."""
    import ctypes as C
    import torch
    import bnhip
    g = torch.Generator(device="cuda").manual_seed(0)
    q = torch.randn((S, 2048), generator=g, device="cuda")
    k = torch.randn((S, 256), generator=g, device="cuda")
    v = torch.randn((S, 256), generator=g, device="cuda")
    o = torch.empty((S, 2048), device="cuda")
    fused = lambda i: bnhip.fused_head_attention(q, k, v, 32, 4, 64, o=o, scale=0.125)
    graph_ms = time_graph(fused, 20, max(steps, 20), warmup, check=o)
    eager_ms = time_launches(fused, max(steps, 20), warmup)
    kr, vr = torch.empty((S, 2048), device="cuda"), torch.empty((S, 2048), device="cuda")
    sc, p, oc = (torch.empty((S, S), device="cuda"), torch.empty((S, S), device="cuda"),
                 torch.empty((S, 2048), device="cuda"))
    V = lambda t: C.byref(bnhip.view(t))
    st = bnhip.stream_of()
    krt = kr.t()

    def chain(i):
        bnhip.call("bn_repeat_kv", V(k), V(kr), 64, 8, st)
        bnhip.call("bn_repeat_kv", V(v), V(vr), 64, 8, st)
        bnhip.call("bn_matmul", V(q), V(krt), V(sc), st)
        bnhip.call("bn_unary", bnhip.BN_MUL_SCALAR, V(sc), 0.125, V(sc), st)
        bnhip.call("bn_softmax", V(sc), V(p), 1, 0, st)
        bnhip.call("bn_matmul", V(p), V(vr), V(oc), st)
    chain_ms = time_launches(chain, max(steps, 20), warmup)
    torch.cuda.synchronize()
    diff = float(((o - oc).abs().max() / oc.abs().max()).item())
    flop = 2 * 2 * 2048 * (S * (S + 1) // 2)   # the chain's causal QK^T and PV, 2048 wide
    nbytes = 4 * (2 * S * 2048 + 2 * S * 256)  # q in, o out, k and v in
    gbs = nbytes / (graph_ms * 1e-3) / 1e9
    return {"config": "Sq = Sk = 128, 32/4 heads, head_dim 64, fp32, causal",
            "roofline": dict(roofline("hbm", gbs, PEAK_HBM_GBS, "GB/s"),
                             note="latency-bound launch: 2.36 MB and 67 MFLOP (the chain's "
                                  "causal products) take under 1 us at either roofline"),
            "device_us": round(graph_ms * 1e3, 2), "eager_us_per_launch": round(eager_ms * 1e3, 2),
            "chain_eager_us": round(chain_ms * 1e3, 2),
            "chain_flop_causal": flop, "max_rel_diff_vs_chain": diff,
            "algorithmic_bytes": 4 * (2 * S * 2048 + 2 * S * 256),
            "note": "device_us from graph replays; the chain = repeat_kv x2, bn_matmul (library "
                    "GEMM), scale, softmax, bn_matmul, launched eagerly"}


def bench_fused_head_long(steps, warmup, sizes=(512, 2048)):
    """bn_fused_head_attention on longer prompts (32/4 heads, head_dim 64,
    fp32, causal), where it runs on the matrix cores: group sums of Q, 32 x
    128 score blocks on v_mfma_f32_32x32x2f32, a log-sum-exp merge (three
    launches and a pool allocation per call).  Eager launches back to back,
    events on the stream; the work counted is the causal half of the two
    products at the group-summed width (2 x 2 x 256 flops per visible pair)."""
    import torch
    import bnhip
    res = {}
    for S in sizes:
        g = torch.Generator(device="cuda").manual_seed(S)
        q = torch.randn((S, 2048), generator=g, device="cuda")
        k = torch.randn((S, 256), generator=g, device="cuda")
        v = torch.randn((S, 256), generator=g, device="cuda")
        o = torch.empty((S, 2048), device="cuda")
        fused = lambda i: bnhip.fused_head_attention(q, k, v, 32, 4, 64, o=o, scale=0.125)
        ms = time_launches(fused, max(steps, 20), warmup)
        flop = 2 * 2 * 256 * (S * (S + 1) // 2)
        tf = flop / (ms * 1e-3) / 1e12
        res[f"S{S}"] = {"us_per_call": round(ms * 1e3, 2), "flop": flop,
                        "roofline": roofline("mfma", tf, PEAK_FP32_TFLOPS, "TFLOP/s")}
    res["note"] = ("eager calls (host launch of three kernels and a pool round trip per call: "
                   "host-bound at 512 rows); device times per kernel in the rocprofv3 summary")
    return res


def cpu_baseline_block(x, ws):
    """Config 1 on the CPU oracle (single thread), the reference's fused-head chain."""
    import numpy as np
    from oracle import oracle as O
    t0 = time.perf_counter()
    xn = O.rmsnorm(x, np.ones((1, x.shape[1]), np.float32), 1e-5)
    O.gqa_layer(xn, *ws, 32, 4, 10000.0, 0, per_head=False)
    el = time.perf_counter() - t0
    return cpu_result(round(el * 1e3, 2), "ms per block",
                      "the whole config-1 block once (RMSNorm + projections + fused-head "
                      "attention + output projection), fp32 oracle")


def bench_tinyllama(prompt=512, new_tokens=128, cpu=True, warmup_tokens=2):
    """Config 4: TinyLLaMA-1.1B (random init, fp32) prefill of a 512-token seeded
    prompt + 128 greedy decode steps with a KV cache.

    path_device_ms is the config's metric: the device time of its attention
    (prefill and decode), RoPE and RMSNorm kernels over one generate, from
    graph replays of each kind's logged launches.  The decode steps rotate Q
    and K inside the QKV projection (qkv_rope): that launch is mostly the
    projection, so its time is reported beside the metric, not in it.
    Each kind carries a roofline of its own (algorithmic bytes or flops of its
    launches over its device time); `roofline` is the largest kind's.
    native_*: the same generate with the decode loop in native code
    (bn_llama_decode, the product's loop), timed with events on its stream
    and priced against HBM: every step streams all weights once."""
    import numpy as np
    import torch
    from tinyllama import TinyLlama, TinyLlamaConfig
    cfg = TinyLlamaConfig()
    m = TinyLlama(cfg, max_len=prompt + new_tokens, seed=1)
    ids = torch.from_numpy(np.random.default_rng(3).integers(0, 32000, prompt)).cuda()

    def reset():
        for L in m.layers:
            L["k_cache"].zero_()
            L["v_cache"].zero_()
        m.length = 0
    if warmup_tokens:
        m.generate(ids, warmup_tokens)  # warm-up (kernels, library handles)
        reset()
    torch.cuda.synchronize()
    m.path_log = []
    t0 = time.perf_counter()
    toks, path_ms = m.generate(ids, new_tokens, time_path=True)
    wall = time.perf_counter() - t0
    log, m.path_log = m.path_log, None
    by_kind = path_replay_ms(log)
    work = {}
    for k, _, w in log:
        work[k] = work.get(k, 0) + w
    metric_kinds = ("prefill_attention", "decode_attention", "rope", "rmsnorm")
    rl = {}
    for k in metric_kinds:
        if k not in by_kind:
            continue
        if k == "prefill_attention":
            v = work[k] / (by_kind[k] * 1e-3) / 1e12
            rl[k] = roofline("mfma", v, PEAK_FP32_TFLOPS, "TFLOP/s")
        else:
            v = work[k] / (by_kind[k] * 1e-3) / 1e9
            rl[k] = roofline("hbm", v, PEAK_HBM_GBS, "GB/s")
        rl[k]["work_per_generate"] = work[k]
        rl[k]["device_ms"] = round(by_kind[k], 3)
    dominant = max(rl, key=lambda k: by_kind[k])
    res = {"prompt": prompt, "new_tokens": new_tokens, "wall_s": round(wall, 3),
           "path_device_ms": round(sum(by_kind[k] for k in metric_kinds if k in by_kind), 3),
           "path_device_ms_by_kind": {k: round(by_kind[k], 3) for k in metric_kinds if k in by_kind},
           "qkv_rope_device_ms": round(by_kind.get("qkv_rope", 0.0), 3),
           "path_device_note": "each kind's launches of the generate (prompt + 128 steps) "
                               "captured into one graph in launch order and replayed; ms per "
                               "replay, no host gaps. path_device_ms = prefill attention + decode "
                               "attention + RoPE (the prompt's bn_rope) + RMSNorm (plain and fused "
                               "with the residual add). qkv_rope_device_ms = the decode steps' "
                               "QKV projections with the rotation in their epilogue (the steps' "
                               "RoPE, inseparable from the projection), kept out of the total",
           "roofline": dict(rl[dominant], kind=dominant),
           "rooflines": rl,
           "path_ms": round(path_ms, 3),
           "path_kernels": "RMSNorm (plain and fused with the residual add), RoPE (prompt: "
                           "bn_rope; decode steps: fused into the QKV projection kernel), GQA "
                           "prefill, GQA decode (fp32)",
           "first_tokens": [int(t) for t in toks[:8].cpu()], "cache_length_end": m.length}
    # the same generation with the decode loop in native code (bn_llama_decode):
    # one call runs every decode step, no host round trip per token
    reset()
    m.generate_native(ids, max(warmup_tokens, 1))
    reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ntoks = m.generate_native(ids, new_tokens)
    torch.cuda.synchronize()
    res["native_wall_s"] = round(time.perf_counter() - t0, 3)
    res["native_tokens_match"] = bool(torch.equal(ntoks.cpu(), toks.cpu()))
    # the decode loop alone, events on its stream: 128 steps after the prompt
    reset()
    logits = m.prefill(ids)
    first = int(torch.argmax(logits[-1]))
    out = torch.empty(new_tokens, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    s_, e_ = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s_.record()
    m.decode_native(first, new_tokens, out)
    e_.record()
    torch.cuda.synchronize()
    nat_ms = s_.elapsed_time(e_)
    h, I, V, kv = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size, \
        cfg.num_key_value_heads * cfg.head_dim
    w_layer = h * (h + 2 * kv) + h * h + h * 2 * I + I * h + 2 * h  # projections + norms
    nat_bytes = 0
    for t in range(new_tokens):
        L = prompt + t + 1  # cache length after the step's append
        nat_bytes += 4 * (cfg.num_hidden_layers * (w_layer + 2 * L * kv + 2 * kv) + h * V + h + h)
    gbs = nat_bytes / (nat_ms * 1e-3) / 1e9
    res["native_decode_ms"] = round(nat_ms, 3)
    res["native_roofline"] = dict(roofline("hbm", gbs, PEAK_HBM_GBS, "GB/s"),
                                  bytes_per_generate=nat_bytes,
                                  note="128 native decode steps: every fp32 weight (22 layers' "
                                       "projections and norms, lm_head, final norm) read once "
                                       "per step, the KV caches read and one row appended per "
                                       "layer, the embedding row; event time on the loop's "
                                       "stream (launch gaps included)")
    res["native_tokens_match_decode_only"] = bool(torch.equal(out[:new_tokens - 1].long().cpu(),
                                                              toks[1:].cpu()))
    if cpu:
        res["cpu_baseline"] = cpu_baseline_tinyllama(m, ids)
    return res


def path_replay_ms(log, steps=5):
    """Device time (ms) of logged launches by kind: each kind's launches are
    captured into one graph, in launch order, and the graph is replayed."""
    import torch
    out = {}
    for kind in sorted({e[0] for e in log}):
        fns = [e[1] for e in log if e[0] == kind]
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for fn in fns:
                fn()
        out[kind] = time_launches(lambda i: g.replay(), steps, 1)
        del g
    return out


def cpu_baseline_tinyllama(m, ids):
    """Oracle on the layer-0 prefill path inputs of the GPU model (teacher-forced),
    single thread, extrapolated x22 layers (labelled).  The projections that feed
    RoPE are numpy GEMMs outside the timed regions."""
    from oracle import oracle as O
    cfg = m.cfg
    L0 = m.layers[0]
    x = m.embed[ids].cpu().numpy()
    w = L0["ln1"].cpu().numpy()
    t0 = time.perf_counter()
    xn = O.rmsnorm(x, w, cfg.rms_norm_eps)
    t_norm = time.perf_counter() - t0
    hq, hk = cfg.hidden_size, cfg.num_key_value_heads * cfg.head_dim
    qkv = xn @ L0["wqkv"].cpu().numpy()  # the model's fused [hidden, hq + 2*hk] projection
    q, k, v = qkv[:, :hq].copy(), qkv[:, hq:hq + hk].copy(), qkv[:, hq + hk:].copy()
    S = x.shape[0]
    t0 = time.perf_counter()
    qr, kr = O.rope(q, 0, 64, 1e4), O.rope(k, 0, 64, 1e4)
    O.gqa_prefill(qr.reshape(1, S, 32, 64), kr.reshape(1, S, 4, 64), v.reshape(1, S, 4, 64),
                  0.125, True, 0)
    t_attn = time.perf_counter() - t0
    layer_s = 2 * t_norm + t_attn  # two RMSNorms per decoder layer
    return cpu_result(round(layer_s * cfg.num_hidden_layers * 1e3, 1),
                      "ms (prefill path kernels, 22 layers, extrapolated from layer 0)",
                      f"layer 0 of the prefill: 2 RMSNorm + RoPE(q, k) + per-head causal GQA "
                      f"over {S} tokens on the GPU run's inputs, fp32 oracle, "
                      f"{layer_s:.2f} s; decode steps not included")


def cpu_baseline_prefill(budget_s=12.0):
    """CPU oracle (single thread) on whole (batch, head) pairs of config 2."""
    import numpy as np
    from oracle import oracle as O
    S, D = 2048, 64
    r = np.random.default_rng(0)
    done, fl, t0 = 0, 0, time.perf_counter()
    while done < 128 and (time.perf_counter() - t0) < budget_s:
        q = r.standard_normal((1, S, 1, D)).astype(np.float32)
        k = r.standard_normal((1, S, 1, D)).astype(np.float32)
        v = r.standard_normal((1, S, 1, D)).astype(np.float32)
        O.gqa_prefill(q, k, v, 0.125, True, 0)
        done += 1
        fl += prefill_flops(1, S, 1, D)
    el = time.perf_counter() - t0
    return cpu_result(round(fl / el / 1e12, 6), "TFLOP/s",
                      f"{done} of 128 (batch, head) pairs of config 2 (S=2048, D=64, causal), "
                      f"fp32 oracle, {el:.1f} s; the oracle computes full S x S scores as the "
                      f"reference chain does, so only the causal half is counted as work")


def cpu_baseline_decode(ragged=False, budget_s=6.0, seed=2):
    """The oracle's decode (single thread) on whole sequences of config 3 (the
    bench's own lengths when ragged); bytes counted at bf16 size."""
    import numpy as np
    from oracle import oracle as O
    L, H, Hkv, D = 4096, 32, 4, 64
    r = np.random.default_rng(seed)
    lens = r.integers(512, 4097, 64).astype(np.int32) if ragged else np.full(64, L, np.int32)
    done, nb, t0 = 0, 0, time.perf_counter()
    while done < 64 and (time.perf_counter() - t0) < budget_s:
        Lb = int(lens[done])
        q = r.standard_normal((1, H, D)).astype(np.float32)
        kc = r.standard_normal((1, Lb, Hkv, D)).astype(np.float32)
        vc = r.standard_normal((1, Lb, Hkv, D)).astype(np.float32)
        O.gqa_decode(q, kc, vc, np.array([Lb], np.int32), 0.125)
        done += 1
        nb += decode_bytes([Lb], Hkv, D, 1, H, 2)
    el = time.perf_counter() - t0
    what = "ragged lengths U[512,4096]" if ragged else "L=4096"
    return cpu_result(round(nb / el / 1e9, 4), "GB/s",
                      f"{done} of 64 sequences of config 3 ({what}), fp32 oracle, {el:.1f} s, "
                      f"bytes counted at bf16 size")


def cpu_baseline_rows(kind, rows=512, w=2048, reps_s=3.0):
    """The oracle's RMSNorm+RoPE / residual add + RMSNorm / SwiGLU (single
    thread) on `rows` rows of the GPU workload's width; GB/s at bf16 size."""
    import numpy as np
    from oracle import oracle as O
    r = np.random.default_rng(9)
    x = r.standard_normal((rows, w)).astype(np.float32)
    d = r.standard_normal((rows, w)).astype(np.float32)
    wt = np.ones((1, w), np.float32)
    fn = {"rmsnorm_rope": lambda: O.rmsnorm_rope(x, wt, 1e-5, 0, 64, 1e4),
          "add_rmsnorm": lambda: O.add_rmsnorm(x, d, wt, 1e-5),
          "silu_mul": lambda: O.silu_mul(x, d)}[kind]
    per_row = {"rmsnorm_rope": 2, "add_rmsnorm": 4, "silu_mul": 3}[kind] * w * 2
    n, t0 = 0, time.perf_counter()
    while n == 0 or time.perf_counter() - t0 < reps_s:
        fn()
        n += 1
    el = (time.perf_counter() - t0) / n
    return cpu_result(round(rows * per_row / el / 1e9, 4), "GB/s",
                      f"{rows} rows x {w} of the GPU workload's shape, fp32 oracle "
                      f"(silu_mul: numpy fp32, the op has no loop of its own to restate), "
                      f"{n} repetitions, bytes counted at bf16 size")


def cpu_baseline_prefill_long(rows=32):
    """Config 5's prefill on the oracle: the last `rows` query rows of S=16384
    (all 32 heads, every key they see), extrapolated to the whole causal
    triangle by flop count (labelled)."""
    import numpy as np
    from oracle import oracle as O
    S, H, Hkv, D = 16384, 32, 4, 64
    r = np.random.default_rng(4)
    q = r.standard_normal((1, rows, H, D)).astype(np.float32)
    k = r.standard_normal((1, S, Hkv, D)).astype(np.float32)
    v = r.standard_normal((1, S, Hkv, D)).astype(np.float32)
    t0 = time.perf_counter()
    O.gqa_prefill(q, k, v, 0.125, True, S - rows)
    el = time.perf_counter() - t0
    fl = 4 * H * D * sum(S - rows + i + 1 for i in range(rows))
    return cpu_result(round(fl / el / 1e12, 6), "TFLOP/s",
                      f"last {rows} query rows of S=16384, all heads, fp32 oracle, {el:.1f} s "
                      f"(rate extrapolated to the full causal prefill)")


def cpu_baseline_linear(m_rows=8):
    """The QKV projection + RoPE on the oracle: op_mm's sequential-k fp32 loop
    (or_matmul) then op_rope, on `m_rows` rows of [2048] x [2048, 2560]."""
    import numpy as np
    from oracle import oracle as O
    r = np.random.default_rng(6)
    x = r.standard_normal((m_rows, 2048)).astype(np.float32)
    w = (r.standard_normal((2048, 2560)) / 45.0).astype(np.float32)
    t0 = time.perf_counter()
    y = O.matmul(x, w)
    O.rope(np.ascontiguousarray(y[:, :2304]), 7, 64, 1e4)
    el = time.perf_counter() - t0
    return cpu_result(round(2 * m_rows * 2048 * 2560 / el / 1e12, 6), "TFLOP/s",
                      f"{m_rows} rows, op_mm restated (sequential k, fp32) + op_rope, {el:.2f} s")


def cpu_baseline_backward(S=2048, H=8):
    """The oracle's attention backward (the reference chain's backward
    primitives composed in numpy fp64, BLAS held to one thread) on one KV
    group of config 2: B=1, S=2048, 8 query heads, 1 KV head."""
    import numpy as np
    from threadpoolctl import threadpool_limits
    from oracle import oracle as O
    r = np.random.default_rng(5)
    q = r.standard_normal((1, S, H, 64)).astype(np.float32)
    k = r.standard_normal((1, S, 1, 64)).astype(np.float32)
    v = r.standard_normal((1, S, 1, 64)).astype(np.float32)
    do = r.standard_normal((1, S, H, 64)).astype(np.float32)
    with threadpool_limits(1):
        t0 = time.perf_counter()
        O.gqa_prefill_backward(q, k, v, do, 0.125, True, 0)
        el = time.perf_counter() - t0
    fl = 5 * prefill_flops(1, S, H, 64) // 2
    return cpu_result(round(fl / el / 1e12, 6), "TFLOP/s",
                      f"one KV group of config 2 (S={S}, {H} query heads), oracle backward "
                      f"in numpy fp64 on one BLAS thread, {el:.1f} s")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--warm-seconds", type=float, default=1.0,
                    help="minimum untimed warm-up per workload, seconds of back-to-back launches")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--tl-warmup", type=int, default=2,
                    help="config 4: warm-up decode tokens before the timed generate (0: none, "
                         "so a kernel trace holds exactly one prefill + 128 steps)")
    ap.add_argument("--decode-token-major", choices=("beside", "skip"), default="beside",
                    help="config 3's token-major cache figure beside the head-major one, or "
                         "skipped (profiling runs whose counters must cover one layout)")
    ap.add_argument("--only", default="",
                    help="comma list of extra workloads (default: all but copy): "
                         "decode,ragged,planned,fp32,norm,long,addnorm,swiglu,linear,bwd,block,tinyllama,copy; "
                         "'head' = headline prefill only")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the attention path has no multi-GPU code)",
              file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    only = set(filter(None, args.only.split(",")))
    want = lambda k: not only or k in only
    K, W = args.steps, args.warmup
    globals()["WARM_SECONDS"] = args.warm_seconds

    head = bench_prefill(4, 2048, 32, 4, "bf16", K, W)
    out = {"metric": METRIC, "value": head["value"], "unit": "TFLOP/s", "n_gpus": 1,
           "steps": K, "warmup": W, "ms_per_step": head["ms_per_launch"],
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
           "data": "synthetic N(0,1) from a fixed seed (torch.Generator 0)",
           "config": {"workload": "causal GQA prefill (config 2)", "batch": 4,
                      "seq_len": 2048, "n_heads": 32, "n_kv_heads": 4, "head_dim": 64,
                      "scale": 0.125, "flops_per_step": head["flops_per_launch"]},
           "roofline": head["roofline"]}
    print(f"prefill bf16: {head['value']} TFLOP/s ({head['ms_per_launch']} ms)", file=sys.stderr,
          flush=True)
    # config 3 in the head-major cache layout (bn_gqa_decode_strided), the
    # token-major one (bn_gqa_decode) beside it
    beside =args.decode_token_major == "beside"
    for sel, key, kind in (("decode", "decode", "uniform"), ("ragged", "decode_ragged", "ragged")):
        if want(sel):
            out[key] = bench_decode(kind, K, W, layout="head_major")
            if beside:
                out[key]["token_major"] = bench_decode(kind, K, W)
            print(f"{key}: {out[key]['value']} GB/s (token-major "
                  f"{out[key]['token_major']['value'] if beside else 'skipped'})", file=sys.stderr,
                  flush=True)
    if want("planned"):
        out["decode_planned"] = bench_decode_planned(K, W)
        print(f"decode planned: { {k: v['planned']['value'] for k, v in out['decode_planned'].items() if k != 'roofline'} }",
              file=sys.stderr, flush=True)
    if want("fp32"):
        out["prefill_fp32"] = bench_prefill(4, 2048, 32, 4, "fp32", max(K // 2, 3), 2)
        print(f"prefill fp32: {out['prefill_fp32']['value']} TFLOP/s", file=sys.stderr, flush=True)
    if want("norm"):
        out["rmsnorm_rope"] = bench_rmsnorm_rope(K, W)
        print(f"rmsnorm_rope: {out['rmsnorm_rope']['value']} GB/s", file=sys.stderr, flush=True)
    if want("long"):
        out["prefill_long"] = bench_prefill(1, 16384, 32, 4, "bf16", max(K // 4, 3), 1)
        print(f"prefill S=16384: {out['prefill_long']['value']} TFLOP/s", file=sys.stderr,
              flush=True)
    if want("addnorm"):
        out["add_rmsnorm"] = bench_add_rmsnorm(K, W)
        print(f"add_rmsnorm: {out['add_rmsnorm']['value']} GB/s", file=sys.stderr, flush=True)
    if want("swiglu"):
        out["silu_mul"] = bench_silu_mul(K, W)
        print(f"silu_mul: {out['silu_mul']['value']} GB/s", file=sys.stderr, flush=True)
    if want("linear"):
        out["linear_rope"] = bench_linear(K, W)
        print(f"linear_rope: {out['linear_rope']}", file=sys.stderr, flush=True)
    if want("bwd"):
        out["prefill_backward"] = bench_backward(K, W)
        print(f"prefill backward: {out['prefill_backward']['value']} TFLOP/s "
              f"({out['prefill_backward']['ms_per_launch']} ms)", file=sys.stderr, flush=True)
    if want("block"):
        out["attention_block"], blk_inputs = bench_block(K, W)
        if not args.no_cpu:
            out["attention_block"]["cpu_baseline"] = cpu_baseline_block(*blk_inputs)
        print(f"config 1 block: {out['attention_block']}", file=sys.stderr, flush=True)
    if want("tinyllama"):
        out["tinyllama"] = bench_tinyllama(cpu=not args.no_cpu, warmup_tokens=args.tl_warmup)
        print(f"config 4: {out['tinyllama']}", file=sys.stderr, flush=True)
    if "copy" in only:
        out["copy"] = bench_copy(K, W)
        print(f"copy: {out['copy']['value']} GB/s", file=sys.stderr, flush=True)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline_prefill()
        cpu = {"decode": lambda: cpu_baseline_decode(False),
               "decode_ragged": lambda: cpu_baseline_decode(True),
               "decode_planned": lambda: dict(cpu_baseline_decode(True),
                                              note="the ragged pattern's oracle run (the planned path "
                                                   "computes the same rows)"),
               # the oracle computes in fp32 whatever the GPU dtype: the same sample
               "prefill_fp32": lambda: dict(out["cpu_baseline"],
                                            note="same oracle run as the headline's (fp32)"),
               "rmsnorm_rope": lambda: cpu_baseline_rows("rmsnorm_rope"),
               "prefill_long": cpu_baseline_prefill_long,
               "add_rmsnorm": lambda: cpu_baseline_rows("add_rmsnorm"),
               "silu_mul": lambda: cpu_baseline_rows("silu_mul", w=5632),
               "linear_rope": cpu_baseline_linear,
               "prefill_backward": cpu_baseline_backward}
        for key, fn in cpu.items():
            if key in out:
                out[key]["cpu_baseline"] = fn()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
