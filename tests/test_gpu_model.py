"""GPU parity of the layer-level paths: config 1 (one attention block
through the `bten` surface, fused-head as the reference computes it and
per-head GQA) and config 4's TinyLLaMA driver (teacher-forced, kernel by
kernel, against the CPU oracle on the inputs the GPU run produced)."""
import math

import numpy as np
import pytest
import torch

import bnhip
import bten
from gpu_util import FP32_TOL, assert_close, require_gpu
from llama_layers import GroupedQueryAttention, RMSNorm
from oracle import oracle as O
from tinyllama import TinyLlama, TinyLlamaConfig

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def config1_inputs(S=128, hidden=2048, H=32, Hkv=4):
    r = np.random.default_rng(0)
    x = r.standard_normal((S, hidden)).astype(np.float32)
    rw = np.random.default_rng(1)
    D = hidden // H
    ws = [(rw.standard_normal(s) * 0.02).astype(np.float32)
          for s in ((hidden, hidden), (hidden, Hkv * D), (hidden, Hkv * D), (hidden, hidden))]
    return x, ws


@pytest.mark.parametrize("mode", ["fused_head", "fused_head_ops", "per_head"])
def test_config1_attention_block(mode):
    """RMSNorm(eps 1e-5) -> Q/K/V -> RoPE -> causal softmax(QK^T/8) V -> O, fp32."""
    x, (wq, wk, wv, wo) = config1_inputs()
    cfg = bten.LLaMAConfig()
    norm = RMSNorm(2048, eps=1e-5)
    attn = GroupedQueryAttention(cfg, mode=mode)
    attn.load_weights(wq, wk, wv, wo)
    xt = bten.TensorF(128, 2048)
    xt.copy_from_numpy(x)
    out = attn(norm(xt), position_offset=0).to_numpy()
    xn = O.rmsnorm(x, np.ones((1, 2048), np.float32), 1e-5)
    ref = O.gqa_layer(xn, wq, wk, wv, wo, 32, 4, 10000.0, 0, per_head=(mode == "per_head"))
    assert_close(out, ref, FP32_TOL, f"config 1 {mode}")


def test_config1_fused_head_kernel_equals_op_chain():
    """bten.fused_head_attention against the same chain op by op on the device
    (repeat_kv, QK^T, scale, softmax, PV) on config 1's shapes."""
    r = np.random.default_rng(4)
    q, k, v = (bten.TensorF(128, w) for w in (2048, 256, 256))
    for t in (q, k, v):
        t.copy_from_numpy(r.standard_normal(t.shape).astype(np.float32))
    one = bten.fused_head_attention(q, k, v, 32, 4, 64, 0.125, True, 0).to_numpy()
    kr, vr = bten.repeat_kv(k, 8, 64), bten.repeat_kv(v, 8, 64)
    chain = ((q @ kr.T) * 0.125).softmax(True, 0) @ vr
    assert_close(one, chain.to_numpy(), FP32_TOL, "fused kernel vs op chain")


def test_config1_offset_and_views():
    # decode-style call: a later position offset through the fused-head chain
    x, (wq, wk, wv, wo) = config1_inputs(S=16, hidden=256, H=8, Hkv=2)
    cfg = bten.LLaMAConfig()
    cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads = 256, 8, 2
    attn = GroupedQueryAttention(cfg)
    attn.load_weights(wq, wk, wv, wo)
    xt = bten.TensorF(16, 256)
    xt.copy_from_numpy(x)
    out = attn(xt, position_offset=5).to_numpy()
    ref = O.gqa_layer(x, wq, wk, wv, wo, 8, 2, 10000.0, 5, per_head=False)
    assert_close(out, ref, FP32_TOL, "offset 5")


def small_llama(layers=2, vocab=512, max_len=96, out_major=True):
    cfg = TinyLlamaConfig(vocab_size=vocab, num_hidden_layers=layers)
    return TinyLlama(cfg, max_len=max_len, seed=1, out_major=out_major)


def test_tinyllama_kernels_teacher_forced():
    """Every RMSNorm (plain and fused with the residual add) / RoPE / QKV
    projection with fused RoPE (decode steps) / prefill / decode launch of a
    2-layer run is recomputed by the oracle from the inputs the GPU used."""
    m = small_llama()
    m.trace = []
    ids = torch.from_numpy(np.random.default_rng(3).integers(0, 512, 64)).cuda()
    m.generate(ids, 3)
    seen = set()
    for name, ins, out, kw in m.trace:
        seen.add(name)
        if name == "rmsnorm":
            ref = O.rmsnorm(ins[0], ins[1], kw["eps"])
        elif name == "add_rmsnorm":
            ref = np.stack(O.add_rmsnorm(ins[0], ins[1], ins[2], kw["eps"]))
        elif name == "rope":
            ref = O.rope(ins[0], kw["offset"], kw["head_dim"], kw["theta"])
        elif name == "linear_rope":
            ref = O.linear_rope(ins[0], ins[1], kw["rope_cols"], kw["offset"], kw["head_dim"],
                                kw["theta"])
        elif name == "prefill":
            ref = O.gqa_prefill(ins[0], ins[1], ins[2], 0.125, True, 0)
        else:
            q, kc, vc = ins
            ref = O.gqa_decode(q, kc, vc, np.array([kw["length"]], np.int32), 0.125)
        assert_close(out, ref, FP32_TOL, f"{name} {kw}")
    assert seen == {"rmsnorm", "add_rmsnorm", "rope", "linear_rope", "prefill", "decode"}


def test_tinyllama_cache_matches_recompute():
    """Logits of a cached decode step equal the last row of a fresh prefill
    over the whole prefix (the reference's generate recomputes the prefix,
    llama_model.py:135-141)."""
    ids = torch.from_numpy(np.random.default_rng(4).integers(0, 512, 40)).cuda()
    m = small_llama()
    logits = m.prefill(ids)
    tok = torch.argmax(logits[-1])
    step_logits = m.step(tok)
    fresh = small_llama()
    ref_logits = fresh.prefill(torch.cat([ids, tok.view(1)]))
    a, b = step_logits.cpu().numpy(), ref_logits.cpu().numpy()
    assert float(np.max(np.abs(a - b)) / np.max(np.abs(b))) < 1e-4


@pytest.mark.parametrize("out_major", [True, False])
@pytest.mark.parametrize("prompt,new", [(40, 12), (7, 1), (1, 30)])
def test_native_decode_matches_generate(prompt, new, out_major):
    """bn_llama_decode runs the decode loop natively (gather, layers, lm_head,
    argmax, next token fed on the device).  Its QKV projection also appends K
    and V to the caches and its gate|up projection writes silu(gate) * up --
    in the output-major kernel's epilogue (out_major) or in the split-k
    reduction, whose slabs are summed in the order of the unfused one -- so
    the generated tokens and every layer's KV cache are bit-identical to
    generate(), which runs the ops one by one."""
    ids = torch.from_numpy(np.random.default_rng(7 + prompt).integers(0, 512, prompt)).cuda()
    a, b = small_llama(out_major=out_major), small_llama(out_major=out_major)
    ref, _ = a.generate(ids, new)
    got = b.generate_native(ids, new)
    torch.cuda.synchronize()
    assert torch.equal(ref.cpu(), got.cpu()), (ref.tolist(), got.tolist())
    assert a.length == b.length == prompt + new
    for La, Lb in zip(a.layers, b.layers):
        assert torch.equal(La["k_cache"], Lb["k_cache"]) and torch.equal(La["v_cache"], Lb["v_cache"])


@pytest.mark.parametrize("hidden,heads,kv_heads,layers", [(1024, 16, 2, 2), (3072, 48, 6, 2),
                                                          (2048, 32, 4, 1), (2048, 32, 4, 3)])
def test_native_decode_matches_generate_other_widths(hidden, heads, kv_heads, layers):
    """hidden 1024: the decode-step norms formed in the projections' x
    staging cover one 16-byte chunk per thread; hidden 3072: wider than the
    one-wave norm kernels' rows, so the native loop launches the norm kernels
    as the step loop does; 1 and 3 layers: the two residual buffers swap an
    odd number of times per step.  Tokens and caches bit-identical to
    generate()."""
    cfg = TinyLlamaConfig(vocab_size=512, hidden_size=hidden, intermediate_size=1024,
                          num_hidden_layers=layers, num_attention_heads=heads,
                          num_key_value_heads=kv_heads)
    a, b = (TinyLlama(cfg, max_len=64, seed=2) for _ in range(2))
    ids = torch.from_numpy(np.random.default_rng(11).integers(0, 512, 9)).cuda()
    ref, _ = a.generate(ids, 12)
    got = b.generate_native(ids, 12)
    torch.cuda.synchronize()
    assert torch.equal(ref.cpu(), got.cpu()), (ref.tolist(), got.tolist())
    for La, Lb in zip(a.layers, b.layers):
        assert torch.equal(La["k_cache"], Lb["k_cache"]) and torch.equal(La["v_cache"], Lb["v_cache"])


def test_native_decode_continues_and_rejects_overflow():
    """Two native calls in a row continue where the first stopped (the second
    starts from the first call's last token at the next position); a call
    that would pass max_len is refused before any launch."""
    ids = torch.from_numpy(np.random.default_rng(3).integers(0, 512, 20)).cuda()
    a, b = small_llama(max_len=64), small_llama(max_len=64)
    ref, _ = a.generate(ids, 16)
    b.prefill(ids)
    first = int(ref[0])
    out = torch.empty(16, dtype=torch.int32, device="cuda")
    b.decode_native(first, 6, out[:6])
    torch.cuda.synchronize()
    b.decode_native(int(out[5]), 10, out[6:])
    assert torch.equal(torch.cat([ref[:1].cpu().int(), out[:15].cpu()]), ref.cpu().int())
    for La, Lb in zip(a.layers, b.layers):
        assert torch.equal(La["k_cache"], Lb["k_cache"])
    with pytest.raises(bnhip.BnError, match="max_len"):
        b.decode_native(0, 64 - b.length + 1, torch.empty(64, dtype=torch.int32, device="cuda"))


# ------------------------------------------------------------ LLaMAModelCpp
def small_cpp_config():
    c = bten.LLaMAConfig()
    (c.vocab_size, c.hidden_size, c.intermediate_size, c.num_hidden_layers,
     c.num_attention_heads, c.num_key_value_heads) = (512, 256, 384, 2, 4, 2)
    return c


def oracle_model_forward(w, ids, c, per_head):
    """llama_model.hpp:52-80 with the decoder layer of llama_layers.hpp:241-272,
    composed from the oracle's restatements (fp64 products rounded to fp32)."""
    f = lambda a: np.asarray(a, np.float32)
    mm = lambda a, b: f(np.asarray(a, np.float64) @ np.asarray(b, np.float64))
    eps, H, Hkv = c.rms_norm_eps, c.num_attention_heads, c.num_key_value_heads
    x = w["embed_tokens"].to_numpy()[ids]
    for L in w["layers"]:
        t = {k: v.to_numpy() for k, v in L.items()}
        xn = O.rmsnorm(x, t["input_layernorm"], eps)
        attn = O.gqa_layer(xn, t["q_proj"], t["k_proj"], t["v_proj"], t["o_proj"], H, Hkv,
                           c.rope_theta, 0, per_head=per_head)
        h = f(x + attn)
        xn2 = O.rmsnorm(h, t["post_attention_layernorm"], eps)
        act = O.silu_mul(mm(xn2, t["gate_proj"]), mm(xn2, t["up_proj"]))
        x = f(h + mm(act, t["down_proj"]))
    return mm(O.rmsnorm(x, w["final_norm"].to_numpy(), eps), w["lm_head"].to_numpy())


@pytest.mark.parametrize("attention", ["fused_head", "per_head"])
def test_llama_model_cpp_forward_vs_oracle(attention):
    """bten.LLaMAModelCpp.forward (llama_bindings.hpp:37-58): the ids are one
    causal sequence, logits for every row; fused-head is the reference
    layer's own chain (llama_layers.hpp:96-109)."""
    c = small_cpp_config()
    m = bten.LLaMAModelCpp(c, attention=attention)
    ids = np.random.default_rng(5).integers(0, 512, 24).astype(np.uint32)
    got = m.forward(ids)
    assert got.shape == (24, 512) and got.dtype == np.float32
    ref = oracle_model_forward(m.weights(), ids, c, attention == "per_head")
    assert_close(got, ref, FP32_TOL, f"LLaMAModelCpp {attention}")


def test_llama_model_cpp_device_weights_equal_host_weights():
    # bn_fill_uniform on the device and the host twin give the same bits
    c = small_cpp_config()
    d, h = bten.LLaMAModelCpp(c, True), bten.LLaMAModelCpp(c, False)
    wd, wh = d.weights(), h.weights()
    for name in ("embed_tokens", "lm_head"):
        np.testing.assert_array_equal(wd[name].to_numpy(), wh[name].to_numpy())
    for Ld, Lh in zip(wd["layers"], wh["layers"]):
        for k in Ld:
            np.testing.assert_array_equal(Ld[k].to_numpy(), Lh[k].to_numpy())


def test_llama_model_cpp_benchmark_and_memory():
    c = small_cpp_config()
    m = bten.LLaMAModelCpp(c)
    ids = np.ones(8, np.uint32)
    assert m.forward_timed(ids) > 0.0
    r = m.benchmark(8, num_warmup=1, num_iterations=3)
    assert set(r) == {"forward_time_ms", "tokens_per_second", "memory_used_bytes", "num_parameters"}
    assert r["forward_time_ms"] > 0 and r["tokens_per_second"] > 0
    assert r["num_parameters"] == c.count_parameters() == m.count_parameters()
    assert r["memory_used_bytes"] == m.get_gpu_memory_usage() or r["memory_used_bytes"] > 0
    assert m.get_gpu_memory_usage() > 0
    with pytest.raises(RuntimeError, match="outside the vocabulary"):
        m.forward(np.array([1, 512], np.uint32))
    assert m.forward(np.zeros(0, np.uint32)).shape == (0, 512)


def test_embedding_gather_and_uniform_fill():
    import ctypes as C
    V = lambda t: C.byref(bnhip.view(t))
    table = torch.randn(50, 96, device="cuda")
    ids = torch.tensor([3, 49, 0, 50, 7, -1], dtype=torch.int32, device="cuda")  # -1: id 2^32-1
    out = torch.full((6, 96), float("nan"), device="cuda")
    bnhip.call("bn_embedding", V(table), ids.data_ptr(), 6, V(out), None)
    torch.cuda.synchronize()
    want = table.cpu().numpy()[[3, 49, 0, 0, 7, 0]]
    want[[3, 5]] = 0.0                           # ids past the table: zero rows
    np.testing.assert_array_equal(out.cpu().numpy(), want)
    for dt in (torch.float32, torch.bfloat16):
        y = torch.empty((37, 91), dtype=dt, device="cuda")
        bnhip.call("bn_fill_uniform", V(y), -0.5, 1.5, 12345, None)
        yt = torch.empty((91, 37), dtype=dt, device="cuda").t()   # strided: same values
        bnhip.call("bn_fill_uniform", V(yt), -0.5, 1.5, 12345, None)
        torch.cuda.synchronize()
        a = y.float().cpu().numpy()
        assert a.min() >= -0.5 and a.max() <= 1.5 and abs(float(a.mean()) - 0.5) < 0.05
        np.testing.assert_array_equal(a, yt.float().cpu().numpy())
