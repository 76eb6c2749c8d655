"""Config 4 at its stated size: TinyLLaMA-1.1B (22 layers, hidden 2048,
32/4 heads, SwiGLU 5632, vocab 32000, fp32, random weights), a 512-token
seeded prompt, then 128 greedy decode steps with the KV cache growing from
513 to 640 keys (llama_model.hpp:52-80, llama_layers.hpp:241-272).

The oracle checks, teacher-forced (each kernel recomputed from the inputs the
GPU run gave it, so greedy near-ties cannot cascade), every path launch --
RMSNorm, residual add + RMSNorm, RoPE, the QKV projection with RoPE, prefill
and decode attention -- of layers 0, 10 and 21 in the prompt pass and in the
decode steps at cache lengths 513, 576 and 640.  The native decode loop must
reproduce the Python step loop's 128 tokens and all 22 layers' caches bit for
bit, and the cached logits of the last step must equal the last row of a
fresh prefill over the whole 640-token sequence.
"""
import numpy as np
import pytest
import torch

from gpu_util import FP32_TOL, assert_close, require_gpu
from oracle import oracle as O
from tinyllama import TinyLlama, TinyLlamaConfig

pytestmark = pytest.mark.gpu
PROMPT, NEW, MAX_LEN = 512, 128, 640
LAYERS = (0, 10, 21)
DECODE_POS = (512, 575, 639)  # position of the token fed; cache length = pos + 1


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def prompt_ids():
    return torch.from_numpy(np.random.default_rng(3).integers(0, 32000, PROMPT)).cuda()


@pytest.fixture(scope="module")
def traced():
    print("config 4: 22-layer model, traced generate (512 + 128)", flush=True)
    m = TinyLlama(TinyLlamaConfig(), max_len=MAX_LEN, seed=1)
    m.trace = []
    m.trace_select = lambda layer, pos0: layer in LAYERS and pos0 in (0,) + DECODE_POS
    toks, _ = m.generate(prompt_ids(), NEW)
    trace, m.trace = m.trace, None
    return m, toks, trace


def oracle_of(name, ins, kw):
    if name == "rmsnorm":
        return O.rmsnorm(ins[0], ins[1], kw["eps"])
    if name == "add_rmsnorm":
        return np.stack(O.add_rmsnorm(ins[0], ins[1], ins[2], kw["eps"]))
    if name == "rope":
        return O.rope(ins[0], kw["offset"], kw["head_dim"], kw["theta"])
    if name == "linear_rope":
        return O.linear_rope(ins[0], ins[1], kw["rope_cols"], kw["offset"], kw["head_dim"],
                             kw["theta"])
    if name == "prefill":
        return O.gqa_prefill(ins[0], ins[1], ins[2], 0.125, True, 0)
    q, kc, vc = ins
    return O.gqa_decode(q, kc, vc, np.array([kw["length"]], np.int32), 0.125)


def test_config4_prompt_kernels_teacher_forced(traced):
    _, _, trace = traced
    seen = set()
    for name, ins, out, kw in trace:
        if kw["pos0"] != 0:
            continue
        seen.add((kw["layer"], name))
        assert_close(out, oracle_of(name, ins, kw), FP32_TOL, f"prompt layer {kw['layer']} {name}")
    want = {(layer, n) for layer in LAYERS for n in ("add_rmsnorm", "rope", "prefill")}
    assert want | {(0, "rmsnorm")} == seen


def test_config4_decode_kernels_teacher_forced(traced):
    _, _, trace = traced
    seen = set()
    for name, ins, out, kw in trace:
        if kw["pos0"] == 0:
            continue
        seen.add((kw["layer"], kw["pos0"], name))
        if name == "decode":
            assert kw["length"] == kw["pos0"] + 1
        assert_close(out, oracle_of(name, ins, kw), FP32_TOL,
                     f"decode pos {kw['pos0']} layer {kw['layer']} {name}")
    want = {(layer, p, n) for layer in LAYERS for p in DECODE_POS
            for n in ("add_rmsnorm", "linear_rope", "decode")}
    want |= {(0, p, "rmsnorm") for p in DECODE_POS}
    assert want == seen


def test_config4_native_decode_matches_generate(traced):
    m, toks, _ = traced
    print("config 4: native decode loop, 128 steps", flush=True)
    b = TinyLlama(TinyLlamaConfig(), max_len=MAX_LEN, seed=1)
    got = b.generate_native(prompt_ids(), NEW)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), toks.cpu()), "native tokens differ from the Python step loop"
    assert b.length == m.length == MAX_LEN
    for i, (La, Lb) in enumerate(zip(m.layers, b.layers)):
        assert torch.equal(La["k_cache"], Lb["k_cache"]), f"layer {i} K cache"
        assert torch.equal(La["v_cache"], Lb["v_cache"]), f"layer {i} V cache"


def test_config4_cached_logits_match_recompute(traced):
    """The reference's generate reruns the whole prefix for every token
    (llama_model.py:135-141); the cached decode's logits at position 639 must
    equal the last row of a fresh prefill over all 640 tokens."""
    m, toks, _ = traced
    print("config 4: fresh prefill over 640 tokens", flush=True)
    c = TinyLlama(TinyLlamaConfig(), max_len=MAX_LEN, seed=1)
    ref = c.prefill(torch.cat([prompt_ids(), toks.view(-1)]))
    a, b = m.last_logits.cpu().numpy(), ref.cpu().numpy()
    assert_close(a, b, FP32_TOL, "logits at position 639: cached decode vs recompute")
