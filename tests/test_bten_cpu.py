"""Host-side behaviour of the `bten` module that needs no GPU: host tensors,
views, numpy round trips, indexing errors, and the reference's error
behaviour for GPU-only ops on host tensors (py_tensor_shim.hh, tensor.cuh,
op_rmsnorm.cuh:142-150, op_rope.cuh:108-117, op_softmax.cuh:160-165)."""
import numpy as np
import pytest

import bten


def host(a, cls=bten.TensorF):
    t = cls(a.shape[0], a.shape[1], False)
    t.copy_from_numpy(a)
    return t


def test_host_roundtrip_and_repr():
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    t = host(a)
    assert t.shape == (3, 4) and not t.is_cuda
    np.testing.assert_array_equal(t.to_numpy(), a)
    assert repr(t) == "dtype=float32 Tensor(3, 4, on_device=false)"
    u = host(np.arange(6, dtype=np.uint32).reshape(2, 3), bten.TensorU32)
    assert repr(u).startswith("dtype=uint32") and u.to_numpy().dtype == np.uint32


def test_views_share_storage_and_gather():
    a = np.arange(20, dtype=np.float32).reshape(4, 5)
    t = host(a)
    np.testing.assert_array_equal(t.T.to_numpy(), a.T)
    np.testing.assert_array_equal(t.transpose().to_numpy(), a.T)
    s = t.slice(1, 3, 2, 5)
    np.testing.assert_array_equal(s.to_numpy(), a[1:3, 2:5])
    np.testing.assert_array_equal(t[1:3, 2:].to_numpy(), a[1:3, 2:])
    np.testing.assert_array_equal(t[2].to_numpy(), a[2:3])
    np.testing.assert_array_equal(t[:, -1].to_numpy(), a[:, 4:5])
    s.fill(-1.0)   # writes through the view
    b = a.copy()
    b[1:3, 2:5] = -1
    np.testing.assert_array_equal(t.to_numpy(), b)
    s.copy_from_numpy(np.full((2, 3), 7, np.float32))
    b[1:3, 2:5] = 7
    np.testing.assert_array_equal(t.to_numpy(), b)


def test_indexing_errors():
    t = bten.TensorF(4, 5, False)
    with pytest.raises(IndexError, match="step=1"):
        t[::2]
    with pytest.raises(IndexError, match="Index out of range"):
        t[7]
    with pytest.raises(IndexError, match="2D indexing"):
        t[1, 2, 3]
    with pytest.raises(TypeError, match="integers, slices, or None"):
        t["a"]
    with pytest.raises(RuntimeError, match="Slice index out of range"):
        t.slice(0, 5, 0, 1)
    with pytest.raises(RuntimeError, match="Expected 2D NumPy array"):
        t.copy_from_numpy(np.zeros(3, np.float32))
    with pytest.raises(RuntimeError, match="Shape mismatch"):
        t.copy_from_numpy(np.zeros((2, 2), np.float32))


def test_gpu_only_ops_raise_on_host_tensors():
    x = host(np.ones((4, 64), np.float32))
    w = host(np.ones((1, 64), np.float32))
    with pytest.raises(RuntimeError, match="^RMSNorm: only GPU implementation available$"):
        x.rmsnorm(w, 1e-5)
    with pytest.raises(RuntimeError, match="^RoPE: only GPU implementation available$"):
        x.rope(0, 64, 10000.0)
    with pytest.raises(RuntimeError, match="^Softmax: only GPU implementation available$"):
        x.softmax(True, 0)
    with pytest.raises(RuntimeError, match="only GPU implementation available"):
        x @ host(np.ones((64, 2), np.float32))
    # shapes are validated before the device, as in the reference
    with pytest.raises(RuntimeError, match="weight shape must be"):
        x.rmsnorm(host(np.ones((1, 32), np.float32)))
    with pytest.raises(RuntimeError, match="divisible by head_dim"):
        x.rope(0, 48)
    with pytest.raises(RuntimeError, match="only GPU implementation available"):
        bten.gqa_prefill(x, x, x, 1, 1, 1, 64)
    with pytest.raises(RuntimeError, match="only GPU implementation available"):
        bten.gqa_prefill_lse(x, x, x, 1, 1, 1, 64)
    lse = bten.TensorF(1, 4, False)
    with pytest.raises(RuntimeError, match="only GPU implementation available"):
        bten.gqa_prefill_backward(x, x, x, x, x, lse, 1, 1, 1, 64)


def test_defaults_match_reference_signatures():
    # py_tensor_shim.hh:280-305 defaults (1e-6f prints as its float value)
    import re
    def has(fn, name, val):
        return re.search(name + r": [^=,]*= " + re.escape(val), fn.__doc__) is not None
    assert has(bten.TensorF.rmsnorm, "eps", "9.999999974752427e-07")
    assert has(bten.TensorF.rope, "position_offset", "0")
    assert has(bten.TensorF.rope, "head_dim", "64")
    assert has(bten.TensorF.rope, "theta", "10000.0")
    assert has(bten.TensorF.softmax, "causal", "False")
    assert has(bten.TensorF.softmax, "seq_offset", "0")
    assert has(bten.TensorF.__init__, "is_cuda", "True")
    c = bten.LLaMAConfig.tinyllama_1_1b()
    assert (c.hidden_size, c.num_attention_heads, c.num_key_value_heads, c.head_dim(),
            c.num_kv_groups()) == (2048, 32, 4, 64, 8)
    assert c.validate() is None            # void in llama_config.hpp:42-51
    with pytest.raises(RuntimeError, match="divisible by num_key_value_heads"):
        bad = bten.LLaMAConfig()
        bad.num_key_value_heads = 5
        bad.validate()
    bten.randgen_seed(1234)
    bten.randgen_seed(42)


def splitmix_uniform(seed, n):
    # SplitMix64 (Steele, Lea & Flood 2014) of seed + (i+1)*golden, top 24 bits
    M = (1 << 64) - 1
    out = np.empty(n, np.float32)
    for i in range(n):
        z = (seed + (i + 1) * 0x9E3779B97F4A7C15) & M
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        z ^= z >> 31
        out[i] = np.float32(z >> 40) * np.float32(1.0 / 16777216.0)
    return out


def small_cfg():
    c = bten.LLaMAConfig()
    (c.vocab_size, c.hidden_size, c.intermediate_size, c.num_hidden_layers,
     c.num_attention_heads, c.num_key_value_heads) = (96, 128, 160, 2, 2, 1)
    return c


def test_llama_config_count_parameters_and_repr():
    # llama_config.hpp:82-105 at TinyLLaMA-1.1B
    c = bten.LLaMAConfig.tinyllama_1_1b()
    h, kv, I, V, L = 2048, 256, 5632, 32000, 22
    per_layer = h * h + 2 * h * kv + h * h + 3 * h * I + 2 * h
    assert c.count_parameters() == V * h + L * per_layer + h + h * V == 1100048384
    assert repr(c) == ("LLaMAConfig(\n  vocab_size=32000,\n  hidden_size=2048,\n  num_layers=22,\n"
                       "  num_heads=32,\n  num_kv_heads=4,\n  intermediate_size=5632\n)")


def test_llama_model_cpp_on_host():
    """LLaMAModelCpp(config, on_device=False): built on the host (the
    reference allocates host tensors), parameter count and memory as the
    reference reports them, and forward raises where the reference's first
    GPU-only op (op_rmsnorm, op_rmsnorm.cuh:148-150) throws."""
    c = small_cfg()
    m = bten.LLaMAModelCpp(c, False)
    assert m.count_parameters() == c.count_parameters()
    assert m.get_gpu_memory_usage() == 0
    with pytest.raises(RuntimeError, match="RMSNorm: only GPU implementation available"):
        m.forward(np.array([1, 2, 3], np.uint32))
    w = m.weights()
    assert len(w["layers"]) == 2
    np.testing.assert_array_equal(w["final_norm"].to_numpy(), np.ones((1, 128), np.float32))
    q = w["layers"][1]["q_proj"].to_numpy()
    assert q.shape == (128, 128) and w["layers"][1]["k_proj"].shape == (128, 64)
    assert w["layers"][0]["gate_proj"].shape == (128, 160)
    emb = w["embed_tokens"].to_numpy()
    assert emb.shape == (96, 128) and emb.min() >= -0.02 and emb.max() <= 0.02
    # the uniform fill restated: lo + (hi - lo) * u with u from SplitMix64 of
    # the tensor's seed stream (embed_tokens is stream 1 of randgen seed 42)
    seed = (42 * 0x100000001B3 + 1) & ((1 << 64) - 1)
    u = splitmix_uniform(seed, 96 * 128).astype(np.float64)
    want = (u * np.float64(np.float32(0.02) - np.float32(-0.02)) + np.float64(np.float32(-0.02)))
    np.testing.assert_array_equal(emb.ravel(), want.astype(np.float32))
    # loading through a view writes the model's weight
    w["layers"][0]["v_proj"].copy_from_numpy(np.full((128, 64), 0.5, np.float32))
    assert np.all(m.weights()["layers"][0]["v_proj"].to_numpy() == 0.5)


def test_llama_model_cpp_signature_defaults():
    import re
    doc = bten.LLaMAModelCpp.benchmark.__doc__
    assert re.search(r"num_warmup: [^=,]*= 5\b", doc) and re.search(r"num_iterations: [^=,]*= 100\b", doc)
    assert re.search(r"on_device: [^=,]*= True", bten.LLaMAModelCpp.__init__.__doc__)
    with pytest.raises(RuntimeError, match="fused_head"):
        bten.LLaMAModelCpp(small_cfg(), False, "bogus")


@pytest.mark.parametrize("field", ["num_hidden_layers", "vocab_size", "intermediate_size"])
@pytest.mark.parametrize("value", [0, -1])
def test_llama_model_cpp_refuses_empty_sizes(field, value):
    """A model with no layers (or no vocabulary / MLP) is refused at
    construction: its forward would index layer 0 of an empty stack."""
    c = small_cfg()
    setattr(c, field, value)
    with pytest.raises(RuntimeError, match="must be positive"):
        bten.LLaMAModelCpp(c, False)


def test_bf16_host_tensor_rounds_to_nearest_even():
    vals = np.array([[1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 3.14159265, 0.0]],
                    np.float32)
    t = host(vals, bten.TensorBF16)
    got = t.to_numpy()
    exp = (vals.view(np.uint32).astype(np.uint64) + 0x7FFF +
           ((vals.view(np.uint32) >> 16) & 1)) >> 16
    exp = (exp.astype(np.uint32) << 16).view(np.float32)
    np.testing.assert_array_equal(got, exp)
    assert repr(t).startswith("dtype=bfloat16")
