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
    assert c.validate()
    bten.randgen_seed(1234)


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
