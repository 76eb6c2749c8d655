// bten.cpp -- the pybind11 module `bten`: the reference's op surface
// (src/bindings.cu:12-25, src/py_tensor_shim.hh:30-310) rebuilt as host C++
// over the C ABI of libbnhip.so (include/bn_hip.h).  No HIP header is
// included here: device memory, copies and kernels are reached only through
// bn_* entry points.
//
// Same module, class, method and argument names and defaults as the
// reference, so mygrad/llama callers run unchanged:
//   TensorF / TensorU32 (py_tensor_shim.hh:184-254), float-only ops
//   (:256-310), randgen_seed (bindings.cu:16-18), LLaMAConfig and
//   LLaMAModelCpp (llama_bindings.hpp:31-122).
// Additions (new names only): TensorBF16, Tensor*.rmsnorm_rope, gqa_prefill,
// gqa_prefill_lse, gqa_prefill_backward, fused_head_attention,
// gqa_decode, repeat_kv, add_rmsnorm, silu_mul, pool_stats / pool_trim / pool_set_limit,
// synchronize, set_stream / get_stream.
//
// Host tensors (is_cuda=False) support construction, copies, fill, views and
// repr.  The compute ops raise "<Op>: only GPU implementation available" on
// them, as the reference's rmsnorm/rope/softmax/mm do (op_rmsnorm.cuh:148-150,
// op_rope.cuh:112-114, op_softmax.cuh:163-165, op_mm_optimized.cuh:77-79);
// there is no CPU compute path in this module.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>

#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "bn_hip.h"

namespace py = pybind11;

namespace {

void *g_stream = nullptr;  // NULL = legacy default stream, as the reference
unsigned long long g_randgen_seed = 42;  // src/randgen.cu

// bn_status -> Python exception (runtime_error -> RuntimeError, as the
// reference's std::runtime_error / CUDA_OK throws).
void check(int st) {
  if (st == BN_OK) return;
  const char *msg = bn_last_error();
  std::string m = (msg && *msg) ? msg : "bn error " + std::to_string(st);
  if (st == BN_ERR_OOM) throw std::bad_alloc();
  throw std::runtime_error(m);
}

struct Storage {
  void *ptr = nullptr;
  size_t bytes = 0;
  bool on_device = false;
  Storage(size_t n, bool dev) : bytes(n), on_device(dev) {
    if (dev) {
      check(bn_alloc(&ptr, n, g_stream));
    } else if (n) {
      ptr = std::malloc(n);
      if (!ptr) throw std::runtime_error("Failed to malloc cpu memory");  // tensor.cuh:72
    }
  }
  ~Storage() {
    if (on_device)
      bn_free(ptr, g_stream);  // stream-ordered: no device synchronisation
    else
      std::free(ptr);
  }
  Storage(const Storage &) = delete;
  Storage &operator=(const Storage &) = delete;
};

template <int DT> struct DTypeInfo;
template <> struct DTypeInfo<BN_F32> {
  using host_t = float;
  static constexpr size_t size = 4;
  static const char *name() { return "float32"; }
};
template <> struct DTypeInfo<BN_U32> {
  using host_t = uint32_t;
  static constexpr size_t size = 4;
  static const char *name() { return "uint32"; }
};
template <> struct DTypeInfo<BN_BF16> {
  using host_t = float;  // numpy side is float32; storage is bf16
  static constexpr size_t size = 2;
  static const char *name() { return "bfloat16"; }
};

uint16_t f32_to_bf16_host(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
float bf16_to_f32_host(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// 2-D strided view over shared storage: the fields of Tensor<T>
// (tensor.cuh:45-52); transpose and slice share the storage.
template <int DT>
class PyTensor {
 public:
  using Info = DTypeInfo<DT>;
  using host_t = typename Info::host_t;
  std::shared_ptr<Storage> ref;
  int32_t h = 0, w = 0, stride_h = 0, stride_w = 1;
  int64_t offset = 0;
  bool on_device = true;

  PyTensor(int h_, int w_, bool is_cuda) : h(h_), w(w_), stride_h(w_), stride_w(1), on_device(is_cuda) {
    if (h_ < 0 || w_ < 0) throw std::runtime_error("Tensor dimensions must be non-negative");
    ref = std::make_shared<Storage>((size_t)h_ * (size_t)w_ * Info::size, is_cuda);
  }
  PyTensor() = default;

  bn_view view() const {
    bn_view v;
    v.data = ref ? ref->ptr : nullptr;
    v.offset = offset;
    v.h = h;
    v.w = w;
    v.stride_h = stride_h;
    v.stride_w = stride_w;
    v.dtype = DT;
    v.on_device = on_device ? 1 : 0;
    return v;
  }
  bool contiguous() const { return stride_w == 1 && (stride_h == w || h <= 1); }
  char *base() const { return (char *)ref->ptr + offset * (int64_t)Info::size; }

  std::pair<int, int> shape() const { return {h, w}; }
  bool is_cuda() const { return on_device; }

  // host staging buffer (raw storage format) <-> this view
  void upload_raw(const void *src) {
    size_t bytes = (size_t)h * w * Info::size;
    if (bytes == 0) return;
    if (contiguous()) {
      check(bn_memcpy(base(), src, bytes, on_device ? 0 : 3, g_stream));
      return;
    }
    if (!on_device) {
      const char *s = (const char *)src;
      for (int r = 0; r < h; ++r)
        for (int c = 0; c < w; ++c)
          std::memcpy((char *)ref->ptr + (offset + (int64_t)r * stride_h + (int64_t)c * stride_w) * Info::size,
                      s + ((size_t)r * w + c) * Info::size, Info::size);
      return;
    }
    PyTensor<DT> tmp(h, w, true);  // dense staging tensor, then a strided device copy
    check(bn_memcpy(tmp.base(), src, bytes, 0, g_stream));
    bn_view sv = tmp.view(), dv = view();
    check(bn_copy(&sv, &dv, g_stream));
  }
  void download_raw(void *dst) const {
    size_t bytes = (size_t)h * w * Info::size;
    if (bytes == 0) return;
    if (contiguous()) {
      check(bn_memcpy(dst, base(), bytes, on_device ? 1 : 3, g_stream));
      return;
    }
    if (!on_device) {
      char *d = (char *)dst;
      for (int r = 0; r < h; ++r)
        for (int c = 0; c < w; ++c)
          std::memcpy(d + ((size_t)r * w + c) * Info::size,
                      (const char *)ref->ptr + (offset + (int64_t)r * stride_h + (int64_t)c * stride_w) * Info::size,
                      Info::size);
      return;
    }
    PyTensor<DT> tmp(h, w, true);
    bn_view sv = view(), dv = tmp.view();
    check(bn_copy(&sv, &dv, g_stream));
    check(bn_memcpy(dst, tmp.base(), bytes, 1, g_stream));
  }

  // py_tensor_shim.hh:47-65
  void copy_from_numpy(py::array_t<host_t, py::array::c_style | py::array::forcecast> arr) {
    if (arr.ndim() != 2) throw std::runtime_error("Expected 2D NumPy array");
    if (arr.shape(0) != h || arr.shape(1) != w) throw std::runtime_error("Shape mismatch");
    if (DT == BN_BF16) {
      std::vector<uint16_t> tmp((size_t)h * w);
      const float *src = reinterpret_cast<const float *>(arr.data());
      for (size_t i = 0; i < tmp.size(); ++i) tmp[i] = f32_to_bf16_host(src[i]);
      upload_raw(tmp.data());
    } else {
      upload_raw(arr.data());
    }
  }

  // py_tensor_shim.hh:68-80 (gathers the view's own elements)
  py::array to_numpy() const {
    py::array_t<host_t> out({(py::ssize_t)h, (py::ssize_t)w});
    if (DT == BN_BF16) {
      std::vector<uint16_t> tmp((size_t)h * w);
      download_raw(tmp.data());
      float *dst = reinterpret_cast<float *>(out.mutable_data());
      for (size_t i = 0; i < tmp.size(); ++i) dst[i] = bf16_to_f32_host(tmp[i]);
    } else {
      download_raw(out.mutable_data());
    }
    return out;
  }

  void fill(double v) {
    if (on_device) {
      bn_view dv = view();
      check(bn_fill(&dv, v, g_stream));
      return;
    }
    for (int r = 0; r < h; ++r)
      for (int c = 0; c < w; ++c) {
        char *p = (char *)ref->ptr + (offset + (int64_t)r * stride_h + (int64_t)c * stride_w) * Info::size;
        if (DT == BN_F32) {
          float f = (float)v;
          std::memcpy(p, &f, 4);
        } else if (DT == BN_U32) {
          uint32_t u = (uint32_t)v;
          std::memcpy(p, &u, 4);
        } else {
          uint16_t b = f32_to_bf16_host((float)v);
          std::memcpy(p, &b, 2);
        }
      }
  }

  PyTensor transpose() const {  // tensor.cuh:133-145
    PyTensor t = *this;
    t.h = w;
    t.w = h;
    t.stride_h = stride_w;
    t.stride_w = stride_h;
    return t;
  }

  PyTensor slice_view(int sh, int eh, int sw, int ew) const {  // tensor.cuh:149-171
    if (sh >= eh || eh > h || sw >= ew || ew > w)
      throw std::runtime_error("Slice index out of range: " + std::to_string(sh) + ":" +
                               std::to_string(eh) + "," + std::to_string(sw) + ":" +
                               std::to_string(ew) + " for tensor " + repr_core());
    PyTensor t = *this;
    t.h = eh - sh;
    t.w = ew - sw;
    t.offset = offset + (int64_t)sh * stride_h + (int64_t)sw * stride_w;
    return t;
  }

  PyTensor getitem(py::object index) const {  // py_tensor_shim.hh:90-152
    auto parse_dim = [&](py::handle obj, int dim) -> std::pair<int, int> {
      if (obj.is(py::ellipsis()) || obj.is_none()) return {0, dim};
      if (py::isinstance<py::slice>(obj)) {
        Py_ssize_t start = 0, stop = 0, step = 0, len = 0;
        if (!obj.cast<py::slice>().compute(dim, &start, &stop, &step, &len))
          throw py::error_already_set();
        if (step != 1) throw py::index_error("Tensor slicing only supports step=1");
        return {(int)start, (int)stop};
      }
      if (py::isinstance<py::int_>(obj)) {
        int idx = obj.cast<int>();
        if (idx < 0) idx += dim;
        if (idx < 0 || idx >= dim) throw py::index_error("Index out of range");
        return {idx, idx + 1};
      }
      throw py::type_error("Tensor indices must be integers, slices, or None");
    };
    py::tuple tup = py::isinstance<py::tuple>(index) ? index.cast<py::tuple>() : py::make_tuple(index);
    if (tup.size() > 2) throw py::index_error("Tensor only supports 2D indexing");
    py::object i0 = tup.size() > 0 ? py::reinterpret_borrow<py::object>(tup[0]) : py::ellipsis();
    py::object i1 = tup.size() > 1 ? py::reinterpret_borrow<py::object>(tup[1]) : py::ellipsis();
    auto [a, b] = parse_dim(i0, h);
    auto [c, d] = parse_dim(i1, w);
    return slice_view(a, b, c, d);
  }

  std::string repr_core() const {
    std::ostringstream oss;
    oss << "Tensor(" << h << ", " << w << ", on_device=" << (on_device ? "true" : "false") << ")";
    return oss.str();
  }
  std::string repr() const { return "dtype=" + std::string(Info::name()) + " " + repr_core(); }

  PyTensor like() const { return PyTensor(h, w, on_device); }
};

using TF = PyTensor<BN_F32>;
using TU = PyTensor<BN_U32>;
using TB = PyTensor<BN_BF16>;

template <int DT>
PyTensor<DT> binary(int op, const PyTensor<DT> &a, const PyTensor<DT> &b) {
  PyTensor<DT> out = a.like();
  bn_view av = a.view(), bv = b.view(), ov = out.view();
  check(bn_binary(op, &av, &bv, &ov, g_stream));
  return out;
}

template <int DT>
TU equal(const PyTensor<DT> &a, const PyTensor<DT> &b) {
  TU out(a.h, a.w, a.on_device);
  bn_view av = a.view(), bv = b.view(), ov = out.view();
  check(bn_binary(BN_EQ, &av, &bv, &ov, g_stream));
  return out;
}

TF unary(int op, const TF &x, float c) {
  TF out = x.like();
  bn_view xv = x.view(), ov = out.view();
  check(bn_unary(op, &xv, c, &ov, g_stream));
  return out;
}

TU scalar_u32(int op, const TU &x, uint32_t c) {
  TU cst(1, x.w, x.on_device);  // one row, broadcast down the rows
  cst.fill((double)c);
  return binary<BN_U32>(op, x, cst);
}

template <int DT>
PyTensor<DT> sum_axis(const PyTensor<DT> &x, int axis) {
  int oh = x.h, ow = x.w;
  if (axis == 0) oh = 1;
  else if (axis == 1) ow = 1;
  else throw std::runtime_error("Invalid axis, must be 0 or 1");
  PyTensor<DT> out(oh, ow, x.on_device);
  bn_view xv = x.view(), ov = out.view();
  check(bn_sum(&xv, &ov, axis, g_stream));
  return out;
}

template <int DT>
TU argmax(const PyTensor<DT> &x) {
  TU out(x.h, 1, x.on_device);
  bn_view xv = x.view(), ov = out.view();
  check(bn_argmax(&xv, &ov, g_stream));
  return out;
}

TF matmul(const TF &a, const TF &b) {
  TF out(a.h, b.w, a.on_device);
  bn_view av = a.view(), bv = b.view(), ov = out.view();
  check(bn_matmul(&av, &bv, &ov, g_stream));
  return out;
}

template <int DT>
PyTensor<DT> rmsnorm(const PyTensor<DT> &x, const PyTensor<DT> &wt, float eps) {
  PyTensor<DT> out = x.like();
  bn_view xv = x.view(), wv = wt.view(), ov = out.view();
  check(bn_rmsnorm(&xv, &wv, &ov, eps, g_stream));
  return out;
}

template <int DT>
PyTensor<DT> rope(const PyTensor<DT> &x, int off, int hd, float theta) {
  PyTensor<DT> out = x.like();
  bn_view xv = x.view(), ov = out.view();
  check(bn_rope(&xv, &ov, off, hd, theta, g_stream));
  return out;
}

template <int DT>
PyTensor<DT> rmsnorm_rope(const PyTensor<DT> &x, const PyTensor<DT> &wt, float eps, int off,
                          int hd, float theta) {
  PyTensor<DT> out = x.like();
  bn_view xv = x.view(), wv = wt.view(), ov = out.view();
  check(bn_rmsnorm_rope(&xv, &wv, &ov, eps, off, hd, theta, g_stream));
  return out;
}

template <int DT>
py::tuple add_rmsnorm(const PyTensor<DT> &x, const PyTensor<DT> &delta, const PyTensor<DT> &wt,
                      float eps) {
  PyTensor<DT> h = x.like(), out = x.like();
  bn_view xv = x.view(), dv = delta.view(), wv = wt.view(), hv = h.view(), ov = out.view();
  check(bn_add_rmsnorm(&xv, &dv, &wv, &hv, &ov, eps, g_stream));
  return py::make_tuple(h, out);
}

template <int DT>
PyTensor<DT> silu_mul(const PyTensor<DT> &gate, const PyTensor<DT> &up) {
  PyTensor<DT> out = gate.like();
  bn_view gv = gate.view(), uv = up.view(), ov = out.view();
  check(bn_silu_mul(&gv, &uv, &ov, g_stream));
  return out;
}

template <int DT>
PyTensor<DT> softmax(const PyTensor<DT> &x, bool causal, int off) {
  PyTensor<DT> out = x.like();
  bn_view xv = x.view(), ov = out.view();
  check(bn_softmax(&xv, &ov, causal ? 1 : 0, off, g_stream));
  return out;
}

template <int DT>
PyTensor<DT> repeat_kv(const PyTensor<DT> &kv, int n_rep, int head_dim) {
  if (n_rep <= 0) throw std::runtime_error("repeat_kv: n_rep must be positive");
  PyTensor<DT> out(kv.h, kv.w * n_rep, kv.on_device);
  bn_view iv = kv.view(), ov = out.view();
  check(bn_repeat_kv(&iv, &ov, head_dim, n_rep, g_stream));
  return out;
}

template <int DT>
void require_rows(const PyTensor<DT> &t, const char *op, const char *name) {
  if (!t.on_device) throw std::runtime_error(std::string(op) + ": only GPU implementation available");
  if (t.stride_w != 1) throw std::runtime_error(std::string(op) + ": " + name + " rows must be contiguous (stride_w == 1)");
}

// q [batch*seq_q, n_heads*head_dim], k/v [batch*seq_kv, n_kv_heads*head_dim]
template <int DT>
PyTensor<DT> gqa_prefill(const PyTensor<DT> &q, const PyTensor<DT> &k, const PyTensor<DT> &v,
                         int batch, int n_heads, int n_kv_heads, int head_dim, py::object scale,
                         bool causal, int seq_offset) {
  const char *op = "GQA prefill";
  require_rows(q, op, "q");
  require_rows(k, op, "k");
  require_rows(v, op, "v");
  if (batch <= 0 || q.h % batch || k.h % batch || v.h != k.h)
    throw std::runtime_error("GQA prefill: rows of q and k/v must be batch * seq_len");
  if (q.w != n_heads * head_dim || k.w != n_kv_heads * head_dim || v.w != k.w)
    throw std::runtime_error("GQA prefill: widths must be n_heads*head_dim and n_kv_heads*head_dim");
  if (k.stride_h != v.stride_h) throw std::runtime_error("GQA prefill: k and v row strides differ");
  float sc = scale.is_none() ? (float)(1.0 / std::sqrt((double)head_dim)) : scale.cast<float>();
  const int seq_q = q.h / batch, seq_kv = k.h / batch;
  PyTensor<DT> out(q.h, q.w, true);
  // k and v carry separate bases; same strides
  check(bn_gqa_prefill(DT, q.base(), k.base(), v.base(), out.base(), batch, seq_q, seq_kv, n_heads,
                       n_kv_heads, head_dim, (int64_t)seq_q * q.stride_h, q.stride_h,
                       (int64_t)seq_kv * k.stride_h, k.stride_h, (int64_t)seq_q * out.stride_h,
                       out.stride_h, sc, causal ? 1 : 0, seq_offset, g_stream));
  return out;
}

// The fused-head chain of llama_layers.hpp:83-109 (repeat_kv, q @ k_rep^T,
// * scale, causal softmax, @ v_rep) in one launch: q [seq_q, n_heads*head_dim],
// k/v [seq_kv, n_kv_heads*head_dim], fp32; returns [seq_q, n_heads*head_dim]
TF fused_head_attention(const TF &q, const TF &k, const TF &v, int n_heads, int n_kv_heads,
                        int head_dim, py::object scale, bool causal, int seq_offset) {
  float sc = scale.is_none() ? (float)(1.0 / std::sqrt((double)head_dim)) : scale.cast<float>();
  TF out(q.h, q.w, q.on_device);
  bn_view qv = q.view(), kv = k.view(), vv = v.view(), ov = out.view();
  check(bn_fused_head_attention(&qv, &kv, &vv, &ov, n_heads, n_kv_heads, head_dim, sc,
                                causal ? 1 : 0, seq_offset, g_stream));
  return out;
}

// gqa_prefill that also returns lse, TensorF [batch*n_heads, seq_q]: the
// natural-log row log-sum-exp the backward recomputes the probabilities from
template <int DT>
py::tuple gqa_prefill_lse(const PyTensor<DT> &q, const PyTensor<DT> &k, const PyTensor<DT> &v,
                          int batch, int n_heads, int n_kv_heads, int head_dim, py::object scale,
                          bool causal, int seq_offset) {
  const char *op = "GQA prefill";
  require_rows(q, op, "q");
  require_rows(k, op, "k");
  require_rows(v, op, "v");
  if (batch <= 0 || q.h % batch || k.h % batch || v.h != k.h)
    throw std::runtime_error("GQA prefill: rows of q and k/v must be batch * seq_len");
  if (q.w != n_heads * head_dim || k.w != n_kv_heads * head_dim || v.w != k.w)
    throw std::runtime_error("GQA prefill: widths must be n_heads*head_dim and n_kv_heads*head_dim");
  if (k.stride_h != v.stride_h) throw std::runtime_error("GQA prefill: k and v row strides differ");
  float sc = scale.is_none() ? (float)(1.0 / std::sqrt((double)head_dim)) : scale.cast<float>();
  const int seq_q = q.h / batch, seq_kv = k.h / batch;
  PyTensor<DT> out(q.h, q.w, true);
  TF lse(batch * n_heads, seq_q, true);
  check(bn_gqa_prefill_lse(DT, q.base(), k.base(), v.base(), out.base(), (float *)lse.base(), batch,
                           seq_q, seq_kv, n_heads, n_kv_heads, head_dim,
                           (int64_t)seq_q * q.stride_h, q.stride_h, (int64_t)seq_kv * k.stride_h,
                           k.stride_h, (int64_t)seq_q * out.stride_h, out.stride_h, sc,
                           causal ? 1 : 0, seq_offset, g_stream));
  return py::make_tuple(out, lse);
}

// (dq, dk, dv) of gqa_prefill from its output o, lse and the gradient dout
// (bf16 kernels; TensorF inputs are rejected by the C ABI)
template <int DT>
py::tuple gqa_prefill_backward(const PyTensor<DT> &q, const PyTensor<DT> &k, const PyTensor<DT> &v,
                               const PyTensor<DT> &o, const PyTensor<DT> &dout, const TF &lse,
                               int batch, int n_heads, int n_kv_heads, int head_dim,
                               py::object scale, bool causal, int seq_offset) {
  const char *op = "GQA prefill backward";
  for (auto t : {&q, &k, &v, &o, &dout}) require_rows(*t, op, "inputs");
  if (batch <= 0 || q.h % batch || k.h % batch || v.h != k.h || o.h != q.h || dout.h != q.h)
    throw std::runtime_error("GQA prefill backward: rows of q/o/dout and k/v must be batch * seq_len");
  if (q.w != n_heads * head_dim || k.w != n_kv_heads * head_dim || v.w != k.w || o.w != q.w ||
      dout.w != q.w)
    throw std::runtime_error("GQA prefill backward: widths must be n_heads*head_dim and n_kv_heads*head_dim");
  if (k.stride_h != v.stride_h || o.stride_h != dout.stride_h)
    throw std::runtime_error("GQA prefill backward: k/v and o/dout row strides must match");
  const int seq_q = q.h / batch, seq_kv = k.h / batch;
  if (!lse.on_device || !lse.contiguous() || lse.h != batch * n_heads || lse.w != seq_q)
    throw std::runtime_error("GQA prefill backward: lse must be a contiguous device TensorF [batch*n_heads, seq_q]");
  float sc = scale.is_none() ? (float)(1.0 / std::sqrt((double)head_dim)) : scale.cast<float>();
  PyTensor<DT> dq(q.h, q.w, true), dk(k.h, k.w, true), dv(v.h, v.w, true);
  // dq takes q's row stride, dk/dv k's: fresh tensors are dense, so q/k must be too
  if (q.stride_h != dq.stride_h || k.stride_h != dk.stride_h)
    throw std::runtime_error("GQA prefill backward: q and k/v must have dense rows");
  check(bn_gqa_prefill_backward(DT, q.base(), k.base(), v.base(), o.base(), dout.base(),
                                (const float *)lse.base(), dq.base(), dk.base(), dv.base(), batch,
                                seq_q, seq_kv, n_heads, n_kv_heads, head_dim,
                                (int64_t)seq_q * q.stride_h, q.stride_h, (int64_t)seq_kv * k.stride_h,
                                k.stride_h, (int64_t)seq_q * o.stride_h, o.stride_h, sc,
                                causal ? 1 : 0, seq_offset, nullptr, 0, g_stream));
  return py::make_tuple(dq, dk, dv);
}

// q [batch, n_heads*head_dim]; caches [batch*max_len, n_kv_heads*head_dim];
// seq_lens: TensorU32 holding batch lengths
template <int DT>
PyTensor<DT> gqa_decode(const PyTensor<DT> &q, const PyTensor<DT> &kc, const PyTensor<DT> &vc,
                        const TU &lens, int n_heads, int n_kv_heads, int head_dim,
                        py::object scale) {
  const char *op = "GQA decode";
  require_rows(q, op, "q");
  require_rows(kc, op, "k_cache");
  require_rows(vc, op, "v_cache");
  if (!lens.on_device) throw std::runtime_error("GQA decode: seq_lens must be a device tensor");
  if (!q.contiguous() || !kc.contiguous() || !vc.contiguous() || !lens.contiguous())
    throw std::runtime_error("GQA decode: q, caches and seq_lens must be contiguous");
  const int batch = q.h;
  if (lens.h * lens.w != batch) throw std::runtime_error("GQA decode: seq_lens must hold one length per row of q");
  if (batch == 0) return PyTensor<DT>(0, q.w, true);
  if (kc.h % batch || vc.h != kc.h || kc.w != vc.w)
    throw std::runtime_error("GQA decode: cache rows must be batch * max_len");
  if (q.w != n_heads * head_dim || kc.w != n_kv_heads * head_dim)
    throw std::runtime_error("GQA decode: widths must be n_heads*head_dim and n_kv_heads*head_dim");
  float sc = scale.is_none() ? (float)(1.0 / std::sqrt((double)head_dim)) : scale.cast<float>();
  PyTensor<DT> out(q.h, q.w, true);
  check(bn_gqa_decode(DT, q.base(), kc.base(), vc.base(), (const int32_t *)lens.base(), out.base(),
                      batch, kc.h / batch, n_heads, n_kv_heads, head_dim, sc, nullptr, 0, g_stream));
  return out;
}

template <int DT>
py::class_<PyTensor<DT>> bind_common(py::module_ &m, const char *pyname) {
  using Self = PyTensor<DT>;
  using H = typename Self::host_t;
  auto cls = py::class_<Self>(m, pyname)
    .def(py::init<int, int, bool>(), py::arg("h"), py::arg("w"), py::arg("is_cuda") = true)
    .def_property_readonly("shape", &Self::shape)
    .def_property_readonly("is_cuda", &Self::is_cuda)
    .def("to_numpy", &Self::to_numpy)
    .def("copy_from_numpy", &Self::copy_from_numpy)
    .def("fill", [](Self &me, H v) { me.fill((double)v); }, py::arg("value"))
    .def("transpose", &Self::transpose)
    .def("slice", &Self::slice_view, py::arg("start_h"), py::arg("end_h"), py::arg("start_w"),
         py::arg("end_w"))
    .def_property_readonly("T", &Self::transpose)
    .def("__getitem__", &Self::getitem)
    .def("__repr__", &Self::repr);
  return cls;
}

template <int DT>
void bind_float_ops(py::class_<PyTensor<DT>> &cls) {
  using Self = PyTensor<DT>;
  cls.def("rmsnorm", [](const Self &me, const Self &w, float eps) { return rmsnorm<DT>(me, w, eps); },
          py::arg("weight"), py::arg("eps") = 1e-6f)
    .def("rope", [](const Self &me, int off, int hd, float th) { return rope<DT>(me, off, hd, th); },
         py::arg("position_offset") = 0, py::arg("head_dim") = 64, py::arg("theta") = 10000.0f)
    .def("softmax", [](const Self &me, bool causal, int off) { return softmax<DT>(me, causal, off); },
         py::arg("causal") = false, py::arg("seq_offset") = 0)
    .def("rmsnorm_rope",
         [](const Self &me, const Self &w, float eps, int off, int hd, float th) {
           return rmsnorm_rope<DT>(me, w, eps, off, hd, th);
         },
         py::arg("weight"), py::arg("eps") = 1e-6f, py::arg("position_offset") = 0,
         py::arg("head_dim") = 64, py::arg("theta") = 10000.0f);
}

// ---------------------------------------------------------------- LLaMA
// Same fields and defaults as llama_config.hpp:13-32 (TinyLLaMA-1.1B).
struct LlamaCfg {
  int vocab_size = 32000, hidden_size = 2048, intermediate_size = 5632, num_hidden_layers = 22,
      num_attention_heads = 32, num_key_value_heads = 4, max_position_embeddings = 2048;
  float rms_norm_eps = 1e-6f, rope_theta = 10000.0f;
  int head_dim() const { return hidden_size / num_attention_heads; }
  void validate() const {  // llama_config.hpp:42-51
    if (num_attention_heads <= 0 || hidden_size % num_attention_heads != 0)
      throw std::runtime_error("hidden_size must be divisible by num_attention_heads");
    if (num_key_value_heads <= 0 || num_attention_heads % num_key_value_heads != 0)
      throw std::runtime_error("num_attention_heads must be divisible by num_key_value_heads");
  }
  // llama_config.hpp:82-105, in size_t throughout (the reference forms
  // vocab_size * hidden_size in int)
  size_t count_parameters() const {
    const size_t h = hidden_size, kv = (size_t)num_key_value_heads * head_dim(),
                 I = intermediate_size, V = vocab_size;
    const size_t per_layer = h * h + 2 * h * kv + h * h + 3 * h * I + 2 * h;
    return V * h + per_layer * (size_t)num_hidden_layers + h + h * V;
  }
  std::string to_string() const {  // llama_config.hpp:68-78
    return "LLaMAConfig(\n  vocab_size=" + std::to_string(vocab_size) + ",\n  hidden_size=" +
           std::to_string(hidden_size) + ",\n  num_layers=" + std::to_string(num_hidden_layers) +
           ",\n  num_heads=" + std::to_string(num_attention_heads) + ",\n  num_kv_heads=" +
           std::to_string(num_key_value_heads) + ",\n  intermediate_size=" +
           std::to_string(intermediate_size) + "\n)";
  }
};

// Host twin of the device uniform fill (bn_fill_uniform): SplitMix64 of the
// seed and the logical index, so host and device models get equal weights.
float uniform01_host(uint64_t seed, uint64_t index) {
  uint64_t z = seed + (index + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  return (float)(uint32_t)(z >> 40) * (1.0f / 16777216.0f);
}

void fill_uniform(TF &t, float lo, float hi, uint64_t seed) {
  if (t.on_device) {
    bn_view v = t.view();
    check(bn_fill_uniform(&v, lo, hi, seed, g_stream));
    return;
  }
  float *p = (float *)t.base();
  for (int64_t i = 0; i < (int64_t)t.h * t.w; ++i)
    p[i] = std::fma(uniform01_host(seed, (uint64_t)i), hi - lo, lo);
}

// LLaMAModel (llama_model.hpp:19-198) behind the PyLLaMAModel binding
// (llama_bindings.hpp:31-96): token ids -> logits through the decoder layers
// (llama_layers.hpp:241-272), all on the path's kernels.
//   * Weights: embed_tokens and lm_head uniform in [-0.02, 0.02] as the
//     reference fills them (llama_model.hpp:27,37; op_uniform_fill with the
//     randgen_seed), norm weights ones; the projections, which the reference
//     leaves uninitialised (bare cudaMalloc), get the same uniform fill.  Each
//     tensor has its own stream of the seed.
//   * Layout: Q|K|V and gate|up are stored concatenated ([hidden, (H+2Hkv)D],
//     [hidden, 2I]) so each is one GEMM; weights() returns the reference's
//     per-projection tensors as column views of them (loading through those
//     views writes the model's weights).
//   * attention = "fused_head" (default) computes the reference's chain
//     (llama_layers.hpp:96-109: Q K_rep^T over all heads at once, scale,
//     causal softmax, @ V_rep) with bn_fused_head_attention, one launch;
//     "per_head" runs per-head GQA on bn_gqa_prefill.
//   * Embedding gathers on the device (bn_embedding) instead of copying the
//     whole table to the host and back (llama_model.hpp:161-198).
class LlamaModelCpp {
 public:
  LlamaModelCpp(const LlamaCfg &cfg, bool on_device, const std::string &attention)
      : cfg_(cfg), on_device_(on_device) {
    cfg_.validate();
    // the reference's constructor allocates whatever it is given; the forward
    // here reads layer 0 and sizes buffers from these, so they must be positive
    if (cfg_.num_hidden_layers <= 0 || cfg_.vocab_size <= 0 || cfg_.hidden_size <= 0 ||
        cfg_.intermediate_size <= 0)
      throw std::runtime_error(
          "LLaMAModelCpp: num_hidden_layers, vocab_size, hidden_size and intermediate_size must be positive");
    if (attention != "fused_head" && attention != "per_head")
      throw std::runtime_error("LLaMAModelCpp: attention must be 'fused_head' or 'per_head'");
    per_head_ = attention == "per_head";
    const int h = cfg_.hidden_size, kv = cfg_.num_key_value_heads * cfg_.head_dim(),
              I = cfg_.intermediate_size;
    uint64_t stream_id = 0;
    auto uniform = [&](int rows, int cols) {
      TF t(rows, cols, on_device_);
      fill_uniform(t, -0.02f, 0.02f, g_randgen_seed * 0x100000001B3ull + (++stream_id));
      return t;
    };
    auto ones = [&]() {
      TF t(1, h, on_device_);
      t.fill(1.0);
      return t;
    };
    embed_ = uniform(cfg_.vocab_size, h);
    for (int l = 0; l < cfg_.num_hidden_layers; ++l) {
      Layer L;
      L.ln1 = ones();
      L.wqkv = uniform(h, h + 2 * kv);
      L.wo = uniform(h, h);
      L.ln2 = ones();
      L.wgu = uniform(h, 2 * I);
      L.wd = uniform(I, h);
      layers_.push_back(std::move(L));
    }
    ln_f_ = ones();
    lm_head_ = uniform(h, cfg_.vocab_size);
    if (on_device_) check(bn_stream_synchronize(g_stream));
  }

  // llama_bindings.hpp:37-58: ids (batch,) -> logits (batch, vocab)
  py::array forward(py::array_t<uint32_t, py::array::c_style | py::array::forcecast> ids) {
    TF logits = run(ids);
    return logits.to_numpy();
  }

  // llama_bindings.hpp:60-71 / llama_model.hpp:86-118: milliseconds of one
  // forward (ids already on the device), host clock between stream syncs
  float forward_timed(py::array_t<uint32_t, py::array::c_style | py::array::forcecast> ids) {
    TU dev_ids = upload_ids(ids);
    if (on_device_) check(bn_stream_synchronize(g_stream));
    const auto t0 = std::chrono::steady_clock::now();
    TF logits = run_device(dev_ids);
    if (on_device_) check(bn_stream_synchronize(g_stream));
    const auto t1 = std::chrono::steady_clock::now();
    return std::chrono::duration<float, std::milli>(t1 - t0).count();
  }

  // llama_model.hpp:209-266: token id 1 in every row, warm-up, mean time
  py::dict benchmark(int batch_size, int num_warmup, int num_iterations) {
    if (batch_size <= 0 || num_iterations <= 0)
      throw std::runtime_error("benchmark: batch_size and num_iterations must be positive");
    py::array_t<uint32_t> ids(batch_size);
    for (int i = 0; i < batch_size; ++i) ids.mutable_at(i) = 1;
    for (int i = 0; i < num_warmup; ++i) run(ids);
    float total = 0.f;
    for (int i = 0; i < num_iterations; ++i) total += forward_timed(ids);
    py::dict d;
    const float ms = total / num_iterations;
    d["forward_time_ms"] = ms;
    d["tokens_per_second"] = batch_size * 1000.0f / ms;
    d["memory_used_bytes"] = get_gpu_memory_usage();
    d["num_parameters"] = count_parameters();
    return d;
  }

  size_t count_parameters() const { return cfg_.count_parameters(); }

  size_t get_gpu_memory_usage() const {  // llama_model.hpp:125-131
    if (!on_device_) return 0;
    size_t free_b = 0, total_b = 0;
    check(bn_mem_get_info(&free_b, &total_b));
    return total_b - free_b;
  }

  // Additive: the weights as TensorF views under the reference's accessor
  // names (llama_model.hpp:140-143, llama_layers.hpp accessors).
  py::dict weights() const {
    const int h = cfg_.hidden_size, kv = cfg_.num_key_value_heads * cfg_.head_dim(),
              I = cfg_.intermediate_size;
    py::dict d;
    d["embed_tokens"] = embed_;
    d["final_norm"] = ln_f_;
    d["lm_head"] = lm_head_;
    py::list layers;
    for (const Layer &L : layers_) {
      py::dict ld;
      ld["input_layernorm"] = L.ln1;
      ld["q_proj"] = L.wqkv.slice_view(0, h, 0, h);
      ld["k_proj"] = L.wqkv.slice_view(0, h, h, h + kv);
      ld["v_proj"] = L.wqkv.slice_view(0, h, h + kv, h + 2 * kv);
      ld["o_proj"] = L.wo;
      ld["post_attention_layernorm"] = L.ln2;
      ld["gate_proj"] = L.wgu.slice_view(0, h, 0, I);
      ld["up_proj"] = L.wgu.slice_view(0, h, I, 2 * I);
      ld["down_proj"] = L.wd;
      layers.append(ld);
    }
    d["layers"] = layers;
    return d;
  }

 private:
  struct Layer {
    TF ln1, wqkv, wo, ln2, wgu, wd;
  };
  LlamaCfg cfg_;
  bool on_device_;
  bool per_head_ = false;
  TF embed_, ln_f_, lm_head_;
  std::vector<Layer> layers_;

  TU upload_ids(const py::array_t<uint32_t, py::array::c_style | py::array::forcecast> &ids) {
    if (ids.ndim() != 1) throw std::runtime_error("LLaMAModelCpp: input_ids must be 1-D (batch,)");
    const int n = (int)ids.shape(0);
    for (int i = 0; i < n; ++i)
      if (ids.at(i) >= (uint32_t)cfg_.vocab_size)
        throw std::runtime_error("LLaMAModelCpp: token id " + std::to_string(ids.at(i)) +
                                 " outside the vocabulary of " + std::to_string(cfg_.vocab_size));
    TU t(n, 1, on_device_);
    if (n) t.upload_raw(ids.data());
    return t;
  }

  TF run(const py::array_t<uint32_t, py::array::c_style | py::array::forcecast> &ids) {
    return run_device(upload_ids(ids));
  }

  // llama_model.hpp:52-80 with the layer of llama_layers.hpp:241-272; each
  // residual add runs fused with the RMSNorm that follows it (bn_add_rmsnorm:
  // the same sum, then the same normalisation)
  TF run_device(const TU &ids) {
    const int n = ids.h, h = cfg_.hidden_size, D = cfg_.head_dim(),
              kv = cfg_.num_key_value_heads * D, I = cfg_.intermediate_size,
              G = cfg_.num_attention_heads / cfg_.num_key_value_heads;
    const float eps = cfg_.rms_norm_eps, theta = cfg_.rope_theta;
    // the first op on a host model is the reference's first throw
    if (!on_device_) throw std::runtime_error("RMSNorm: only GPU implementation available");
    if (n == 0) return TF(0, cfg_.vocab_size, true);
    TF hdn(n, h, true);
    {
      bn_view tv = embed_.view(), ov = hdn.view();
      check(bn_embedding(&tv, (const uint32_t *)ids.base(), n, &ov, g_stream));
    }
    TF x = rmsnorm<BN_F32>(hdn, layers_[0].ln1, eps);
    for (size_t l = 0; l < layers_.size(); ++l) {
      const Layer &L = layers_[l];
      TF qkv = matmul(x, L.wqkv);
      {  // RoPE on the Q and K columns, in place (one launch)
        TF qk = qkv.slice_view(0, n, 0, h + kv);
        bn_view v = qk.view();
        check(bn_rope(&v, &v, 0, D, theta, g_stream));
      }
      TF q = qkv.slice_view(0, n, 0, h), k = qkv.slice_view(0, n, h, h + kv),
         v = qkv.slice_view(0, n, h + kv, h + 2 * kv);
      TF attn;
      if (per_head_) {
        attn = gqa_prefill<BN_F32>(q, k, v, 1, cfg_.num_attention_heads, cfg_.num_key_value_heads,
                                   D, py::none(), true, 0);
      } else {
        if (kv <= 512 && kv % 16 == 0 && D % 4 == 0) {
          // repeat_kv, q @ k_rep^T, * scale, causal softmax, @ v_rep: one launch
          attn = fused_head_attention(q, k, v, cfg_.num_attention_heads,
                                      cfg_.num_key_value_heads, D, py::none(), true, 0);
        } else {  // KV widths past the fused kernel's LDS budget: the chain op by op
          TF krep = G > 1 ? repeat_kv<BN_F32>(k, G, D) : k;
          TF vrep = G > 1 ? repeat_kv<BN_F32>(v, G, D) : v;
          TF scores = matmul(q, krep.transpose());
          TF scaled = unary(BN_MUL_SCALAR, scores, (float)(1.0 / std::sqrt((double)D)));
          attn = matmul(softmax<BN_F32>(scaled, true, 0), vrep);
        }
      }
      TF o = matmul(attn, L.wo);
      TF x2 = hdn.like();
      {
        bn_view hv = hdn.view(), ov = o.view(), wv = L.ln2.view(), yv = x2.view();
        check(bn_add_rmsnorm(&hv, &ov, &wv, &hv, &yv, eps, g_stream));  // hdn += o
      }
      TF gu = matmul(x2, L.wgu);
      TF act = silu_mul<BN_F32>(gu.slice_view(0, n, 0, I), gu.slice_view(0, n, I, 2 * I));
      TF mlp = matmul(act, L.wd);
      const TF &next_w = l + 1 < layers_.size() ? layers_[l + 1].ln1 : ln_f_;
      x = hdn.like();
      bn_view hv = hdn.view(), mv = mlp.view(), wv = next_w.view(), yv = x.view();
      check(bn_add_rmsnorm(&hv, &mv, &wv, &hv, &yv, eps, g_stream));  // hdn += mlp
    }
    return matmul(x, lm_head_);
  }
};

}  // namespace

PYBIND11_MODULE(bten, m) {
  m.doc() = "BareNet op surface on MI355X (gfx950) HIP kernels via libbnhip's C ABI";

  m.def("randgen_seed", [](unsigned long long seed) { g_randgen_seed = seed; }, "Set random seed");

  // ------------------------------------------------------------ TensorF
  auto tf = bind_common<BN_F32>(m, "TensorF");
  tf.def("__add__", [](const TF &a, const TF &b) { return binary<BN_F32>(BN_ADD, a, b); }, py::arg("other"))
    .def("__add__", [](const TF &a, float c) { return unary(BN_ADD_SCALAR, a, c); }, py::arg("scalar"))
    .def("__sub__", [](const TF &a, const TF &b) { return binary<BN_F32>(BN_SUB, a, b); }, py::arg("other"))
    .def("__mul__", [](const TF &a, const TF &b) { return binary<BN_F32>(BN_MUL, a, b); }, py::arg("other"))
    .def("__mul__", [](const TF &a, float c) { return unary(BN_MUL_SCALAR, a, c); }, py::arg("scalar"))
    .def("__eq__", [](const TF &a, const TF &b) { return equal<BN_F32>(a, b); }, py::arg("other"))
    .def("sum", [](const TF &a, int axis) { return sum_axis<BN_F32>(a, axis); }, py::arg("axis"))
    .def("argmax", [](const TF &a) { return argmax<BN_F32>(a); })
    .def("__matmul__", &matmul, py::arg("other"))
    .def("relu", [](const TF &a) { return unary(BN_RELU, a, 0.f); })
    .def("relu_back",
         [](const TF &me, const TF &dout) {
           TF din = me.like();
           bn_view a = me.view(), b = dout.view(), c = din.view();
           check(bn_unary_backward(BN_RELU_BACK, &a, &b, &c, g_stream));
           return din;
         },
         py::arg("DOut"))
    .def("silu", [](const TF &a) { return unary(BN_SILU, a, 0.f); })
    .def("silu_back",
         [](const TF &me, const TF &dout) {
           TF din = me.like();
           bn_view a = me.view(), b = dout.view(), c = din.view();
           check(bn_unary_backward(BN_SILU_BACK, &a, &b, &c, g_stream));
           return din;
         },
         py::arg("DOut"))
    .def("rmsnorm_back",
         [](const TF &me, const TF &w, const TF &gout, TF &gw, float eps) {
           TF gin = me.like();
           bn_view a = me.view(), b = w.view(), c = gout.view(), d = gin.view(), e = gw.view();
           check(bn_rmsnorm_backward(&a, &b, &c, &d, &e, eps, g_stream));
           return gin;
         },
         py::arg("weight"), py::arg("grad_out"), py::arg("grad_weight"), py::arg("eps") = 1e-6f)
    .def("rope_back",
         [](const TF &gout, int off, int hd, float th) {
           TF gin = gout.like();
           bn_view a = gout.view(), b = gin.view();
           check(bn_rope_backward(&a, &b, off, hd, th, g_stream));
           return gin;
         },
         py::arg("position_offset") = 0, py::arg("head_dim") = 64, py::arg("theta") = 10000.0f)
    .def("softmax_back",
         [](const TF &out, const TF &gout) {
           TF gin = out.like();
           bn_view a = out.view(), b = gout.view(), c = gin.view();
           check(bn_softmax_backward(&a, &b, &c, g_stream));
           return gin;
         },
         py::arg("grad_out"))
    .def("to_bf16", [](const TF &a) {
      TB out(a.h, a.w, a.on_device);
      if (!a.on_device) throw std::runtime_error("to_bf16: only GPU implementation available");
      bn_view x = a.view(), y = out.view();
      check(bn_copy(&x, &y, g_stream));
      return out;
    });
  bind_float_ops<BN_F32>(tf);

  // ----------------------------------------------------------- TensorU32
  auto tu = bind_common<BN_U32>(m, "TensorU32");
  tu.def("__add__", [](const TU &a, const TU &b) { return binary<BN_U32>(BN_ADD, a, b); }, py::arg("other"))
    .def("__add__", [](const TU &a, uint32_t c) { return scalar_u32(BN_ADD, a, c); }, py::arg("scalar"))
    .def("__sub__", [](const TU &a, const TU &b) { return binary<BN_U32>(BN_SUB, a, b); }, py::arg("other"))
    .def("__mul__", [](const TU &a, const TU &b) { return binary<BN_U32>(BN_MUL, a, b); }, py::arg("other"))
    .def("__mul__", [](const TU &a, uint32_t c) { return scalar_u32(BN_MUL, a, c); }, py::arg("scalar"))
    .def("__eq__", [](const TU &a, const TU &b) { return equal<BN_U32>(a, b); }, py::arg("other"))
    .def("sum", [](const TU &a, int axis) { return sum_axis<BN_U32>(a, axis); }, py::arg("axis"))
    .def("argmax", [](const TU &a) { return argmax<BN_U32>(a); });

  // ---------------------------------------------------------- TensorBF16
  auto tb = bind_common<BN_BF16>(m, "TensorBF16");
  bind_float_ops<BN_BF16>(tb);
  tb.def("to_f32", [](const TB &a) {
    TF out(a.h, a.w, a.on_device);
    if (!a.on_device) throw std::runtime_error("to_f32: only GPU implementation available");
    bn_view x = a.view(), y = out.view();
    check(bn_copy(&x, &y, g_stream));
    return out;
  });

  // ----------------------------------------------------- fused attention
  m.def("fused_head_attention", &fused_head_attention, py::arg("query"), py::arg("key"),
        py::arg("value"), py::arg("n_heads") = 32, py::arg("n_kv_heads") = 4,
        py::arg("head_dim") = 64, py::arg("scale") = py::none(), py::arg("causal") = true,
        py::arg("seq_offset") = 0);
  m.def("gqa_prefill", &gqa_prefill<BN_F32>, py::arg("q"), py::arg("k"), py::arg("v"),
        py::arg("batch") = 1, py::arg("n_heads") = 32, py::arg("n_kv_heads") = 4,
        py::arg("head_dim") = 64, py::arg("scale") = py::none(), py::arg("causal") = true,
        py::arg("seq_offset") = 0);
  m.def("gqa_prefill", &gqa_prefill<BN_BF16>, py::arg("q"), py::arg("k"), py::arg("v"),
        py::arg("batch") = 1, py::arg("n_heads") = 32, py::arg("n_kv_heads") = 4,
        py::arg("head_dim") = 64, py::arg("scale") = py::none(), py::arg("causal") = true,
        py::arg("seq_offset") = 0);
  for (int bf = 0; bf < 2; ++bf) {
    auto args_lse = [&](auto fn) {
      m.def("gqa_prefill_lse", fn, py::arg("q"), py::arg("k"), py::arg("v"), py::arg("batch") = 1,
            py::arg("n_heads") = 32, py::arg("n_kv_heads") = 4, py::arg("head_dim") = 64,
            py::arg("scale") = py::none(), py::arg("causal") = true, py::arg("seq_offset") = 0);
    };
    auto args_bwd = [&](auto fn) {
      m.def("gqa_prefill_backward", fn, py::arg("q"), py::arg("k"), py::arg("v"), py::arg("o"),
            py::arg("dout"), py::arg("lse"), py::arg("batch") = 1, py::arg("n_heads") = 32,
            py::arg("n_kv_heads") = 4, py::arg("head_dim") = 64, py::arg("scale") = py::none(),
            py::arg("causal") = true, py::arg("seq_offset") = 0);
    };
    if (bf) {
      args_lse(&gqa_prefill_lse<BN_BF16>);
      args_bwd(&gqa_prefill_backward<BN_BF16>);
    } else {
      args_lse(&gqa_prefill_lse<BN_F32>);
      args_bwd(&gqa_prefill_backward<BN_F32>);
    }
  }
  m.def("gqa_decode", &gqa_decode<BN_F32>, py::arg("q"), py::arg("k_cache"), py::arg("v_cache"),
        py::arg("seq_lens"), py::arg("n_heads") = 32, py::arg("n_kv_heads") = 4,
        py::arg("head_dim") = 64, py::arg("scale") = py::none());
  m.def("gqa_decode", &gqa_decode<BN_BF16>, py::arg("q"), py::arg("k_cache"), py::arg("v_cache"),
        py::arg("seq_lens"), py::arg("n_heads") = 32, py::arg("n_kv_heads") = 4,
        py::arg("head_dim") = 64, py::arg("scale") = py::none());
  m.def("add_rmsnorm", &add_rmsnorm<BN_F32>, py::arg("x"), py::arg("delta"), py::arg("weight"),
        py::arg("eps") = 1e-6, "(x + delta, RMSNorm(x + delta) * weight) in one pass");
  m.def("add_rmsnorm", &add_rmsnorm<BN_BF16>, py::arg("x"), py::arg("delta"), py::arg("weight"),
        py::arg("eps") = 1e-6);
  m.def("silu_mul", &silu_mul<BN_F32>, py::arg("gate"), py::arg("up"), "silu(gate) * up");
  m.def("silu_mul", &silu_mul<BN_BF16>, py::arg("gate"), py::arg("up"));
  m.def("repeat_kv", &repeat_kv<BN_F32>, py::arg("kv"), py::arg("n_rep"), py::arg("head_dim") = 64);
  m.def("repeat_kv", &repeat_kv<BN_BF16>, py::arg("kv"), py::arg("n_rep"), py::arg("head_dim") = 64);

  // ------------------------------------------------------ runtime / pool
  m.def("synchronize", []() { check(bn_stream_synchronize(g_stream)); });
  // Tensors free stream-ordered on the stream current at their destruction.
  // Switching streams first waits for the outgoing stream, so every kernel
  // that touched a tensor has finished or is ordered before its free.
  m.def("set_stream", [](uintptr_t s) {
          void *next = reinterpret_cast<void *>(s);
          if (next != g_stream) check(bn_stream_synchronize(g_stream));
          g_stream = next;
        }, py::arg("stream"),
        "Launch on this hipStream_t handle (0 = legacy default stream); waits for the current stream first");
  m.def("get_stream", []() { return reinterpret_cast<uintptr_t>(g_stream); });
  m.def("pool_stats", []() {
    bn_pool_stats s;
    check(bn_pool_get_stats(&s));
    py::dict d;
    d["bytes_in_use"] = s.bytes_in_use;
    d["peak_bytes_in_use"] = s.peak_bytes_in_use;
    d["bytes_reserved"] = s.bytes_reserved;
    d["n_allocs"] = s.n_allocs;
    d["n_frees"] = s.n_frees;
    d["n_live"] = s.n_live;
    return d;
  });
  m.def("pool_reset_peak", []() { check(bn_pool_reset_peak()); });
  m.def("pool_trim", [](size_t keep) { check(bn_pool_trim(keep)); }, py::arg("min_bytes_to_keep") = 0);
  m.def("pool_set_limit", [](size_t lim) { check(bn_pool_set_limit(lim)); }, py::arg("limit_bytes"));
  m.def("device_count", []() {
    int n = 0;
    check(bn_device_count(&n));
    return n;
  });

  // --------------------------------------------------------- LLaMAConfig
  // llama_bindings.hpp:99-111 (plus the eps/theta/max_position fields of
  // llama_config.hpp:21-24, readable and writable here)
  using Config = LlamaCfg;
  py::class_<Config>(m, "LLaMAConfig")
    .def(py::init<>())
    .def_readwrite("vocab_size", &Config::vocab_size)
    .def_readwrite("hidden_size", &Config::hidden_size)
    .def_readwrite("intermediate_size", &Config::intermediate_size)
    .def_readwrite("num_hidden_layers", &Config::num_hidden_layers)
    .def_readwrite("num_attention_heads", &Config::num_attention_heads)
    .def_readwrite("num_key_value_heads", &Config::num_key_value_heads)
    .def_readwrite("max_position_embeddings", &Config::max_position_embeddings)
    .def_readwrite("rms_norm_eps", &Config::rms_norm_eps)
    .def_readwrite("rope_theta", &Config::rope_theta)
    .def("head_dim", &Config::head_dim)
    .def("num_kv_groups", [](const Config &c) { return c.num_attention_heads / c.num_key_value_heads; })
    .def("validate", &Config::validate)
    .def("count_parameters", &Config::count_parameters)
    .def_static("tinyllama_1_1b", []() {
      Config c;
      c.validate();
      return c;
    })
    .def("__repr__", &Config::to_string);

  // ------------------------------------------------------- LLaMAModelCpp
  // llama_bindings.hpp:113-122; `attention` is additive (default: the
  // reference's fused-head chain), weights() too
  py::class_<LlamaModelCpp>(m, "LLaMAModelCpp")
    .def(py::init<const Config &, bool, const std::string &>(), py::arg("config"),
         py::arg("on_device") = true, py::arg("attention") = "fused_head")
    .def("forward", &LlamaModelCpp::forward, py::arg("input_ids"))
    .def("forward_timed", &LlamaModelCpp::forward_timed, py::arg("input_ids"))
    .def("benchmark", &LlamaModelCpp::benchmark, py::arg("batch_size"), py::arg("num_warmup") = 5,
         py::arg("num_iterations") = 100)
    .def("count_parameters", &LlamaModelCpp::count_parameters)
    .def("get_gpu_memory_usage", &LlamaModelCpp::get_gpu_memory_usage)
    .def("weights", &LlamaModelCpp::weights);
}
