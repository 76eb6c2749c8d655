// bn_elemwise.hip -- the rest of the op surface the attention layers call:
// row softmax (causal / offset), fp32 matmul on strided views, the device
// repeat_kv mapping, and the elementwise / reduction helpers.
//
// Reference kernels replaced:
//   op_softmax_kernel / op_softmax_causal_kernel / op_softmax_backward_kernel
//     (src/ops/op_softmax.cuh:8-246)
//   op_mm_kernel / op_mm_tiled_kernel (src/ops/op_mm.cuh:23-57,
//     src/ops/op_mm_optimized.cuh:13-87)
//   repeat_kv host loop (src/llama/llama_layers.hpp:131-175)
//   functor kernels of src/ops/op_elemwise.cuh:169-283, op_silu.cuh:33-48,
//     op_reduction.cuh:36-109
#include <rocblas/rocblas.h>

#include <cfloat>

#include "bn_common.hpp"

namespace bn {
namespace {

// ------------------------------------------------------------- softmax
// One 256-thread workgroup per row with the reference's reduction shape:
// thread t owns columns t, t+256, ... and partials meet in an LDS tree
// (op_softmax.cuh:96-143), so the fp32 sums associate as the reference's.
template <typename T>
__global__ __launch_bounds__(256) void softmax_kernel(DView<const T> x, DView<T> y, int causal,
                                                      int seq_offset) {
  __shared__ float red[256];
  const int row = blockIdx.x, tid = threadIdx.x;
  const long q = causal ? (long)row + seq_offset : (long)x.w;  // :89
  float m = -INFINITY;
  for (int i = tid; i < x.w; i += 256)
    if (i <= q) {
      float v = Elem<T>::load(&x.at(row, i));
      if (v > m) m = v;
    }
  red[tid] = m;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (tid < s && red[tid + s] > red[tid]) red[tid] = red[tid + s];
    __syncthreads();
  }
  const float mx = red[0];
  __syncthreads();
  float sum = 0.f;
  for (int i = tid; i < x.w; i += 256) {
    if (i <= q) {
      float e = expf(Elem<T>::load(&x.at(row, i)) - mx);
      Elem<T>::store(&y.at(row, i), e);
      sum += e;
    } else {
      Elem<T>::store(&y.at(row, i), 0.f);  // :129
    }
  }
  red[tid] = sum;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (tid < s) red[tid] += red[tid + s];
    __syncthreads();
  }
  const float total = red[0];
  for (int i = tid; i < x.w; i += 256)
    if (i <= q) Elem<T>::store(&y.at(row, i), Elem<T>::load(&y.at(row, i)) / total);
}

__global__ __launch_bounds__(256) void softmax_backward_kernel(DView<const float> y,
                                                               DView<const float> dy,
                                                               DView<float> dx) {
  __shared__ float red[256];
  const int row = blockIdx.x, tid = threadIdx.x;
  float s = 0.f;
  for (int i = tid; i < y.w; i += 256) s += y.at(row, i) * dy.at(row, i);
  red[tid] = s;
  __syncthreads();
  for (int k = 128; k > 0; k >>= 1) {
    if (tid < k) red[tid] += red[tid + k];
    __syncthreads();
  }
  const float tot = red[0];
  for (int i = tid; i < y.w; i += 256) dx.at(row, i) = y.at(row, i) * (dy.at(row, i) - tot);
}

// -------------------------------------------------------------- matmul
// fp32 c = a @ b on arbitrary strided views (op_mm, op_mm.cuh:39-57) on the
// fp32 matrix cores: v_mfma_f32_32x32x2f32 (lane l supplies A[l%32][l/32] and
// B[l/32][l%32]; D[8(i/4) + 4(l/32) + i%4][l%32] lands in register i).
// A 256-thread workgroup owns a 64x64 output tile, each wave a 32x32 block;
// k steps of 32 are staged through k-major LDS tiles (conflict-free operand
// reads), the next step's tile prefetched into registers, coalesced along
// whichever dimension of each view has unit stride (so transposed views such
// as key.T load as well as row-major ones).  Small outputs split k across
// workgroups into partial slabs that a second kernel sums in a fixed order
// (deterministic).  Products and sums are fp32; the association differs from
// op_mm_tiled_kernel's single running sum (op_mm_optimized.cuh:35-62).
typedef float mf32x16_t __attribute__((ext_vector_type(16)));
constexpr int MT = 64, KT = 32, LP = MT + 4;

__global__ __launch_bounds__(256) void matmul_kernel(DView<const float> a, DView<const float> b,
                                                     DView<float> c, float *part, int kchunk) {
  __shared__ float As[KT][LP];  // As[k][m]
  __shared__ float Bs[KT][LP];  // Bs[k][n]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int row0 = blockIdx.y * MT, col0 = blockIdx.x * MT;
  const int kb = blockIdx.z * kchunk, ke = min(kb + kchunk, a.w);
  // staging maps: 8 elements per thread per matrix, consecutive along the
  // unit-stride dimension when there is one
  const bool a_krow = a.sw == 1 || a.sh != 1;  // a's k dimension is the contiguous one (or neither)
  const bool b_nrow = b.sw == 1 || b.sh != 1;
  const int am = a_krow ? tid >> 2 : (tid & 7) * 8, ak = a_krow ? (tid & 3) * 8 : tid >> 3;
  const int bk = b_nrow ? tid >> 3 : (tid & 3) * 8, bn = b_nrow ? (tid & 7) * 8 : tid >> 2;
  float ra[8], rb[8];
  auto gload = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int m = row0 + am + (a_krow ? 0 : e), k = k0 + ak + (a_krow ? e : 0);
      ra[e] = (m < a.h && k < ke) ? a.at(m, k) : 0.f;
      const int kk = k0 + bk + (b_nrow ? 0 : e), n = col0 + bn + (b_nrow ? e : 0);
      rb[e] = (kk < ke && n < b.w) ? b.at(kk, n) : 0.f;
    }
  };
  auto lstore = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      As[ak + (a_krow ? e : 0)][am + (a_krow ? 0 : e)] = ra[e];
      Bs[bk + (b_nrow ? 0 : e)][bn + (b_nrow ? e : 0)] = rb[e];
    }
  };
  mf32x16_t acc = {};
  if (kb < ke) gload(kb);
  for (int k0 = kb; k0 < ke; k0 += KT) {
    __syncthreads();  // previous step's operand reads are done
    lstore();
    __syncthreads();
    if (k0 + KT < ke) gload(k0 + KT);
#pragma unroll
    for (int kk = 0; kk < KT; kk += 2) {
      const float av = As[kk + (lane >> 5)][wm * 32 + (lane & 31)];
      const float bv = Bs[kk + (lane >> 5)][wn * 32 + (lane & 31)];
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc, 0, 0, 0);
    }
  }
  const int n = col0 + wn * 32 + (lane & 31);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int m = row0 + wm * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
    if (m < c.h && n < c.w) {
      if (part)
        part[((int64_t)blockIdx.z * c.h + m) * c.w + n] = acc[i];
      else
        c.at(m, n) = acc[i];
    }
  }
}

// c = sum over the k slabs, slab 0 first
__global__ __launch_bounds__(256) void matmul_reduce_kernel(const float *part, int nsplit,
                                                            DView<float> c) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t mn = (int64_t)c.h * c.w;
  if (idx >= mn) return;
  float s = 0.f;
  for (int z = 0; z < nsplit; ++z) s += part[z * mn + idx];
  c.at((int)(idx / c.w), (int)(idx % c.w)) = s;
}

// ---------------------------------------------------------- elementwise
template <typename T>
__global__ void repeat_kv_kernel(DView<const T> kv, DView<T> out, int head_dim, int n_rep) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)out.h * out.w) return;
  const int r = (int)(idx / out.w), c = (int)(idx % out.w);
  const int dst_head = c / head_dim, d = c % head_dim;
  // destination head kv_h*n_rep + rep reads source head kv_h (llama_layers.hpp:159-163)
  out.at(r, c) = kv.at(r, (dst_head / n_rep) * head_dim + d);
}

__device__ __forceinline__ float b_at(const DView<const float> &b, int i, int j) {
  if (b.h == 1) return b.at(0, j);  // op_elemwise.cuh:232-238
  if (b.w == 1) return b.at(i, 0);
  return b.at(i, j);
}

__global__ void binary_kernel(int op, DView<const float> a, DView<const float> b, DView<float> y,
                              DView<uint32_t> yu) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)a.h * a.w) return;
  const int i = (int)(idx / a.w), j = (int)(idx % a.w);
  const float x = a.at(i, j), z = b_at(b, i, j);
  switch (op) {
    case BN_ADD: y.at(i, j) = x + z; break;
    case BN_SUB: y.at(i, j) = x - z; break;
    case BN_MUL: y.at(i, j) = x * z; break;
    default: yu.at(i, j) = (x == z) ? 1u : 0u; break;
  }
}

__global__ void binary_u32_kernel(int op, DView<const uint32_t> a, DView<const uint32_t> b,
                                  DView<uint32_t> y) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)a.h * a.w) return;
  const int i = (int)(idx / a.w), j = (int)(idx % a.w);
  const uint32_t x = a.at(i, j);
  const uint32_t z = b.h == 1 ? b.at(0, j) : (b.w == 1 ? b.at(i, 0) : b.at(i, j));
  switch (op) {
    case BN_ADD: y.at(i, j) = x + z; break;
    case BN_SUB: y.at(i, j) = x - z; break;
    case BN_MUL: y.at(i, j) = x * z; break;
    default: y.at(i, j) = (x == z) ? 1u : 0u; break;
  }
}

__global__ void unary_kernel(int op, DView<const float> x, float c, DView<float> y) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)x.h * x.w) return;
  const int i = (int)(idx / x.w), j = (int)(idx % x.w);
  const float v = x.at(i, j);
  float r;
  switch (op) {
    case BN_RELU: r = v > 0.f ? v : 0.f; break;               // ReluFunc
    case BN_SILU: r = v / (1.0f + expf(-v)); break;           // op_silu.cuh SiLUFunc
    case BN_ADD_SCALAR: r = v + c; break;                     // AddConstFunc
    default: r = c * v; break;                                // MultiplyConstFunc
  }
  y.at(i, j) = r;
}

__global__ void unary_backward_kernel(int op, DView<const float> x, DView<const float> dy,
                                      DView<float> dx) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)x.h * x.w) return;
  const int i = (int)(idx / x.w), j = (int)(idx % x.w);
  const float v = x.at(i, j), g = dy.at(i, j);
  if (op == BN_RELU_BACK) {
    dx.at(i, j) = v > 0.f ? g : 0.f;
  } else {
    float sg = 1.0f / (1.0f + expf(-v));
    dx.at(i, j) = g * (sg + v * (sg * (1.0f - sg)));
  }
}

template <typename T>
__global__ void fill_kernel(DView<T> y, T v) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)y.h * y.w) return;
  y.at((int)(idx / y.w), (int)(idx % y.w)) = v;
}

// Uniform [lo, hi) fill from a counter-based generator: element (i, j) of an
// h x w view gets the SplitMix64 output (Steele, Lea & Flood, "Fast
// splittable pseudorandom number generators", OOPSLA 2014) of
// seed + (i*w + j + 1) * 0x9E3779B97F4A7C15, whose top 24 bits scale to
// [0, 1).  The value depends only on (seed, logical index): the same for any
// launch shape, stride or device.
__device__ __forceinline__ float uniform01(uint64_t seed, uint64_t index) {
  uint64_t z = seed + (index + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  return (float)(uint32_t)(z >> 40) * (1.0f / 16777216.0f);
}

template <typename T>
__global__ void fill_uniform_kernel(DView<T> y, float lo, float span, uint64_t seed) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)y.h * y.w) return;
  const float v = fmaf(uniform01(seed, (uint64_t)idx), span, lo);
  Elem<T>::store(&y.at((int)(idx / y.w), (int)(idx % y.w)), v);
}

template <typename Tin, typename Tout>
__global__ void copy_kernel(DView<const Tin> x, DView<Tout> y) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)x.h * x.w) return;
  const int i = (int)(idx / x.w), j = (int)(idx % x.w);
  if constexpr (std::is_same<Tin, Tout>::value)
    y.at(i, j) = x.at(i, j);
  else
    Elem<Tout>::store(&y.at(i, j), Elem<Tin>::load(&x.at(i, j)));
}

// op_reduction_kernel_colwise / _rowwise: sequential accumulation from
// element 0 (op_reduction.cuh:36-92); argmax keeps the first maximum.
template <typename T>
__global__ void sum_kernel(DView<const T> x, DView<T> y, int axis) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (axis == 0) {
    if (idx >= x.w) return;
    T acc = x.at(0, idx);
    for (int r = 1; r < x.h; ++r) acc = x.at(r, idx) + acc;
    y.at(0, idx) = acc;
  } else {
    if (idx >= x.h) return;
    T acc = x.at(idx, 0);
    for (int c = 1; c < x.w; ++c) acc = x.at(idx, c) + acc;
    y.at(idx, 0) = acc;
  }
}

// argmax: one workgroup per row.  The sequential rule (accumulator starts at
// column 0, takes x when x > accumulator) returns column 0 when x[0] is NaN
// (nothing compares greater) and otherwise the first column holding the
// largest non-NaN value (a NaN elsewhere never compares greater).  Each
// thread scans columns t, t + 256, ... keeping its first maximum; the
// candidates merge by larger value, then smaller column -- the same answer.
template <typename T>
__device__ __forceinline__ bool is_nan_val(T v) {
  if constexpr (std::is_same<T, float>::value) return v != v;
  else return false;
}

template <typename T>
__global__ __launch_bounds__(256) void argmax_kernel(DView<const T> x, DView<uint32_t> y) {
  constexpr uint32_t NONE = 0xffffffffu;
  __shared__ T sv[256];
  __shared__ uint32_t si[256];
  const int r = blockIdx.x, t = threadIdx.x;
  if (is_nan_val(x.at(r, 0))) {
    if (t == 0) y.at(r, 0) = 0;
    return;
  }
  T best = T{};
  uint32_t bi = NONE;
  constexpr int U = 8;  // loads in flight per thread; columns still visited in order
  for (int c0 = t; c0 < x.w; c0 += 256 * U) {
    T v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = c0 + 256 * u < x.w ? x.at(r, c0 + 256 * u) : T{};
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + 256 * u;
      if (c < x.w && !is_nan_val(v[u]) && (bi == NONE || v[u] > best)) {
        best = v[u];
        bi = (uint32_t)c;
      }
    }
  }
  sv[t] = best;
  si[t] = bi;
  __syncthreads();
  for (int half = 128; half > 0; half >>= 1) {
    if (t < half) {
      const T v = sv[t + half];
      const uint32_t i = si[t + half];
      // equal values: the smaller column wins
      if (i != NONE && (si[t] == NONE || v > sv[t] || (v == sv[t] && i < si[t]))) {
        sv[t] = v;
        si[t] = i;
      }
    }
    __syncthreads();
  }
  if (t == 0) y.at(r, 0) = si[0];
}

// argmax of contiguous fp32 rows (16-byte aligned, width a multiple of 4):
// 1024 threads, each scanning 16-byte chunks t, t + 1024, ... in column
// order with four chunks in flight (two rounds for a 32000-wide row), x[0]
// loaded with the first round instead of before it; the candidates merge
// by the same rule as argmax_kernel (larger value, then smaller column),
// by wave shuffles and one LDS step.
__global__ __launch_bounds__(1024) void argmax_rows_f32_kernel(const float *x, int64_t rs, int w,
                                                               uint32_t *y, int64_t ys) {
  constexpr uint32_t NONE = 0xffffffffu;
  constexpr int U = 4;
  __shared__ float sv[16];
  __shared__ uint32_t si[16];
  const int r = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const float *row = x + (int64_t)r * rs;
  const int nch = w / 4;
  const float x0 = row[0];
  float best = 0.f;
  uint32_t bi = NONE;
  for (int c0 = t; c0 < nch; c0 += 1024 * U) {
    float4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = *(const float4 *)(row + 4 * min(c0 + 1024 * u, nch - 1));
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + 1024 * u;
      const float e4[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (c < nch && !(e4[e] != e4[e]) && (bi == NONE || e4[e] > best)) {
          best = e4[e];
          bi = (uint32_t)(4 * c + e);
        }
    }
  }
  // (v, i) beats (bv, bidx): a candidate against none, a larger value, or an
  // equal value at a smaller column -- a total order, so both lanes of a
  // butterfly pair keep the same winner
  auto merge = [&](int width) {
    for (int m = width; m >= 1; m >>= 1) {
      const float ov = __shfl_xor(best, m, 64);
      const uint32_t oi = (uint32_t)__shfl_xor((int)bi, m, 64);
      if (oi != NONE && (bi == NONE || ov > best || (ov == best && oi < bi))) {
        best = ov;
        bi = oi;
      }
    }
  };
  merge(32);
  if (lane == 0) {
    sv[wave] = best;
    si[wave] = bi;
  }
  __syncthreads();
  if (wave > 0) return;
  best = lane < 16 ? sv[lane] : 0.f;
  bi = lane < 16 ? si[lane] : NONE;
  merge(8);
  if (lane == 0) y[(int64_t)r * ys] = x0 != x0 ? 0u : bi;  // NaN at column 0: column 0
}

inline dim3 grid1d(int64_t n) { return dim3((unsigned)((n + 255) / 256)); }

// Plain GEMMs (each operand row-major or a transposed view, output row-major)
// go to rocBLAS's fp32 GEMM; other strided views take matmul_kernel.  One
// rocBLAS handle per thread, bound to the library's device.
bool unit_stride(const bn_view *v, bool &transposed, int64_t &ld) {
  if (v->stride_w == 1 && v->stride_h >= v->w) {
    transposed = false;
    ld = v->stride_h;
    return ld >= 1;
  }
  if (v->stride_h == 1 && v->stride_w >= v->h) {
    transposed = true;
    ld = v->stride_w;
    return ld >= 1;
  }
  return false;
}

int blas_gemm(const bn_view *a, const bn_view *b, const bn_view *c, hipStream_t s, bool &done) {
  done = false;
  bool ta, tb, tc;
  int64_t lda, ldb, ldc;
  if (!unit_stride(a, ta, lda) || !unit_stride(b, tb, ldb) || !unit_stride(c, tc, ldc) || tc)
    return BN_OK;
  if (lda > INT32_MAX || ldb > INT32_MAX || ldc > INT32_MAX) return BN_OK;
  thread_local rocblas_handle handle = nullptr;
  if (!handle) {
    if (rocblas_create_handle(&handle) != rocblas_status_success) {
      handle = nullptr;
      return fail(BN_ERR_HIP, "Matrix multiply: rocblas_create_handle failed");
    }
  }
  if (rocblas_set_stream(handle, s) != rocblas_status_success)
    return fail(BN_ERR_HIP, "Matrix multiply: rocblas_set_stream failed");
  // row-major C = A B  <=>  column-major C^T = B^T A^T; a row-major view is
  // its transpose in column-major, a transposed view needs op T
  const float one = 1.f, zero = 0.f;
  const float *ap = (const float *)a->data + a->offset;
  const float *bp = (const float *)b->data + b->offset;
  float *cp = (float *)c->data + c->offset;
  const rocblas_status r =
      rocblas_sgemm(handle, tb ? rocblas_operation_transpose : rocblas_operation_none,
                    ta ? rocblas_operation_transpose : rocblas_operation_none, c->w, c->h, a->w,
                    &one, bp, (rocblas_int)ldb, ap, (rocblas_int)lda, &zero, cp,
                    (rocblas_int)ldc);
  if (r != rocblas_status_success)
    return fail(BN_ERR_HIP, std::string("Matrix multiply: rocblas_sgemm: ") +
                                rocblas_status_to_string(r));
  done = true;
  return BN_OK;
}

}  // namespace
}  // namespace bn

using namespace bn;

extern "C" {

int bn_softmax(const bn_view *x, const bn_view *y, int causal, int seq_offset, void *stream) {
  const unsigned mask = (1u << BN_F32) | (1u << BN_BF16);
  int st;
  if ((st = check_view(x, "Softmax", "input", mask))) return st;
  if ((st = check_view(y, "Softmax", "output", mask))) return st;
  if (!same_shape(x, y)) return fail(BN_ERR_SHAPE, "Softmax: input/output shape mismatch");
  if (x->dtype != y->dtype) return fail(BN_ERR_UNSUPPORTED, "Softmax: input and output dtypes differ");
  if ((st = require_device("Softmax", {x, y}))) return st;
  if ((st = ensure_device())) return st;
  if (x->h == 0) return BN_OK;
  hipStream_t s = as_stream(stream);
  if (x->dtype == BN_F32)
    hipLaunchKernelGGL(softmax_kernel<float>, dim3(x->h), dim3(256), 0, s, dview<const float>(x),
                       dview<float>(y), causal ? 1 : 0, seq_offset);
  else
    hipLaunchKernelGGL(softmax_kernel<bf16_t>, dim3(x->h), dim3(256), 0, s,
                       dview<const bf16_t>(x), dview<bf16_t>(y), causal ? 1 : 0, seq_offset);
  BN_LAUNCH_CHECK();
  return BN_OK;
}

int bn_softmax_backward(const bn_view *y, const bn_view *dy, const bn_view *dx, void *stream) {
  const unsigned mask = 1u << BN_F32;
  int st;
  if ((st = check_view(y, "Softmax backward", "output", mask))) return st;
  if ((st = check_view(dy, "Softmax backward", "grad_output", mask))) return st;
  if ((st = check_view(dx, "Softmax backward", "grad_input", mask))) return st;
  if (!same_shape(y, dy) || !same_shape(y, dx))
    return fail(BN_ERR_SHAPE, "Softmax backward: shape mismatch");
  if ((st = require_device("Softmax backward", {y, dy, dx}))) return st;
  if ((st = ensure_device())) return st;
  if (y->h == 0) return BN_OK;
  hipLaunchKernelGGL(softmax_backward_kernel, dim3(y->h), dim3(256), 0, as_stream(stream),
                     dview<const float>(y), dview<const float>(dy), dview<float>(dx));
  BN_LAUNCH_CHECK();
  return BN_OK;
}

int bn_matmul(const bn_view *a, const bn_view *b, const bn_view *c, void *stream) {
  const unsigned mask = 1u << BN_F32;
  int st;
  if ((st = check_view(a, "Matrix multiply", "a", mask))) return st;
  if ((st = check_view(b, "Matrix multiply", "b", mask))) return st;
  if ((st = check_view(c, "Matrix multiply", "out", mask))) return st;
  if (a->h != c->h || b->w != c->w || a->w != b->h)  // op_mm.cuh:13-15
    return fail(BN_ERR_SHAPE, "a,b,out tensor shape mismatch a:(" + std::to_string(a->h) + ", " +
                                  std::to_string(a->w) + "), b:(" + std::to_string(b->h) + ", " +
                                  std::to_string(b->w) + "), out:(" + std::to_string(c->h) +
                                  ", " + std::to_string(c->w) + ")");
  if ((st = require_device("Matrix multiply", {a, b, c}))) return st;
  if ((st = ensure_device())) return st;
  if (c->h == 0 || c->w == 0) return BN_OK;
  if (a->w > 0) {
    bool done = false;
    if ((st = blas_gemm(a, b, c, as_stream(stream), done))) return st;
    if (done) return BN_OK;
  }
  const int tiles = ((c->w + MT - 1) / MT) * ((c->h + MT - 1) / MT);
  // split k while the grid is small and every slab keeps >= 128 of k
  int nsplit = 1;
  while (nsplit < 16 && tiles * nsplit < 256 && a->w / (2 * nsplit) >= 128) nsplit *= 2;
  const int kchunk = ((a->w + nsplit - 1) / nsplit + KT - 1) / KT * KT;
  nsplit = a->w == 0 ? 1 : (a->w + kchunk - 1) / kchunk;
  hipStream_t s = as_stream(stream);
  float *part = nullptr;
  if (nsplit > 1) {
    void *ws = nullptr;
    if ((st = bn_alloc(&ws, (size_t)nsplit * c->h * c->w * sizeof(float), stream))) return st;
    part = (float *)ws;
  }
  dim3 grid((c->w + MT - 1) / MT, (c->h + MT - 1) / MT, nsplit);
  hipLaunchKernelGGL(matmul_kernel, grid, dim3(256), 0, s, dview<const float>(a),
                     dview<const float>(b), dview<float>(c), part, kchunk > 0 ? kchunk : KT);
  hipError_t e = hipGetLastError();
  st = e == hipSuccess ? BN_OK : hip_fail(e, __FILE__, __LINE__);
  if (st == BN_OK && part) {
    const int64_t mn = (int64_t)c->h * c->w;
    hipLaunchKernelGGL(matmul_reduce_kernel, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, s,
                       part, nsplit, dview<float>(c));
    e = hipGetLastError();
    st = e == hipSuccess ? BN_OK : hip_fail(e, __FILE__, __LINE__);
  }
  if (part) {
    const int st2 = bn_free(part, stream);
    if (st == BN_OK) st = st2;
  }
  return st;
}

int bn_repeat_kv(const bn_view *kv, const bn_view *out, int head_dim, int n_rep, void *stream) {
  const unsigned mask = (1u << BN_F32) | (1u << BN_BF16);
  int st;
  if ((st = check_view(kv, "repeat_kv", "kv", mask))) return st;
  if ((st = check_view(out, "repeat_kv", "out", mask))) return st;
  if (head_dim <= 0 || n_rep <= 0 || kv->w % head_dim != 0)
    return fail(BN_ERR_SHAPE, "repeat_kv: kv width must be a multiple of head_dim");
  if (out->h != kv->h || (int64_t)out->w != (int64_t)kv->w * n_rep)
    return fail(BN_ERR_SHAPE, "repeat_kv: out must be [rows, kv_width * n_rep]");
  if (kv->dtype != out->dtype) return fail(BN_ERR_UNSUPPORTED, "repeat_kv: dtypes differ");
  if ((st = require_device("repeat_kv", {kv, out}))) return st;
  if ((st = ensure_device())) return st;
  const int64_t n = (int64_t)out->h * out->w;
  if (n == 0) return BN_OK;
  if (kv->dtype == BN_F32)
    hipLaunchKernelGGL(repeat_kv_kernel<float>, grid1d(n), dim3(256), 0, as_stream(stream),
                       dview<const float>(kv), dview<float>(out), head_dim, n_rep);
  else
    hipLaunchKernelGGL(repeat_kv_kernel<bf16_t>, grid1d(n), dim3(256), 0, as_stream(stream),
                       dview<const bf16_t>(kv), dview<bf16_t>(out), head_dim, n_rep);
  BN_LAUNCH_CHECK();
  return BN_OK;
}

int bn_binary(int op, const bn_view *a, const bn_view *b, const bn_view *y, void *stream) {
  if (op < BN_ADD || op > BN_EQ) return fail(BN_ERR_INVALID_ARG, "bn_binary: unknown op");
  const unsigned mask = (1u << BN_F32) | (1u << BN_U32);
  int st;
  if ((st = check_view(a, "elementwise", "a", mask))) return st;
  if ((st = check_view(b, "elementwise", "b", mask))) return st;
  if ((st = check_view(y, "elementwise", "out", mask))) return st;
  if (!same_shape(a, y)) return fail(BN_ERR_SHAPE, "out, a tensor shape mismatch");
  bool ok = (a->h == b->h && a->w == b->w) || (a->h == b->h && b->w == 1) ||
            (a->w == b->w && b->h == 1);  // ensure_bcast_shape_device, op_elemwise.cuh:294-300
  if (!ok) return fail(BN_ERR_SHAPE, "a,b shape mismatch");
  if (a->dtype != b->dtype) return fail(BN_ERR_UNSUPPORTED, "elementwise: a and b dtypes differ");
  const int want_out = (op == BN_EQ) ? BN_U32 : a->dtype;
  if (y->dtype != want_out) return fail(BN_ERR_UNSUPPORTED, "elementwise: wrong output dtype");
  if ((st = require_device("elementwise", {a, b, y}))) return st;
  if ((st = ensure_device())) return st;
  const int64_t n = (int64_t)a->h * a->w;
  if (n == 0) return BN_OK;
  hipStream_t s = as_stream(stream);
  if (a->dtype == BN_F32) {
    DView<float> yf = dview<float>(y);
    DView<uint32_t> yu = dview<uint32_t>(y);
    hipLaunchKernelGGL(binary_kernel, grid1d(n), dim3(256), 0, s, op, dview<const float>(a),
                       dview<const float>(b), yf, yu);
  } else {
    hipLaunchKernelGGL(binary_u32_kernel, grid1d(n), dim3(256), 0, s, op,
                       dview<const uint32_t>(a), dview<const uint32_t>(b), dview<uint32_t>(y));
  }
  BN_LAUNCH_CHECK();
  return BN_OK;
}

int bn_unary(int op, const bn_view *x, float scalar, const bn_view *y, void *stream) {
  if (op < BN_RELU || op > BN_MUL_SCALAR) return fail(BN_ERR_INVALID_ARG, "bn_unary: unknown op");
  const unsigned mask = 1u << BN_F32;
  int st;
  if ((st = check_view(x, "elementwise", "input", mask))) return st;
  if ((st = check_view(y, "elementwise", "output", mask))) return st;
  if (!same_shape(x, y)) return fail(BN_ERR_SHAPE, "out, a tensor shape mismatch");
  if ((st = require_device("elementwise", {x, y}))) return st;
  if ((st = ensure_device())) return st;
  const int64_t n = (int64_t)x->h * x->w;
  if (n == 0) return BN_OK;
  hipLaunchKernelGGL(unary_kernel, grid1d(n), dim3(256), 0, as_stream(stream), op,
                     dview<const float>(x), scalar, dview<float>(y));
  BN_LAUNCH_CHECK();
  return BN_OK;
}

int bn_unary_backward(int op, const bn_view *x, const bn_view *dy, const bn_view *dx,
                      void *stream) {
  if (op != BN_RELU_BACK && op != BN_SILU_BACK)
    return fail(BN_ERR_INVALID_ARG, "bn_unary_backward: unknown op");
  const unsigned mask = 1u << BN_F32;
  int st;
  if ((st = check_view(x, "elementwise backward", "input", mask))) return st;
  if ((st = check_view(dy, "elementwise backward", "grad_output", mask))) return st;
  if ((st = check_view(dx, "elementwise backward", "grad_input", mask))) return st;
  if (!same_shape(x, dy) || !same_shape(x, dx)) return fail(BN_ERR_SHAPE, "elementwise backward: shape mismatch");
  if ((st = require_device("elementwise backward", {x, dy, dx}))) return st;
  if ((st = ensure_device())) return st;
  const int64_t n = (int64_t)x->h * x->w;
  if (n == 0) return BN_OK;
  hipLaunchKernelGGL(unary_backward_kernel, grid1d(n), dim3(256), 0, as_stream(stream), op,
                     dview<const float>(x), dview<const float>(dy), dview<float>(dx));
  BN_LAUNCH_CHECK();
  return BN_OK;
}

int bn_fill(const bn_view *y, double value, void *stream) {
  const unsigned mask = (1u << BN_F32) | (1u << BN_BF16) | (1u << BN_U32);
  int st;
  if ((st = check_view(y, "fill", "tensor", mask))) return st;
  if ((st = require_device("fill", {y}))) return st;
  if ((st = ensure_device())) return st;
  const int64_t n = (int64_t)y->h * y->w;
  if (n == 0) return BN_OK;
  hipStream_t s = as_stream(stream);
  if (y->dtype == BN_F32) {
    hipLaunchKernelGGL(fill_kernel<float>, grid1d(n), dim3(256), 0, s, dview<float>(y), (float)value);
  } else if (y->dtype == BN_U32) {
    hipLaunchKernelGGL(fill_kernel<uint32_t>, grid1d(n), dim3(256), 0, s, dview<uint32_t>(y),
                       (uint32_t)value);
  } else {
    float f = (float)value;
    uint32_t u;
    std::memcpy(&u, &f, 4);
    u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even (finite values)
    hipLaunchKernelGGL(fill_kernel<bf16_t>, grid1d(n), dim3(256), 0, s, dview<bf16_t>(y),
                       (bf16_t)(u >> 16));
  }
  BN_LAUNCH_CHECK();
  return BN_OK;
}

int bn_fill_uniform(const bn_view *y, float lo, float hi, uint64_t seed, void *stream) {
  const unsigned mask = (1u << BN_F32) | (1u << BN_BF16);
  int st;
  if ((st = check_view(y, "uniform fill", "tensor", mask))) return st;
  if (!std::isfinite(lo) || !std::isfinite(hi) || !(hi > lo))
    return fail(BN_ERR_INVALID_ARG, "uniform fill: need finite lo < hi");
  if ((st = require_device("uniform fill", {y}))) return st;
  if ((st = ensure_device())) return st;
  const int64_t n = (int64_t)y->h * y->w;
  if (n == 0) return BN_OK;
  hipStream_t s = as_stream(stream);
  if (y->dtype == BN_F32)
    hipLaunchKernelGGL(fill_uniform_kernel<float>, grid1d(n), dim3(256), 0, s, dview<float>(y), lo,
                       hi - lo, seed);
  else
    hipLaunchKernelGGL(fill_uniform_kernel<bf16_t>, grid1d(n), dim3(256), 0, s, dview<bf16_t>(y),
                       lo, hi - lo, seed);
  BN_LAUNCH_CHECK();
  return BN_OK;
}

int bn_sum(const bn_view *x, const bn_view *y, int axis, void *stream) {
  const unsigned mask = (1u << BN_F32) | (1u << BN_U32);
  int st;
  if ((st = check_view(x, "sum", "input", mask))) return st;
  if ((st = check_view(y, "sum", "output", mask))) return st;
  if (axis != 0 && axis != 1) return fail(BN_ERR_INVALID_ARG, "Invalid axis, must be 0 or 1");
  if (x->dtype != y->dtype) return fail(BN_ERR_UNSUPPORTED, "sum: dtypes differ");
  if ((axis == 0 && (y->h != 1 || y->w != x->w)) || (axis == 1 && (y->w != 1 || y->h != x->h)))
    return fail(BN_ERR_SHAPE, "sum: output shape mismatch");
  if ((st = require_device("sum", {x, y}))) return st;
  if ((st = ensure_device())) return st;
  const int n = axis == 0 ? x->w : x->h;
  if (n == 0 || x->h == 0 || x->w == 0) return BN_OK;
  if (x->dtype == BN_F32)
    hipLaunchKernelGGL(sum_kernel<float>, grid1d(n), dim3(256), 0, as_stream(stream),
                       dview<const float>(x), dview<float>(y), axis);
  else
    hipLaunchKernelGGL(sum_kernel<uint32_t>, grid1d(n), dim3(256), 0, as_stream(stream),
                       dview<const uint32_t>(x), dview<uint32_t>(y), axis);
  BN_LAUNCH_CHECK();
  return BN_OK;
}

int bn_argmax(const bn_view *x, const bn_view *y, void *stream) {
  int st;
  if ((st = check_view(x, "argmax", "input", (1u << BN_F32) | (1u << BN_U32)))) return st;
  if ((st = check_view(y, "argmax", "output", 1u << BN_U32))) return st;
  if (y->h != x->h || y->w != 1) return fail(BN_ERR_SHAPE, "argmax: output must be (rows, 1)");
  if ((st = require_device("argmax", {x, y}))) return st;
  if ((st = ensure_device())) return st;
  if (x->h == 0 || x->w == 0) return BN_OK;
  if (x->h > 0x7fffffff) return fail(BN_ERR_UNSUPPORTED, "argmax: too many rows");
  if (x->dtype == BN_F32 && rows_aligned(x, 16) && x->w % 4 == 0)
    hipLaunchKernelGGL(argmax_rows_f32_kernel, dim3((unsigned)x->h), dim3(1024), 0, as_stream(stream),
                       (const float *)x->data + x->offset, (int64_t)x->stride_h, (int)x->w,
                       (uint32_t *)y->data + y->offset, (int64_t)y->stride_h);
  else if (x->dtype == BN_F32)
    hipLaunchKernelGGL(argmax_kernel<float>, dim3((unsigned)x->h), dim3(256), 0, as_stream(stream),
                       dview<const float>(x), dview<uint32_t>(y));
  else
    hipLaunchKernelGGL(argmax_kernel<uint32_t>, dim3((unsigned)x->h), dim3(256), 0, as_stream(stream),
                       dview<const uint32_t>(x), dview<uint32_t>(y));
  BN_LAUNCH_CHECK();
  return BN_OK;
}

int bn_copy(const bn_view *x, const bn_view *y, void *stream) {
  const unsigned mask = (1u << BN_F32) | (1u << BN_BF16) | (1u << BN_U32);
  int st;
  if ((st = check_view(x, "copy", "input", mask))) return st;
  if ((st = check_view(y, "copy", "output", mask))) return st;
  if (!same_shape(x, y)) return fail(BN_ERR_SHAPE, "copy: shape mismatch");
  if ((x->dtype == BN_U32) != (y->dtype == BN_U32))
    return fail(BN_ERR_UNSUPPORTED, "copy: U32 converts to U32 only");
  if ((st = require_device("copy", {x, y}))) return st;
  if ((st = ensure_device())) return st;
  const int64_t n = (int64_t)x->h * x->w;
  if (n == 0) return BN_OK;
  hipStream_t s = as_stream(stream);
  dim3 g = grid1d(n);
  if (x->dtype == BN_U32)
    hipLaunchKernelGGL((copy_kernel<uint32_t, uint32_t>), g, dim3(256), 0, s,
                       dview<const uint32_t>(x), dview<uint32_t>(y));
  else if (x->dtype == BN_F32 && y->dtype == BN_F32)
    hipLaunchKernelGGL((copy_kernel<float, float>), g, dim3(256), 0, s, dview<const float>(x),
                       dview<float>(y));
  else if (x->dtype == BN_F32)
    hipLaunchKernelGGL((copy_kernel<float, bf16_t>), g, dim3(256), 0, s, dview<const float>(x),
                       dview<bf16_t>(y));
  else if (y->dtype == BN_F32)
    hipLaunchKernelGGL((copy_kernel<bf16_t, float>), g, dim3(256), 0, s, dview<const bf16_t>(x),
                       dview<float>(y));
  else
    hipLaunchKernelGGL((copy_kernel<bf16_t, bf16_t>), g, dim3(256), 0, s,
                       dview<const bf16_t>(x), dview<bf16_t>(y));
  BN_LAUNCH_CHECK();
  return BN_OK;
}

}  // extern "C"
