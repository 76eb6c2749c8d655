// bn_norm_rope.hip -- RMSNorm, RoPE and the fused RMSNorm->RoPE kernel.
//
// Reference kernels replaced: op_rmsnorm_kernel (src/ops/op_rmsnorm.cuh:8-53),
// op_rmsnorm_backward_kernel (:55-133), op_rope_kernel_simple
// (src/ops/op_rope.cuh:55-99), op_rope_backward_kernel (:128-169).
//
// Fast path (rows contiguous and 16-byte aligned, which is every layer
// tensor): one 64-lane wave per row, 16-byte vector loads, the row held in
// registers between the sum of squares and the write (one HBM read, one HBM
// write per element).  RoPE angles: position*freq in fp32 as the reference
// forms them (op_rope.cuh:82-83), sin/cos from the accurate device libm.
// Any other view (transposes, column slices, odd widths) takes a strided
// path with one workgroup per row.
#include <algorithm>

#include "bn_common.hpp"

namespace bn {
namespace {

// 16-byte chunk <-> VEC floats
template <typename T> struct Chunk;
typedef uint32_t raw16_t __attribute__((ext_vector_type(4)));  // one 16-byte chunk
__device__ __forceinline__ raw16_t load_raw(const void *p) { return *reinterpret_cast<const raw16_t *>(p); }
// Outputs written once are stored non-temporal (kept out of L2/MALL); the
// SwiGLU inputs, two streams read once, are loaded non-temporal too.
// Measured on bf16 [16384, 2048] / [16384, 5632]: non-temporal stores +1.5%
// (RMSNorm+RoPE), +14% (residual add + RMSNorm), +5% (SwiGLU); non-temporal
// loads +7% on SwiGLU but -14% on RMSNorm+RoPE, whose 67 MB input stays in
// the 256 MB MALL, and -5% on the residual add with the stores also
// non-temporal.
__device__ __forceinline__ raw16_t load_stream(const void *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const raw16_t *>(p));
}
__device__ __forceinline__ void store_stream(void *p, raw16_t v) {
  __builtin_nontemporal_store(v, reinterpret_cast<raw16_t *>(p));
}

template <> struct Chunk<float> {
  static constexpr int VEC = 4;
  __device__ static __forceinline__ void cvt(raw16_t t, float (&v)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(t[i]);
  }
  __device__ static __forceinline__ void load(const float *p, float (&v)[4]) {
    float4 t = *reinterpret_cast<const float4 *>(p);
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
  }
  __device__ static __forceinline__ void store(float *p, const float (&v)[4]) {
    store_stream(p, raw16_t{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                            __float_as_uint(v[3])});
  }
};
template <> struct Chunk<bf16_t> {
  static constexpr int VEC = 8;
  __device__ static __forceinline__ void cvt(raw16_t t, float (&v)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(t[i] << 16);
      v[2 * i + 1] = __uint_as_float(t[i] & 0xffff0000u);
    }
  }
  __device__ static __forceinline__ void load(const bf16_t *p, float (&v)[8]) {
    uint4 t = *reinterpret_cast<const uint4 *>(p);
    uint32_t u[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(u[i] << 16);
      v[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
    }
  }
  __device__ static __forceinline__ void store(bf16_t *p, const float (&v)[8]) {
    uint32_t u[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      u[i] = (uint32_t)f32_to_bf16(v[2 * i]) | ((uint32_t)f32_to_bf16(v[2 * i + 1]) << 16);
    store_stream(p, raw16_t{u[0], u[1], u[2], u[3]});
  }
};

constexpr int kRowsPerBlock = 4;  // 4 waves, one row each
constexpr int kMaxChunks = 8;     // chunks per lane kept in registers (at most)
static_assert(64 * kMaxChunks * 4 == kNormRowF32, "fp32 rows of the one-wave kernels");

// y = rope?(x / rms * w); requires cols % VEC == 0, cols <= 64*NCH*VEC,
// head_dim % VEC == 0 when ROPE.  NCH = 16-byte chunks per lane.
template <typename T, bool ROPE, int NCH>
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(
    const T *__restrict__ x, int64_t x_rs, const T *__restrict__ w, int64_t w_off,
    T *__restrict__ y, int64_t y_rs, int rows, int cols, float eps, int pos_off,
    int head_dim, RopeFreqs freqs) {
  constexpr int VEC = Chunk<T>::VEC;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T *xr = x + (int64_t)row * x_rs;
  const int nchunks = cols / VEC;
  // every x and weight chunk of the row is requested before the first use
  // (clamped indices, no branch), so a short call pays one memory latency
  raw16_t xraw[NCH], wraw[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int cc = min(lane + 64 * i, nchunks - 1);
    xraw[i] = load_raw(xr + cc * VEC);
    wraw[i] = load_raw(w + w_off + cc * VEC);
  }
  float v[NCH][VEC];
  // sum of squares as one fma chain in element order (spelled out, so the
  // compiler cannot pick another contraction: projections that form this
  // norm in their own staging reproduce these bits)
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    Chunk<T>::cvt(xraw[i], v[i]);
    if (lane + 64 * i < nchunks) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) ss = fmaf(v[i][j], v[i][j], ss);
    }
  }
  ss = wave_sum(ss);
  const float mean_sq = ss / (float)cols;   // op_rmsnorm.cuh:44
  const float rms = sqrtf(mean_sq + eps);   // :45
  const float inv_rms = 1.0f / rms;
  T *yr = y + (int64_t)row * y_rs;
  const float pos = (float)(row + pos_off);
  int cached_p0 = -1;
  float cs[VEC / 2], sn[VEC / 2];
  // A row has head_dim/2 distinct angles.  When every chunk of a lane starts
  // at the same offset within its head (64*VEC a multiple of head_dim), lane
  // l evaluates angle l % (head_dim/2) once and each lane collects its VEC/2
  // angles from the lanes that hold them: one sincosf per lane instead of
  // VEC/2, the same values.
  if (ROPE && head_dim <= 128 && (64 * VEC) % head_dim == 0) {
    const int half = head_dim >> 1;
    float s1, c1;
    sincosf(pos * freqs.f[lane % half], &s1, &c1);  // op_rope.cuh:83
    const int p0 = ((lane * VEC) % head_dim) >> 1;
#pragma unroll
    for (int j = 0; j < VEC / 2; ++j) {
      sn[j] = __shfl(s1, p0 + j, 64);
      cs[j] = __shfl(c1, p0 + j, 64);
    }
    cached_p0 = p0;
  }
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    int c = lane + 64 * i;
    if (c < nchunks) {
      float wv[VEC];
      Chunk<T>::cvt(wraw[i], wv);
      float o[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) o[j] = (v[i][j] * inv_rms) * wv[j];
      if (ROPE) {
        int p0 = ((c * VEC) % head_dim) >> 1;
        if (p0 != cached_p0) {
#pragma unroll
          for (int j = 0; j < VEC / 2; ++j) {
            float ang = pos * freqs.f[p0 + j];  // op_rope.cuh:83
            sincosf(ang, &sn[j], &cs[j]);
          }
          cached_p0 = p0;
        }
#pragma unroll
        for (int j = 0; j < VEC / 2; ++j) {
          float x0 = o[2 * j], x1 = o[2 * j + 1];
          o[2 * j] = x0 * cs[j] - x1 * sn[j];      // op_rope.cuh:94
          o[2 * j + 1] = x0 * sn[j] + x1 * cs[j];  // :96
        }
      }
      Chunk<T>::store(yr + c * VEC, o);
    }
  }
}

// Residual add fused with the next RMSNorm (the decoder layer's
// h = x + delta; y = RMSNorm(h) * w, llama_layers.hpp:241-272): one wave per
// row, h written once and normalised from registers (bf16: the rounded h, as
// a separate add would store it).  h may alias x (in-place residual update):
// each lane reads its chunks before writing them.
template <typename T, int NCH>
__global__ __launch_bounds__(256) void add_rmsnorm_rows_kernel(
    const T *x, int64_t x_rs, const T *__restrict__ dlt, int64_t d_rs, const T *__restrict__ w,
    T *h, int64_t h_rs, T *__restrict__ y, int64_t y_rs, int rows, int cols, float eps) {
  constexpr int VEC = Chunk<T>::VEC;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nchunks = cols / VEC;
  raw16_t xraw[NCH], draw[NCH], wraw[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int cc = min(lane + 64 * i, nchunks - 1);
    xraw[i] = load_raw(x + (int64_t)row * x_rs + cc * VEC);
    draw[i] = load_raw(dlt + (int64_t)row * d_rs + cc * VEC);
    wraw[i] = load_raw(w + cc * VEC);
  }
  float v[NCH][VEC];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    float dv[VEC];
    Chunk<T>::cvt(xraw[i], v[i]);
    Chunk<T>::cvt(draw[i], dv);
#pragma unroll
    for (int j = 0; j < VEC; ++j) v[i][j] = Elem<T>::round(v[i][j] + dv[j]);
    if (lane + 64 * i < nchunks) {
      Chunk<T>::store(h + (int64_t)row * h_rs + (lane + 64 * i) * VEC, v[i]);
#pragma unroll
      for (int j = 0; j < VEC; ++j) ss = fmaf(v[i][j], v[i][j], ss);  // one fma chain, as above
    }
  }
  ss = wave_sum(ss);
  const float rms = sqrtf(ss / (float)cols + eps);  // op_rmsnorm.cuh:44-45
  const float inv_rms = 1.0f / rms;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = lane + 64 * i;
    if (c < nchunks) {
      float wv[VEC], o[VEC];
      Chunk<T>::cvt(wraw[i], wv);
#pragma unroll
      for (int j = 0; j < VEC; ++j) o[j] = (v[i][j] * inv_rms) * wv[j];
      Chunk<T>::store(y + (int64_t)row * y_rs + c * VEC, o);
    }
  }
}

// SwiGLU activation: out = silu(gate) * up with silu(g) = g / (1 + exp(-g))
// (op_silu.cuh:8-14 followed by op_multiply), one pass over 16-byte chunks:
// each thread requests its SCPT chunks of gate and up before the first use.
constexpr int SCPT = 4;
template <typename T>
__global__ __launch_bounds__(256) void silu_mul_rows_kernel(const T *__restrict__ g, int64_t g_rs,
                                                            const T *__restrict__ u, int64_t u_rs,
                                                            T *__restrict__ o, int64_t o_rs,
                                                            int rows, int cols) {
  constexpr int VEC = Chunk<T>::VEC;
  const int cpr = cols / VEC;  // chunks per row
  const int64_t n = (int64_t)rows * cpr;
  const int64_t first = (int64_t)blockIdx.x * 256 * SCPT + threadIdx.x;
  raw16_t graw[SCPT], uraw[SCPT];
  int64_t goff[SCPT], uoff[SCPT], ooff[SCPT];
#pragma unroll
  for (int k = 0; k < SCPT; ++k) {
    const int64_t idx = min(first + 256 * k, n - 1);  // clamped: in range, stored only if valid
    const int r = (int)(idx / cpr), cc = (int)(idx - (int64_t)r * cpr);
    goff[k] = (int64_t)r * g_rs + cc * VEC;
    uoff[k] = (int64_t)r * u_rs + cc * VEC;
    ooff[k] = (int64_t)r * o_rs + cc * VEC;
    graw[k] = load_stream(g + goff[k]);
    uraw[k] = load_stream(u + uoff[k]);
  }
#pragma unroll
  for (int k = 0; k < SCPT; ++k) {
    if (first + 256 * k >= n) break;
    float gv[VEC], uv[VEC], ov[VEC];
    Chunk<T>::cvt(graw[k], gv);
    Chunk<T>::cvt(uraw[k], uv);
#pragma unroll
    for (int j = 0; j < VEC; ++j) ov[j] = swiglu_silu(gv[j]) * uv[j];
    Chunk<T>::store(o + ooff[k], ov);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void silu_mul_strided_kernel(DView<const T> g, DView<const T> u,
                                                               DView<T> o) {
  const int64_t n = (int64_t)o.h * o.w;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < n;
       idx += (int64_t)gridDim.x * 256) {
    const int r = (int)(idx / o.w), c = (int)(idx - (int64_t)r * o.w);
    const float gv = Elem<T>::load(&g.at(r, c));
    Elem<T>::store(&o.at(r, c), swiglu_silu(gv) * Elem<T>::load(&u.at(r, c)));
  }
}

template <typename T>
__global__ __launch_bounds__(256) void add_strided_kernel(DView<const T> a, DView<const T> b,
                                                          DView<T> c) {
  const int64_t n = (int64_t)c.h * c.w;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < n;
       idx += (int64_t)gridDim.x * 256) {
    const int r = (int)(idx / c.w), col = (int)(idx - (int64_t)r * c.w);
    Elem<T>::store(&c.at(r, col), Elem<T>::load(&a.at(r, col)) + Elem<T>::load(&b.at(r, col)));
  }
}

// Strided fallback: one 256-thread block per row, per-thread strided partial
// sums and an LDS tree (the reference's reduction shape, op_rmsnorm.cuh:25-41).
template <typename T, bool ROPE>
__global__ __launch_bounds__(256) void rmsnorm_strided_kernel(DView<const T> x, DView<const T> w,
                                                              DView<T> y, float eps, int pos_off,
                                                              int head_dim, RopeFreqs freqs) {
  __shared__ float red[256];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  float ss = 0.f;
  for (int i = tid; i < x.w; i += 256) {
    float v = Elem<T>::load(&x.at(row, i));
    ss += v * v;
  }
  red[tid] = ss;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (tid < s) red[tid] += red[tid + s];
    __syncthreads();
  }
  const float rms = sqrtf(red[0] / (float)x.w + eps);
  const float inv_rms = 1.0f / rms;
  if (!ROPE) {
    for (int i = tid; i < x.w; i += 256)
      Elem<T>::store(&y.at(row, i), Elem<T>::load(&x.at(row, i)) * inv_rms *
                                        Elem<T>::load(&w.at(0, i)));
  } else {
    const float pos = (float)(row + pos_off);
    for (int k = tid; k < x.w / 2; k += 256) {
      int c0 = 2 * k;
      int p = (c0 % head_dim) >> 1;
      float x0 = Elem<T>::load(&x.at(row, c0)) * inv_rms * Elem<T>::load(&w.at(0, c0));
      float x1 = Elem<T>::load(&x.at(row, c0 + 1)) * inv_rms * Elem<T>::load(&w.at(0, c0 + 1));
      float sn, cs;
      sincosf(pos * freqs.f[p], &sn, &cs);
      Elem<T>::store(&y.at(row, c0), x0 * cs - x1 * sn);
      Elem<T>::store(&y.at(row, c0 + 1), x0 * sn + x1 * cs);
    }
  }
}

// RoPE on any view: one thread per (row, pair); pair k covers columns 2k, 2k+1,
// which is (head*head_dim + 2p, +1) with p = k % (head_dim/2) (op_rope.cuh:72-77).
template <typename T, bool INVERSE>
__global__ __launch_bounds__(256) void rope_kernel(DView<const T> x, DView<T> y, int pos_off,
                                                   int head_dim, RopeFreqs freqs) {
  const int pairs = x.w >> 1;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)x.h * pairs) return;
  const int row = (int)(idx / pairs);
  const int k = (int)(idx - (int64_t)row * pairs);
  const int p = k % (head_dim >> 1);
  const float ang = (float)(row + pos_off) * freqs.f[p];
  float sn, cs;
  sincosf(ang, &sn, &cs);
  const float x0 = Elem<T>::load(&x.at(row, 2 * k));
  const float x1 = Elem<T>::load(&x.at(row, 2 * k + 1));
  if (!INVERSE) {
    Elem<T>::store(&y.at(row, 2 * k), x0 * cs - x1 * sn);
    Elem<T>::store(&y.at(row, 2 * k + 1), x0 * sn + x1 * cs);
  } else {  // op_rope.cuh:163-168, transpose of the rotation
    Elem<T>::store(&y.at(row, 2 * k), x0 * cs + x1 * sn);
    Elem<T>::store(&y.at(row, 2 * k + 1), -x0 * sn + x1 * cs);
  }
}

// op_rmsnorm_backward_kernel arithmetic (op_rmsnorm.cuh:75-132), fp32.
__global__ __launch_bounds__(256) void rmsnorm_backward_kernel(DView<const float> x,
                                                               DView<const float> w,
                                                               DView<const float> dy,
                                                               DView<float> dx,
                                                               DView<float> dw, float eps) {
  __shared__ float red[2][256];
  const int row = blockIdx.x, tid = threadIdx.x;
  float ss = 0.f, sg = 0.f;
  for (int i = tid; i < x.w; i += 256) {
    float xv = x.at(row, i);
    ss += xv * xv;
    sg += dy.at(row, i) * w.at(0, i) * xv;
  }
  red[0][tid] = ss;
  red[1][tid] = sg;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (tid < s) {
      red[0][tid] += red[0][tid + s];
      red[1][tid] += red[1][tid + s];
    }
    __syncthreads();
  }
  const float rms = sqrtf(red[0][0] / (float)x.w + eps);
  const float inv_rms = 1.0f / rms;
  const float inv_rms3 = inv_rms * inv_rms * inv_rms;
  const float sum_grad = red[1][0];
  for (int i = tid; i < x.w; i += 256) {
    float xv = x.at(row, i), g = dy.at(row, i), wv = w.at(0, i);
    dx.at(row, i) = g * wv * inv_rms + (-inv_rms3 * xv * sum_grad / (float)x.w);
    atomicAdd(&dw.at(0, i), g * (xv * inv_rms));  // summed over rows, as :131
  }
}

__global__ void zero_row_kernel(DView<float> v) {
  int i = blockIdx.x * 256 + threadIdx.x;
  if (i < v.w) v.at(0, i) = 0.f;
}

template <typename T, bool ROPE>
int launch_rmsnorm(const bn_view *x, const bn_view *weight, const bn_view *y, float eps,
                   int pos_off, int head_dim, const RopeFreqs &fr, hipStream_t s) {
  const int rows = x->h, cols = x->w;
  if (rows == 0 || cols == 0) return BN_OK;
  constexpr int VEC = Chunk<T>::VEC;
  const bool fast = rows_aligned(x, 16) && rows_aligned(y, 16) && rows_aligned(weight, 16) &&
                    cols % VEC == 0 && cols <= 64 * kMaxChunks * VEC &&
                    (!ROPE || head_dim % VEC == 0);
  if (fast) {
    const T *xp = reinterpret_cast<const T *>(x->data) + x->offset;
    const T *wp = reinterpret_cast<const T *>(weight->data) + weight->offset;
    T *yp = reinterpret_cast<T *>(y->data) + y->offset;
    dim3 grid((rows + kRowsPerBlock - 1) / kRowsPerBlock);
    if (cols <= 64 * 4 * VEC)
      hipLaunchKernelGGL((rmsnorm_rows_kernel<T, ROPE, 4>), grid, dim3(256), 0, s, xp,
                         (int64_t)x->stride_h, wp, (int64_t)0, yp, (int64_t)y->stride_h, rows,
                         cols, eps, pos_off, head_dim, fr);
    else
      hipLaunchKernelGGL((rmsnorm_rows_kernel<T, ROPE, kMaxChunks>), grid, dim3(256), 0, s, xp,
                         (int64_t)x->stride_h, wp, (int64_t)0, yp, (int64_t)y->stride_h, rows,
                         cols, eps, pos_off, head_dim, fr);
  } else {
    DView<const T> xv = dview<const T>(x), wv = dview<const T>(weight);
    DView<T> yv = dview<T>(y);
    hipLaunchKernelGGL((rmsnorm_strided_kernel<T, ROPE>), dim3(rows), dim3(256), 0, s, xv, wv,
                       yv, eps, pos_off, head_dim, fr);
  }
  BN_LAUNCH_CHECK();
  return BN_OK;
}

int rmsnorm_common(const char *op, const bn_view *x, const bn_view *weight, const bn_view *y,
                   float eps, bool rope, int pos_off, int head_dim, float theta, void *stream) {
  const unsigned mask = (1u << BN_F32) | (1u << BN_BF16);
  int st;
  if ((st = check_view(x, op, "input", mask))) return st;
  if ((st = check_view(weight, op, "weight", mask))) return st;
  if ((st = check_view(y, op, "output", mask))) return st;
  if (!same_shape(x, y)) return fail(BN_ERR_SHAPE, std::string(op) + ": input/output shape mismatch");
  if (weight->h != 1 || weight->w != x->w)
    return fail(BN_ERR_SHAPE, std::string(op) + ": weight shape must be (1, hidden_dim)");
  if (x->dtype != y->dtype || x->dtype != weight->dtype)
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": input, weight and output dtypes differ");
  RopeFreqs fr;
  if (rope) {
    if ((st = make_rope_freqs(op, head_dim, theta, &fr))) return st;
    if (x->w % head_dim != 0)
      return fail(BN_ERR_SHAPE, std::string(op) + ": hidden_dim must be divisible by head_dim");
  }
  if ((st = require_device(op, {x, weight, y}))) return st;
  if ((st = ensure_device())) return st;
  hipStream_t s = as_stream(stream);
  if (x->dtype == BN_F32)
    return rope ? launch_rmsnorm<float, true>(x, weight, y, eps, pos_off, head_dim, fr, s)
                : launch_rmsnorm<float, false>(x, weight, y, eps, pos_off, head_dim, fr, s);
  return rope ? launch_rmsnorm<bf16_t, true>(x, weight, y, eps, pos_off, head_dim, fr, s)
              : launch_rmsnorm<bf16_t, false>(x, weight, y, eps, pos_off, head_dim, fr, s);
}

template <bool INVERSE>
int rope_common(const char *op, const bn_view *x, const bn_view *y, int pos_off, int head_dim,
                float theta, void *stream) {
  const unsigned mask = (1u << BN_F32) | (1u << BN_BF16);
  int st;
  if ((st = check_view(x, op, "input", mask))) return st;
  if ((st = check_view(y, op, "output", mask))) return st;
  if (!same_shape(x, y)) return fail(BN_ERR_SHAPE, std::string(op) + ": input/output shape mismatch");
  if (x->dtype != y->dtype)
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": input and output dtypes differ");
  if (head_dim <= 0 || x->w % head_dim != 0)
    return fail(BN_ERR_SHAPE, std::string(op) + ": hidden_dim must be divisible by head_dim");
  RopeFreqs fr;
  if ((st = make_rope_freqs(op, head_dim, theta, &fr))) return st;
  if ((st = require_device(op, {x, y}))) return st;
  if ((st = ensure_device())) return st;
  const int64_t n = (int64_t)x->h * (x->w / 2);
  if (n == 0) return BN_OK;
  dim3 grid((unsigned)((n + 255) / 256));
  hipStream_t s = as_stream(stream);
  if (x->dtype == BN_F32)
    hipLaunchKernelGGL((rope_kernel<float, INVERSE>), grid, dim3(256), 0, s,
                       dview<const float>(x), dview<float>(y), pos_off, head_dim, fr);
  else
    hipLaunchKernelGGL((rope_kernel<bf16_t, INVERSE>), grid, dim3(256), 0, s,
                       dview<const bf16_t>(x), dview<bf16_t>(y), pos_off, head_dim, fr);
  BN_LAUNCH_CHECK();
  return BN_OK;
}

inline unsigned grid_for(int64_t n) { return (unsigned)std::min<int64_t>((n + 255) / 256, 8192); }

template <typename T>
int launch_add_rmsnorm(const bn_view *x, const bn_view *d, const bn_view *w, const bn_view *h,
                       const bn_view *y, float eps, hipStream_t s) {
  const int rows = x->h, cols = x->w;
  constexpr int VEC = Chunk<T>::VEC;
  const bool fast = rows_aligned(x, 16) && rows_aligned(d, 16) && rows_aligned(h, 16) &&
                    rows_aligned(y, 16) && rows_aligned(w, 16) && cols % VEC == 0 &&
                    cols <= 64 * kMaxChunks * VEC;
  if (fast) {
    const T *xp = (const T *)x->data + x->offset, *dp = (const T *)d->data + d->offset;
    const T *wp = (const T *)w->data + w->offset;
    T *hp = (T *)h->data + h->offset, *yp = (T *)y->data + y->offset;
    dim3 grid((rows + kRowsPerBlock - 1) / kRowsPerBlock);
    if (cols <= 64 * 4 * VEC)
      hipLaunchKernelGGL((add_rmsnorm_rows_kernel<T, 4>), grid, dim3(256), 0, s, xp,
                         (int64_t)x->stride_h, dp, (int64_t)d->stride_h, wp, hp,
                         (int64_t)h->stride_h, yp, (int64_t)y->stride_h, rows, cols, eps);
    else
      hipLaunchKernelGGL((add_rmsnorm_rows_kernel<T, kMaxChunks>), grid, dim3(256), 0, s, xp,
                         (int64_t)x->stride_h, dp, (int64_t)d->stride_h, wp, hp,
                         (int64_t)h->stride_h, yp, (int64_t)y->stride_h, rows, cols, eps);
    BN_LAUNCH_CHECK();
    return BN_OK;
  }
  // any other views: the add, then RMSNorm of h (two launches)
  hipLaunchKernelGGL((add_strided_kernel<T>), dim3(grid_for((int64_t)rows * cols)), dim3(256), 0, s,
                     dview<const T>(x), dview<const T>(d), dview<T>(h));
  BN_LAUNCH_CHECK();
  RopeFreqs fr;
  return launch_rmsnorm<T, false>(h, w, y, eps, 0, 2, fr, s);
}

template <typename T>
int launch_silu_mul(const bn_view *g, const bn_view *u, const bn_view *o, hipStream_t s) {
  const int rows = g->h, cols = g->w;
  constexpr int VEC = Chunk<T>::VEC;
  const int64_t n = (int64_t)rows * cols;
  if (rows_aligned(g, 16) && rows_aligned(u, 16) && rows_aligned(o, 16) && cols % VEC == 0)
    hipLaunchKernelGGL((silu_mul_rows_kernel<T>), dim3((unsigned)((n / VEC + 256 * SCPT - 1) / (256 * SCPT))),
                       dim3(256), 0, s,
                       (const T *)g->data + g->offset, (int64_t)g->stride_h,
                       (const T *)u->data + u->offset, (int64_t)u->stride_h,
                       (T *)o->data + o->offset, (int64_t)o->stride_h, rows, cols);
  else
    hipLaunchKernelGGL((silu_mul_strided_kernel<T>), dim3(grid_for(n)), dim3(256), 0, s,
                       dview<const T>(g), dview<const T>(u), dview<T>(o));
  BN_LAUNCH_CHECK();
  return BN_OK;
}

}  // namespace
}  // namespace bn

using namespace bn;

extern "C" {

int bn_rmsnorm(const bn_view *x, const bn_view *weight, const bn_view *y, float eps,
               void *stream) {
  return rmsnorm_common("RMSNorm", x, weight, y, eps, false, 0, 2, 1.f, stream);
}

int bn_rmsnorm_rope(const bn_view *x, const bn_view *weight, const bn_view *y, float eps,
                    int position_offset, int head_dim, float theta, void *stream) {
  return rmsnorm_common("RMSNorm+RoPE", x, weight, y, eps, true, position_offset, head_dim,
                        theta, stream);
}

int bn_add_rmsnorm(const bn_view *x, const bn_view *delta, const bn_view *weight,
                   const bn_view *h, const bn_view *y, float eps, void *stream) {
  const char *op = "Add+RMSNorm";
  const unsigned mask = (1u << BN_F32) | (1u << BN_BF16);
  int st;
  if ((st = check_view(x, op, "input", mask))) return st;
  if ((st = check_view(delta, op, "residual", mask))) return st;
  if ((st = check_view(weight, op, "weight", mask))) return st;
  if ((st = check_view(h, op, "sum", mask))) return st;
  if ((st = check_view(y, op, "output", mask))) return st;
  if (!same_shape(x, delta) || !same_shape(x, h) || !same_shape(x, y))
    return fail(BN_ERR_SHAPE, std::string(op) + ": input/residual/sum/output shape mismatch");
  if (weight->h != 1 || weight->w != x->w)
    return fail(BN_ERR_SHAPE, std::string(op) + ": weight shape must be (1, hidden_dim)");
  if (delta->dtype != x->dtype || h->dtype != x->dtype || y->dtype != x->dtype ||
      weight->dtype != x->dtype)
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": dtypes differ");
  if ((st = require_device(op, {x, delta, weight, h, y}))) return st;
  if ((st = ensure_device())) return st;
  if (x->h == 0 || x->w == 0) return BN_OK;
  hipStream_t s = as_stream(stream);
  return x->dtype == BN_F32 ? launch_add_rmsnorm<float>(x, delta, weight, h, y, eps, s)
                            : launch_add_rmsnorm<bf16_t>(x, delta, weight, h, y, eps, s);
}

int bn_silu_mul(const bn_view *gate, const bn_view *up, const bn_view *out, void *stream) {
  const char *op = "SiLU*up";
  const unsigned mask = (1u << BN_F32) | (1u << BN_BF16);
  int st;
  if ((st = check_view(gate, op, "gate", mask))) return st;
  if ((st = check_view(up, op, "up", mask))) return st;
  if ((st = check_view(out, op, "output", mask))) return st;
  if (!same_shape(gate, up) || !same_shape(gate, out))
    return fail(BN_ERR_SHAPE, std::string(op) + ": gate/up/output shape mismatch");
  if (up->dtype != gate->dtype || out->dtype != gate->dtype)
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": dtypes differ");
  if ((st = require_device(op, {gate, up, out}))) return st;
  if ((st = ensure_device())) return st;
  if (gate->h == 0 || gate->w == 0) return BN_OK;
  hipStream_t s = as_stream(stream);
  return gate->dtype == BN_F32 ? launch_silu_mul<float>(gate, up, out, s)
                               : launch_silu_mul<bf16_t>(gate, up, out, s);
}

int bn_rope(const bn_view *x, const bn_view *y, int position_offset, int head_dim, float theta,
            void *stream) {
  return rope_common<false>("RoPE", x, y, position_offset, head_dim, theta, stream);
}

int bn_rope_backward(const bn_view *dy, const bn_view *dx, int position_offset, int head_dim,
                     float theta, void *stream) {
  return rope_common<true>("RoPE backward", dy, dx, position_offset, head_dim, theta, stream);
}

int bn_rmsnorm_backward(const bn_view *x, const bn_view *weight, const bn_view *dy,
                        const bn_view *dx, const bn_view *dweight, float eps, void *stream) {
  const char *op = "RMSNorm backward";
  const unsigned mask = 1u << BN_F32;
  int st;
  if ((st = check_view(x, op, "input", mask))) return st;
  if ((st = check_view(weight, op, "weight", mask))) return st;
  if ((st = check_view(dy, op, "grad_output", mask))) return st;
  if ((st = check_view(dx, op, "grad_input", mask))) return st;
  if ((st = check_view(dweight, op, "grad_weight", mask))) return st;
  if (!same_shape(x, dy) || !same_shape(x, dx)) return fail(BN_ERR_SHAPE, "RMSNorm backward: shape mismatch");
  if (weight->h != 1 || weight->w != x->w || dweight->h != 1 || dweight->w != x->w)
    return fail(BN_ERR_SHAPE, "RMSNorm backward: weight shape must be (1, hidden_dim)");
  if ((st = require_device(op, {x, weight, dy, dx, dweight}))) return st;
  if ((st = ensure_device())) return st;
  hipStream_t s = as_stream(stream);
  if (x->w == 0) return BN_OK;
  hipLaunchKernelGGL(zero_row_kernel, dim3((x->w + 255) / 256), dim3(256), 0, s,
                     dview<float>(dweight));
  BN_LAUNCH_CHECK();
  if (x->h == 0) return BN_OK;
  hipLaunchKernelGGL(rmsnorm_backward_kernel, dim3(x->h), dim3(256), 0, s,
                     dview<const float>(x), dview<const float>(weight), dview<const float>(dy),
                     dview<float>(dx), dview<float>(dweight), eps);
  BN_LAUNCH_CHECK();
  return BN_OK;
}

}  // extern "C"
