// bn_common.hpp -- internal helpers shared by the libbnhip translation units:
// error reporting behind the C ABI, host-side view validation, device-side
// strided views and bf16 conversion.  Not part of the public interface.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <initializer_list>
#include <string>
#include <type_traits>

#include "bn_hip.h"

namespace bn {

// ----------------------------------------------------------------- errors
void set_error(const std::string &msg);
inline int fail(int status, const std::string &msg) {
  set_error(msg);
  return status;
}
int hip_fail(hipError_t err, const char *file, int line);

// Returns from the enclosing C-ABI function with BN_ERR_HIP on error.
#define BN_HIP_TRY(expr)                                              \
  do {                                                                \
    hipError_t bn_e_ = (expr);                                        \
    if (bn_e_ != hipSuccess) return ::bn::hip_fail(bn_e_, __FILE__, __LINE__); \
  } while (0)

// After a kernel launch: report launch-configuration errors.
#define BN_LAUNCH_CHECK() BN_HIP_TRY(hipGetLastError())

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// Makes sure the library's device is current on the calling thread.
int ensure_device();
// The device bn_init selected (valid after ensure_device()).
int library_device();
// Looks up, once per device, the device address of the decode scratch array
// (bn_decode.hip); called by bn_init with `device` current.
int decode_scratch_setup(int device);
// Compute units of the library's device (0 if the query fails); call after
// ensure_device().
int device_cu_count();

// bn_linear_rope with the split-k reduction's epilogue chosen by the caller
// (bn_linear.hip): kLinEpiPlain is bn_linear_rope's own (the rotation of the
// first rope_cols columns; with k_dst, columns [app_col, app_col + app_w) of
// row r are also stored to k_dst + r*app_rs and the next app_w columns to
// v_dst + r*app_rs: a QKV projection's K and V appended to the caches);
// kLinEpiSilu reads the output as [gate | up] halves and writes
// y = silu(gate) * up, y [m, n/2].  The slabs are summed in one order for
// every epilogue, so a fused epilogue gives the bits of the unfused ops.
// The epilogues need the split-k path (always taken for m <= 8).
constexpr int kLinEpiPlain = 0, kLinEpiSilu = 1;
// fp32 row width up to which bn_rmsnorm / bn_add_rmsnorm run their one-wave
// row kernels (64 lanes x 8 chunks of 4; wider rows take a strided kernel
// with another summation order)
constexpr int kNormRowF32 = 2048;
// fp32 elements of x an output-major few-rows projection stages in LDS
// (64 KB per workgroup: rows staged x k padded to 256 for fp32)
constexpr int kGemvStagedMax = 16384;
// A normalised input for an output-major projection of one fp32 row (a
// decode step; k <= kNormRowF32): the kernel reads x as the residual stream
// h and projects rmsnorm(h + d) * w instead (d null: rmsnorm(h) * w), formed as
// add_rmsnorm / rmsnorm form it, so the product has the bits of the norm
// kernel followed by the projection; h_out (not null) receives h + d.  h_out
// must not alias h or d (other workgroups still read them).
struct LinNorm {
  const float *d, *w;
  float *h_out;
  float eps;
};
// A merged input for an output-major projection of one fp32 row: x is the
// attention output of a split short-cache decode (decode_short_partials),
// formed in the staging from its partial records -- x[h*64 + d] merges the
// n_split records of query head h (`part`: [n_heads][n_split][kDecRec]) over
// the valid splits of the sequence's length (`lens[0]`, device, clamped to
// [0, max_len]) -- with the arithmetic of the decode's own combine kernel,
// so the product has the bits of bn_gqa_decode followed by the projection.
struct LinMerge {
  const float *part;
  const int32_t *lens;
  int n_split, max_len;
  int len;  // >= 0: the sequence's length, given by the host (lens is not read)
};
int linear_run(const bn_view *x, const bn_view *w, const bn_view *y, int rope_cols,
               int position_offset, int head_dim, float theta, void *workspace,
               size_t workspace_bytes, int epi, float *k_dst, float *v_dst, int app_col, int app_w,
               int64_t app_rs, void *stream, const LinNorm *nrm = nullptr,
               const LinMerge *mrg = nullptr);

// ------------------------------------------------ split decode partials
// A split decode writes, per (sequence, query head), n_split records of
// kDecRec floats: m (the split's largest score, log2 units), l (its sum of
// exp2(s - m)) and acc[64] (its sum of exp2(s - m) * v).  Splits at or past
// the sequence's valid count hold no keys and are never read as numbers.
constexpr int kDecRec = 66;
// The short-cache split decode (fp32 caches of at most kShortMaxLen keys,
// at most kShortMaxUnits (sequence, query head) pairs): kShortSplits splits
// per (sequence, query head), each of short_split_chunk(len) keys.
constexpr int kShortMaxLen = 1024, kShortMaxUnits = 256, kShortSplits = 4;
__host__ __device__ inline int short_split_chunk(int len, int n_split) {
  const int c = ((len + n_split - 1) / n_split + 3) & ~3;  // whole 4-key lane groups
  return c < 4 ? 4 : c;
}
// Launches the short-cache split decode alone: fp32 q [batch, n_heads, 64],
// caches [batch, max_len, n_kv_heads, 64], partial records into `part`
// ([batch * n_heads][kShortSplits][kDecRec]); the caller merges them
// (bn_decode.hip's combine, or an output projection's LinMerge staging).
// Shapes are the caller's to check: short_path_ok() true.
// host_len >= 0: every sequence's length, given by the host (seq_lens is
// not read; a decode loop knows its position).
bool short_path_ok(int dtype, int batch, int max_len, int n_heads);
int decode_short_partials(const float *q, const float *k_cache, const float *v_cache,
                          const int32_t *seq_lens, int host_len, float *part, int batch, int max_len,
                          int n_heads, int n_kv_heads, float scale, hipStream_t s);

// The merge of 4 consecutive d of one (sequence, head) over records
// [0, nvalid), in groups of 8 records (loads of a group first, then its
// merge, with the running max rescaled between groups).  Records at or past
// nvalid are read from an in-range slot and skipped by a select (never
// multiplied by a zero weight: they may hold Inf or NaN).
struct DecMerge {
  float ms[8], ls[8];
  float4 as[8];
  float M, L, A[4];
  __device__ __forceinline__ void start() {
    M = -INFINITY;
    L = 0.f;
    A[0] = A[1] = A[2] = A[3] = 0.f;
  }
  // SYS: system-scope loads, past the caches (records another workgroup of
  // the same launch wrote through to memory); the same values either way
  template <bool SYS = false>
  __device__ __forceinline__ void load8(const float *part, int n_split, int s0, int d0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float *ps = part + min(s0 + j, n_split - 1) * kDecRec;
      if constexpr (SYS) {
        auto rd = [](const float *a) { return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM); };
        ms[j] = rd(ps);
        ls[j] = rd(ps + 1);
        as[j] = make_float4(rd(ps + 2 + d0), rd(ps + 3 + d0), rd(ps + 4 + d0), rd(ps + 5 + d0));
      } else {
        const float2 ml = *reinterpret_cast<const float2 *>(ps);  // 264-byte records: 8-byte aligned
        ms[j] = ml.x;
        ls[j] = ml.y;
        as[j] = make_float4(ps[2 + d0], ps[3 + d0], ps[4 + d0], ps[5 + d0]);
      }
    }
  }
  // the same values in two parts: acc from the records, (m, l) from a table
  // of pairs (stride 2 floats; e.g. gathered into LDS)
  __device__ __forceinline__ void load_acc8(const float *part, int n_split, int s0, int d0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float *ps = part + min(s0 + j, n_split - 1) * kDecRec;
      as[j] = make_float4(ps[2 + d0], ps[3 + d0], ps[4 + d0], ps[5 + d0]);
    }
  }
  __device__ __forceinline__ void load_ml8(const float *ml, int n_split, int s0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float2 v = *reinterpret_cast<const float2 *>(ml + 2 * min(s0 + j, n_split - 1));
      ms[j] = v.x;
      ls[j] = v.y;
    }
  }
  __device__ __forceinline__ void merge8(int s0, int nvalid) {
    float mx = M;
#pragma unroll
    for (int j = 0; j < 8; ++j) mx = s0 + j < nvalid ? fmaxf(mx, ms[j]) : mx;
    const float mu = mx == -INFINITY ? 0.f : mx;       // nothing valid yet: weights stay 0
    const float fo = __builtin_amdgcn_exp2f(M - mu);  // M = -inf -> 0
    L *= fo;
    A[0] *= fo; A[1] *= fo; A[2] *= fo; A[3] *= fo;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const bool ok = s0 + j < nvalid;
      const float f = __builtin_amdgcn_exp2f(ms[j] - mu);
      L = ok ? fmaf(ls[j], f, L) : L;
      A[0] = ok ? fmaf(as[j].x, f, A[0]) : A[0];
      A[1] = ok ? fmaf(as[j].y, f, A[1]) : A[1];
      A[2] = ok ? fmaf(as[j].z, f, A[2]) : A[2];
      A[3] = ok ? fmaf(as[j].w, f, A[3]) : A[3];
    }
    M = mx;
  }
  // the merged values (an empty sequence: zeros)
  __device__ __forceinline__ float4 result() const {
    const float inv = L > 0.f ? 1.0f / L : 0.f;
    return make_float4(A[0] * inv, A[1] * inv, A[2] * inv, A[3] * inv);
  }
};

// ------------------------------------------------------------ validation
inline size_t dtype_size(int dt) { return dt == BN_BF16 ? 2 : 4; }

// Checks a view's fields; `op` prefixes the message ("RMSNorm", ...).
// dtype_mask: bit (1 << dtype) set for each accepted dtype.
int check_view(const bn_view *v, const char *op, const char *name, unsigned dtype_mask,
               bool need_device = false);

// The reference validates shapes first and the device last (op_rmsnorm.cuh:
// 142-150); GPU-only ops end their validation with this check.
inline int require_device(const char *op, std::initializer_list<const bn_view *> vs) {
  for (const bn_view *v : vs)
    if (!v->on_device)
      return fail(BN_ERR_NOT_DEVICE, std::string(op) + ": only GPU implementation available");
  return BN_OK;
}

inline bool same_shape(const bn_view *a, const bn_view *b) {
  return a->h == b->h && a->w == b->w;
}

// True when the view is row-major contiguous within rows (stride_w == 1) and
// every row starts on a `align`-byte boundary.
inline bool rows_aligned(const bn_view *v, int align) {
  size_t es = dtype_size(v->dtype);
  uintptr_t base = reinterpret_cast<uintptr_t>(v->data) + (uintptr_t)(v->offset * (int64_t)es);
  return v->stride_w == 1 && (base % align) == 0 &&
         ((size_t)((int64_t)v->stride_h * (int64_t)es) % align) == 0;
}

// ----------------------------------------------------- device-side views
template <typename T>
struct DView {
  T *p;  // already offset to element (0, 0)
  int h, w;
  int64_t sh, sw;
  __device__ __forceinline__ T &at(int r, int c) const { return p[r * sh + c * sw]; }
};

template <typename T>
inline DView<T> dview(const bn_view *v) {
  DView<T> d;
  d.p = reinterpret_cast<T *>(v->data) + v->offset;
  d.h = v->h;
  d.w = v->w;
  d.sh = v->stride_h;
  d.sw = v->stride_w;
  return d;
}

// ------------------------------------------------------------------ bf16
// bf16 values are stored as raw 16-bit patterns; conversions are exact
// (bf16 -> f32) and round-to-nearest-even (f32 -> bf16).
typedef uint16_t bf16_t;

__device__ __forceinline__ float bf16_to_f32(bf16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
  __bf16 h = (__bf16)f;  // v_cvt_pk_bf16_f32 on gfx950: RNE, NaN-preserving
  return __builtin_bit_cast(bf16_t, h);
}

template <typename T> struct Elem;
template <> struct Elem<float> {
  __device__ static __forceinline__ float load(const float *p) { return *p; }
  __device__ static __forceinline__ void store(float *p, float v) { *p = v; }
  __device__ static __forceinline__ float round(float v) { return v; }  // value as stored
};
template <> struct Elem<bf16_t> {
  __device__ static __forceinline__ float load(const bf16_t *p) { return bf16_to_f32(*p); }
  __device__ static __forceinline__ void store(bf16_t *p, float v) { *p = f32_to_bf16(v); }
  __device__ static __forceinline__ float round(float v) { return bf16_to_f32(f32_to_bf16(v)); }
};

// ------------------------------------------------------------ SwiGLU
// SwiGLU's silu(g) = g / (1 + e^-g) (op_silu.cuh SiLUFunc) as one exp2 and
// one reciprocal instead of the library expf and an IEEE division (about a
// fifth of the instructions; the fused SwiGLU kernels issue them for every
// element): within 1e-5 relative of the exact value while e^-g is finite,
// -0 or 0 where it overflows, as the exact quotient rounds.  Every SwiGLU
// kernel (standalone and in the projection's reduction) uses this one form,
// so their results agree bit for bit.
__device__ __forceinline__ float swiglu_silu(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.4426950408889634f));
}

// --------------------------------------------------------- wave reductions
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

// RoPE frequencies formed on the host as the reference forms them
// (op_rope.cuh:82): e = (float)(2p)/head_dim, freq = (float)(1.0/(double)theta^e).
constexpr int kMaxRopePairs = 256;
struct RopeFreqs {
  float f[kMaxRopePairs];
};
int make_rope_freqs(const char *op, int head_dim, float theta, RopeFreqs *out);

}  // namespace bn
