// bn_linear.hip -- the GQA layer's projections on gfx950 MFMA with RoPE in
// the epilogue: y = x @ w, then the reference's rotation (op_rope.cuh:55-99)
// on the first rope_cols columns of y -- the Q and K heads of a fused QKV
// weight -- at position position_offset + row.  rope_cols = 0 is the plain
// projection (the output projection, llama_layers.hpp:112).
//
// A workgroup computes a 64x64 tile of y^T = w^T x^T with 4 waves of 32x32:
// lane = output row, registers = 16 output columns, so each rotation pair
// (2p, 2p+1) sits in adjacent registers of one lane.  w and x tiles are
// staged through LDS (double-buffered, one barrier per k step).  fp32 runs
// v_mfma_f32_32x32x2_f32 on w rows and x columns read straight from LDS;
// bf16 runs v_mfma_f32_32x32x16_bf16 with the w^T fragments read by
// ds_read_b64_tr_b16 and the x fragments in the same k order.  Small grids
// split k: each slab writes fp32 partial sums and linear_reduce_kernel adds
// them in slab order and applies the rotation (deterministic, no atomics).
// A few rows (decode steps) stream w instead: row-major w through
// linear_small_kernel's k slabs (and the same reduction), an output-major w
// (the transposed view of an [n, k] matrix) through linear_gemv_t_kernel,
// one launch with the epilogue and no partials.
#include <algorithm>

#include "bn_common.hpp"

namespace bn {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int TN = 64, TM = 64;  // workgroup tile: output columns x output rows

template <typename T>
struct LinCfg;
// k per LDS stage (measured: doubling it to 64 / 128 loses 8% (fp32) and 17%
// (bf16, 2048 rows) -- half the workgroups fit a compute unit)
template <>
struct LinCfg<float> {
  static constexpr int KT = 32;  // k per LDS stage
  static constexpr int WP = TN + 4;       // Ws[k][n] pitch, elements
  static constexpr int XP = KT + 4;       // Xs[m][k] pitch
};
template <>
struct LinCfg<bf16_t> {
  static constexpr int KT = 64;
  static constexpr int WP = TN + 8;  // 144 B rows: conflict-free transposed 16-bit reads
  static constexpr int XP = KT + 8;
};

struct LinParams {
  const void *x, *w;
  void *y;
  float *part;  // [nsplit][m][n] fp32 partial sums, or null
  int64_t x_rs, w_rs, y_rs;
  int m, n, k, kchunk;  // kchunk: k per slab, a multiple of the stage depth
  int rope_cols, head_dim, pos0;
  // epilogue extras of the split-k reduction and of the output-major
  // few-rows kernel (decode steps, fp32): columns
  // [app_col, app_col + app_w) of row r also go to k_dst + r*app_rs and
  // [app_col + app_w, app_col + 2*app_w) to v_dst + r*app_rs (the K and V
  // rows of a QKV projection appended to the caches); null: none
  float *k_dst, *v_dst;
  int app_col, app_w;
  int64_t app_rs;
  // normalised input of the output-major kernel (LinNorm): x is h
  const float *nd, *nw;
  float *nh_out;
  float neps;
  // merged input of the output-major kernel (LinMerge): x is formed from a
  // split decode's partial records
  const float *mpart;
  const int32_t *mlens;
  int msplit, mmax_len, mlen;
};

// epilogues: EPI_PLAIN writes y (rotated in the first rope_cols columns);
// EPI_SILU takes the sums as gate | up halves and writes y = silu(gate) * up,
// the width of one half
constexpr int EPI_PLAIN = kLinEpiPlain, EPI_SILU = kLinEpiSilu;

__device__ __forceinline__ bf16x4_t tr16(const bf16_t *lds) {
  const s16x4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4_t *)(__attribute__((address_space(3))) void *)lds);
  return __builtin_bit_cast(bf16x4_t, r);
}

template <typename T>
__device__ __forceinline__ void store4(T *dst, const float (&v)[4]);
template <>
__device__ __forceinline__ void store4<float>(float *dst, const float (&v)[4]) {
  *(float4 *)dst = make_float4(v[0], v[1], v[2], v[3]);
}
template <>
__device__ __forceinline__ void store4<bf16_t>(bf16_t *dst, const float (&v)[4]) {
  const uint32_t lo = (uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
  const uint32_t hi = (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
  *(uint2 *)dst = make_uint2(lo, hi);
}

// rotation of the pairs (gn, gn+1) and (gn+2, gn+3) of row gm that lie in
// the first rope_cols columns (op_rope.cuh:79-98: fp32 angle position*freq)
__device__ __forceinline__ void rope4(float (&v)[4], int gm, int gn, const LinParams &p,
                                      const RopeFreqs &fr) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int c = gn + 2 * j;
    if (c < p.rope_cols) {
      const float ang = (float)(p.pos0 + gm) * fr.f[(c % p.head_dim) >> 1];
      float sn, cs;
      sincosf(ang, &sn, &cs);
      const float x0 = v[2 * j], x1 = v[2 * j + 1];
      v[2 * j] = x0 * cs - x1 * sn;
      v[2 * j + 1] = x0 * sn + x1 * cs;
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256, 2) void linear_kernel(LinParams p, RopeFreqs fr) {
  using C = LinCfg<T>;
  constexpr int KT = C::KT, WP = C::WP, XP = C::XP;
  constexpr int VE = 16 / (int)sizeof(T);  // elements per 16-byte chunk
  constexpr int WCH = TN / VE, XCH = KT / VE;  // chunks per w row, per x row
  __shared__ __attribute__((aligned(16))) T Ws[2][KT * WP];  // Ws[k][n]
  __shared__ __attribute__((aligned(16))) T Xs[2][TM * XP];  // Xs[m][k]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31, hf = lane >> 5;
  const int n_off = 32 * (wave & 1), m_off = 32 * (wave >> 1);
  const int n0 = blockIdx.x * TN, m0 = blockIdx.y * TM;
  const int kb = blockIdx.z * p.kchunk, ke = min(kb + p.kchunk, p.k);
  const T *X = (const T *)p.x, *W = (const T *)p.w;

  // staging: NCH 16-byte chunks of w and of x per thread per stage (KT x TN
  // of w and TM x KT of x hold the same number of chunks)
  constexpr int NCH = KT * TN / VE / 256;
  static_assert(NCH * 256 * VE == KT * TN && TM * KT == KT * TN, "staging covers both tiles");
  u32x4_t wr[NCH], xr[NCH];
  auto gload = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = tid + 256 * i;
      const int gk = k0 + c / WCH, gn = n0 + (c % WCH) * VE;
      wr[i] = (gk < ke && gn < p.n) ? *(const u32x4_t *)(W + gk * p.w_rs + gn) : u32x4_t{0u, 0u, 0u, 0u};
      const int gm = m0 + c / XCH, gk2 = k0 + (c % XCH) * VE;
      xr[i] = (gm < p.m && gk2 < ke) ? *(const u32x4_t *)(X + gm * p.x_rs + gk2) : u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  auto lstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = tid + 256 * i;
      *(u32x4_t *)(&Ws[buf][(c / WCH) * WP + (c % WCH) * VE]) = wr[i];
      *(u32x4_t *)(&Xs[buf][(c / XCH) * XP + (c % XCH) * VE]) = xr[i];
    }
  };
  // two accumulators over alternating k steps: independent MFMA chains
  f32x16_t acc[2] = {f32x16_t{}, f32x16_t{}};
  const bool busy = m0 + m_off < p.m && n0 + n_off < p.n;  // wave-uniform
  const int tr_off = (4 * hf + ((lane & 15) >> 2)) * WP + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const int nst = ke > kb ? (ke - kb + KT - 1) / KT : 0;
  if (nst > 0) gload(kb);
  for (int s = 0; s < nst; ++s) {
    const int buf = s & 1;
    lstore(buf);
    __syncthreads();  // also: every wave finished stage s-2, the last reader of buf
    if (s + 1 < nst) gload(kb + (s + 1) * KT);
    if (!busy) continue;
    const T *ws = Ws[buf], *xs = Xs[buf];
    if constexpr (sizeof(T) == 4) {
      // A = w^T: lane holds w[k = 2kk + hf][n]; B = x^T: lane holds x[m][k]
#pragma unroll
      for (int kk = 0; kk < KT / 2; ++kk) {
        const float a = ws[(2 * kk + hf) * WP + n_off + r32];
        const float b = xs[(m_off + r32) * XP + 2 * kk + hf];
        acc[kk & 1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[kk & 1], 0, 0, 0);
      }
    } else {
      // A = w^T by transposed reads: slot j of lane half hf is k = 16u +
      // 8(j/4) + 4hf + j%4; B = x^T in the same k order
#pragma unroll
      for (int u = 0; u < KT / 16; ++u) {
        const bf16_t *wp = ws + 16 * u * WP + tr_off + n_off;
        const bf16x4_t alo = tr16(wp), ahi = tr16(wp + 8 * WP);
        const bf16x8_t a = {alo[0], alo[1], alo[2], alo[3], ahi[0], ahi[1], ahi[2], ahi[3]};
        const bf16_t *xp = xs + (m_off + r32) * XP + 16 * u + 4 * hf;
        const bf16x4_t blo = *(const bf16x4_t *)xp, bhi = *(const bf16x4_t *)(xp + 8);
        const bf16x8_t b = {blo[0], blo[1], blo[2], blo[3], bhi[0], bhi[1], bhi[2], bhi[3]};
        acc[u & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[u & 1], 0, 0, 0);
      }
    }
  }
  if (!busy) return;
  const int gm = m0 + m_off + r32;
  if (gm >= p.m) return;
  // acc[.][4g + e] = y^T[n = n_off + 8g + 4hf + e][m]: four consecutive columns
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int gn = n0 + n_off + 8 * g + 4 * hf;
    if (gn >= p.n) continue;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = acc[0][4 * g + e] + acc[1][4 * g + e];
    if (p.part) {
      *(float4 *)(p.part + ((int64_t)blockIdx.z * p.m + gm) * p.n + gn) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      rope4(v, gm, gn, p, fr);
      store4<T>((T *)p.y + gm * p.y_rs + gn, v);
    }
  }
}

// Split-k slab sums, in one order for every caller and epilogue: wave w of
// a 256-thread workgroup adds slabs w, w+4, w+8, ... in increasing order
// (loads 8 deep), and the four wave sums meet in LDS as ((s0 + s1) + s2) + s3.
// Lane l owns columns 4l..4l+3 of the workgroup's 256-column strip; grid y
// is the row.  Four waves per strip spread the slab reads of a few-row
// projection over 4x the threads of a one-thread-per-column sum.
__device__ __forceinline__ float4 add4(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}
__device__ __forceinline__ float4 slab_sum_wave(const float *src, int nsplit, int64_t stride, int w) {
  constexpr int B = 8;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = w; s0 < nsplit; s0 += 4 * B) {
    float4 a[B];
#pragma unroll
    for (int j = 0; j < B; ++j)
      a[j] = *(const float4 *)(src + (int64_t)min(s0 + 4 * j, nsplit - 1) * stride);
#pragma unroll
    for (int j = 0; j < B; ++j)
      if (s0 + 4 * j < nsplit) acc = add4(acc, a[j]);
  }
  return acc;
}

template <typename T, int EPI>
__global__ __launch_bounds__(256) void linear_reduce_kernel(LinParams p, RopeFreqs fr, int nsplit) {
  __shared__ float4 red[EPI == EPI_SILU ? 2 : 1][3][64];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gm = blockIdx.y;
  const int width = EPI == EPI_SILU ? p.n / 2 : p.n;  // output columns
  const int gn = blockIdx.x * 256 + lane * 4;
  const int gc = min(gn, width - 4);  // clamped: loads stay in the row
  const int64_t mn = (int64_t)p.m * p.n;
  const float *src = p.part + (int64_t)gm * p.n + gc;
  float4 a = slab_sum_wave(src, nsplit, mn, w);
  float4 b = make_float4(0.f, 0.f, 0.f, 0.f);
  if (EPI == EPI_SILU) b = slab_sum_wave(src + width, nsplit, mn, w);
  if (w > 0) {
    red[0][w - 1][lane] = a;
    if constexpr (EPI == EPI_SILU) red[1][w - 1][lane] = b;
  }
  __syncthreads();
  if (w > 0 || gn >= width) return;
  a = add4(add4(add4(a, red[0][0][lane]), red[0][1][lane]), red[0][2][lane]);
  float v[4] = {a.x, a.y, a.z, a.w};
  if constexpr (EPI == EPI_SILU) {
    b = add4(add4(add4(b, red[1][0][lane]), red[1][1][lane]), red[1][2][lane]);
    const float u[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = swiglu_silu(v[j]) * u[j];  // as silu_mul_rows_kernel
  } else {
    rope4(v, gm, gn, p, fr);
    if (p.k_dst) {  // K | V columns appended to the caches (fp32)
      const int c = gn - p.app_col;
      if (c >= 0 && c < 2 * p.app_w) {
        float *dst = (c < p.app_w ? p.k_dst + c : p.v_dst + (c - p.app_w)) + gm * p.app_rs;
        *(float4 *)dst = make_float4(v[0], v[1], v[2], v[3]);
      }
    }
  }
  store4<T>((T *)p.y + gm * p.y_rs + gn, v);
}

// Few rows (decode steps): streaming w once is the whole cost, so the
// matrix cores would idle on 31 of 32 rows.  One workgroup per (column strip,
// k slab): each lane owns 16 bytes of columns, the 4 waves take interleaved k
// rows of the slab (8 loads of w in flight per lane), x of the slab is staged
// in LDS and read as a broadcast, and the waves' sums meet in LDS.  The slab
// sums go to the partials (fp32 [nsplit][m][n]) for linear_reduce_kernel.
constexpr int SMALL_M = 8;
constexpr int SK_MAX = 256;  // k rows per slab, at most

template <typename T, int MR>
__global__ __launch_bounds__(256) void linear_small_kernel(LinParams p) {
  constexpr int VE = 16 / (int)sizeof(T);
  constexpr int COLS = 64 * VE;  // columns per workgroup
  __shared__ float xs[MR][SK_MAX];
  __shared__ float red[3][MR][COLS];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gn = blockIdx.x * COLS + lane * VE;
  const int kb = blockIdx.y * p.kchunk, ke = min(kb + p.kchunk, p.k);
  const int nk = ke - kb;
  const T *X = (const T *)p.x, *W = (const T *)p.w;
  for (int i = tid; i < MR * nk; i += 256) {
    const int r = i / nk, kk = i % nk;
    xs[r][kk] = r < p.m ? Elem<T>::load(X + r * p.x_rs + kb + kk) : 0.f;
  }
  __syncthreads();
  float acc[MR][VE];
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int e = 0; e < VE; ++e) acc[r][e] = 0.f;
  const bool col_ok = gn < p.n;
  constexpr int U = 8;  // loads in flight per lane
  for (int k0 = wave; k0 < nk; k0 += 4 * U) {
    u32x4_t wv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = k0 + 4 * u;
      // w is read once per call: non-temporal, kept out of L2/MALL
      wv[u] = (col_ok && kk < nk) ? __builtin_nontemporal_load((const u32x4_t *)(W + (kb + kk) * p.w_rs + gn))
                                  : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = min(k0 + 4 * u, nk - 1);  // a zero w chunk past the slab adds nothing
      float wf[VE];
      if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int e = 0; e < 4; ++e) wf[e] = __uint_as_float(wv[u][e]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          wf[2 * e] = __uint_as_float(wv[u][e] << 16);
          wf[2 * e + 1] = __uint_as_float(wv[u][e] & 0xffff0000u);
        }
      }
#pragma unroll
      for (int r = 0; r < MR; ++r) {
        const float xv = xs[r][kk];
#pragma unroll
        for (int e = 0; e < VE; ++e) acc[r][e] = fmaf(xv, wf[e], acc[r][e]);
      }
    }
  }
  if (wave > 0) {
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
      for (int e = 0; e < VE; ++e) red[wave - 1][r][lane * VE + e] = acc[r][e];
  }
  __syncthreads();
  if (wave > 0 || !col_ok) return;
#pragma unroll
  for (int r = 0; r < MR; ++r) {
    if (r >= p.m) break;
    float v[VE];
#pragma unroll
    for (int e = 0; e < VE; ++e)
      v[e] = ((acc[r][e] + red[0][r][lane * VE + e]) + red[1][r][lane * VE + e]) + red[2][r][lane * VE + e];
    float *dst = p.part + ((int64_t)blockIdx.y * p.m + r) * p.n + gn;
#pragma unroll
    for (int e = 0; e < VE; e += 4) *(float4 *)(dst + e) = make_float4(v[e], v[e + 1], v[e + 2], v[e + 3]);
  }
}

// Few rows against an output-major weight: w viewed [k, n] with stride_h 1,
// so the k weights of each output are contiguous (a row of the [n, k]
// matrix the view transposes).  Every output then streams as one contiguous
// row and needs no k split, no partials and no second launch.  A wave owns
// two outputs -- a rotation pair (2p, 2p+1), or for EPI_SILU the gate column
// j and the up column j + n/2 -- and reads their weight rows 16 bytes per
// lane through buffer descriptors whose range ends at k (loads past it
// return zeros and move no data), GV_ROUND loads per row and lane per round.
// The first round is requested before x is staged (the two round trips
// overlap).  Each lane sums its k positions in increasing order, a
// wave sum gives the dot product, and the wave applies the epilogue (the
// rotation and the K/V cache append, or silu(gate) * up) and stores.  x is
// staged in LDS once per workgroup as fp32.
constexpr int GV_M = 4;        // rows of x, at most
constexpr int GV_ROUND = 8;    // 16-byte loads per weight row and lane in a round
constexpr int GV_XMAX = kGemvStagedMax; // fp32 elements of x in LDS: staged rows x padded k (64 KB)

// NRM: x = rmsnorm(h + d) * w formed in the staging (one fp32 row of at
// most kNormRowF32 elements: two 16-byte chunks per thread).  MRG: x = the
// merged attention output of a split short-cache decode (one fp32 row).
template <typename T, int MR, int EPI, bool NRM = false, bool MRG = false>
__global__ __launch_bounds__(256) void linear_gemv_t_kernel(LinParams p, RopeFreqs fr) {
  // [MR][kp], zeros past k; NRM: then h + d [kp]
  extern __shared__ __attribute__((aligned(16))) float gxs[];
  constexpr int VE = 16 / (int)sizeof(T);  // k per 16-byte load
  constexpr int SPAN = 64 * VE;            // k per wave-wide load
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kp = (p.k + SPAN - 1) / SPAN * SPAN;
  const int nl = kp / SPAN;  // wave-wide loads per weight row

  // this wave's outputs and weight rows (clamped: a wave past the last
  // output loads a valid row and exits after the staging barrier)
  const int width = EPI == EPI_SILU ? p.n / 2 : p.n;  // output columns
  const int j0 = EPI == EPI_SILU ? blockIdx.x * 4 + wave : (blockIdx.x * 4 + wave) * 2;
  const bool active = j0 < width;  // wave-uniform
  const int jc = active ? j0 : 0;
  const int r0 = jc, r1 = EPI == EPI_SILU ? jc + width : jc + 1;
  // w_rs: elements between consecutive outputs' rows
  auto rsrc = [&](int row) __attribute__((always_inline)) {
    const uint64_t a = (uint64_t)((const T *)p.w + (int64_t)row * p.w_rs);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    return __builtin_amdgcn_make_buffer_rsrc((void *)(((uint64_t)hi << 32) | lo), (short)0,
                                             p.k * (int)sizeof(T), 0x00020000);
  };
  const __amdgpu_buffer_rsrc_t ra = rsrc(r0), rb = rsrc(r1);
  auto issue = [&](u32x4_t (&a)[GV_ROUND], u32x4_t (&b)[GV_ROUND], int l0) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < GV_ROUND; ++u) {
      const int off = ((l0 + u) * SPAN + lane * VE) * (int)sizeof(T);  // past k: zeros
      // each weight byte is read once per call: non-temporal
      a[u] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 2));
      b[u] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 2));
    }
  };
  float acc[2][MR];
#pragma unroll
  for (int r = 0; r < MR; ++r) acc[0][r] = acc[1][r] = 0.f;
  auto consume = [&](const u32x4_t (&a)[GV_ROUND], const u32x4_t (&b)[GV_ROUND], int l0)
      __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < GV_ROUND; ++u) {
      // slots past the padded row carry no weights: skipped (wave-uniform),
      // so an Inf in x meets no zero weight (fma(0, Inf) would be NaN)
      if (l0 + u >= nl) break;
      const int xo = (l0 + u) * SPAN + lane * VE;
      float wa[VE], wb[VE];
      if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int e = 0; e < 4; ++e) { wa[e] = __uint_as_float(a[u][e]); wb[e] = __uint_as_float(b[u][e]); }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          wa[2 * e] = __uint_as_float(a[u][e] << 16);
          wa[2 * e + 1] = __uint_as_float(a[u][e] & 0xffff0000u);
          wb[2 * e] = __uint_as_float(b[u][e] << 16);
          wb[2 * e + 1] = __uint_as_float(b[u][e] & 0xffff0000u);
        }
      }
#pragma unroll
      for (int r = 0; r < MR; ++r) {
        const float *xr = gxs + r * kp + xo;
#pragma unroll
        for (int e = 0; e < VE; e += 4) {
          const float4 x4 = *(const float4 *)(xr + e);
          acc[0][r] = fmaf(wa[e], x4.x, acc[0][r]);
          acc[0][r] = fmaf(wa[e + 1], x4.y, acc[0][r]);
          acc[0][r] = fmaf(wa[e + 2], x4.z, acc[0][r]);
          acc[0][r] = fmaf(wa[e + 3], x4.w, acc[0][r]);
          acc[1][r] = fmaf(wb[e], x4.x, acc[1][r]);
          acc[1][r] = fmaf(wb[e + 1], x4.y, acc[1][r]);
          acc[1][r] = fmaf(wb[e + 2], x4.z, acc[1][r]);
          acc[1][r] = fmaf(wb[e + 3], x4.w, acc[1][r]);
        }
      }
    }
  };

  u32x4_t a0[GV_ROUND], b0[GV_ROUND];
  if constexpr (NRM) {
    // x = rmsnorm(h + d) * nw (one fp32 row, k <= kNormRowF32: one pass), each
    // element formed as add_rmsnorm_rows_kernel (d given) or
    // rmsnorm_rows_kernel form it: h + d, the sum of squares in their order
    // (lane l of one wave over chunks l, l + 64, ... in turn as one fma
    // chain, then the wave sum), 1 / sqrtf(ss / k + eps), (v * inv) * w.
    // Every wave of every workgroup forms the same sum from h + d staged in
    // LDS; workgroup 0 also stores h + d to nh_out (the next residual).  The
    // h, d and norm-weight loads go out before the first weight round, so
    // they return first (in order) and the norm is formed while the weights
    // are on their way; no loop or branch sits between them and their use.
    static_assert(MR == 1 && sizeof(T) == 4, "the normalised input is one fp32 row");
    constexpr int XB = kNormRowF32 / 1024;  // 16-byte chunks per thread
    constexpr int CPL = kNormRowF32 / 256;  // 16-byte chunks per lane of one wave
    const float *H = (const float *)p.x;
    const float *D = p.nd ? p.nd : H;  // no d: a second read of h, not used
    const int cpr = kp / 4, nch = p.k / 4;
    float *raw = gxs + kp;
    u32x4_t hr[XB], dr[XB], wr[XB];
#pragma unroll
    for (int u = 0; u < XB; ++u) {
      const int kk = min((u * 256 + tid) * 4, p.k - 4);
      hr[u] = *(const u32x4_t *)(H + kk);
      dr[u] = *(const u32x4_t *)(D + kk);
      wr[u] = *(const u32x4_t *)(p.nw + kk);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep them ahead of the weight loads
    issue(a0, b0, 0);
    float v[XB][4];
#pragma unroll
    for (int u = 0; u < XB; ++u) {
      const int c = u * 256 + tid, kk = c * 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float h = __uint_as_float(hr[u][e]);
        v[u][e] = p.nd ? h + __uint_as_float(dr[u][e]) : h;
      }
      if (c < cpr) {
        const bool ok = kk < p.k;
        const float4 hv = ok ? make_float4(v[u][0], v[u][1], v[u][2], v[u][3]) : make_float4(0.f, 0.f, 0.f, 0.f);
        *(float4 *)(raw + kk) = hv;
        if (ok && p.nh_out && blockIdx.x == 0) *(float4 *)(p.nh_out + kk) = hv;
      }
    }
    __syncthreads();
    // chunks past the row add exact zeros (fma(0, 0, ss) = ss)
    float4 h4[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) h4[i] = *(const float4 *)(raw + min(lane + 64 * i, nch - 1) * 4);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const bool in = lane + 64 * i < nch;
      const float4 z = in ? h4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
      ss = fmaf(z.x, z.x, ss);
      ss = fmaf(z.y, z.y, ss);
      ss = fmaf(z.z, z.z, ss);
      ss = fmaf(z.w, z.w, ss);
    }
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)p.k + p.neps);  // op_rmsnorm.cuh:44-45
#pragma unroll
    for (int u = 0; u < XB; ++u) {
      const int c = u * 256 + tid, kk = c * 4;
      if (c < cpr) {
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = kk < p.k ? (v[u][e] * inv) * __uint_as_float(wr[u][e]) : 0.f;
        *(float4 *)(gxs + kk) = make_float4(o[0], o[1], o[2], o[3]);
      }
    }
  } else if constexpr (MRG) {
    // x[4c .. 4c+3] (query head 4c / 64, d = 4c mod 64) merged from the
    // head's partial records exactly as decode_combine_kernel merges them
    // (DecMerge), after the first weight round is requested.  The records'
    // (m, l) pairs are gathered into LDS once per workgroup (every chunk of
    // a head needs them); each thread requests its chunks' acc slices, two
    // chunks per pass, before any merge.
    static_assert(MR == 1 && sizeof(T) == 4, "the merged input is one fp32 row");
    issue(a0, b0, 0);
    const int cpr = kp / 4, nch = p.k / 4, S = p.msplit, nrec = (p.k >> 6) * S;
    float *gml = gxs + kp;  // (m, l) of record r at gml[2r]
    DecMerge mg[2];
    auto acc_of = [&](int c0) __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int kk = min(c0 + u * 256 + tid, nch - 1) * 4;  // in range: the merge is discarded
        mg[u].load_acc8(p.mpart + (int64_t)(kk >> 6) * S * kDecRec, S, 0, kk & 63);
      }
    };
    acc_of(0);
    for (int r = tid; r < nrec; r += 256)
      *(float2 *)(gml + 2 * r) = *(const float2 *)(p.mpart + (int64_t)r * kDecRec);
    int len = p.mlen >= 0 ? p.mlen : p.mlens[0];
    len = len < 0 ? 0 : (len > p.mmax_len ? p.mmax_len : len);
    const int chunk = short_split_chunk(len, S);
    const int nvalid = (len + chunk - 1) / chunk;
    __syncthreads();
    for (int c0 = 0; c0 < cpr; c0 += 512) {
      if (c0 > 0) acc_of(c0);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int c = c0 + u * 256 + tid;
        const int kk = min(c, nch - 1) * 4;
        const float *ml = gml + 2 * (kk >> 6) * S;
        mg[u].load_ml8(ml, S, 0);
        mg[u].start();
        mg[u].merge8(0, nvalid);
        for (int s0 = 8; s0 < nvalid; s0 += 8) {
          mg[u].load_acc8(p.mpart + (int64_t)(kk >> 6) * S * kDecRec, S, s0, kk & 63);
          mg[u].load_ml8(ml, S, s0);
          mg[u].merge8(s0, nvalid);
        }
        if (c < cpr) *(float4 *)(gxs + c * 4) = c < nch ? mg[u].result() : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  } else {
    issue(a0, b0, 0);
    // x rows in 16-byte chunks: thread tid takes chunks tid + 256u of every
    // row, XB per row requested before any is stored (clamped addresses,
    // zeros selected afterwards: no branch around a load).  One pass covers
    // 256*XB chunks per row; longer rows loop.
    constexpr int XB = 8 / MR;
    const T *X = (const T *)p.x;
    const int cpr = kp / VE;  // chunks per row
    auto stage = [&](int cb) __attribute__((always_inline)) {
      u32x4_t v[MR][XB];
#pragma unroll
      for (int r = 0; r < MR; ++r)
#pragma unroll
        for (int u = 0; u < XB; ++u) {
          const int kk = min((cb + u * 256 + tid) * VE, p.k - VE);
          v[r][u] = *(const u32x4_t *)(X + min(r, p.m - 1) * p.x_rs + kk);
        }
#pragma unroll
      for (int r = 0; r < MR; ++r)
#pragma unroll
        for (int u = 0; u < XB; ++u) {
          const int c = cb + u * 256 + tid, kk = c * VE;
          if (c < cpr) {
            const bool ok = r < p.m && kk < p.k;
            float *d = gxs + r * kp + kk;
            if constexpr (sizeof(T) == 4) {
              *(float4 *)d = ok ? make_float4(__uint_as_float(v[r][u][0]), __uint_as_float(v[r][u][1]),
                                              __uint_as_float(v[r][u][2]), __uint_as_float(v[r][u][3]))
                                : make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                d[2 * e] = ok ? __uint_as_float(v[r][u][e] << 16) : 0.f;
                d[2 * e + 1] = ok ? __uint_as_float(v[r][u][e] & 0xffff0000u) : 0.f;
              }
            }
          }
        }
    };
    stage(0);
    for (int cb = 256 * XB; cb < cpr; cb += 256 * XB) stage(cb);
  }
  __syncthreads();
  if (!active) return;  // a whole wave; no barrier follows
  // longer rows: one round after the other (keeping the next round in flight
  // while one is consumed measured slower on config 4's down projection)
  for (int l0 = 0; l0 < nl; l0 += GV_ROUND) {
    if (l0 > 0) issue(a0, b0, l0);
    __builtin_amdgcn_sched_barrier(0);
    consume(a0, b0, l0);
  }
#pragma unroll
  for (int r = 0; r < MR; ++r) {
    acc[0][r] = wave_sum(acc[0][r]);
    acc[1][r] = wave_sum(acc[1][r]);
  }
  // lane r stores row r's outputs
  float v0 = acc[0][0], v1 = acc[1][0];
#pragma unroll
  for (int r = 1; r < MR; ++r)
    if (lane == r) { v0 = acc[0][r]; v1 = acc[1][r]; }
  if (lane >= p.m) return;
  const int gm = lane;
  T *yrow = (T *)p.y + gm * p.y_rs;
  if constexpr (EPI == EPI_SILU) {
    Elem<T>::store(yrow + j0, swiglu_silu(v0) * v1);  // as silu_mul_rows_kernel
  } else {
    if (j0 < p.rope_cols) {  // op_rope.cuh:79-98: fp32 angle position*freq
      const float ang = (float)(p.pos0 + gm) * fr.f[(j0 % p.head_dim) >> 1];
      float sn, cs;
      sincosf(ang, &sn, &cs);
      const float x0 = v0, x1 = v1;
      v0 = x0 * cs - x1 * sn;
      v1 = x0 * sn + x1 * cs;
    }
    if (p.k_dst) {  // K | V columns appended to the caches (fp32)
      const int c = j0 - p.app_col;
      if (c >= 0 && c < 2 * p.app_w) {
        float *dst = (c < p.app_w ? p.k_dst + c : p.v_dst + (c - p.app_w)) + gm * p.app_rs;
        dst[0] = v0;
        dst[1] = v1;
      }
    }
    Elem<T>::store(yrow + j0, v0);
    Elem<T>::store(yrow + j0 + 1, v1);
  }
}

// slabs of the few-rows path: about kSmallWg workgroups, slabs of
// 32..SK_MAX rows in multiples of 32
constexpr int kSmallWg = 512;
void plan_small(int dtype, int n, int k, int *nsplit, int *kchunk) {
  const int cols = 64 * (dtype == BN_BF16 ? 8 : 4);
  const int strips = (n + cols - 1) / cols;
  const int want = std::max(1, kSmallWg / strips);
  int kc = (k + want - 1) / want;
  kc = std::min(std::max((kc + 31) / 32 * 32, 32), SK_MAX);
  *kchunk = kc;
  *nsplit = k > 0 ? (k + kc - 1) / kc : 1;
}

// k slabs: as many as still fit the grid in one round of resident
// workgroups (kLinSlots: 4 per compute unit of an MI355X -- 36 KB of LDS
// each), each slab at least two stages deep.  A fixed device size keeps the
// plan, and so the workspace size, independent of the device queried.
constexpr int64_t kLinSlots = 1024;
void plan_split(int dtype, int m, int n, int k, int *nsplit, int *kchunk) {
  const int KT = dtype == BN_BF16 ? LinCfg<bf16_t>::KT : LinCfg<float>::KT;
  const int64_t tiles = (int64_t)((n + TN - 1) / TN) * ((m + TM - 1) / TM);
  const int stages = (k + KT - 1) / KT;
  int ns = (int)std::min<int64_t>(kLinSlots / tiles, std::max(1, stages / 2));
  ns = std::max(ns, 1);
  const int per = (stages + ns - 1) / ns;
  *kchunk = std::max(per, 1) * KT;
  *nsplit = k > 0 ? (k + *kchunk - 1) / *kchunk : 1;
}

// ------------------------------------------------ output-major, many rows
// y[m][n] = sum_k x[m][k] w[n][k] with w output-major (each output's k
// weights contiguous) and more rows than the few-rows kernel stages (m > 4;
// fp32) on v_mfma_f32_32x32x2f32: one workgroup per 32 rows x 128 outputs,
// wave w on the 32 outputs n0 + 32w ..; k in stages of 32 staged through
// LDS (x: 32 rows, w: 128 rows of 128 bytes each, every thread one 16-byte
// chunk of x and four of w per stage, whole cache lines per row), two stage
// buffers (one barrier per stage), the next stage's loads in flight while
// this one is multiplied.  Lane (r, hf) reads 16 bytes of its x row and of
// its w row at k offset 8u + 4hf: the operands of four MFMAs (contraction
// pairs {8u + e, 8u + 4 + e}).  The epilogue rotates the pairs (2p, 2p+1) of
// the first rope_cols columns (op_rope.cuh:79-98, fp32 angle (pos0 + m) *
// freq) with the neighbouring lane's value, and stores.  Workgroups that
// read the same weight rows go to one XCD.
constexpr int NT_BM = 32, NT_BN = 128, NT_KS = 32, NT_P = NT_KS + 4;  // LDS row pitch (floats)
typedef float f32x16_nt __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256) void linear_nt_kernel(LinParams p, RopeFreqs fr) {
  __shared__ __attribute__((aligned(16))) float xs[2][NT_BM * NT_P];
  __shared__ __attribute__((aligned(16))) float ws[2][NT_BN * NT_P];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, r32 = lane & 31, hf = lane >> 5;
  const int n_rt = (p.m + NT_BM - 1) / NT_BM;
  // workgroups are dealt to the 8 XCDs in turn: logical unit u's XCD is
  // u / (grid / 8), so consecutive units -- the row tiles of one column
  // tile -- share an L2
  int u = blockIdx.x;
  if ((gridDim.x & 7) == 0) u = (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
  const int rt = u % n_rt, ct = u / n_rt;
  const int m0 = rt * NT_BM, n0 = ct * NT_BN;
  const int nst = (p.k + NT_KS - 1) / NT_KS;
  // staging: thread tid holds chunk c = tid of x (row c / 8, k 4*(c % 8))
  // and chunks tid + 256j of w; rows past m / n read a valid row (their
  // outputs are not stored), k past p.k reads zeros
  const int cr = tid >> 3, ck = 4 * (tid & 7);
  const float *xg = (const float *)p.x + (int64_t)min(m0 + cr, p.m - 1) * p.x_rs + ck;
  const float *wg[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) wg[j] = (const float *)p.w + (int64_t)min(n0 + cr + 32 * j, p.n - 1) * p.w_rs + ck;
  float4 xr, wr[4];
  auto gload = [&](int st) __attribute__((always_inline)) {
    const int k0 = st * NT_KS;
    const bool ok = k0 + ck < p.k;  // k is a multiple of 4: a chunk is all in or all out
    xr = ok ? *(const float4 *)(xg + k0) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < 4; ++j) wr[j] = ok ? *(const float4 *)(wg[j] + k0) : make_float4(0.f, 0.f, 0.f, 0.f);
  };
  auto lstore = [&](int b) __attribute__((always_inline)) {
    *(float4 *)(&xs[b][cr * NT_P + ck]) = xr;
#pragma unroll
    for (int j = 0; j < 4; ++j) *(float4 *)(&ws[b][(cr + 32 * j) * NT_P + ck]) = wr[j];
  };
  f32x16_nt acc = f32x16_nt{};
  gload(0);
  lstore(0);
  __syncthreads();
  for (int st = 0; st < nst; ++st) {
    const int b = st & 1;
    if (st + 1 < nst) gload(st + 1);
    const float *xa = &xs[b][r32 * NT_P + 4 * hf];
    const float *wa = &ws[b][(32 * w + r32) * NT_P + 4 * hf];
#pragma unroll
    for (int uu = 0; uu < NT_KS / 8; ++uu) {
      const float4 a = *(const float4 *)(xa + 8 * uu);
      const float4 bb = *(const float4 *)(wa + 8 * uu);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, bb.x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, bb.y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, bb.z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, bb.w, acc, 0, 0, 0);
    }
    if (st + 1 < nst) lstore(b ^ 1);  // buffer b ^ 1 was last read in stage st - 1
    __syncthreads();
  }

  // register i of acc is row m0 + 8(i/4) + 4hf + i%4 of column n0 + 32w + r32;
  // a rotation pair is the even column's lane and the next one.  The tile's
  // angles (pos0 + m) * freq take one sincosf each, shared through LDS (the
  // staging buffers are free after the last barrier): row r, frequency
  // index q of the tile's columns (q < 64 covers head_dim <= 128 and any
  // 128 columns: (n % head_dim) / 2 for n in [n0, n0 + 128))
  const int gn = n0 + 32 * w + r32;
  const bool even = (r32 & 1) == 0;
  const bool rot = (gn & ~1) < p.rope_cols;
  static_assert(NT_BM * 64 * 2 <= NT_BN * NT_P, "the angle table fits one w staging buffer");
  float2 *sc = reinterpret_cast<float2 *>(&ws[0][0]);  // [NT_BM][64] (sin, cos)
  const bool table = n0 < p.rope_cols && p.head_dim <= 128;  // uniform
  if (table) {
    const int nq = min(p.head_dim / 2, 64);
    for (int e = tid; e < NT_BM * 64; e += 256) {
      const int r = e >> 6, q = e & 63;
      float sn = 0.f, cs = 1.f;
      if (q < nq) sincosf((float)(p.pos0 + m0 + r) * fr.f[q], &sn, &cs);
      sc[e] = make_float2(sn, cs);
    }
    __syncthreads();
  }
  const int q = rot ? ((gn & ~1) % p.head_dim) >> 1 : 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = 8 * (i >> 2) + 4 * hf + (i & 3), gm = m0 + row;
    float v = acc[i];
    const float o = __shfl_xor(v, 1, 64);  // the pair's other column
    if (rot) {  // op_rope.cuh:79-98: fp32 angle position * freq
      float2 t;
      if (table) {
        t = sc[row * 64 + q];
      } else {  // head_dim above 128: the angle of this element
        sincosf((float)(p.pos0 + gm) * fr.f[q], &t.x, &t.y);
      }
      const float x0 = even ? v : o, x1 = even ? o : v;
      v = even ? x0 * t.y - x1 * t.x : x0 * t.x + x1 * t.y;
    }
    if (gm < p.m && gn < p.n) ((float *)p.y)[(int64_t)gm * p.y_rs + gn] = v;
  }
}

}  // namespace
}  // namespace bn

using namespace bn;

// the few-rows path always goes through the partials (its reduction applies
// the rotation); the tiled path only when it splits k
static void plan(int dtype, int m, int n, int k, bool *small, int *nsplit, int *kchunk) {
  *small = m <= SMALL_M && k > 0;
  if (*small)
    plan_small(dtype, n, k, nsplit, kchunk);
  else
    plan_split(dtype, m, n, k, nsplit, kchunk);
}

extern "C" size_t bn_linear_rope_workspace_size(int dtype, int m, int n, int k) {
  if ((dtype != BN_F32 && dtype != BN_BF16) || m <= 0 || n <= 0 || k <= 0) return 0;
  int ns, kc;
  bool small;
  plan(dtype, m, n, k, &small, &ns, &kc);
  return (small || ns > 1) ? (size_t)ns * m * n * sizeof(float) : 0;
}

namespace bn {

namespace {
// output-major w with more than four rows (linear_nt_kernel; fp32, plain
// epilogue): x and w rows 16-byte aligned and k a multiple of 4 (checked by
// the caller's layout test)
int nt_run(const bn_view *x, const bn_view *w, const bn_view *y, int rope_cols, int position_offset,
           int head_dim, const RopeFreqs &fr, const char *op, void *stream) {
  int st;
  if ((st = require_device(op, {x, w, y}))) return st;
  if (y->h == 0 || y->w == 0) return BN_OK;
  if ((st = ensure_device())) return st;
  LinParams p = {};
  p.x = (const float *)x->data + x->offset;
  p.w = (const float *)w->data + w->offset;
  p.y = (float *)y->data + y->offset;
  p.x_rs = x->stride_h; p.w_rs = w->stride_w; p.y_rs = y->stride_h;
  p.m = x->h; p.n = w->w; p.k = x->w;
  p.rope_cols = rope_cols; p.head_dim = rope_cols ? head_dim : 2; p.pos0 = position_offset;
  const int64_t tiles = (int64_t)((p.m + NT_BM - 1) / NT_BM) * ((p.n + NT_BN - 1) / NT_BN);
  if (tiles > 0x7fffffff) return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": too many output tiles");
  hipLaunchKernelGGL(linear_nt_kernel, dim3((unsigned)tiles), dim3(256), 0, as_stream(stream), p, fr);
  BN_LAUNCH_CHECK();
  return BN_OK;
}

// output-major w (linear_gemv_t_kernel): shapes and the rotation table are
// checked by linear_run; this checks the layout the kernel reads
int gemv_t_run(const bn_view *x, const bn_view *w, const bn_view *y, int rope_cols,
               int position_offset, int head_dim, const RopeFreqs &fr, int epi, float *k_dst,
               float *v_dst, int app_col, int app_w, int64_t app_rs, const LinNorm *nrm,
               const LinMerge *mrg, const char *op, void *stream) {
  const int dt = x->dtype;
  const int64_t ve = dt == BN_BF16 ? 8 : 4;  // elements per 16 bytes
  const size_t es = dtype_size(dt);
  const int m = x->h, n = w->w, k = x->w;
  const int64_t kp = (k + 64 * ve - 1) / (64 * ve) * (64 * ve);
  auto base_ok = [&](const bn_view *v) {
    return ((reinterpret_cast<uintptr_t>(v->data) + (uintptr_t)(v->offset * (int64_t)es)) & 15u) == 0;
  };
  auto rows_ok = [&](const bn_view *v) {
    return (int64_t)v->h * v->w == 0 || (v->stride_w == 1 && v->stride_h % ve == 0 && base_ok(v));
  };
  // x is staged and w streamed 16 bytes at a time; y is stored one element
  // at a time (any row stride)
  const bool y_ok = (int64_t)y->h * y->w == 0 || y->stride_w == 1;
  if (!rows_ok(x) || !y_ok || !base_ok(w) || w->stride_w % ve || k % ve || y->w % 2)
    return fail(BN_ERR_UNSUPPORTED,
                std::string(op) + ": an output-major w needs 16-byte aligned rows of x and w, k a "
                                  "multiple of 16 bytes, contiguous rows of y and an even output width");
  if (m > GV_M && !nrm && !mrg && !k_dst && epi == EPI_PLAIN && dt == BN_F32)
    return nt_run(x, w, y, rope_cols, position_offset, head_dim, fr, op, stream);
  // the kernel stages mr rows (3 rows run the 4-row instance)
  const int mr = m <= 1 ? 1 : (m <= 2 ? 2 : 4);
  if (m > GV_M || (int64_t)mr * kp > GV_XMAX)
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": an output-major w takes at most " +
                                        std::to_string(GV_M) + " rows of x and " +
                                        std::to_string(GV_XMAX) + " staged x elements");
  if (k_dst && (dt != BN_F32 || app_col < 0 || app_col % 4 || app_w % 4 || app_col + 2 * app_w > n))
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": bad K/V append columns");
  const char *hx = (const char *)x->data + x->offset * (int64_t)es;
  if (mrg) {  // one fp32 row: n_heads * 64 merged attention outputs
    if (nrm || dt != BN_F32 || m != 1 || k % 64 || !mrg->part || (!mrg->lens && mrg->len < 0) ||
        mrg->n_split <= 0 || mrg->max_len <= 0 || kp + (int64_t)(k / 64) * mrg->n_split * 2 > GV_XMAX)
      return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": a merged input is one fp32 row of whole heads");
  }
  if (nrm) {  // one fp32 row of h, staged in one pass; h_out written while h and d are read
    if (dt != BN_F32 || m != 1 || k < 4 || k > kNormRowF32 || !nrm->w)
      return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": a normalised input is one fp32 row of 4.." +
                                          std::to_string(kNormRowF32) + " elements with its weight");
    if ((reinterpret_cast<uintptr_t>(nrm->d) | reinterpret_cast<uintptr_t>(nrm->w) |
         reinterpret_cast<uintptr_t>(nrm->h_out)) & 15u)
      return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": the norm's rows must be 16-byte aligned");
    auto overlaps = [&](const void *a, const void *b) {
      const char *pa = (const char *)a, *pb = (const char *)b;
      return a && b && pa < pb + (size_t)k * 4 && pb < pa + (size_t)k * 4;
    };
    if (overlaps(nrm->h_out, hx) || overlaps(nrm->h_out, nrm->d))
      return fail(BN_ERR_INVALID_ARG, std::string(op) + ": the norm's h_out must not overlap h or d");
  }
  int st;
  if ((st = require_device(op, {x, w, y}))) return st;
  if (y->h == 0 || y->w == 0) return BN_OK;
  if ((st = ensure_device())) return st;
  LinParams p = {};
  p.x = (const char *)x->data + x->offset * (int64_t)es;
  p.w = (const char *)w->data + w->offset * (int64_t)es;
  p.y = (char *)y->data + y->offset * (int64_t)es;
  p.x_rs = x->stride_h; p.w_rs = w->stride_w; p.y_rs = y->stride_h;
  p.m = m; p.n = n; p.k = k;
  p.rope_cols = rope_cols; p.head_dim = rope_cols ? head_dim : 2; p.pos0 = position_offset;
  p.k_dst = k_dst; p.v_dst = v_dst; p.app_col = app_col; p.app_w = app_w; p.app_rs = app_rs;
  if (nrm) {
    p.nd = nrm->d; p.nw = nrm->w; p.nh_out = nrm->h_out; p.neps = nrm->eps;
  }
  if (mrg) {
    p.mpart = mrg->part; p.mlens = mrg->lens; p.msplit = mrg->n_split; p.mmax_len = mrg->max_len;
    p.mlen = mrg->len;
  }
  // a merged input also holds every record's (m, l) pair
  const size_t lds = (size_t)(nrm ? 2 : mr) * kp * sizeof(float) +
                     (mrg ? (size_t)(k / 64) * mrg->n_split * 2 * sizeof(float) : 0);
  // four waves per workgroup, two weight rows (one output pair, or one
  // gate | up output) per wave
  const int waves = n / 2;
  const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
  hipStream_t s = as_stream(stream);
#define BN_GV(T, MR, E, ...) \
  hipLaunchKernelGGL((linear_gemv_t_kernel<T, MR, E, ##__VA_ARGS__>), grid, block, lds, s, p, fr)
#define BN_GV_M(T, E)                 \
  do {                                \
    if (mr == 1) BN_GV(T, 1, E);      \
    else if (mr == 2) BN_GV(T, 2, E); \
    else BN_GV(T, 4, E);              \
  } while (0)
  if (nrm) {
    if (epi == EPI_SILU) BN_GV(float, 1, EPI_SILU, true);
    else BN_GV(float, 1, EPI_PLAIN, true);
  } else if (mrg) {
    if (epi == EPI_SILU) BN_GV(float, 1, EPI_SILU, false, true);
    else BN_GV(float, 1, EPI_PLAIN, false, true);
  } else if (dt == BN_F32) {
    if (epi == EPI_SILU) BN_GV_M(float, EPI_SILU);
    else BN_GV_M(float, EPI_PLAIN);
  } else {
    if (epi == EPI_SILU) BN_GV_M(bf16_t, EPI_SILU);
    else BN_GV_M(bf16_t, EPI_PLAIN);
  }
#undef BN_GV_M
#undef BN_GV
  BN_LAUNCH_CHECK();
  return BN_OK;
}
}  // namespace

// bn_linear_rope with a reduction epilogue (EPI_SILU: y is [m, n/2]) and
// optional K/V appends (LinParams::k_dst); the epilogues exist on the
// split-k paths, which the few-rows projections always take, and on the
// output-major few-rows kernel.
int linear_run(const bn_view *x, const bn_view *w, const bn_view *y, int rope_cols,
               int position_offset, int head_dim, float theta, void *workspace,
               size_t workspace_bytes, int epi, float *k_dst, float *v_dst, int app_col, int app_w,
               int64_t app_rs, void *stream, const LinNorm *nrm, const LinMerge *mrg) {
  const char *op = epi == EPI_SILU ? "Linear+SwiGLU" : "Linear";
  const unsigned mask = (1u << BN_F32) | (1u << BN_BF16);
  int st;
  if ((st = check_view(x, op, "x", mask))) return st;
  if ((st = check_view(w, op, "w", mask))) return st;
  if ((st = check_view(y, op, "y", mask))) return st;
  if (x->dtype != w->dtype || x->dtype != y->dtype)
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": x, w and y must share one dtype");
  const int64_t y_cols = epi == EPI_SILU ? (int64_t)w->w / 2 : w->w;
  if (x->w != w->h || y->h != x->h || y->w != y_cols || (epi == EPI_SILU && w->w % 8))
    return fail(BN_ERR_SHAPE, std::string(op) + ": shape mismatch x:(" + std::to_string(x->h) +
                                  ", " + std::to_string(x->w) + "), w:(" + std::to_string(w->h) +
                                  ", " + std::to_string(w->w) + "), y:(" + std::to_string(y->h) +
                                  ", " + std::to_string(y->w) + ")");
  RopeFreqs fr{};
  if (rope_cols != 0) {
    if ((st = make_rope_freqs(op, head_dim, theta, &fr))) return st;
    if (rope_cols < 0 || rope_cols > y->w || rope_cols % head_dim != 0)
      return fail(BN_ERR_SHAPE, std::string(op) +
                                    ": rope_cols must be a multiple of head_dim within the output width");
  }
  const int dt = x->dtype;
  const int64_t ve = dt == BN_BF16 ? 8 : 4;  // elements per 16 bytes
  const size_t es = dtype_size(dt);
  // views with no elements (k = 0) are never read: their layout is free
  auto ok = [&](const bn_view *v) {
    if ((int64_t)v->h * v->w == 0) return true;
    return v->stride_w == 1 && v->stride_h % ve == 0 &&
           ((reinterpret_cast<uintptr_t>(v->data) + (uintptr_t)(v->offset * (int64_t)es)) & 15u) == 0;
  };
  auto unit = [](const bn_view *v) { return (int64_t)v->h * v->w == 0 || v->stride_w == 1; };
  // an output-major w (stride_h == 1: each output's k weights contiguous) takes
  // the few-rows streaming kernel without a k split
  if ((int64_t)w->h * w->w > 0 && w->stride_h == 1 && w->stride_w != 1)
    return gemv_t_run(x, w, y, rope_cols, position_offset, head_dim, fr, epi, k_dst, v_dst, app_col,
                      app_w, app_rs, nrm, mrg, op, stream);
  if (nrm || mrg)
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": a normalised or merged input needs an output-major w");
  if (!unit(x) || !unit(w) || !unit(y))
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": rows must be contiguous (stride_w == 1)");
  if (!ok(x) || !ok(w) || !ok(y) || x->w % ve || y->w % ve)
    return fail(BN_ERR_UNSUPPORTED, std::string(op) +
                                        ": rows must start 16-byte aligned and widths be multiples of 16 bytes");
  if ((st = require_device(op, {x, w, y}))) return st;
  if (y->h == 0 || y->w == 0) return BN_OK;
  const int m = y->h, n = w->w, k = x->w;
  int nsplit, kchunk;
  bool small;
  plan(dt, m, n, k, &small, &nsplit, &kchunk);
  if ((epi != EPI_PLAIN || k_dst) && !(small || nsplit > 1))
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": the fused epilogue needs the split-k path");
  if (k_dst && (dt != BN_F32 || app_col < 0 || app_col % 4 || app_w % 4 || app_col + 2 * app_w > n))
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": bad K/V append columns");
  const size_t need = (small || nsplit > 1) ? (size_t)nsplit * m * n * sizeof(float) : 0;
  if (workspace && workspace_bytes < need)
    return fail(BN_ERR_INVALID_ARG, std::string(op) + ": workspace of " +
                                        std::to_string(workspace_bytes) + " bytes, need " +
                                        std::to_string(need));
  if (workspace && (reinterpret_cast<uintptr_t>(workspace) & 15u))
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": workspace must be 16-byte aligned");
  // grid limits: row tiles on grid y (at most 65535), reduction threads
  if ((!small && (m + TM - 1) / TM > 65535) || ((small || nsplit > 1) && m > 65535))
    return fail(BN_ERR_UNSUPPORTED, std::string(op) + ": problem too large");
  if ((st = ensure_device())) return st;
  hipStream_t s = as_stream(stream);
  void *ws = workspace;
  bool own = false;
  if (need && !ws) {
    if ((st = bn_alloc(&ws, need, stream))) return st;
    own = true;
  }
  LinParams p;
  p.x = (const char *)x->data + x->offset * (int64_t)es;
  p.w = (const char *)w->data + w->offset * (int64_t)es;
  p.y = (char *)y->data + y->offset * (int64_t)es;
  p.part = need ? (float *)ws : nullptr;
  p.x_rs = x->stride_h; p.w_rs = w->stride_h; p.y_rs = y->stride_h;
  p.m = m; p.n = n; p.k = k; p.kchunk = kchunk;
  p.rope_cols = rope_cols; p.head_dim = rope_cols ? head_dim : 2; p.pos0 = position_offset;
  p.k_dst = k_dst; p.v_dst = v_dst; p.app_col = app_col; p.app_w = app_w; p.app_rs = app_rs;
  if (small) {
    const int cols = 64 * (dt == BN_BF16 ? 8 : 4);
    dim3 grid((unsigned)((n + cols - 1) / cols), (unsigned)nsplit);
#define BN_SMALL(T, MR) hipLaunchKernelGGL((linear_small_kernel<T, MR>), grid, dim3(256), 0, s, p)
    if (dt == BN_F32) {
      if (m <= 1) BN_SMALL(float, 1);
      else if (m <= 2) BN_SMALL(float, 2);
      else if (m <= 4) BN_SMALL(float, 4);
      else BN_SMALL(float, 8);
    } else {
      if (m <= 1) BN_SMALL(bf16_t, 1);
      else if (m <= 2) BN_SMALL(bf16_t, 2);
      else if (m <= 4) BN_SMALL(bf16_t, 4);
      else BN_SMALL(bf16_t, 8);
    }
#undef BN_SMALL
  } else {
    dim3 grid((unsigned)((n + TN - 1) / TN), (unsigned)((m + TM - 1) / TM), (unsigned)nsplit);
    if (dt == BN_F32)
      hipLaunchKernelGGL(linear_kernel<float>, grid, dim3(256), 0, s, p, fr);
    else
      hipLaunchKernelGGL(linear_kernel<bf16_t>, grid, dim3(256), 0, s, p, fr);
  }
  hipError_t e = hipGetLastError();
  if (e == hipSuccess && need) {
    const dim3 rg((unsigned)((y->w + 255) / 256), (unsigned)m);
    if (epi == EPI_SILU) {
      if (dt == BN_F32)
        hipLaunchKernelGGL((linear_reduce_kernel<float, EPI_SILU>), rg, dim3(256), 0, s, p, fr, nsplit);
      else
        hipLaunchKernelGGL((linear_reduce_kernel<bf16_t, EPI_SILU>), rg, dim3(256), 0, s, p, fr, nsplit);
    } else {
      if (dt == BN_F32)
        hipLaunchKernelGGL((linear_reduce_kernel<float, EPI_PLAIN>), rg, dim3(256), 0, s, p, fr, nsplit);
      else
        hipLaunchKernelGGL((linear_reduce_kernel<bf16_t, EPI_PLAIN>), rg, dim3(256), 0, s, p, fr, nsplit);
    }
    e = hipGetLastError();
  }
  st = e == hipSuccess ? BN_OK : hip_fail(e, __FILE__, __LINE__);
  if (own) {
    const int st2 = bn_free(ws, stream);
    if (st == BN_OK) st = st2;
  }
  return st;
}

}  // namespace bn

extern "C" int bn_linear_rope(const bn_view *x, const bn_view *w, const bn_view *y, int rope_cols,
                              int position_offset, int head_dim, float theta, void *workspace,
                              size_t workspace_bytes, void *stream) {
  return linear_run(x, w, y, rope_cols, position_offset, head_dim, theta, workspace, workspace_bytes,
                    EPI_PLAIN, nullptr, nullptr, 0, 0, 0, stream);
}
